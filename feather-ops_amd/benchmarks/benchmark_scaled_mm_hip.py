#!/usr/bin/env python3
"""Kernel benchmark and tile sweep of the fp16/bf16 x fp8 scaled matmul on the shape grid in cells.py.

Same role and options as the reference's `bench/benchmark_scaled_mm_hip.py` (whole grid or groups or
explicit cells, the heuristic against an explicit tile list, a square sweep): per cell it times
`torch_mm` (torch's matmul on the already-dequantized bf16 weight: the optimistic control, which does
not pay for dequantization), `auto` (the tile `select_scaled_mm_config` picks) and, with `--tiles`,
every listed tile, interleaved (see protocol.py). It prints TFLOP/s per provider, the best tile and how
far the heuristic's pick is from it, and with `--json` writes every measurement for refitting.

Run from `feather-ops_amd/`:

    python -m benchmarks.benchmark_scaled_mm_hip                        # whole grid, heuristic vs torch.mm
    python -m benchmarks.benchmark_scaled_mm_hip --groups baseline,h3
    python -m benchmarks.benchmark_scaled_mm_hip --tiles                # every instantiated tile as well
    python -m benchmarks.benchmark_scaled_mm_hip --tiles "2,2,4,4,8,1;8,1,4,1,4,0"
    python -m benchmarks.benchmark_scaled_mm_hip --cells "4096,12288,3072" --cold
    python -m benchmarks.benchmark_scaled_mm_hip --tiles --splits 2,3,4,6,8   # split-K candidates too
    python -m benchmarks.benchmark_scaled_mm_hip --groups text-16 --graph      # kernel time, no host gaps

`auto` is the whole heuristic (tile and split count, and for bf16 activations whether to widen them in a
pass of their own first). Where it widens first (on every cell with `--widen-all`), `widened` times that pass
plus the fp16-activation pick and `in_place` the bf16 pick widening them inside the kernel, and the summary
line gives the first's speedup over the second. With `--splits`, every listed tile (ring or
streaming) whose grid has fewer tiles than the GPU has compute units is also timed split `S` ways (named
`(tile)/S`), for each `S` that keeps at most four workgroups per CU (`--split-any-grid`: whatever the
grid, under that same cap). Every provider calls its op directly
(split launches with one preallocated workspace per cell), so the Python layer's per-call cost is not
timed; `--graph` also takes the op dispatch out (replays of captured batches), which matters for kernels
of a few microseconds.
"""

import argparse
import json
import math
import pathlib
import sys

import torch

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1]))

from benchmarks.cells import GROUPS, cells  # noqa: E402
from benchmarks.protocol import measure, paired_speedup  # noqa: E402
from feather_ops.scaled_mm import (  # noqa: E402
    _auto_choice,
    prepack_b_for_scaled_mm,
    select_scaled_mm_config,
    select_scaled_mm_splits,
    set_weight_streaming,
)
from feather_ops.tiles import SCALED_MM_TILES, gemm_block_sizes, split_workspace_bytes  # noqa: E402

_CUS = 256


def _blocks(m: int, n: int, tile: tuple[int, ...]) -> int:
    bm, bn, _ = gemm_block_sizes(tile)
    return -(-m // bm) * -(-n // bn)

_DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
_FP8 = {"e5m2": torch.float8_e5m2, "e4m3fn": torch.float8_e4m3fn}


def parse_tiles(text: str) -> list[tuple[int, ...]]:
    if text == "":
        return list(SCALED_MM_TILES)
    tiles = []
    for chunk in text.split(";"):
        tile = tuple(int(v) for v in chunk.split(","))
        if len(tile) != 6:
            raise SystemExit(f"--tiles entry {chunk!r} should hold 6 comma-separated integers "
                             "(block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch)")
        if tile not in SCALED_MM_TILES:
            raise SystemExit(f"{tile} is not one of the compiled tiles (feather_ops.tiles.SCALED_MM_TILES)")
        tiles.append(tile)
    return tiles


def weight_copies(n: int, k: int, cold: bool, copies: int | None = None) -> int:
    """Copies of the prepacked weight to rotate over: `copies` if given, else enough to exceed the 256 MB MALL
    twice when cold and one otherwise."""
    if copies is not None:
        return copies
    if not cold:
        return 1
    k_pad = -(-k // 128) * 128
    return int(min(16, max(1, math.ceil(512e6 / (k_pad * n)))))


def run_cell(m: int, n: int, k: int, tiles, args) -> dict:
    a_dtype, out_dtype = _DT[args.a_dtype], _DT[args.out_dtype]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    a = torch.randn((m, k), generator=gen, device="cuda").to(a_dtype)
    fp8 = _FP8[args.fp8]
    b_kn = torch.randn((k, n), generator=gen, device="cuda").to(fp8)
    scale = torch.tensor(2.34, device="cuda", dtype=torch.float32)
    bias = torch.randn(n, generator=gen, device="cuda").to(out_dtype) if args.bias else None
    copies = weight_copies(n, k, args.cold, args.copies)
    packed = prepack_b_for_scaled_mm(b_kn)
    packs = [packed] + [packed.clone() for _ in range(copies - 1)]
    control_w = (b_kn.t().float() * scale).to(torch.bfloat16).contiguous()
    control_a = a.to(torch.bfloat16)
    del b_kn
    out = torch.empty((m, n), device="cuda", dtype=out_dtype)
    op = torch.ops.feather_ops.scaled_mm.default

    picked = tuple(select_scaled_mm_config(m, n, k, a_dtype, fp8, out_dtype))
    picked_splits = select_scaled_mm_splits(m, n, k, picked, a_dtype)
    wide_tile, wide_splits, widen = _auto_choice(m, n, k, a_dtype)
    # bf16 activations: time the widening pass + fp16-activation pick against the in-place bf16 pick where the
    # heuristic widens first, or on every cell with --widen-all (the data its rule is fitted on)
    compare_widen = a_dtype == torch.bfloat16 and (widen or args.widen_all)
    if compare_widen and not widen:
        wide_tile = tuple(select_scaled_mm_config(m, n, k, torch.float16))
        wide_splits = select_scaled_mm_splits(m, n, k, wide_tile, torch.float16)
    split_cases = [(tile, splits) for tile in tiles for splits in args.splits
                   if (_blocks(m, n, tile) < _CUS or args.split_any_grid) and _blocks(m, n, tile) * splits <= 4 * _CUS
                   and split_workspace_bytes(m, n, k, tile, splits) > 0]
    if picked_splits > 1:
        split_cases.append((picked, picked_splits))
    # One zeroed workspace for every split launch of the cell (each leaves its counters at zero), passed
    # to the op directly, so that a launch allocates nothing and can be captured.
    ws_cases = split_cases + ([(wide_tile, wide_splits)] if compare_widen and wide_splits > 1 else [])
    ws_bytes = max([split_workspace_bytes(m, n, k, tile, splits) for tile, splits in ws_cases], default=0)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    split_op = torch.ops.feather_ops.scaled_mm_splitk.default

    def launcher(tile, splits):
        if splits == 1:
            return lambda i: op(a, packs[i % copies], scale, bias, out, *tile)
        return lambda i: split_op(a, packs[i % copies], scale, bias, out, ws, splits, *tile)

    providers = {"torch_mm": lambda i: torch.mm(control_a, control_w.t())}
    for tile in tiles:
        providers[str(tile)] = launcher(tile, 1)
    for tile, splits in split_cases:
        providers[f"{tile}/{splits}"] = launcher(tile, splits)
    auto_name = str(picked) if picked_splits == 1 else f"{picked}/{picked_splits}"
    if compare_widen:
        # `widened`: the widening pass plus the fp16-activation pick; `in_place`: the bf16 pick widening the
        # activations inside the kernel; `auto` is whichever of the two the heuristic runs
        a16 = torch.empty((m, k), dtype=torch.float16, device="cuda")
        widen_op = torch.ops.feather_ops.widen_bf16.default

        def widened(i):
            widen_op(a, a16)
            if wide_splits == 1:
                op(a16, packs[i % copies], scale, bias, out, *wide_tile)
            else:
                split_op(a16, packs[i % copies], scale, bias, out, ws, wide_splits, *wide_tile)

        providers["widened"] = widened
        if auto_name not in providers:
            providers["in_place"] = launcher(picked, picked_splits)
    elif auto_name not in providers:  # when the sweep includes the pick, `auto` is that measurement
        providers["auto"] = launcher(picked, picked_splits)
    res = measure(providers, warmup=args.warmup, rounds=args.rounds, target_ms=args.target_ms, graph=args.graph)
    if compare_widen and "in_place" not in res:
        res["in_place"] = res[auto_name]
    if "auto" not in res:
        res["auto"] = res["widened"] if widen else res["in_place"] if compare_widen else res[auto_name]
    tflops = {name: 2.0 * m * n * k / (r.median_ms * 1e-3) / 1e12 for name, r in res.items()}
    tile_names = [name for name in providers if name not in ("torch_mm", "auto")] or ["auto"]
    best = max(tile_names, key=lambda name: tflops[name])
    return {
        "M": m, "N": n, "K": k, "weight_copies": copies, "picked": list(picked), "picked_splits": picked_splits,
        "widened_first": widen, "widened_tile": list(wide_tile) if compare_widen else None,
        "widened_splits": wide_splits if compare_widen else None,
        "widened_vs_in_place": paired_speedup(res["widened"], res["in_place"]) if compare_widen else None,
        "best": best,
        "tflops": tflops, "median_ms": {name: r.median_ms for name, r in res.items()},
        "spread": {name: (r.p80_ms - r.p20_ms) / r.median_ms for name, r in res.items()},
        "auto_vs_torch_mm": paired_speedup(res["auto"], res["torch_mm"]),
        "auto_vs_best": tflops["auto"] / tflops[best],
    }


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--cells", default=None, help="'M,N,K;M,N,K' instead of the grid")
    parser.add_argument("--groups", default="", help=f"comma-separated groups of cells.py: {','.join(GROUPS)}")
    parser.add_argument("--square", action="store_true", help="N^3 for N in 512..8192 instead of the grid")
    parser.add_argument("--tiles", nargs="?", const="", default=None, help="'m,n,u,rm,rn,p;...', or nothing for all")
    parser.add_argument("--splits", default="", help="'2,3,4': split-K counts to time for underfilled grids")
    parser.add_argument("--split-any-grid", action="store_true",
                        help="time the split counts on grids of a CU's worth of tiles or more too")
    parser.add_argument("--a-dtype", choices=list(_DT), default="bf16")
    parser.add_argument("--out-dtype", choices=list(_DT), default="bf16")
    parser.add_argument("--fp8", choices=list(_FP8), default="e5m2", help="weight format")
    parser.add_argument("--no-bias", dest="bias", action="store_false")
    parser.add_argument("--cold", action="store_true", help="rotate weight copies past the 256 MB MALL")
    parser.add_argument("--copies", type=int, default=None,
                        help="rotate exactly this many weight copies (a working set of that many weights)")
    parser.add_argument("--weight-streaming", choices=["auto", "on", "off"], default=None,
                        help="non-temporal weight loads (feather_ops.set_weight_streaming); default: leave the mode")
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--rounds", type=int, default=5)
    parser.add_argument("--target-ms", type=float, default=20.0)
    parser.add_argument("--widen-all", action="store_true",
                        help="bf16 activations: time the widening pass + fp16-activation pick on every cell")
    parser.add_argument("--graph", action="store_true",
                        help="time replays of captured batches (kernel time without host launch overhead)")
    parser.add_argument("--json", dest="json_path", default=None)
    args = parser.parse_args()
    if not torch.cuda.is_available():
        print("needs a GPU", file=sys.stderr)
        return 2

    if args.copies is not None and args.copies < 1:
        parser.error("--copies must be at least 1")
    if args.weight_streaming is not None:
        set_weight_streaming(args.weight_streaming)
    tiles = parse_tiles(args.tiles) if args.tiles is not None else []
    args.splits = [int(v) for v in args.splits.split(",") if v.strip()]
    if args.square:
        shapes = [("square", s, s, s) for s in (512, 1024, 2048, 4096, 8192)]
    elif args.cells:
        shapes = [("custom", *(int(v) for v in c.split(","))) for c in args.cells.split(";")]
    else:
        shapes = cells({g.strip() for g in args.groups.split(",") if g.strip()} or None)

    results = []
    print(f"{'cell':34s} {'torch_mm':>9s} {'auto':>9s} {'best':>9s}  auto/best  auto/torch  picked -> best", flush=True)
    for group, m, n, k in shapes:
        r = run_cell(m, n, k, tiles, args)
        r["group"] = group
        results.append(r)
        t = r["tflops"]
        print(f"{group + ' ' + f'{m}x{n}x{k}':34s} {t['torch_mm']:9.1f} {t['auto']:9.1f} {t[r['best']]:9.1f}"
              f"  {r['auto_vs_best']:9.3f}  {r['auto_vs_torch_mm']:10.3f}  {tuple(r['picked'])}"
              f"{'/' + str(r['picked_splits']) if r['picked_splits'] > 1 else ''} -> {r['best']}"
              + (f"  [{'widened first' if r['widened_first'] else 'widened (not picked)'} on "
                 f"{tuple(r['widened_tile'])}{'/' + str(r['widened_splits']) if r['widened_splits'] > 1 else ''}: "
                 f"x{r['widened_vs_in_place']:.3f} over in place]" if r["widened_tile"] else ""), flush=True)
        if args.json_path:  # after every cell, so a run cut short keeps what it measured
            pathlib.Path(args.json_path).write_text(json.dumps({"args": vars(args), "results": results}, indent=1))
        torch.cuda.empty_cache()
    geo = lambda xs: math.exp(sum(math.log(x) for x in xs) / len(xs))  # noqa: E731
    print(f"geomean over {len(results)} cells: auto/best {geo([r['auto_vs_best'] for r in results]):.3f}, "
          f"auto/torch_mm {geo([r['auto_vs_torch_mm'] for r in results]):.3f}", flush=True)
    if args.json_path:
        pathlib.Path(args.json_path).write_text(json.dumps({"args": vars(args), "results": results}, indent=1))
    return 0


if __name__ == "__main__":
    with torch.inference_mode():
        sys.exit(main())
