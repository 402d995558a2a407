#!/usr/bin/env python3
"""Same-box A/B of two builds of libfeather_ops_gfx950.so through the C ABI.

Per cell both builds launch the heuristic's pick of the package being imported (tile and split count, or
`--tile` for every cell) on the same inputs, interleaved round by round (protocol.py), and the outputs are
compared bit for bit. The build under test is `--new` (default: the package's own library), the control
`--old`; an older commit's library comes from building that commit in a worktree, e.g.

    git worktree add /tmp/old <commit> && make -C /tmp/old/feather-ops_amd -j8
    python -m benchmarks.compare_builds --old /tmp/old/feather-ops_amd/feather_ops/libfeather_ops_gfx950.so \
        --cells "4096,12288,3072;4096,3072,3072"
    python -m benchmarks.compare_builds --old ... --groups all --ring-only --a-dtype bf16

Run from `feather-ops_amd/` on the GPU. Prints per cell the median time of each build, new/old and whether
the outputs are bit-identical, then the geometric mean of new/old.
"""

import argparse
import ctypes
import json
import math
import sys

import torch

from feather_ops import _lib
from feather_ops.scaled_mm import select_scaled_mm_config, select_scaled_mm_splits
from feather_ops.scaled_mm import prepack_b_for_scaled_mm
from feather_ops.tiles import split_workspace_bytes

from .cells import GROUPS, cells
from .protocol import measure

_DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
_FP8 = {"e5m2": torch.float8_e5m2, "e4m3fn": torch.float8_e4m3fn}


def bind(path: str) -> ctypes.CDLL:
    lib = ctypes.CDLL(path)
    lib.launch_scaled_mm.restype = ctypes.c_bool
    lib.launch_scaled_mm.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_void_p]
    lib.feather_scaled_mm_splitk.restype = ctypes.c_bool
    lib.feather_scaled_mm_splitk.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                                    ctypes.c_void_p]
    return lib


def run_cell(libs: dict, m: int, n: int, k: int, args) -> dict:
    a_dtype = _DT[args.a_dtype]
    fp8 = _FP8[args.fp8]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    a = torch.randn((m, k), generator=gen, device="cuda").to(a_dtype)
    packed = prepack_b_for_scaled_mm(torch.randn((k, n), generator=gen, device="cuda").to(fp8))
    scale = torch.tensor(2.34, device="cuda", dtype=torch.float32)
    tile = tuple(args.tile) if args.tile else tuple(select_scaled_mm_config(m, n, k, a_dtype, fp8, a_dtype))
    splits = 1 if args.tile else select_scaled_mm_splits(m, n, k, tile, a_dtype)
    tiles = {"new": tile, "old": tuple(args.old_tile) if args.old_tile else tile}
    stream = torch.cuda.current_stream().cuda_stream
    outs = {name: torch.empty((m, n), device="cuda", dtype=a_dtype) for name in libs}
    ws_bytes = split_workspace_bytes(m, n, k, tile, splits) if splits > 1 else 0
    workspaces = {name: torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda") for name in libs}
    bf16 = a_dtype == torch.bfloat16

    def provider(name):
        lib, out, ws, tile = libs[name], outs[name], workspaces[name], tiles[name]

        def launch(_i):
            if splits > 1:
                ok = lib.feather_scaled_mm_splitk(a.data_ptr(), packed.data_ptr(), scale.data_ptr(), None,
                                                  out.data_ptr(), m, n, k, 1, 0, fp8 == torch.float8_e5m2, bf16,
                                                  bf16, *tile[:5], bool(tile[5]), splits, ws.data_ptr(), ws_bytes,
                                                  stream)
            else:
                ok = lib.launch_scaled_mm(a.data_ptr(), packed.data_ptr(), scale.data_ptr(), None, out.data_ptr(),
                                          m, n, k, 1, 0, fp8 == torch.float8_e5m2, bf16, bf16, *tile[:5],
                                          bool(tile[5]), stream)
            if not ok:
                raise RuntimeError(f"launch refused for {m}x{n}x{k} tile {tile} splits {splits}")
        return launch

    res = measure({name: provider(name) for name in libs}, warmup=args.warmup, rounds=args.rounds,
                  target_ms=args.target_ms)
    same = torch.equal(outs["new"].view(torch.int16), outs["old"].view(torch.int16))
    new_ms, old_ms = res["new"].median_ms, res["old"].median_ms
    return {"M": m, "N": n, "K": k, "tile": list(tile), "old_tile": list(tiles["old"]), "splits": splits,
            "new_us": new_ms * 1e3, "old_us": old_ms * 1e3, "new_over_old": new_ms / old_ms, "bit_identical": same}


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--old", required=True, help="control build of libfeather_ops_gfx950.so")
    p.add_argument("--new", default=str(_lib.LIBRARY), help="build under test (default: the package's)")
    p.add_argument("--cells", help="'M,N,K;M,N,K' instead of groups")
    p.add_argument("--groups", default="baseline", help="comma-separated groups of cells.py, or 'all'")
    p.add_argument("--ring-only", action="store_true", help="only cells whose pick is an LDS ring tile")
    p.add_argument("--tile", type=lambda s: [int(x) for x in s.split(",")], help="pin one tile for every cell")
    p.add_argument("--old-tile", type=lambda s: [int(x) for x in s.split(",")],
                   help="the control build's tile, if not the same (with --tile; unsplit launches)")
    p.add_argument("--a-dtype", choices=sorted(_DT), default="fp16")
    p.add_argument("--fp8", choices=sorted(_FP8), default="e5m2")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--rounds", type=int, default=9)
    p.add_argument("--target-ms", type=float, default=5.0)
    p.add_argument("--json", dest="json_path")
    args = p.parse_args()
    if not torch.cuda.is_available():
        print("no GPU", file=sys.stderr)
        return 1
    if args.old_tile and not args.tile:
        print("--old-tile needs --tile", file=sys.stderr)
        return 1
    if args.cells:
        todo = [tuple(int(x) for x in c.split(",")) for c in args.cells.split(";") if c.strip()]
    else:
        groups = None if args.groups == "all" else set(args.groups.split(","))
        unknown = set() if groups is None else groups - set(GROUPS)
        if unknown:
            print(f"unknown groups: {sorted(unknown)}", file=sys.stderr)
            return 1
        todo = list(dict.fromkeys((m, n, k) for _, m, n, k in cells(groups)))
    libs = {"new": bind(args.new), "old": bind(args.old)}
    rows = []
    for m, n, k in todo:
        if args.ring_only and not args.tile:
            pick = select_scaled_mm_config(m, n, k, _DT[args.a_dtype], _FP8[args.fp8], _DT[args.a_dtype])
            if not pick[5]:
                continue
        r = run_cell(libs, m, n, k, args)
        rows.append(r)
        old_tile = "" if r["old_tile"] == r["tile"] else f" (old {tuple(r['old_tile'])})"
        print(f"{m}x{n}x{k} tile {tuple(r['tile'])}{old_tile} s{r['splits']}: new {r['new_us']:.2f} us  "
              f"old {r['old_us']:.2f} us  new/old {r['new_over_old']:.3f}  "
              f"{'bit-identical' if r['bit_identical'] else 'DIFFERENT'}", flush=True)
    if rows:
        g = math.exp(sum(math.log(r["new_over_old"]) for r in rows) / len(rows))
        print(f"geomean new/old over {len(rows)} cells: {g:.4f} (min {min(r['new_over_old'] for r in rows):.3f}, "
              f"max {max(r['new_over_old'] for r in rows):.3f})")
    if args.json_path:
        with open(args.json_path, "w") as f:
            json.dump({"args": vars(args), "results": rows}, f, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
