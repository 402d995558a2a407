"""Benchmark of the fp16/bf16 x fp8e5m2 scaled matmul on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]

Headline workload (BASELINE.json metric): C3, the DiT MLP up-projection, A fp16 [4096, 3072] x W e5m2
[12288, 3072] (prepacked [192, 12288, 16], per-tensor scale) -> fp16 [4096, 12288]. One step is one
`scaled_mm_hip` call on inputs already resident in HBM; K steps are timed with HIP events on the stream
the kernels run on, bracketed by device synchronisation. value = TFLOP/s = 2*M*N*K / time per step.

Also reported: the skinny HBM-bound cell C4 (A fp16 [16, 4096] x W e5m2 [14336, 4096]) as GB/s of
algorithmic bytes, timed over a HIP graph of launches that rotate over 8 distinct weight copies (8 x
58.7 MB > the 256 MB MALL, so each launch streams its weight from HBM), the bf16 cell C2, a split-K
cell (an underfilled grid, 512 x 5120 x 5376, with the best unsplit tile beside it), and the CPU oracle
(oracle/scaled_mm_oracle.c, all host cores) on a row sample of C3 as `cpu_baseline`.

Prints one JSON line (the driver's contract) on rank 0.
"""

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT, ROOT / "feather-ops_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

PEAK_FP16_TFLOPS = 2516.6  # MI355X dense fp16/bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E

# HBM bytes per launch, by (cell, tile): rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of `bench.py --only <cell>`
# (KiB per dispatch), scaled by the factors a 512 MiB device-to-device copy gives the same counters
# (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000). Re-measure when the kernel changes; a tile without a
# measurement reports null.
MEASURED_TRAFFIC_BYTES = {
    ("c3", (2, 2, 4, 4, 8, 1)): (190033 * 2.0 + 107814 * 1.0) * 1024,
    ("c4", (8, 1, 4, 1, 4, 0)): (29219 * 2.0 + 448 * 1.0) * 1024,
}


def algorithmic_bytes(m: int, k: int, n: int, bias: bool = False) -> int:
    """Each byte once: A (2MK) + prepacked weight (K_pad*N) + output (2MN) + scale (4) [+ bias (2N)]."""
    k_pad = -(-k // 128) * 128
    return 2 * m * k + k_pad * n + 2 * m * n + 4 + (2 * n if bias else 0)


def make_device_inputs(m, k, n, a_fmt, copies=1, seed=0, fp8="e5m2"):
    """The benchmark workload, generated on the GPU: A ~ N(0, 1) [M, K] in fp16 or bf16, W ~ N(0, 0.02)
    [N, K] quantized to e5m2 (or e4m3fn) with the per-tensor scale max|W| / 57344 (448), prepacked by the
    package's own `prepack_b_for_scaled_mm`. Returns (a, [prepacked weight x copies], scale)."""
    import torch

    import feather_ops

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    a_dtype = torch.bfloat16 if a_fmt == "bf16" else torch.float16
    a = torch.randn((m, k), generator=gen, device="cuda", dtype=torch.float32).to(a_dtype)
    w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    fp8_dtype, fp8_max = (torch.float8_e4m3fn, 448.0) if fp8 == "e4m3fn" else (torch.float8_e5m2, 57344.0)
    scale = w.abs().max() / fp8_max
    w8 = (w / scale).to(fp8_dtype)
    del w
    b0 = feather_ops.prepack_b_for_scaled_mm(w8.t().contiguous())
    del w8
    bs = [b0] + [b0.clone() for _ in range(copies - 1)]
    return a, bs, scale.reshape(()).to(torch.float32)


def time_c3(steps: int, warmup: int):
    import torch

    import feather_ops

    m, k, n = 4096, 3072, 12288
    a, bs, s = make_device_inputs(m, k, n, "fp16")
    b = bs[0]
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, b.dtype, torch.float16)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default
    for _ in range(warmup):
        feather_ops.scaled_mm_hip(a, b, s, None, torch.float16)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        op(a, b, s, None, out, *tile)
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop) / steps
    flops = 2.0 * m * n * k
    return {"m": m, "k": k, "n": n, "tile": list(tile), "ms": ms, "wall_s": wall, "tflops": flops / (ms * 1e-3) / 1e12,
            "bytes": algorithmic_bytes(m, k, n)}


def time_e4m3_cell(steps: int = 100, warmup: int = 10):
    """The C3 shape with e4m3fn weights (the other fp8 format the API takes), timed like C3."""
    import torch

    import feather_ops

    m, k, n = 4096, 3072, 12288
    a, bs, s = make_device_inputs(m, k, n, "fp16", fp8="e4m3fn")
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.float16)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default
    for _ in range(warmup):
        op(a, bs[0], s, None, out, *tile)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        op(a, bs[0], s, None, out, *tile)
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    return {"tile": list(tile), "us": ms * 1e3, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def time_c4(reps: int = 50, copies: int = 8):
    import torch

    import feather_ops

    m, k, n = 16, 4096, 14336
    a, bs, s = make_device_inputs(m, k, n, "fp16", copies=copies)
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.float16)
    outs = [torch.empty((m, n), dtype=torch.float16, device="cuda") for _ in range(copies)]
    op = torch.ops.feather_ops.scaled_mm.default
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(copies):
            op(a, bs[i], s, None, outs[i], *tile)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    launches = copies * 4
    with torch.cuda.graph(graph):
        for i in range(launches):
            op(a, bs[i % copies], s, None, outs[i % copies], *tile)
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / (reps * launches)
    nbytes = algorithmic_bytes(m, k, n)
    return {"m": m, "k": k, "n": n, "tile": list(tile), "us": us, "gbps": nbytes / (us * 1e-6) / 1e9,
            "bytes": nbytes, "weight_copies": copies}


def time_c2(steps: int = 100, warmup: int = 10):
    """C2, the bf16-activation cell (bf16 [4096, 3072] x e5m2 [3072, 3072] -> bf16), TFLOP/s."""
    import torch

    import feather_ops

    m, k, n = 4096, 3072, 3072
    a, bs, s = make_device_inputs(m, k, n, "bf16")
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default
    for _ in range(warmup):
        op(a, bs[0], s, None, out, *tile)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        op(a, bs[0], s, None, out, *tile)
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    return {"tile": list(tile), "us": ms * 1e3, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def time_split_cell(m: int, k: int, n: int, unsplit_tile, copies: int = 1, steps: int = 100, warmup: int = 10):
    """A split-K cell: the heuristic's pick (split along K) and an unsplit tile on fp16 [m, k] x e5m2 [n, k]
    -> fp16, each launched back to back through the op with one preallocated workspace (so the Python
    layer's per-call cost is not timed), rotating over `copies` weights. Returns us, TFLOP/s and GB/s of
    algorithmic bytes for both."""
    import torch

    import feather_ops
    from feather_ops.scaled_mm import select_scaled_mm_splits
    from feather_ops.tiles import split_workspace_bytes

    a, bs, s = make_device_inputs(m, k, n, "fp16", copies=copies)
    tile = tuple(feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.float16))
    splits = select_scaled_mm_splits(m, n, k, tile, a.dtype)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(split_workspace_bytes(m, n, k, tile, splits), 1), dtype=torch.uint8, device="cuda")
    nbytes = 2 * m * k + -(-k // 128) * 128 * n + 2 * m * n + 4
    res = {"tile": list(tile), "splits": splits, "unsplit_tile": list(unsplit_tile)}
    for name, t, sp in (("auto", tile, splits), ("unsplit", tuple(unsplit_tile), 1)):
        def launch(i, t=t, sp=sp):
            if sp == 1:
                torch.ops.feather_ops.scaled_mm.default(a, bs[i % copies], s, None, out, *t)
            else:
                torch.ops.feather_ops.scaled_mm_splitk.default(a, bs[i % copies], s, None, out, ws, sp, *t)
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            launch(i)
        stop.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / steps
        res[name] = {"us": ms * 1e3, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12,
                     "gbps": nbytes / (ms * 1e-3) / 1e9}
    return res


def run_only(which: str, steps: int, warmup: int, tile=None) -> None:
    """One kernel, `warmup + steps` eager launches, nothing else: the target of rocprofv3 --pmc runs.

    c3 / c4: the scaled_mm kernel on that cell (c4 rotates over 8 weight copies); copy: torch's
    device-to-device copy of a 512 MiB buffer, whose FETCH_SIZE / WRITE_SIZE calibrate the counters
    (1 x 512 MiB read and 1 x 512 MiB written per launch); torch_c3: torch's fp16 matmul (hipBLASLt) on
    the C3 shape with the weight already dequantized to fp16, the library control a counter comparison
    is made against.
    """
    import torch

    import feather_ops

    if which == "torch_c3":
        a = torch.randn(4096, 3072, device="cuda", dtype=torch.float16)
        w = torch.randn(12288, 3072, device="cuda", dtype=torch.float16)
        for _ in range(warmup + steps):
            torch.mm(a, w.t())
        torch.cuda.synchronize()
        return
    if which == "copy":
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(warmup + steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    m, k, n, copies = (4096, 3072, 12288, 1) if which == "c3" else (16, 4096, 14336, 8)
    a, bs, s = make_device_inputs(m, k, n, "fp16", copies=copies)
    if tile is None:
        tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.float16)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default
    for i in range(warmup + steps):
        op(a, bs[i % copies], s, None, out, *tile)
    torch.cuda.synchronize()


def time_cpu_oracle(budget_s: float = 20.0):
    """The oracle on host cores over a row sample of the C3 workload (the same device-generated inputs,
    copied to the host), scaled to TFLOP/s. The oracle is the checker; it is only timed here."""
    import numpy as np
    import torch

    from oracle import naive as oracle

    m, k, n = 4096, 3072, 12288
    a, bs, s = make_device_inputs(m, k, n, "fp16")
    a_bits = a.view(torch.int16).cpu().numpy().view(np.uint16)
    packed = bs[0].view(torch.uint8).cpu().numpy()
    scale = float(s.item())
    del a, bs, s
    threads = min(16, oracle.cpu_count())
    rows = 32
    t0 = time.perf_counter()
    oracle.scaled_mm(a_bits, oracle.F16, packed, oracle.E5M2, scale, None, oracle.F16,
                     rows=np.arange(rows), threads=threads)
    t_probe = time.perf_counter() - t0
    rows = int(max(32, min(m, rows * budget_s / max(t_probe, 1e-3))))
    sample = np.linspace(0, m - 1, rows).astype(np.int64)
    t0 = time.perf_counter()
    oracle.scaled_mm(a_bits, oracle.F16, packed, oracle.E5M2, scale, None, oracle.F16, rows=sample, threads=threads)
    t = time.perf_counter() - t0
    try:
        model = next(line.split(":", 1)[1].strip() for line in open("/proc/cpuinfo") if line.startswith("model name"))
    except (OSError, StopIteration):
        model = "unknown"
    return {"value": 2.0 * rows * n * k / t / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"C3 rows: {rows} of {m} evenly spaced (x all {n} columns, K={k}), {t:.1f} s on {model}"}


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    parser.add_argument("--no-secondary", action="store_true",
                        help="skip the C4 (HBM), C2 (bf16), e4m3fn and split-K cells")
    parser.add_argument("--only", choices=["c3", "c4", "copy", "torch_c3"],
                        help="launch one kernel only (for profilers)")
    parser.add_argument("--tile", help="with --only: pin the tile, e.g. 2,4,4,8,4,1")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one GPU's share of the GEMM is "
              "the kernel at its shard's shape); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.only:
        tile = tuple(int(v) for v in args.tile.split(",")) if args.tile else None
        run_only(args.only, args.steps, args.warmup, tile)
        print(f"ran {args.only}: {args.warmup} + {args.steps} launches")
        return 0
    c3 = time_c3(args.steps, args.warmup)
    c4 = None if args.no_secondary else time_c4()
    c2 = None if args.no_secondary else time_c2()
    # 168 tiles of 128 x 128 for 256 CUs; the unsplit control is the best unsplit tile of the sweep
    e4 = None if args.no_secondary else time_e4m3_cell()
    sk = None if args.no_secondary else time_split_cell(512, 5120, 5376, (2, 2, 4, 2, 2, 1))
    # a decoder's down projection at batch 2: 64 tiles of 16 x 64, 67 MB of weight, 8 rotated copies; the
    # unsplit control is the streaming tile the heuristic picks without split-K (16 x 16, 256 blocks)
    dk = None if args.no_secondary else time_split_cell(2, 16384, 4096, (8, 1, 4, 1, 1, 0), copies=8)
    cpu = None if args.no_cpu else time_cpu_oracle()

    line = {
        "metric": "TFLOP/s (% fp16 MFMA peak) at 4096x3072x12288; HBM GB/s at M=16",
        "value": round(c3["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to e5m2 with a per-tensor scale, generated on the GPU)",
        "config": {"workload": "C3 DiT MLP up-projection: fp16 [4096,3072] x e5m2 [12288,3072] -> fp16, scale, no bias",
                   "M": c3["m"], "K": c3["k"], "N": c3["n"], "tile": c3["tile"],
                   "pct_fp16_peak": round(100 * c3["tflops"] / PEAK_FP16_TFLOPS, 2)},
        "roofline": {"bound": "mfma", "achieved": round(c3["tflops"], 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(c3["tflops"] / PEAK_FP16_TFLOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get(("c3", tuple(c3["tile"])))},
    }
    if c4 is not None:
        line["hbm_cell"] = {"workload": "C4 skinny: fp16 [16,4096] x e5m2 [14336,4096] -> fp16",
                            "GBps": round(c4["gbps"], 1), "us_per_launch": round(c4["us"], 3),
                            "frac_hbm_peak": round(c4["gbps"] / PEAK_HBM_GBPS, 4), "tile": c4["tile"],
                            "algorithmic_bytes": c4["bytes"], "weight_copies_rotated": c4["weight_copies"],
                            "traffic": MEASURED_TRAFFIC_BYTES.get(("c4", tuple(c4["tile"])))}
    if c2 is not None:
        line["bf16_cell"] = {"workload": "C2 DiT attention projection: bf16 [4096,3072] x e5m2 [3072,3072] -> bf16",
                             "TFLOPs": round(c2["tflops"], 1), "us_per_launch": round(c2["us"], 2),
                             "frac_fp16_peak": round(c2["tflops"] / PEAK_FP16_TFLOPS, 4), "tile": c2["tile"]}
    if e4 is not None:
        line["e4m3_cell"] = {"workload": "C3 shape with e4m3fn weights: fp16 [4096,3072] x e4m3fn [12288,3072] -> fp16",
                             "TFLOPs": round(e4["tflops"], 1), "us_per_launch": round(e4["us"], 2),
                             "frac_fp16_peak": round(e4["tflops"] / PEAK_FP16_TFLOPS, 4), "tile": e4["tile"]}
    if sk is not None:
        line["splitk_cell"] = {"workload": "underfilled grid: fp16 [512,5120] x e5m2 [5376,5120] -> fp16",
                               "tile": sk["tile"], "splits": sk["splits"],
                               "TFLOPs": round(sk["auto"]["tflops"], 1), "us_per_launch": round(sk["auto"]["us"], 2),
                               "unsplit_64x64_TFLOPs": round(sk["unsplit"]["tflops"], 1)}
    if dk is not None:
        line["decode_split_cell"] = {"workload": "skinny long K: fp16 [2,16384] x e5m2 [4096,16384] -> fp16, "
                                                 "8 rotated weights",
                                     "tile": dk["tile"], "splits": dk["splits"], "GBps": round(dk["auto"]["gbps"], 1),
                                     "us_per_launch": round(dk["auto"]["us"], 2),
                                     "frac_hbm_peak": round(dk["auto"]["gbps"] / PEAK_HBM_GBPS, 4),
                                     "unsplit_tile": dk["unsplit_tile"],
                                     "unsplit_GBps": round(dk["unsplit"]["gbps"], 1)}
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
