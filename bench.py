"""Benchmark of the fp16/bf16 x fp8e5m2 scaled matmul on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--rounds R] [--no-cpu] [--no-secondary]

Headline workload (BASELINE.json metric): C3, the DiT MLP up-projection, A fp16 [4096, 3072] x W e5m2
[12288, 3072] (prepacked [192, 12288, 16], per-tensor scale) -> fp16 [4096, 12288]. One step is one
`feather_ops::scaled_mm` launch on inputs already resident in HBM. Timing protocol, for every cell: W
untimed launches, then rounds of K launches until the clocks settle (at least 1 s of continuous work and
the last three rounds within 2% of each other, at most 6 s), then R timed rounds of K launches, each
bracketed by device synchronisation and timed with HIP events on the stream the kernels run on. The
median round gives ms_per_step; p20 and p80 are reported beside it. value = TFLOP/s = 2*M*N*K / median
time per step.

Also reported: the skinny HBM-bound cell C4 (A fp16 [16, 4096] x W e5m2 [14336, 4096]) as GB/s of
algorithmic bytes, timed over a HIP graph of launches that rotate over 8 distinct weight copies (8 x
58.7 MB > the 256 MB MALL, so each launch streams its weight from HBM), the bf16 cell C2 through the auto
path (with the in-place widening's time and the fp16-activation kernel's beside it), the C3 shape with
e4m3fn weights, the C3 shape with bf16 activations through the auto path (which widens them in a pass of
their own there and runs the fp16-activation kernel; the in-place widening's time beside it), two
split-K cells with the unsplit tile beside each, and `cpu_baseline`: the
reference's CPU path (naive.py's semantics as torch CPU calls with fp32 accumulation) on C1, the
CPU configuration, on the host's cores.

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
# (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000), measured on the kernel sources whose digest is
# TRAFFIC_SOURCES_SHA16 (`kernel_sources_sha16()`). A run whose sources differ, or a tile without a
# measurement, reports traffic null: the figure belongs to the build it was measured on.
TRAFFIC_SOURCES_SHA16 = "95e2f4bcb510343e"
MEASURED_TRAFFIC_BYTES = {
    ("c3", (2, 2, 4, 8, 8, 1)): (147576.5 * 2.0 + 98304 * 1.0) * 1024,
    ("c4", (4, 1, 4, 1, 4, 0)): (29219.6 * 2.0 + 448 * 1.0) * 1024,
}
KERNEL_SOURCES = ("csrc/scaled_mm_kernels.h", "csrc/scaled_mm_wide.h", "csrc/scaled_mm_launch.hip",
                  "csrc/scaled_mm_launch.h", "csrc/feather_tiles.h", "csrc/scaled_mm_api.hip")


def kernel_sources_sha16() -> str:
    """First 16 hex digits of the SHA-256 over the matmul kernels' sources (names and contents, in order)."""
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update(rel.encode())
        h.update((ROOT / "feather-ops_amd" / rel).read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(cell: str, tile) -> float | None:
    """HBM bytes per launch of `cell` on `tile` if they were measured on these kernel sources, else None."""
    if TRAFFIC_SOURCES_SHA16 is None or kernel_sources_sha16() != TRAFFIC_SOURCES_SHA16:
        return None
    return MEASURED_TRAFFIC_BYTES.get((cell, tuple(tile)))


class ClockMonitor:
    """The GPU's shader clock while a load runs, from the SMU's metrics table (amdsmi `gpu_metrics`: the
    current GFX clock of every XCD). The SMU rewrites that table once a second (its `system_clock_counter`,
    in ns, steps by 10^9 between rewrites), so a thread polls it every `period_s` and keeps each rewrite once;
    the table present when start() is called was written before the load window and is dropped. A clock read
    between kernels instead (a few microseconds after the MFMA load stops) already shows it recovering
    toward 2.4 GHz, so the window must be loaded throughout. Unavailable (amdsmi missing, no matching
    device): no rewrites are kept and summary() returns None. `reader` (tests) replaces amdsmi: it returns
    (table counter, [per-XCD MHz])."""

    def __init__(self, period_s: float = 0.002, reader=None):
        self.period_s = period_s
        self.tables = []          # (perf_counter when first seen, table counter, [per-XCD MHz])
        self._stale = None
        self._stop = None
        self._thread = None
        self._read = reader
        if reader is None:
            try:
                import amdsmi

                amdsmi.amdsmi_init()
                handles = amdsmi.amdsmi_get_processor_handles()
                if len(handles) == 1:
                    handle = handles[0]

                    def read():
                        metrics = amdsmi.amdsmi_get_gpu_metrics_info(handle)
                        clks = [c for c in (metrics.get("current_gfxclks") or [])
                                if isinstance(c, int) and 0 < c < 10000]
                        return metrics.get("system_clock_counter"), clks

                    self._read = read
            except Exception:  # amdsmi absent or refused: no clock figure, the benchmark itself is unaffected
                self._read = None

    def _poll(self):
        """Keep the table if it is a rewrite not seen yet; False once the reader fails."""
        import time as _time

        try:
            counter, clks = self._read()
        except Exception:
            return False
        seen = self.tables[-1][1] if self.tables else self._stale
        if clks and counter is not None and counter != seen:
            self.tables.append((_time.perf_counter(), counter, clks))
        return True

    def _run(self):
        while not self._stop.is_set():
            if not self._poll():
                return
            self._stop.wait(self.period_s)

    def start(self):
        import threading

        if self._read is None:
            return
        try:
            self._stale = self._read()[0]
        except Exception:
            self._read = None
            return
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()

    def rewrites(self) -> int:
        return len(self.tables)

    def stop(self):
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
            self._thread = None

    def summary(self) -> dict | None:
        """Median over the window's table rewrites of the mean XCD clock, its range, and each XCD's median;
        None without a rewrite."""
        if not self.tables:
            return None
        means = [sum(c) / len(c) for _, _, c in self.tables]
        n_xcd = min(len(c) for _, _, c in self.tables)
        per_xcd = [_percentile([c[i] for _, _, c in self.tables], 0.5) for i in range(n_xcd)]
        return {"clock_mhz": round(_percentile(means, 0.5), 1), "min_mhz": round(min(means), 1),
                "max_mhz": round(max(means), 1), "per_xcd_mhz": [round(v, 1) for v in per_xcd],
                "table_rewrites": len(means),
                "method": "amdsmi gpu_metrics current_gfxclks (every XCD), each once-a-second rewrite of the SMU's "
                          "table during the timed rounds and the same launches continued after them"}


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


def _percentile(values, q):
    xs = sorted(values)
    pos = q * (len(xs) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(xs) - 1)
    return xs[lo] + (xs[hi] - xs[lo]) * (pos - lo)


def steady_rounds(launch_round, launches: int, rounds: int, warmup: int, min_warm_s: float = 1.0,
                  max_warm_s: float = 6.0, tol: float = 0.02, monitor: "ClockMonitor | None" = None,
                  min_rewrites: int = 3, max_clock_s: float = 5.0) -> dict:
    """Time `launch_round` (enqueues `launches` kernel launches on the current stream) at steady state.

    `warmup` untimed launches' worth of rounds first, then more rounds until the clocks settle (at least
    min_warm_s of continuous work and the last three round times within `tol` of each other; at most
    max_warm_s), then `rounds` timed rounds. Each round is bracketed by device synchronisation and timed
    with HIP events on the launching stream. Returns microseconds per launch: median, p20, p80, plus the
    warm-up actually run. A `monitor` (ClockMonitor) samples the clock from the first timed round on; as its
    table is rewritten once a second, the same rounds continue untimed after the timed ones until it has
    `min_rewrites` rewrites (at most `max_clock_s` of monitoring in all).
    """
    import torch

    stream = torch.cuda.current_stream()

    def one() -> float:
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        launch_round()
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3 / launches

    t0 = time.perf_counter()
    warm = [one() for _ in range(max(1, -(-warmup // launches)))]
    while True:
        elapsed = time.perf_counter() - t0
        if elapsed >= max_warm_s:
            break
        if elapsed >= min_warm_s and len(warm) >= 3 and max(warm[-3:]) <= (1 + tol) * min(warm[-3:]):
            break
        warm.append(one())
    warm_s = time.perf_counter() - t0
    if monitor is not None:
        monitor.start()
    t_mon = time.perf_counter()
    timed = [one() for _ in range(rounds)]
    if monitor is not None:
        while monitor.rewrites() < min_rewrites and time.perf_counter() - t_mon < max_clock_s:
            one()
        monitor.stop()
    return {"us": _percentile(timed, 0.5), "p20_us": _percentile(timed, 0.2), "p80_us": _percentile(timed, 0.8),
            "rounds": rounds, "launches_per_round": launches, "warmup_launches": len(warm) * launches,
            "warmup_s": round(warm_s, 2), "last_warmup_us": warm[-1]}


def _cell_stats(t: dict, flops: float, nbytes: float) -> dict:
    return {"us_per_launch": round(t["us"], 3), "p20_us": round(t["p20_us"], 3), "p80_us": round(t["p80_us"], 3),
            "TFLOPs": round(flops / (t["us"] * 1e-6) / 1e12, 1), "GBps": round(nbytes / (t["us"] * 1e-6) / 1e9, 1)}


def time_c3(steps: int, warmup: int, rounds: int):
    import torch

    import feather_ops

    m, k, n = 4096, 3072, 12288
    a, bs, s = make_device_inputs(m, k, n, "fp16")
    b = bs[0]
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, b.dtype, torch.float16)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default

    def launch_round():
        for _ in range(steps):
            op(a, b, s, None, out, *tile)

    monitor = ClockMonitor()
    t = steady_rounds(launch_round, steps, rounds, warmup, monitor=monitor)
    clock = monitor.summary()
    flops = 2.0 * m * n * k
    return {"m": m, "k": k, "n": n, "tile": list(tile), "t": t, "tflops": flops / (t["us"] * 1e-6) / 1e12,
            "bytes": algorithmic_bytes(m, k, n), "clock": clock}


def time_square_cell(m: int, k: int, n: int, a_fmt: str, fp8: str, steps: int, warmup: int, rounds: int):
    """One MFMA-bound cell on the heuristic's tile, back-to-back launches, steady state."""
    import torch

    import feather_ops

    a, bs, s = make_device_inputs(m, k, n, a_fmt, fp8=fp8)
    out_dtype = torch.bfloat16 if a_fmt == "bf16" else torch.float16
    tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, out_dtype)
    out = torch.empty((m, n), dtype=out_dtype, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default

    def launch_round():
        for _ in range(steps):
            op(a, bs[0], s, None, out, *tile)

    t = steady_rounds(launch_round, steps, rounds, warmup, min_warm_s=0.5)
    return {"tile": list(tile), **_cell_stats(t, 2.0 * m * n * k, algorithmic_bytes(m, k, n))}


def time_bf16_auto_cell(m: int, k: int, n: int, steps: int, warmup: int, rounds: int):
    """bf16 activations through the auto path (`scaled_mm_hip` without a tile: widened first, then the
    fp16-activation kernel, where the heuristic says so) against the kernel widening them in place on the bf16
    pick, back-to-back launches, steady state."""
    import torch

    import feather_ops
    from feather_ops.scaled_mm import _auto_choice

    a, bs, s = make_device_inputs(m, k, n, "bf16")
    tile, splits, widen = _auto_choice(m, n, k, a.dtype)
    in_tile = feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    op = torch.ops.feather_ops.scaled_mm.default

    def auto_round():
        for _ in range(steps):
            feather_ops.scaled_mm_hip(a, bs[0], s, None, torch.bfloat16)

    def in_place_round():
        for _ in range(steps):
            op(a, bs[0], s, None, out, *in_tile)

    flops, nbytes = 2.0 * m * n * k, algorithmic_bytes(m, k, n)
    auto = _cell_stats(steady_rounds(auto_round, steps, rounds, warmup, min_warm_s=0.5), flops, nbytes)
    in_place = _cell_stats(steady_rounds(in_place_round, steps, rounds, warmup, min_warm_s=0.5), flops, nbytes)
    return {"tile": list(tile), "splits": splits, "widened_first": widen, **auto,
            "in_place_tile": list(in_tile), "in_place": in_place}


def time_c4(rounds: int, copies: int = 8, replays: int = 10):
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
    torch.cuda.synchronize()

    def launch_round():
        for _ in range(replays):
            graph.replay()

    t = steady_rounds(launch_round, launches * replays, rounds, launches, min_warm_s=0.5)
    nbytes = algorithmic_bytes(m, k, n)
    return {"m": m, "k": k, "n": n, "tile": list(tile), "t": t, "gbps": nbytes / (t["us"] * 1e-6) / 1e9,
            "bytes": nbytes, "weight_copies": copies}


def time_split_cell(m: int, k: int, n: int, unsplit_tile, rounds: int, copies: int = 1, steps: int = 50,
                    warmup: int = 10):
    """A split-K cell: the heuristic's pick (split along K) and an unsplit tile on fp16 [m, k] x e5m2 [n, k]
    -> fp16, each launched back to back through the op with one preallocated workspace (so the Python
    layer's per-call cost is not timed), rotating over `copies` weights. Returns per-launch stats for both."""
    import torch

    import feather_ops
    from feather_ops.scaled_mm import select_scaled_mm_splits
    from feather_ops.tiles import split_workspace_bytes

    a, bs, s = make_device_inputs(m, k, n, "fp16", copies=copies)
    tile = tuple(feather_ops.select_scaled_mm_config(m, n, k, a.dtype, bs[0].dtype, torch.float16))
    splits = select_scaled_mm_splits(m, n, k, tile, a.dtype)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(split_workspace_bytes(m, n, k, tile, splits), 1), dtype=torch.uint8, device="cuda")
    nbytes = algorithmic_bytes(m, k, n)
    res = {"tile": list(tile), "splits": splits, "unsplit_tile": list(unsplit_tile)}
    for name, t, sp in (("auto", tile, splits), ("unsplit", tuple(unsplit_tile), 1)):
        def launch_round(t=t, sp=sp):
            for i in range(steps):
                if sp == 1:
                    torch.ops.feather_ops.scaled_mm.default(a, bs[i % copies], s, None, out, *t)
                else:
                    torch.ops.feather_ops.scaled_mm_splitk.default(a, bs[i % copies], s, None, out, ws, sp, *t)
        res[name] = _cell_stats(steady_rounds(launch_round, steps, rounds, warmup, min_warm_s=0.5),
                                2.0 * m * n * k, nbytes)
    return res


def run_only(which: str, steps: int, warmup: int, tile=None) -> None:
    """One kernel, `warmup + steps` eager launches, nothing else: the target of rocprofv3 --pmc runs.

    c3 / c4: the scaled_mm kernel on that cell (c4 rotates over 8 weight copies); copy: torch's
    device-to-device copy of a 512 MiB buffer, whose FETCH_SIZE / WRITE_SIZE calibrate the counters
    (1 x 512 MiB read and 1 x 512 MiB written per launch); torch_c3: torch's fp16 matmul (hipBLASLt) on
    the C3 shape with the weight already dequantized to fp16, the library control a counter comparison
    is made against; bf16_c3: the auto path on the C3 shape with bf16 activations (the widening pass, then
    the fp16-activation kernel).
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
    if which == "bf16_c3":
        a, bs, s = make_device_inputs(4096, 3072, 12288, "bf16")
        for _ in range(warmup + steps):
            feather_ops.scaled_mm_hip(a, bs[0], s, None, torch.bfloat16)
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


def _cpu_model() -> str:
    try:
        return next(line.split(":", 1)[1].strip() for line in open("/proc/cpuinfo") if line.startswith("model name"))
    except (OSError, StopIteration):
        return "unknown"


def time_cpu_baseline(runs: int = 9, c3_runs: int = 5):
    """The reference's CPU path on C1, the CPU configuration (seed 0): naive.py's
    semantics as torch CPU calls with fp32 accumulation (`oracle.naive.scaled_mm_torch`: unpack, upcast,
    fp32 matmul, scale, downcast), on every core of this process's CPU share. One warm-up, then the median
    of `runs` runs; the C3 shape beside it (median of `c3_runs`). The oracle is only timed here."""
    import numpy as np
    import torch

    from oracle import naive as oracle

    share = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    threads = min(share, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else share
    torch.set_num_threads(threads)

    def timed(m, k, n, reps):
        a_bits, packed, scale, _ = oracle.make_inputs(m, k, n, oracle.F16, seed=0)
        a = torch.from_numpy(a_bits.view(np.int16)).view(torch.float16)
        bp = torch.from_numpy(packed).view(torch.float8_e5m2)
        s = torch.tensor(scale, dtype=torch.float32)
        oracle.scaled_mm_torch(a, bp, s, None, torch.float16)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            oracle.scaled_mm_torch(a, bp, s, None, torch.float16)
            times.append(time.perf_counter() - t0)
        return _percentile(times, 0.5), _percentile(times, 0.2), _percentile(times, 0.8)

    c1 = timed(256, 1024, 1024, runs)
    c3 = timed(4096, 3072, 12288, c3_runs) if c3_runs else None
    flops1 = 2.0 * 256 * 1024 * 1024
    out = {"value": round(flops1 / c1[0] / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": (f"C1 fp16 [256,1024] x e5m2 [1024,1024] -> fp16, seed 0, whole workload: naive.py semantics "
                      f"as torch CPU calls (unpack, upcast, fp32 matmul, scale, downcast), median of {runs} runs "
                      f"after 1 warm-up: {c1[0] * 1e3:.3f} ms (p20 {c1[1] * 1e3:.3f}, p80 {c1[2] * 1e3:.3f}); "
                      f"{threads} threads, nproc {share}, os.cpu_count {os.cpu_count()}, {_cpu_model()}")}
    if c3 is not None:
        out["c3"] = {"ms": round(c3[0] * 1e3, 2), "p20_ms": round(c3[1] * 1e3, 2), "p80_ms": round(c3[2] * 1e3, 2),
                     "TFLOPs": round(2.0 * 4096 * 3072 * 12288 / c3[0] / 1e12, 4), "runs": c3_runs}
    return out


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--rounds", type=int, default=7, help="timed rounds of --steps launches (at least 5)")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-secondary", action="store_true",
                        help="skip the C4 (HBM), C2 (bf16), e4m3fn, bf16 auto-path and split-K cells")
    parser.add_argument("--only", choices=["c3", "c4", "copy", "torch_c3", "bf16_c3"],
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
    rounds = max(5, args.rounds)
    c3 = time_c3(args.steps, args.warmup, rounds)
    sec = not args.no_secondary
    c4 = time_c4(rounds) if sec else None
    # C2 through the auto path (the widening pass, then the fp16-activation kernel: one round of 256 x 192
    # tiles), the in-place widening on the bf16 pick beside it
    c2 = time_bf16_auto_cell(4096, 3072, 3072, 50, 10, rounds) if sec else None
    # the same shape with fp16 activations: separates the bf16 widening's cost from the kernel's
    c2h = time_square_cell(4096, 3072, 3072, "fp16", "e5m2", 50, 10, rounds) if sec else None
    e4 = time_square_cell(4096, 3072, 12288, "fp16", "e4m3fn", 20, 10, rounds) if sec else None
    bw = time_bf16_auto_cell(4096, 3072, 12288, 20, 10, rounds) if sec else None
    # 168 tiles of 128 x 128 for 256 CUs; the unsplit control is the best unsplit tile of the sweep
    sk = time_split_cell(512, 5120, 5376, (2, 2, 4, 2, 2, 1), rounds) if sec else None
    # a decoder's down projection at batch 2: 64 tiles of 16 x 64, 67 MB of weight, 8 rotated copies; the
    # unsplit control is the streaming tile the heuristic picks without split-K (16 x 16, 256 blocks)
    dk = time_split_cell(2, 16384, 2048, (8, 1, 4, 1, 1, 0), rounds, copies=16) if sec else None
    cpu = None if args.no_cpu else time_cpu_baseline()

    t3 = c3["t"]
    flops3 = 2.0 * c3["m"] * c3["n"] * c3["k"]
    line = {
        "metric": "TFLOP/s (% fp16 MFMA peak) at 4096x3072x12288; HBM GB/s at M=16",
        "value": round(c3["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t3["us"] * 1e-3, 5),
        "clock_mhz": c3["clock"]["clock_mhz"] if c3["clock"] else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to e5m2 with a per-tensor scale, generated on the GPU)",
        "config": {"workload": "C3 DiT MLP up-projection: fp16 [4096,3072] x e5m2 [12288,3072] -> fp16, scale, no bias",
                   "M": c3["m"], "K": c3["k"], "N": c3["n"], "tile": c3["tile"],
                   "pct_fp16_peak": round(100 * c3["tflops"] / PEAK_FP16_TFLOPS, 2)},
        "timing": {"rounds": t3["rounds"], "steps_per_round": args.steps, "statistic": "median round",
                   "p20_ms": round(t3["p20_us"] * 1e-3, 5), "p80_ms": round(t3["p80_us"] * 1e-3, 5),
                   "p20_TFLOPs": round(flops3 / (t3["p80_us"] * 1e-6) / 1e12, 1),
                   "p80_TFLOPs": round(flops3 / (t3["p20_us"] * 1e-6) / 1e12, 1),
                   "warmup_launches": t3["warmup_launches"], "warmup_s": t3["warmup_s"],
                   "warmup_rule": "W launches, then rounds until >= 1 s of work and the last 3 rounds within 2% "
                                  "(at most 6 s)"},
        "roofline": {"bound": "mfma", "achieved": round(c3["tflops"], 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(c3["tflops"] / PEAK_FP16_TFLOPS, 4),
                     "traffic": measured_traffic("c3", c3["tile"]),
                     "traffic_sources_sha16": TRAFFIC_SOURCES_SHA16},
        "kernel_sources_sha16": kernel_sources_sha16(),
    }
    if c3["clock"]:
        line["clock"] = {**c3["clock"], "peak_assumes_mhz": 2400,
                         "frac_at_measured_clock": round(c3["tflops"] / (PEAK_FP16_TFLOPS * c3["clock"]["clock_mhz"]
                                                                         / 2400.0), 4)}
    if c4 is not None:
        t4 = c4["t"]
        line["hbm_cell"] = {"workload": "C4 skinny: fp16 [16,4096] x e5m2 [14336,4096] -> fp16",
                            "GBps": round(c4["gbps"], 1), "us_per_launch": round(t4["us"], 3),
                            "p20_us": round(t4["p20_us"], 3), "p80_us": round(t4["p80_us"], 3),
                            "frac_hbm_peak": round(c4["gbps"] / PEAK_HBM_GBPS, 4), "tile": c4["tile"],
                            "algorithmic_bytes": c4["bytes"], "weight_copies_rotated": c4["weight_copies"],
                            "timed_as": f"HIP graph of 32 launches, {t4['launches_per_round'] // 32} replays per round, "
                                        f"median of {t4['rounds']} rounds (launch gaps included)",
                            "traffic": measured_traffic("c4", c4["tile"])}
    if c2 is not None:
        line["bf16_cell"] = {"workload": "C2 DiT attention projection: bf16 [4096,3072] x e5m2 [3072,3072] -> bf16",
                             **c2, "frac_fp16_peak": round(c2["TFLOPs"] / PEAK_FP16_TFLOPS, 4)}
        if c2h is not None:
            line["bf16_cell"]["fp16_activations"] = {
                "workload": "the same shape with fp16 activations and output", **c2h,
                "frac_fp16_peak": round(c2h["TFLOPs"] / PEAK_FP16_TFLOPS, 4),
                "bf16_over_fp16_time": round(c2["us_per_launch"] / c2h["us_per_launch"], 4)}
    if e4 is not None:
        line["e4m3_cell"] = {"workload": "C3 shape with e4m3fn weights: fp16 [4096,3072] x e4m3fn [12288,3072] -> fp16",
                             **e4, "frac_fp16_peak": round(e4["TFLOPs"] / PEAK_FP16_TFLOPS, 4)}
    if bw is not None:
        line["bf16_wide_cell"] = {"workload": "C3 shape with bf16 activations, auto path: bf16 [4096,3072] x e5m2 "
                                              "[12288,3072] -> bf16 (widening pass included in the time)",
                                  **bw, "frac_fp16_peak": round(bw["TFLOPs"] / PEAK_FP16_TFLOPS, 4)}
    if sk is not None:
        line["splitk_cell"] = {"workload": "underfilled grid: fp16 [512,5120] x e5m2 [5376,5120] -> fp16",
                               "tile": sk["tile"], "splits": sk["splits"], **sk["auto"],
                               "unsplit_tile": sk["unsplit_tile"], "unsplit": sk["unsplit"]}
    if dk is not None:
        line["decode_split_cell"] = {"workload": "skinny long K: fp16 [2,16384] x e5m2 [2048,16384] -> fp16, "
                                                 "16 rotated weights",
                                     "tile": dk["tile"], "splits": dk["splits"], **dk["auto"],
                                     "frac_hbm_peak": round(dk["auto"]["GBps"] / PEAK_HBM_GBPS, 4),
                                     "unsplit_tile": dk["unsplit_tile"], "unsplit": dk["unsplit"]}
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
