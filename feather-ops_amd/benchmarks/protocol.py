"""Timing protocol for the tile sweep: interleaved providers, rotated order, median and p20/p80 per launch.

One measurement of a provider is a batch of back-to-back launches between two HIP events on the current
stream; a case times every provider once per round, in an order rotated by one each round, so clock drift
on the box (5-10% between runs, and within a run while the part heats) hits every provider alike. The
batch size comes from a single-launch estimate so that one batch takes about `target_ms`.

With `graph=True` each provider's batch is captured once into a HIP graph and a measurement is one replay:
the launches then follow each other without the host in between, so a kernel shorter than its launch
path on the host (Python, op dispatch: 5-15 us) is timed by itself. Eager batches time what an eager
caller sees, host overhead included when the kernel is shorter than it.

Cold weights: on MI355X the 256 MB MALL holds most weights, so an L2 flush does not make a launch cold.
A case instead rotates its weight over enough copies that they do not fit in the MALL (see
`benchmark_scaled_mm_hip.py --cold`), which is also what a model does when every layer has its own
weight.
"""

import statistics
from collections.abc import Callable
from dataclasses import dataclass

import torch


def percentile(values: list[float], q: float) -> float:
    """Linear-interpolation percentile of `values` at `q` in [0, 1]."""
    ordered = sorted(values)
    if not ordered:
        raise ValueError("no samples")
    pos = (len(ordered) - 1) * q
    lo = int(pos)
    hi = min(lo + 1, len(ordered) - 1)
    return ordered[lo] + (ordered[hi] - ordered[lo]) * (pos - lo)


@dataclass(frozen=True)
class Measurement:
    median_ms: float
    p20_ms: float
    p80_ms: float
    samples_ms: tuple[float, ...]

    @staticmethod
    def of(samples: list[float]) -> "Measurement":
        return Measurement(statistics.median(samples), percentile(samples, 0.2), percentile(samples, 0.8),
                           tuple(samples))


def rotated_orders(names: list[str], rounds: int) -> list[list[str]]:
    """Round r starts at index r * ceil(n / rounds) mod n, so over the rounds every provider's position
    spreads over the whole round (and over every position equally often when rounds is a multiple of n)."""
    n = len(names)
    step = max(1, -(-n // rounds))
    return [names[(r * step) % n:] + names[:(r * step) % n] for r in range(rounds)]


def _batch_ms(fn: Callable[[int], object], start: int, iters: int) -> float:
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record()
    for i in range(iters):
        fn(start + i)
    end.record()
    end.synchronize()
    return begin.elapsed_time(end) / iters


def _capture(fn: Callable[[int], object], iters: int) -> torch.cuda.CUDAGraph:
    """A graph of `iters` launches of `fn` (indices 0 .. iters - 1), captured on a side stream."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(iters):
            fn(i)
    torch.cuda.synchronize()
    return graph


def _replay_ms(graph: torch.cuda.CUDAGraph, iters: int) -> float:
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record()
    graph.replay()
    end.record()
    end.synchronize()
    return begin.elapsed_time(end) / iters


def measure(providers: dict[str, Callable[[int], object]], *, warmup: int = 5, rounds: int = 5,
            target_ms: float = 20.0, max_iters: int = 64, graph: bool = False) -> dict[str, Measurement]:
    """Time each provider (called with a running launch index, which a provider may use to rotate its
    weight copies) over `rounds` interleaved rounds; with `graph`, as replays of a captured batch."""
    names = list(providers)
    for name in names:
        for i in range(warmup):
            providers[name](i)
    torch.cuda.synchronize()
    iters = {}
    graphs = {}
    for name in names:
        one = max(_batch_ms(providers[name], 0, 1), 1e-4)
        iters[name] = int(min(max(round(target_ms / one), 1), max_iters))
        if graph:
            graphs[name] = _capture(providers[name], iters[name])
            _replay_ms(graphs[name], iters[name])  # warm replay
    samples: dict[str, list[float]] = {name: [] for name in names}
    counter = 0
    for order in rotated_orders(names, rounds):
        for name in order:
            if graph:
                samples[name].append(_replay_ms(graphs[name], iters[name]))
            else:
                samples[name].append(_batch_ms(providers[name], counter, iters[name]))
            counter += iters[name]
    return {name: Measurement.of(v) for name, v in samples.items()}


def paired_speedup(candidate: Measurement, control: Measurement) -> float:
    """Median over rounds of control / candidate (rounds are paired because they ran back to back)."""
    return statistics.median(c / x for c, x in zip(control.samples_ms, candidate.samples_ms))
