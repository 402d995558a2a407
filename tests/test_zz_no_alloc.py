"""The allocation-free split-K entry point, feather_scaled_mm_splitk_noalloc, through the C ABI.

Its output is checked against feather_scaled_mm_splitk's (same kernels, same split order: identical bits)
on a caller-allocated workspace and against the oracle, on two calls in a row (the second with a smaller
input, so it reuses the static array the first one left behind). Launches needing more than the static
array holds are refused on the host (tests/test_boundary.py, on the CPU).
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import check_against_oracle, sample_rows

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 * 1024 + (64 << 20)


@pytest.fixture(scope="module")
def lib():
    from feather_ops import _lib

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    handle = ctypes.CDLL(str(_lib.LIBRARY))
    common = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + [ctypes.c_bool] * 3 + \
        [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_int]
    handle.feather_scaled_mm_splitk.restype = ctypes.c_bool
    handle.feather_scaled_mm_splitk.argtypes = common + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    handle.feather_scaled_mm_splitk_noalloc.restype = ctypes.c_bool
    handle.feather_scaled_mm_splitk_noalloc.argtypes = common + [ctypes.c_void_p]
    handle.feather_splitk_workspace_bytes.restype = ctypes.c_int64
    handle.feather_splitk_workspace_bytes.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int] * 5 + \
        [ctypes.c_bool, ctypes.c_int]
    return handle


def _inputs(m, n, k, a_dtype, out_dtype, seed):
    import feather_ops

    g = torch.Generator("cpu").manual_seed(seed)
    a = torch.randn(m, k, generator=g).to(a_dtype).cuda()
    w = torch.randn(k, n, generator=g).to(torch.float8_e5m2).cuda()
    bp = feather_ops.prepack_b_for_scaled_mm(w)
    s = torch.tensor(0.125, dtype=torch.float32, device="cuda")
    bias = torch.randn(n, generator=g).to(out_dtype).cuda()
    return a, bp, s, bias


def _call(lib, fn, a, bp, s, bias, c, tile, splits, *ws):
    m, k = a.shape
    n = bp.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    return fn(a.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(), m, n, k, 1, 1, True,
              a.dtype == torch.bfloat16, c.dtype == torch.bfloat16, *tile, splits, *ws, stream)


# calls in a row on one GPU's static array, each smaller than the last: the largest split launch the heuristic
# makes (a 128 x 128 ring tile split 4 ways, 48 MiB of partials), a smaller ring launch, then a streaming tile
CASES = [
    (256, 12288, 4096, torch.float16, torch.float16, (2, 2, 4, 4, 4, 1), 4),  # 192 tiles x 4 splits, 48 MiB
    (512, 2048, 2560, torch.float16, torch.float16, (2, 2, 4, 4, 4, 1), 4),   # 64 tiles x 4 splits, 16 MiB
    (16, 1024, 4096, torch.bfloat16, torch.bfloat16, (8, 1, 4, 1, 4, 0), 3),  # 16 tiles x 3 splits
]


def test_noalloc_matches_the_workspace_entry_point_twice_in_a_row(lib):
    for i, (m, n, k, a_dt, out_dt, tile, splits) in enumerate(CASES):
        print(f"noalloc case {i}: {m}x{n}x{k} tile {tile} splits {splits}", flush=True)
        a, bp, s, bias = _inputs(m, n, k, a_dt, out_dt, seed=20 + i)
        need = lib.feather_splitk_workspace_bytes(m, n, k, *tile, splits)
        assert 0 < need <= SCRATCH_BYTES
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        want = torch.empty((m, n), dtype=out_dt, device="cuda")
        assert _call(lib, lib.feather_scaled_mm_splitk, a, bp, s, bias, want, tile, splits, ws.data_ptr(), need)
        got = torch.full((m, n), float("nan"), dtype=out_dt, device="cuda")
        assert _call(lib, lib.feather_scaled_mm_splitk_noalloc, a, bp, s, bias, got, tile, splits)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        check_against_oracle(got, a, bp, s, bias, rows=sample_rows(m, n_random=8) if m * n * k > (1 << 28) else None)
        # the static counters are left zero: the same call again gives the same bits
        again = torch.empty_like(got)
        assert _call(lib, lib.feather_scaled_mm_splitk_noalloc, a, bp, s, bias, again, tile, splits)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), want.view(torch.int16))


def test_noalloc_with_one_split_runs_the_unsplit_kernel(lib):
    """splits = 1 needs no scratch: the unsplit kernel, checked against the oracle. (Launches past the static
    array are refused on the host before any GPU call; tests/test_boundary.py checks that on the CPU.)"""
    m, n, k, tile = 64, 64, 64, (2, 2, 4, 4, 4, 1)
    a, bp, s, bias = _inputs(m, n, k, torch.float16, torch.float16, seed=30)
    c = torch.empty((m, n), dtype=torch.float16, device="cuda")
    assert _call(lib, lib.feather_scaled_mm_splitk_noalloc, a, bp, s, bias, c, tile, 1)
    torch.cuda.synchronize()
    check_against_oracle(c, a, bp, s, bias)
    assert np.isfinite(c.float().cpu().numpy()).all()


def test_noalloc_replays_under_graph_capture(lib):
    """A split noalloc call captured into a HIP graph (after an eager call on the device, as the header asks)
    replays correctly: each replay, with new activations copied into the captured input and eager work on the
    stream between replays, gives the bits of the eager feather_scaled_mm_splitk on the same inputs."""
    m, n, k, tile, splits = 512, 2048, 2560, (2, 2, 4, 4, 4, 1), 4
    a, bp, s, bias = _inputs(m, n, k, torch.float16, torch.float16, seed=40)
    warm = torch.empty((m, n), dtype=torch.float16, device="cuda")
    assert _call(lib, lib.feather_scaled_mm_splitk_noalloc, a, bp, s, bias, warm, tile, splits)  # eager first
    torch.cuda.synchronize()
    need = lib.feather_splitk_workspace_bytes(m, n, k, *tile, splits)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    got = torch.empty((m, n), dtype=torch.float16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            ok = _call(lib, lib.feather_scaled_mm_splitk_noalloc, a, bp, s, bias, got, tile, splits)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert ok
    g = torch.Generator("cpu").manual_seed(41)
    for replay in range(4):
        print(f"noalloc graph replay {replay}", flush=True)
        a.copy_(torch.randn(m, k, generator=g).to(torch.float16).cuda())
        want = torch.empty((m, n), dtype=torch.float16, device="cuda")
        assert _call(lib, lib.feather_scaled_mm_splitk, a, bp, s, bias, want, tile, splits, ws.data_ptr(), need)
        torch.cuda.synchronize()
        got.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), replay
    check_against_oracle(got, a, bp, s, bias, rows=sample_rows(m, n_random=8))
