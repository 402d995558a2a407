"""GPU parity of split-K (`scaled_mm_hip(..., splits=S)`, op `feather_ops::scaled_mm_splitk`, C ABI
`feather_scaled_mm_splitk`) against the CPU oracle.

Split-K changes only the fp32 summation order, so every case meets the same bar as the unsplit kernel
(`check_against_oracle`). Also checked: every ring tile and every streaming tile with ragged M, N and K;
split counts up to the stage (ring) or 64-deep group (streaming) count; bias, per-column scales, bf16
activations (the register-staged path), e4m3fn, both output dtypes; determinism; a shared workspace
reused with alternating inputs and across kernel families (no stale partial sums are read); the
workspace counters back at zero after each call; graph replay; the C ABI called directly; and the
refusals of the op.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import check_against_oracle, sample_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _tensor(shape, dtype, seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).cuda()


def _ring_tiles():
    from feather_ops.tiles import SCALED_MM_TILES

    return [t for t in SCALED_MM_TILES if t[5] == 1]


def _stream_tiles():
    from feather_ops.tiles import SCALED_MM_TILES

    return [t for t in SCALED_MM_TILES if t[5] == 0]


def _stages(k, tile):
    return -(-k // (16 * tile[2]))


@pytest.mark.parametrize("tile", _ring_tiles())
@pytest.mark.parametrize("splits", [2, 3, 5])
def test_every_ring_tile_split(fo, tile, splits):
    """Ragged M, N (N % 16 == 8) and K (the last stage is partly past K); K = 304 has 5 stages."""
    M, N, K = 67, 264, 304
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    scale = torch.tensor(0.75, device="cuda")
    bias = _tensor((N,), torch.bfloat16, seed=2)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile, splits=splits)
    check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("m", [1, 20, 48, 64])
def test_ring_split_with_fewer_rows_than_the_tile(fo, m):
    """The 64 x 128 ring tile split along K at skinny M (the heuristic's 16 < M <= 64 regime): the rows
    past M read as zeros and are never stored."""
    N, K = 1032, 4096
    a = _tensor((m, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e4m3fn, seed=1))
    scale = torch.tensor(0.5, device="cuda")
    bias = _tensor((N,), torch.float16, seed=2)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.float16, tile=(1, 4, 4, 4, 2, 1), splits=4)
    check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("tile", _stream_tiles())
@pytest.mark.parametrize("splits", [2, 3, 7])
def test_every_stream_tile_split(fo, tile, splits):
    """Ragged M (not a multiple of the 16-row fragment), N (N % 16 == 8) and K: K = 1040 is 17 groups of 64,
    the last one a single chunk of 16, so a split can hold fewer groups than the block has K slices."""
    M, N, K = 37, 264, 1040
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    scale = torch.tensor(0.75, device="cuda")
    bias = _tensor((N,), torch.bfloat16, seed=2)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile, splits=splits)
    check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("a_dtype,b_dtype,out_dtype", [(torch.bfloat16, torch.float8_e4m3fn, torch.float16),
                                                       (torch.float16, torch.float8_e5m2, torch.bfloat16)])
def test_stream_split_dtypes_with_column_scales(fo, a_dtype, b_dtype, out_dtype):
    M, N, K = 5, 1032, 2048
    a = _tensor((M, K), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), b_dtype, seed=1))
    scale = (torch.rand(N, generator=torch.Generator().manual_seed(3)) + 0.5).cuda()
    bias = _tensor((N,), out_dtype, seed=2)
    for tile in [(8, 1, 4, 1, 4, 0), (4, 2, 4, 1, 2, 0), (2, 2, 4, 4, 2, 0)]:
        out = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=tile, splits=4)
        check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("m,n,k,tile,splits", [
    (16, 14336, 4096, (8, 1, 4, 1, 4, 0), 2),     # the weight-streaming cell
    (32, 5120, 25600, (2, 2, 4, 2, 2, 0), 4),
    (2, 4096, 16384, (8, 1, 4, 1, 4, 0), 4),
    (1, 3072, 3072, (8, 1, 4, 1, 2, 0), 3),
])
def test_stream_split_full_size(fo, m, n, k, tile, splits):
    a = _tensor((m, k), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    scale = torch.tensor(0.02, device="cuda")
    bias = _tensor((n,), torch.float16, seed=2)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.float16, tile=tile, splits=splits)
    check_against_oracle(out, a, bp, scale, bias, rows=sample_rows(m))


def test_stream_split_count_up_to_the_group_count(fo):
    M, N, K = 16, 128, 1024  # 16 groups of 64, whatever the tile's unroll_k
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    tile = (8, 1, 8, 1, 4, 0)
    unsplit = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile)
    for splits in (2, 16):
        out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=splits)
        check_against_oracle(out, a, bp, None, None)
        assert (out.float() - unsplit.float()).abs().max().item() <= unsplit.float().abs().max().item() * 2**-9
    with pytest.raises(RuntimeError):
        fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=17)


def test_workspace_reuse_across_kernel_families(fo):
    """Ring and streaming split launches alternate on one workspace; the streaming counters (one per
    fragment) and the ring ones (one per wave) share the fixed area, and every call leaves it zero."""
    from feather_ops.scaled_mm import _split_workspaces

    cases = [(16, 5376, 4096, (8, 1, 4, 1, 4, 0), 3), (300, 1000, 2048, (2, 2, 4, 4, 4, 1), 4),
             (3, 2056, 1600, (4, 2, 4, 1, 2, 0), 5), (64, 640, 4096, (2, 2, 4, 4, 2, 0), 8),
             (16, 5376, 4096, (8, 1, 4, 1, 4, 0), 3)]
    for i, (m, n, k, tile, splits) in enumerate(cases):
        a = _tensor((m, k), torch.float16, seed=60 + i)
        bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=70 + i))
        out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=splits)
        check_against_oracle(out, a, bp, None, None, rows=sample_rows(m))
    torch.cuda.synchronize()
    ws = _split_workspaces[(torch.cuda.current_device(), torch.cuda.current_stream().cuda_stream)]
    assert int(ws[: 64 * 1024].view(torch.int32).abs().sum().item()) == 0


@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b_dtype,out_dtype", [(torch.float8_e5m2, torch.float16),
                                               (torch.float8_e5m2, torch.bfloat16),
                                               (torch.float8_e4m3fn, torch.bfloat16)])
def test_dtype_combinations_with_column_scales(fo, a_dtype, b_dtype, out_dtype):
    M, N, K = 200, 512, 1024
    a = _tensor((M, K), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), b_dtype, seed=1))
    scale = (torch.rand(N, generator=torch.Generator().manual_seed(3)) + 0.5).cuda()
    bias = _tensor((N,), out_dtype, seed=2)
    # 128-row tiles and the 64-row ones (deep ring with fp16 activations, shallow with bf16 at M = 200)
    for tile in [(2, 2, 4, 4, 4, 1), (2, 2, 4, 4, 8, 1), (2, 4, 4, 4, 4, 1), (1, 4, 4, 4, 2, 1), (2, 2, 4, 2, 2, 1)]:
        out = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=tile, splits=4)
        check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("m,n,k,splits", [(512, 5376, 5120, 3), (512, 4096, 4096, 4), (1040, 1536, 6144, 4),
                                          (192, 12288, 4096, 2)])
def test_underfilled_grids_full_size(fo, m, n, k, splits):
    """The mid-size cells split-K is for, full size, on a row sample."""
    a = _tensor((m, k), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    scale = torch.tensor(0.02, device="cuda")
    out = fo.scaled_mm_hip(a, bp, scale, None, torch.float16, tile=(2, 2, 4, 4, 4, 1), splits=splits)
    check_against_oracle(out, a, bp, scale, None, rows=sample_rows(m))


def test_split_count_up_to_the_stage_count(fo):
    M, N, K = 96, 128, 1024  # 16 stages of 64
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    for splits in (1, 4, 16):
        out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=(2, 2, 4, 2, 2, 1), splits=splits)
        check_against_oracle(out, a, bp, None, None)
    with pytest.raises(RuntimeError):
        fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=(2, 2, 4, 2, 2, 1), splits=17)


def test_deterministic_and_close_to_unsplit(fo):
    M, N, K = 300, 1000, 2048
    a = _tensor((M, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.01, device="cuda")
    tile = (2, 2, 4, 4, 4, 1)
    x = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=3)
    for _ in range(3):
        y = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=3)
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    ref = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile)
    diff = (x.float() - ref.float()).abs().max().item()
    assert diff <= 2 * ref.float().abs().max().item() * 2**-10  # one or two fp16 ulps of summation order


def test_workspace_reuse_across_shapes(fo):
    """One cached workspace serves calls of different shapes and tiles, small grids after big ones and the
    other way round: the counter area is the same fixed area for every shape and stays zero."""
    shapes = [(512, 5376, 1024, (2, 2, 4, 4, 4, 1), 3), (67, 264, 304, (2, 2, 4, 2, 2, 1), 5),
              (192, 12288, 1024, (2, 2, 4, 4, 4, 1), 2), (130, 520, 512, (4, 2, 4, 4, 8, 1), 4),
              (192, 12288, 1024, (2, 2, 4, 4, 4, 1), 2)]
    for i, (m, n, k, tile, splits) in enumerate(shapes):
        a = _tensor((m, k), torch.float16, seed=i)
        bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=100 + i))
        out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=splits)
        check_against_oracle(out, a, bp, None, None, rows=sample_rows(m))


def test_workspace_reuse_with_alternating_inputs(fo):
    """One stream, one workspace, different inputs each call: a call must never read another call's partial
    sums (they sit at the same workspace addresses), and must leave the counters at zero."""
    from feather_ops.scaled_mm import _split_workspaces
    from feather_ops.tiles import split_workspace_bytes

    M, N, K = 160, 640, 1536
    tile = (2, 2, 4, 4, 4, 1)
    inputs = []
    for seed in range(3):
        a = _tensor((M, K), torch.float16, seed=10 + seed)
        bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=20 + seed))
        inputs.append((a, bp, fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile)))
    for _round in range(2):
        for a, bp, unsplit in inputs:
            out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=6)
            check_against_oracle(out, a, bp, None, None)
            assert (out.float() - unsplit.float()).abs().max().item() <= unsplit.float().abs().max().item() * 2**-9
    torch.cuda.synchronize()
    ws = _split_workspaces[(torch.cuda.current_device(), torch.cuda.current_stream().cuda_stream)]
    tiles = -(-M // 128) * -(-N // 128)
    assert split_workspace_bytes(M, N, K, tile, 6) <= ws.numel()
    counters = ws[: tiles * 4 * 4].view(torch.int32)
    assert int(counters.abs().sum().item()) == 0


def test_concurrent_streams_use_their_own_workspaces(fo):
    """Split launches on two streams at once: each stream has its own workspace, and both results are right."""
    from feather_ops.scaled_mm import _split_workspaces

    M, N, K = 512, 1536, 4096
    tile = (2, 2, 4, 4, 4, 1)
    inputs = [(_tensor((M, K), torch.float16, seed=40 + i),
               fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=50 + i))) for i in range(2)]
    want = [fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile) for a, bp in inputs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = [[], []]
    for _ in range(4):
        for i, stream in enumerate(streams):
            with torch.cuda.stream(stream):
                a, bp = inputs[i]
                outs[i].append(fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile, splits=4))
    torch.cuda.synchronize()
    keys = {(torch.cuda.current_device(), s.cuda_stream) for s in streams}
    assert keys <= set(_split_workspaces)
    assert _split_workspaces[keys.pop()].data_ptr() != _split_workspaces[keys.pop()].data_ptr()
    for i in range(2):
        for out in outs[i]:
            assert (out.float() - want[i].float()).abs().max().item() <= want[i].float().abs().max().item() * 2**-9
    check_against_oracle(outs[1][-1], *inputs[1], None, None, rows=sample_rows(M))


def test_cleared_workspaces_are_recreated_zeroed(fo):
    from feather_ops.scaled_mm import _split_workspaces, clear_split_workspaces

    M, N, K = 256, 512, 4096
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    first = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=(2, 2, 4, 4, 4, 1), splits=4)
    torch.cuda.synchronize()
    clear_split_workspaces()
    assert not _split_workspaces
    again = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=(2, 2, 4, 4, 4, 1), splits=4)
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    assert _split_workspaces


def test_graph_replay_matches_eager(fo):
    """Captured split launches replay correctly, with eager work and syncs between replays."""
    M, N, K = 256, 768, 2048
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.5, device="cuda")
    tile = (2, 2, 4, 4, 4, 1)
    want = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=4)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=4)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=4)
    for _ in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile, splits=4)  # eager work in between
        torch.cuda.synchronize()


def test_c_abi_direct(fo):
    """feather_scaled_mm_splitk through ctypes matches the op bit for bit; a short or misaligned
    workspace is refused before anything is enqueued."""
    from feather_ops import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    lib.feather_scaled_mm_splitk.restype = ctypes.c_bool
    lib.feather_scaled_mm_splitk.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_int] + \
        [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.feather_splitk_workspace_bytes.restype = ctypes.c_int64
    lib.feather_splitk_workspace_bytes.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int] * 5 + \
        [ctypes.c_bool, ctypes.c_int]
    M, N, K = 100, 256, 640
    a = _tensor((M, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.3, device="cuda")
    bias = _tensor((N,), torch.float16, seed=2)
    tile = (2, 2, 4, 4, 4, True)
    want = fo.scaled_mm_hip(a, bp, s, bias, torch.float16, tile=tile, splits=5)
    need = lib.feather_splitk_workspace_bytes(M, N, K, *tile, 5)
    ws = torch.zeros(need + 256, dtype=torch.uint8, device="cuda")
    c = torch.empty_like(want)
    stream = torch.cuda.current_stream().cuda_stream
    args = (a.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(), M, N, K, 1, 1, True, True,
            False, *tile, 5)
    assert lib.feather_scaled_mm_splitk(*args, ws.data_ptr(), need, stream)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), want.view(torch.int16))
    assert not lib.feather_scaled_mm_splitk(*args, ws.data_ptr(), need - 1, stream)
    assert not lib.feather_scaled_mm_splitk(*args, ws.data_ptr() + 16, need, stream)
    torch.cuda.synchronize()
    assert int(ws.count_nonzero().item()) > 0  # the partial sums are there; the counters are zero again
    tiles = 1 * 2
    assert int(ws[: tiles * 4 * 4].view(torch.int32).abs().sum().item()) == 0


def test_op_rejects_bad_split_arguments(fo):
    a = _tensor((64, 256), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((256, 128), torch.float8_e5m2, seed=1))
    c = torch.empty(64, 128, dtype=torch.float16, device="cuda")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    op = torch.ops.feather_ops.scaled_mm_splitk.default
    with pytest.raises(RuntimeError, match="Unsupported config"):
        op(a, bp, None, None, c, ws, 2, 4, 1, 4, 1, 4)          # a streaming tile's numbers as a ring tile
    with pytest.raises(RuntimeError, match="workspace must hold"):
        op(a, bp, None, None, c, ws[:1024], 2, 2, 2, 4, 4, 4)
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        op(a, bp, None, None, c, ws[16:], 2, 2, 2, 4, 4, 4)
    with pytest.raises(RuntimeError, match="uint8"):
        op(a, bp, None, None, c, ws.view(torch.int32), 2, 2, 2, 4, 4, 4)
    with pytest.raises(RuntimeError, match="splits must be"):
        op(a, bp, None, None, c, ws, 0, 2, 2, 4, 4, 4)
    op(a, bp, None, None, c, ws, 4, 2, 2, 4, 4, 4)              # K = 256: 4 stages, 4 splits is fine
    check_against_oracle(c, a, bp, None, None)
    assert np.all(ws[:256].cpu().numpy() == 0)
