"""GPU parity of the per-output-column scale against the CPU oracle.

The reference's naive path (`feather_ops/naive.py:29-33`) multiplies the fp32 product by a 1-D scale,
per output column when `bias_dim=1`; its kernel takes only the per-tensor form. Here the torch op takes
a scale of N elements (and the C ABI `has_scale == 2`) for per-channel quantized weights. Checked over
every tile (ring and stream kernels, ragged N and K), the heuristic's auto path on large shapes (row
sample), every dtype combination, against the per-tensor form (a constant vector must give the same bits),
and the op's and the C ABI's refusals.
"""

import ctypes

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


def _per_channel_weight(k, n, b_dtype=torch.float8_e5m2, seed=1):
    """W [N, K] with row magnitudes spread over 2^-4 .. 2^3, quantized per output channel:
    s[n] = max|W[n, :]| / fp8 max, Wq = fp8(W / s[:, None]). Returns (B = Wq^T [K, N] on the GPU, s)."""
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    w *= torch.exp2(torch.randint(-4, 4, (n, 1), generator=g).float())
    s = (w.abs().amax(dim=1) / torch.finfo(b_dtype).max).float()
    wq = (w / s[:, None]).to(b_dtype)
    return wq.t().contiguous().cuda(), s.cuda()


def _all_tiles():
    from feather_ops.tiles import SCALED_MM_TILES

    return SCALED_MM_TILES


@pytest.mark.parametrize("tile", _all_tiles())
def test_every_tile_per_column_scale(fo, tile):
    M, N, K = 67, 272, 304
    a = _tensor((M, K), torch.float16)
    b, s = _per_channel_weight(K, N)
    bias = _tensor((N,), torch.bfloat16, seed=2)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, s, bias, torch.bfloat16, tile=tile)
    check_against_oracle(out, a, bp, s, bias)


@pytest.mark.parametrize("tile", _all_tiles())
def test_constant_column_scales_equal_the_per_tensor_scale(fo, tile):
    M, N, K = 40, 200, 160
    a = _tensor((M, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    bias = _tensor((N,), torch.float16, seed=2)
    one = fo.scaled_mm_hip(a, bp, torch.tensor(0.37, device="cuda"), bias, torch.float16, tile=tile)
    vec = fo.scaled_mm_hip(a, bp, torch.full((N,), 0.37, device="cuda"), bias, torch.float16, tile=tile)
    assert torch.equal(one.view(torch.int16), vec.view(torch.int16))


@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b_dtype,out_dtype", [(torch.float8_e5m2, torch.float16),
                                               (torch.float8_e5m2, torch.bfloat16),
                                               (torch.float8_e4m3fn, torch.bfloat16),
                                               (torch.float8_e4m3fn, torch.float16)])
def test_dtype_combinations(fo, a_dtype, b_dtype, out_dtype):
    M, N, K = 129, 384, 640
    a = _tensor((M, K), a_dtype)
    b, s = _per_channel_weight(K, N, b_dtype)
    bias = _tensor((N,), out_dtype, seed=2)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, s, bias, out_dtype)
    check_against_oracle(out, a, bp, s, bias)


@pytest.mark.parametrize("m,n,k", [(16, 14336, 4096), (64, 4096, 4096), (2048, 4096, 1024), (4096, 3072, 3072)])
def test_auto_path_on_large_shapes(fo, m, n, k):
    """The heuristic's stream, mid and ring regimes, full-size, on a row sample."""
    a = _tensor((m, k), torch.float16)
    b, s = _per_channel_weight(k, n)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, s, None, torch.float16)
    check_against_oracle(out, a, bp, s, None, rows=sample_rows(m))


def test_op_rejects_bad_column_scales(fo):
    a = _tensor((16, 64), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((64, 32), torch.float8_e5m2, seed=1))
    with pytest.raises(RuntimeError, match="scale must have one element"):
        fo.scaled_mm_hip(a, bp, torch.ones(31, device="cuda"), None, torch.float16)
    with pytest.raises(RuntimeError, match="must be 1D"):
        fo.scaled_mm_hip(a, bp, torch.ones(1, 32, device="cuda"), None, torch.float16)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        fo.scaled_mm_hip(a, bp, torch.ones(33, device="cuda")[1:], None, torch.float16)
    with pytest.raises(RuntimeError, match="contiguous"):
        fo.scaled_mm_hip(a, bp, torch.ones(64, device="cuda")[::2], None, torch.float16)


def test_c_abi_per_column_scale(fo):
    """launch_scaled_mm with has_scale = 2 matches the torch op bit for bit; a misaligned vector is refused."""
    from feather_ops import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    lib.launch_scaled_mm.restype = ctypes.c_bool
    lib.launch_scaled_mm.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_void_p]
    M, N, K = 100, 256, 320
    a = _tensor((M, K), torch.float16)
    b, s = _per_channel_weight(K, N)
    bp = fo.prepack_b_for_scaled_mm(b)
    want = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=(2, 2, 4, 2, 2, 0))
    c = torch.empty_like(want)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.launch_scaled_mm(a.data_ptr(), bp.data_ptr(), s.data_ptr(), None, c.data_ptr(), M, N, K, 2, 0,
                                True, False, False, 2, 2, 4, 2, 2, False, stream)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), want.view(torch.int16))
    shifted = torch.empty(N + 1, device="cuda")
    assert not lib.launch_scaled_mm(a.data_ptr(), bp.data_ptr(), shifted[1:].data_ptr(), None, c.data_ptr(), M, N, K,
                                    2, 0, True, False, False, 2, 2, 4, 2, 2, False, stream)
