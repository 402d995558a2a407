"""GPU weight prepack (`csrc/prepack.hip`, behind `prepack_b_for_scaled_mm` and the C ABI
`feather_prepack_b`) against the oracle's prepack (`oracle/scaled_mm_oracle.c`, the reference's
`scaled_mm.py:137-150` index formula): a byte permutation, so bit-exact, over every byte value, ragged K,
N % 16 == 8 and the benchmark weights. The GEMM parity tests prepack on the GPU too, so this file is
what pins the layout they feed the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import naive as oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _random_codes(k, n, seed):
    return np.random.default_rng(seed).integers(0, 256, size=(k, n), dtype=np.uint8)


@pytest.mark.parametrize("dtype", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("k,n", [(1, 8), (16, 8), (127, 24), (128, 128), (200, 1000), (300, 136), (2560, 5120)])
def test_prepack_matches_the_oracle(fo, dtype, k, n):
    codes = _random_codes(k, n, seed=k * 7 + n)
    b = torch.from_numpy(codes).cuda().view(dtype)
    got = fo.prepack_b_for_scaled_mm(b)
    assert got.dtype == dtype and got.shape == (oracle.k_padded(k) // 16, n, 16)
    np.testing.assert_array_equal(got.view(torch.uint8).cpu().numpy(), oracle.prepack(codes))


@pytest.mark.parametrize("k,n", [(3072, 12288), (4096, 14336)])
def test_prepack_matches_torch_permutation_on_benchmark_weights(fo, k, n):
    """Full benchmark sizes: against torch's own view/permute copy of the same device tensor."""
    b = torch.randint(0, 256, (k, n), dtype=torch.uint8, device="cuda").view(torch.float8_e5m2)
    got = fo.prepack_b_for_scaled_mm(b).view(torch.uint8)
    want = b.view(torch.uint8).view(k // 16, 16, n).permute(0, 2, 1).contiguous()
    assert torch.equal(got, want)


def test_prepack_writes_zero_padding_over_garbage(fo):
    """Pad rows are written as zeros, not left as whatever the output buffer held."""
    from feather_ops import _lib

    k, n = 40, 64
    codes = _random_codes(k, n, seed=3)
    b = torch.from_numpy(codes).cuda()
    out = torch.full((8, n, 16), 0xAB, dtype=torch.uint8, device="cuda")
    lib = ctypes.CDLL(str(_lib.LIBRARY))
    lib.feather_prepack_b.restype = ctypes.c_bool
    lib.feather_prepack_b.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    assert lib.feather_prepack_b(b.data_ptr(), out.data_ptr(), k, n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.prepack(codes))


def test_prepack_feeds_the_gemm(fo):
    """The GEMM on a GPU-prepacked weight equals the GEMM on the oracle-prepacked weight, bit for bit
    (K = 192 pads to 256, so the zero rows are read too)."""
    m, k, n = 33, 192, 96
    g = torch.Generator("cpu").manual_seed(5)
    a = torch.randn((m, k), generator=g).to(torch.float16).cuda()
    codes = (torch.randn((k, n), generator=g) * 4).to(torch.float8_e5m2).view(torch.uint8).numpy()
    gpu_packed = fo.prepack_b_for_scaled_mm(torch.from_numpy(codes).cuda().view(torch.float8_e5m2))
    ref_packed = torch.from_numpy(oracle.prepack(codes)).cuda().view(torch.float8_e5m2)
    out1 = fo.scaled_mm_hip(a, gpu_packed, None, None, torch.float16)
    out2 = fo.scaled_mm_hip(a, ref_packed, None, None, torch.float16)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
