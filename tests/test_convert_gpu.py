"""GPU parity of `feather_ops.bf16_to_fp16` (reference: feather_ops/convert.py:24-34, tests/test_convert.py).

The HIP kernel (csrc/convert.hip) against the oracle's round-toward-zero conversion, bit for bit: every
bf16 code, the reference test's shapes (tests/test_convert.py:7-11) with its own torch comparison, and
lengths whose last elements take the kernel's scalar tail (n % 8 != 0).
"""

import numpy as np
import pytest
import torch

from gpu_helpers import bits_of
from oracle import naive as oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _check_bits(x: torch.Tensor, y: torch.Tensor) -> None:
    want = oracle.bf16_to_f16_rtz(bits_of(x))
    got = bits_of(y)
    nan = np.isnan(want.view(np.float16).astype(np.float32))
    assert np.array_equal(np.isnan(got.view(np.float16).astype(np.float32)), nan)
    assert np.array_equal(got >> 15, want >> 15)  # NaNs keep their sign too
    bad = np.nonzero((got != want) & ~nan)[0]
    assert bad.size == 0, [(hex(int(bits_of(x).ravel()[i])), hex(int(got.ravel()[i])), hex(int(want.ravel()[i])))
                           for i in bad[:8]]


def test_every_bf16_code(fo):
    codes = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).cuda()
    out = fo.bf16_to_fp16(codes)
    assert out.dtype == torch.float16 and out.shape == codes.shape
    _check_bits(codes, out)


@pytest.mark.parametrize("shape", [(1024, 1024), (257, 512), (1, 4096)])
def test_reference_shapes(fo, shape):
    torch.manual_seed(0)
    x = torch.randn(shape, dtype=torch.bfloat16, device="cuda")
    y = fo.bf16_to_fp16(x)
    # the reference test's own comparison (tests/test_convert.py:20)
    torch.testing.assert_close(y, x.to(torch.float16), rtol=0, atol=1e-5)
    _check_bits(x, y)


@pytest.mark.parametrize("n", [2, 6, 8002, 2048 * 7 + 4, 8 * 40001 + 2])
def test_lengths_reaching_the_scalar_tail(fo, n):
    """The last n % 8 elements (or all of them, below 8) take the per-element path; values span every code
    region (subnormal truncation, saturation, inf, NaN) so both paths see each."""
    g = torch.Generator("cpu").manual_seed(n)
    codes = torch.randint(0, 65536, (n,), generator=g, dtype=torch.int32)
    codes[-min(n, 6):] = torch.tensor([0x0001, 0x3380, 0x7f7f, 0x7f80, 0xffc1, 0x8035], dtype=torch.int32)[-min(n, 6):]
    x = codes.to(torch.int16).view(torch.bfloat16).cuda()
    _check_bits(x, fo.bf16_to_fp16(x))


def test_c_abi_matches_the_op(fo):
    """feather_bf16_to_fp16 called through ctypes on torch-owned memory gives the op's bits."""
    import ctypes

    from feather_ops import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    lib.feather_bf16_to_fp16.restype = ctypes.c_bool
    lib.feather_bf16_to_fp16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    x = torch.randn(3, 1001 * 2, dtype=torch.bfloat16, device="cuda") * 1e5
    y = torch.empty(x.shape, dtype=torch.float16, device="cuda")
    assert lib.feather_bf16_to_fp16(x.data_ptr(), y.data_ptr(), x.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), fo.bf16_to_fp16(x).view(torch.int16))
    _check_bits(x, y)
