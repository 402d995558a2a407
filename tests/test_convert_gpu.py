"""GPU parity of `feather_ops.bf16_to_fp16` (reference: feather_ops/convert.py:24-34, tests/test_convert.py)
and of `feather_ops::widen_bf16`, the round-to-nearest-even widening the auto path runs ahead of the
fp16-activation kernel for bf16 activations (naive.py:21's `a.to(torch.float16)`).

The HIP kernels (csrc/convert.hip) against the oracle's round-toward-zero and round-to-nearest-even
conversions, bit for bit: every bf16 code, the reference test's shapes (tests/test_convert.py:7-11) with its
own torch comparison, and lengths whose last elements take the kernel's 16-byte and scalar tails.
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


_RNE_TABLE = None


def _rne_table() -> np.ndarray:
    global _RNE_TABLE
    if _RNE_TABLE is None:
        _RNE_TABLE = oracle.widen_bf16_to_f16(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    return _RNE_TABLE


def _check_bits(x: torch.Tensor, y: torch.Tensor, nearest: bool = False) -> None:
    want = _rne_table()[bits_of(x)] if nearest else oracle.bf16_to_f16_rtz(bits_of(x))
    got = bits_of(y)
    nan = np.isnan(want.view(np.float16).astype(np.float32))
    assert np.array_equal(np.isnan(got.view(np.float16).astype(np.float32)), nan)
    assert np.array_equal(got >> 15, want >> 15)  # NaNs keep their sign too
    bad = np.nonzero((got != want) & ~nan)[0]
    assert bad.size == 0, [(hex(int(bits_of(x).ravel()[i])), hex(int(got.ravel()[i])), hex(int(want.ravel()[i])))
                           for i in bad[:8]]


def _widen(x: torch.Tensor) -> torch.Tensor:
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    torch.ops.feather_ops.widen_bf16.default(x, out)
    return out


_CONVERTERS = {"rtz": lambda fo, x: fo.bf16_to_fp16(x), "rne": lambda fo, x: _widen(x)}


@pytest.mark.parametrize("mode", sorted(_CONVERTERS))
def test_every_bf16_code(fo, mode):
    codes = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).cuda()
    out = _CONVERTERS[mode](fo, codes)
    assert out.dtype == torch.float16 and out.shape == codes.shape
    _check_bits(codes, out, mode == "rne")


@pytest.mark.parametrize("mode", sorted(_CONVERTERS))
@pytest.mark.parametrize("shape", [(1024, 1024), (257, 512), (1, 4096)])
def test_reference_shapes(fo, shape, mode):
    torch.manual_seed(0)
    x = torch.randn(shape, dtype=torch.bfloat16, device="cuda")
    y = _CONVERTERS[mode](fo, x)
    # the reference test's own comparison (tests/test_convert.py:20)
    torch.testing.assert_close(y, x.to(torch.float16), rtol=0, atol=1e-5)
    _check_bits(x, y, mode == "rne")


@pytest.mark.parametrize("mode", sorted(_CONVERTERS))
@pytest.mark.parametrize("n", [2, 6, 8192, 8192 * 2, 8002, 2048 * 7 + 4, 8 * 40001 + 2])
def test_lengths_reaching_the_scalar_tail(fo, n, mode):
    """A block converts 8192 elements with 4 16-byte loads per work-item; the last, partial block takes
    16-byte pieces and its last n % 8 elements (all of them, below 8) the per-element path. Values span every
    code region (subnormal rounding, overflow, inf, NaN) so each path sees each."""
    g = torch.Generator("cpu").manual_seed(n)
    codes = torch.randint(0, 65536, (n,), generator=g, dtype=torch.int32)
    codes[-min(n, 6):] = torch.tensor([0x0001, 0x3380, 0x7f7f, 0x7f80, 0xffc1, 0x8035], dtype=torch.int32)[-min(n, 6):]
    x = codes.to(torch.int16).view(torch.bfloat16).cuda()
    _check_bits(x, _CONVERTERS[mode](fo, x), mode == "rne")


def test_widening_is_the_kernels_own(fo):
    """The widened copy run on the fp16-activation kernel gives the bits of the bf16 kernel, which widens the
    same activations itself: same tile, bf16 output, extreme values included."""
    torch.manual_seed(1)
    m, n, k = 256, 512, 384
    a = (torch.randn((m, k), device="cuda") * 3000).to(torch.bfloat16)
    a[0, :6] = torch.tensor([70000.0, -1e-7, 6e-8, float("inf"), 1e-3, -65520.0], device="cuda").to(torch.bfloat16)
    w = (torch.randn((k, n), device="cuda") * 0.05).to(torch.float8_e5m2)
    packed = fo.prepack_b_for_scaled_mm(w)
    scale = torch.tensor(0.5, device="cuda")
    tile = (2, 2, 4, 4, 4, 1)
    in_place = fo.scaled_mm_hip(a, packed, scale, None, torch.bfloat16, tile=tile)
    widened = fo.scaled_mm_hip(_widen(a), packed, scale, None, torch.bfloat16, tile=tile)
    assert torch.equal(in_place.view(torch.int16), widened.view(torch.int16))


@pytest.mark.parametrize("mode", sorted(_CONVERTERS))
def test_c_abi_matches_the_op(fo, mode):
    """feather_bf16_to_fp16 / feather_widen_bf16 called through ctypes on torch-owned memory give the op's
    bits."""
    import ctypes

    from feather_ops import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    fn = lib.feather_widen_bf16 if mode == "rne" else lib.feather_bf16_to_fp16
    fn.restype = ctypes.c_bool
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    x = torch.randn(3, 1001 * 2, dtype=torch.bfloat16, device="cuda") * 1e5
    y = torch.empty(x.shape, dtype=torch.float16, device="cuda")
    assert fn(x.data_ptr(), y.data_ptr(), x.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), _CONVERTERS[mode](fo, x).view(torch.int16))
    _check_bits(x, y, mode == "rne")
