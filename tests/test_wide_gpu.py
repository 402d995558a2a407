"""GPU parity of the wide kernel (tile (2, 2, 4, 8, 8, 1): 256 x 256, 4 waves of 128 x 128, one workgroup per
CU) against the CPU oracle, and bit for bit against the ring kernel.

The wide kernel has two load paths, chosen per launch: shapes on its grid (M and N multiples of 256, K of 64)
take unmasked loads with the tile and stage in the scalar offset; every other shape masks each load's lanes.
Its epilogue has four forms (bias or not, per-tensor or per-column scale), each a separate code path. These
tests cover both load paths, all four epilogues, every dtype combination, grids of more than one round (more
tiles than CUs), split launches of both paths, and single-stage K. Each accumulator sums the same k order as
the ring kernel's, so the two must agree bit for bit as well as with the oracle.
"""

import pytest
import torch

from gpu_helpers import check_against_oracle, sample_rows

pytestmark = pytest.mark.gpu

WIDE = (2, 2, 4, 8, 8, 1)
RING = (1, 4, 4, 8, 4, 1)


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _tensor(shape, dtype, seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).cuda()


def _inputs(fo, m, n, k, a_dtype, b_dtype, seed=0):
    a = _tensor((m, k), a_dtype, seed=seed)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), b_dtype, seed=seed + 1))
    return a, bp


def _rows(m):
    return None if m <= 600 else sample_rows(m, n_random=24)


@pytest.mark.parametrize("m,n,k", [
    (512, 512, 256),      # on the grid: the unmasked path, 4 tiles
    (256, 4096, 1024),    # on the grid, one tile row
    (300, 264, 208),      # ragged M, N and K
    (257, 520, 2560),     # ragged M and N, K on the grid
    (512, 768, 80),       # M and N on the grid, ragged K (the masked path)
    (1, 256, 64),         # one row, one stage
    (513, 1000, 16),      # K of one chunk
])
@pytest.mark.parametrize("a_dtype,b_dtype,out_dtype", [
    (torch.float16, torch.float8_e5m2, torch.float16),
    (torch.bfloat16, torch.float8_e5m2, torch.bfloat16),
    (torch.float16, torch.float8_e4m3fn, torch.bfloat16),
    (torch.bfloat16, torch.float8_e4m3fn, torch.float16),
])
def test_wide_against_oracle_and_ring(fo, m, n, k, a_dtype, b_dtype, out_dtype):
    a, bp = _inputs(fo, m, n, k, a_dtype, b_dtype, seed=m + n + k)
    scale = torch.tensor(0.625, device="cuda")
    bias = _tensor((n,), out_dtype, seed=7)
    wide = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=WIDE)
    ring = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=RING)
    assert torch.equal(wide.view(torch.int16), ring.view(torch.int16))
    if k < 64 and out_dtype == torch.float16:
        # One fp16 rounding flip (an fp32 summation-order difference) is 2^-10 |y|, over the sqrt(K)-scaled
        # bound (6.3e-4 RMS at K = 16) wherever |y| > 0.64 RMS; with K this short the bf16-output combinations
        # (which accept such flips) and the equality with the ring kernel above carry the check.
        return
    check_against_oracle(wide, a, bp, scale, bias, rows=_rows(m))


@pytest.mark.parametrize("bias_on", [False, True])
@pytest.mark.parametrize("col_scale", [False, True])
@pytest.mark.parametrize("m,n,k", [(512, 512, 448), (264, 392, 528)])
def test_wide_epilogue_forms(fo, bias_on, col_scale, m, n, k):
    """The four epilogues (bias or not x per-tensor or per-column scale), on both load paths. bf16 output: per-
    column scales spread the outputs over a wide range, where one fp16 rounding flip of a large output would
    exceed the sqrt(K)-scaled bound at these K; the bf16 comparison accepts such flips (and equality with the
    ring kernel pins the bits)."""
    a, bp = _inputs(fo, m, n, k, torch.float16, torch.float8_e5m2, seed=3)
    if col_scale:
        g = torch.Generator("cpu").manual_seed(5)
        scale = (torch.rand(n, generator=g) * 2 + 0.1).cuda()
    else:
        scale = torch.tensor(1.25, device="cuda")
    bias = _tensor((n,), torch.bfloat16, seed=9) if bias_on else None
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=WIDE)
    ring = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=RING)
    assert torch.equal(out.view(torch.int16), ring.view(torch.int16))
    check_against_oracle(out, a, bp, scale, bias)


def test_wide_no_scale_no_bias(fo):
    a, bp = _inputs(fo, 256, 512, 128, torch.float16, torch.float8_e5m2)
    out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=WIDE)
    check_against_oracle(out, a, bp, None, None)


@pytest.mark.parametrize("m,n,k", [
    (4096, 12288, 3072),   # C3: 768 tiles, three rounds
    (4352, 4608, 1024),    # 17 x 18 = 306 tiles: a full round and a partial one
    (4100, 4104, 576),     # ragged, 17 x 17 tiles
])
def test_wide_multi_round_grids(fo, m, n, k):
    a, bp = _inputs(fo, m, n, k, torch.float16, torch.float8_e5m2, seed=11)
    scale = torch.tensor(0.02, device="cuda")
    out = fo.scaled_mm_hip(a, bp, scale, None, torch.float16, tile=WIDE)
    ring = fo.scaled_mm_hip(a, bp, scale, None, torch.float16, tile=RING)
    assert torch.equal(out.view(torch.int16), ring.view(torch.int16))
    check_against_oracle(out, a, bp, scale, None, rows=sample_rows(m, n_random=16))


@pytest.mark.parametrize("m,n,k,splits", [
    (512, 512, 2048, 4),   # on the grid
    (300, 264, 1040, 3),   # ragged: the last split holds the partial stage
    (256, 256, 128, 2),    # one stage per split
])
def test_wide_split_k(fo, m, n, k, splits):
    """Split launches of the wide tile (partial sums joined through the workspace) on both load paths; fp32
    summation order differs from the unsplit launch, so the check is against the oracle's bound."""
    a, bp = _inputs(fo, m, n, k, torch.float16, torch.float8_e5m2, seed=13)
    scale = torch.tensor(0.5, device="cuda")
    bias = _tensor((n,), torch.bfloat16, seed=4)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=WIDE, splits=splits)
    check_against_oracle(out, a, bp, scale, bias)
    again = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=WIDE, splits=splits)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))  # deterministic join


def test_wide_nan_inf_propagate(fo):
    """Non-finite activations and weight codes reach the outputs they touch, as in the oracle."""
    m, n, k = 256, 256, 128
    a = _tensor((m, k), torch.float16)
    a[3, 5] = float("inf")
    a[77, 64] = float("nan")
    b = _tensor((k, n), torch.float8_e5m2, seed=1)
    b.view(torch.uint8)[9, 200] = 0x7C   # +inf
    b.view(torch.uint8)[100, 17] = 0x7E  # NaN
    bp = fo.prepack_b_for_scaled_mm(b)
    s = torch.tensor(1.0, device="cuda")
    out = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=WIDE)
    check_against_oracle(out, a, bp, s, None)
