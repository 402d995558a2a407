"""GPU parity of the wide kernel (tiles (2, 2, 4, 8, 8, 1): 256 x 256, 4 waves of 128 x 128, and (2, 2, 4, 8, 6, 1):
256 x 192, 4 waves of 128 x 96; one workgroup per CU) against the CPU oracle, and bit for bit against the ring
kernel.

The wide kernel has two load paths, chosen per launch: shapes on its grid (M a multiple of 256, N of the tile's
width, K of 64) take unmasked loads with the tile and stage in the scalar offset; every other shape masks each
load's lanes.
Its epilogue has four forms (bias or not, per-tensor or per-column scale), each a separate code path. These
tests cover both load paths, all four epilogues, every dtype combination, grids of more than one round (more
tiles than CUs), split launches of both paths, and single-stage K. Each accumulator sums the same k order as
the ring kernel's and both round through the same epilogue arithmetic, so the two must agree bit for bit as well
as with the oracle. A bias-only launch (zero activations) pins the epilogue's column mapping and the bias add
exactly, for both output types and both scale forms.
"""

import pytest
import torch

from gpu_helpers import check_against_oracle, sample_rows

pytestmark = pytest.mark.gpu

WIDE = (2, 2, 4, 8, 8, 1)
WIDE_192 = (2, 2, 4, 8, 6, 1)
WIDE_TILES = [WIDE, WIDE_192]
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


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
@pytest.mark.parametrize("m,n,k", [
    (512, 512, 256),      # on the 256 x 256 grid: the unmasked path, 4 tiles
    (512, 384, 256),      # on the 256 x 192 grid
    (256, 4608, 1024),    # on both grids, one tile row
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
def test_wide_against_oracle_and_ring(fo, tile, m, n, k, a_dtype, b_dtype, out_dtype):
    a, bp = _inputs(fo, m, n, k, a_dtype, b_dtype, seed=m + n + k)
    scale = torch.tensor(0.625, device="cuda")
    bias = _tensor((n,), out_dtype, seed=7)
    wide = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=tile)
    ring = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=RING)
    assert torch.equal(wide.view(torch.int16), ring.view(torch.int16))
    if k < 64 and out_dtype == torch.float16:
        # One fp16 rounding flip (an fp32 summation-order difference) is 2^-10 |y|, over the sqrt(K)-scaled
        # bound (6.3e-4 RMS at K = 16) wherever |y| > 0.64 RMS; with K this short the bf16-output combinations
        # (which accept such flips) and the equality with the ring kernel above carry the check.
        return
    check_against_oracle(wide, a, bp, scale, bias, rows=_rows(m))


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
@pytest.mark.parametrize("bias_on", [False, True])
@pytest.mark.parametrize("col_scale", [False, True])
@pytest.mark.parametrize("m,n,k", [(512, 768, 448), (264, 392, 528)])
def test_wide_epilogue_forms(fo, tile, bias_on, col_scale, m, n, k):
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
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile)
    ring = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=RING)
    assert torch.equal(out.view(torch.int16), ring.view(torch.int16))
    check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("col_scale", [False, True])
@pytest.mark.parametrize("n", [768, 776])
def test_wide_bias_lands_on_its_column(fo, tile, out_dtype, col_scale, n):
    """Zero activations: every output is round(0 * scale) + bias[col] = bias[col] exactly, so any column
    mix-up in the epilogue (which lanes hold which columns, which bias dword feeds which pair) shows. Biases
    are distinct small integers, exact in both output types; N = 776 takes the masked path."""
    m, k = 300, 64
    a = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=2))
    bias = (torch.arange(n, dtype=torch.float32) % 251 - 125).to(out_dtype).cuda()
    scale = (torch.rand(n) + 0.5).cuda() if col_scale else torch.tensor(1.5, device="cuda")
    out = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype, tile=tile)
    assert torch.equal(out, bias.expand(m, n))


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
def test_wide_no_scale_no_bias(fo, tile):
    a, bp = _inputs(fo, 256, 768, 128, torch.float16, torch.float8_e5m2)
    out = fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=tile)
    check_against_oracle(out, a, bp, None, None)


@pytest.mark.parametrize("tile,m,n,k", [
    (WIDE, 4096, 12288, 3072),      # C3: 768 tiles, three rounds
    (WIDE, 4352, 4608, 1024),       # 17 x 18 = 306 tiles: a full round and a partial one
    (WIDE, 4100, 4104, 576),        # ragged, 17 x 17 tiles
    (WIDE_192, 4096, 3072, 3072),   # C2's shape: 16 x 16 = 256 tiles, one round
    (WIDE_192, 4096, 9216, 1024),   # 16 x 48 = 768 tiles, three rounds
    (WIDE_192, 4100, 3080, 576),    # ragged, 17 x 17 tiles
])
def test_wide_multi_round_grids(fo, tile, m, n, k):
    a, bp = _inputs(fo, m, n, k, torch.float16, torch.float8_e5m2, seed=11)
    scale = torch.tensor(0.02, device="cuda")
    out = fo.scaled_mm_hip(a, bp, scale, None, torch.float16, tile=tile)
    ring = fo.scaled_mm_hip(a, bp, scale, None, torch.float16, tile=RING)
    assert torch.equal(out.view(torch.int16), ring.view(torch.int16))
    check_against_oracle(out, a, bp, scale, None, rows=sample_rows(m, n_random=16))


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
@pytest.mark.parametrize("m,n,k,splits", [
    (512, 768, 2048, 4),   # on both grids
    (300, 264, 1040, 3),   # ragged: the last split holds the partial stage
    (256, 768, 128, 2),    # one stage per split
])
def test_wide_split_k(fo, tile, m, n, k, splits):
    """Split launches of the wide tile (partial sums joined through the workspace) on both load paths; fp32
    summation order differs from the unsplit launch, so the check is against the oracle's bound."""
    a, bp = _inputs(fo, m, n, k, torch.float16, torch.float8_e5m2, seed=13)
    scale = torch.tensor(0.5, device="cuda")
    bias = _tensor((n,), torch.bfloat16, seed=4)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile, splits=splits)
    check_against_oracle(out, a, bp, scale, bias)
    again = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile, splits=splits)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))  # deterministic join


@pytest.mark.parametrize("tile", WIDE_TILES, ids=["256x256", "256x192"])
def test_wide_nan_inf_propagate(fo, tile):
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
    out = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile)
    check_against_oracle(out, a, bp, s, None)
