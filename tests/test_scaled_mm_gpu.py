"""GPU parity of `scaled_mm_hip` against the CPU oracle (reference tests: tests/test_scaled_mm_hip.py).

Same shapes, dtypes and tile sweep as the reference's tests (test_scaled_mm_hip.py:16-89), plus the
BASELINE configurations, edge cases (NaN/inf, subnormals, bf16 past fp16's range, N % 16 == 8), the
C ABI called directly, and determinism. Inputs are generated on the CPU with fixed seeds and copied to
the GPU; the oracle evaluates every row for small shapes and a fixed row sample for large ones.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import bits_of, check_against_oracle, sample_rows, to_dev_bits
from oracle import naive as oracle

pytestmark = pytest.mark.gpu

RTOL = 0.01
ATOL = {torch.float16: 2.0, torch.bfloat16: 16.0}

SHAPES = [  # (M, N, K), reference test_scaled_mm_hip.py:16-27
    (1, 128, 128),
    (17, 96, 64),
    (128, 128, 128),
    (256, 256, 256),
    (512, 1024, 5120),
    (4111, 512, 256),
    (4112, 1152, 1152),
    (4304, 4304, 1152),
    (5376, 512, 3072),
    (2048, 1024, 5120),
]
TAIL_SHAPE = (67, 272, 304)
DTYPES = [(torch.float8_e5m2, torch.float16), (torch.float8_e5m2, torch.bfloat16),
          (torch.float8_e4m3fn, torch.bfloat16)]


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _tensor(shape, dtype, seed=0):
    """The reference's `_tensor` (randn -> dtype), drawn on the CPU so the oracle sees the same bits."""
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).cuda()


def _ref_metric(out, a, b_prepacked, scale, bias, rows):
    """The reference's own bound (relative Frobenius <= 1%, max-abs <= ATOL), on the oracle."""
    from gpu_helpers import oracle_ref

    ref = oracle.bits_to_f32(oracle_ref(a, b_prepacked, scale, bias, out.dtype, rows=rows),
                             oracle.BF16 if out.dtype == torch.bfloat16 else oracle.F16).astype(np.float64)
    got = out.float().cpu().numpy()[rows if rows is not None else slice(None)].astype(np.float64)
    diff = np.abs(got - ref)
    rel = np.linalg.norm(diff) / max(np.linalg.norm(ref), 1e-6)
    return rel, diff.max()


def _rows_for(M, N, K):
    return None if M * N * K <= (1 << 27) else sample_rows(M)


@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b_dtype,out_dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_shapes(fo, a_dtype, b_dtype, out_dtype, shape):
    M, N, K = shape
    a = _tensor((M, K), a_dtype)
    b = _tensor((K, N), b_dtype, seed=1)
    scale = torch.tensor(2.34, device="cuda", dtype=torch.float32)
    bias = _tensor((N,), out_dtype, seed=2)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype)
    rows = _rows_for(M, N, K)
    rel, max_abs = _ref_metric(out, a, bp, scale, bias, rows)
    assert rel <= RTOL, f"rel={rel:.3g}"
    assert max_abs <= ATOL[out_dtype], f"max_abs={max_abs:.3g}"
    check_against_oracle(out, a, bp, scale, bias, rows=rows)


def _all_tiles():
    from feather_ops.tiles import SCALED_MM_TILES

    return SCALED_MM_TILES


@pytest.mark.parametrize("tile", _all_tiles())
def test_every_tile(fo, tile):
    M, N, K = TAIL_SHAPE
    a = _tensor((M, K), torch.float16)
    b = _tensor((K, N), torch.float8_e5m2, seed=1)
    scale = torch.tensor(0.75, device="cuda", dtype=torch.float32)
    bias = _tensor((N,), torch.bfloat16, seed=2)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile)
    check_against_oracle(out, a, bp, scale, bias)


@pytest.mark.parametrize("tile", _all_tiles())
def test_every_tile_bf16_in_fp16_out_n_mod_16_is_8(fo, tile):
    M, N, K = 33, 200, 160
    a = _tensor((M, K), torch.bfloat16)
    b = _tensor((K, N), torch.float8_e5m2, seed=1)
    bp = fo.prepack_b_for_scaled_mm(b)
    out = fo.scaled_mm_hip(a, bp, torch.tensor(0.5, device="cuda"), None, torch.float16, tile=tile)
    check_against_oracle(out, a, bp, torch.tensor(0.5), None)


def test_scale_and_bias_are_optional(fo):
    a = _tensor((96, 64), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((64, 128), torch.float8_e5m2, seed=1))
    out = fo.scaled_mm_hip(a, bp, None, None, torch.float16)
    check_against_oracle(out, a, bp, None, None)


def test_heuristic_matches_a_measured_tile(fo):
    a = _tensor((4112, 1152), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((1152, 1152), torch.float8_e5m2, seed=1))
    scale = torch.tensor(1.5, device="cuda", dtype=torch.float32)
    out = fo.scaled_mm_hip(a, bp, scale, None, torch.bfloat16)
    check_against_oracle(out, a, bp, scale, None, rows=sample_rows(4112))


@pytest.mark.parametrize("tile,m,n,splits,deep", [
    ((1, 4, 4, 4, 2, 1), 200, 3000, 1, True),      # 4 x 24 tiles: the deep ring
    ((1, 4, 4, 4, 2, 1), 4160, 1032, 1, False),    # 65 x 9 = 585 tiles: more than 512, the shallow ring
    ((2, 2, 4, 2, 2, 1), 130, 1000, 1, True),
    ((2, 2, 4, 2, 2, 1), 4160, 1032, 1, False),    # 65 x 17 = 1105 tiles: more than 1024
    ((1, 4, 4, 4, 2, 1), 200, 3000, 4, True),      # 96 tiles x 4 splits
    ((1, 4, 4, 4, 2, 1), 1040, 4104, 2, False),    # 17 x 33 tiles x 2 splits = 1122 workgroups
    ((2, 2, 4, 2, 2, 1), 2112, 1032, 2, False),    # 33 x 17 tiles x 2 splits = 1122 workgroups
    ((2, 2, 4, 2, 2, 1), 48, 3000, 3, True),       # bf16 activations too: M <= 64, two column waves
])
@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
def test_deep_and_shallow_ring_variants(fo, tile, m, n, splits, deep, a_dtype):
    """A 64-row ring tile runs its deep-ring instantiation on grids whose workgroups are all resident at once
    and the shallow one beyond, split or not; each against the oracle, bf16 activations included (the
    register-staged path)."""
    from feather_ops.tiles import ring_is_deep

    assert ring_is_deep(m, n, tile, splits) == deep
    if a_dtype == torch.bfloat16:
        deep = ring_is_deep(m, n, tile, splits, a_bf16=True)
    K = 1040
    a = _tensor((m, K), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, n), torch.float8_e4m3fn, seed=1))
    s = torch.tensor(0.25, device="cuda")
    bias = _tensor((n,), torch.bfloat16, seed=2)
    out = fo.scaled_mm_hip(a, bp, s, bias, torch.bfloat16, tile=tile, splits=splits)
    check_against_oracle(out, a, bp, s, bias, rows=None if m < 1000 else sample_rows(m, n_random=16))


# Workgroup counts per launch, and the schedules they get with bf16 activations and in split launches
# (unsplit launches with fp16 activations take reads first everywhere):
@pytest.mark.parametrize("tile,n_tiles,splits", [
    ((2, 2, 4, 4, 8, 1), 132, 1),   # 4 x 132 = 528 workgroups: a full round of 512 reads first, the 16 after it
                                    # (one per CU) interleaved, in one launch
    ((2, 2, 4, 4, 8, 1), 100, 1),   # 400: a partial round that pairs blocks on some CUs, all reads first
    ((2, 2, 4, 4, 8, 1), 60, 1),    # 240: at most one block per CU, all interleaved
    ((1, 4, 4, 8, 4, 1), 132, 1),   # the same block as 128 x 64 waves (reads first with fp16 activations only)
    ((2, 2, 4, 4, 4, 1), 194, 1),   # 776: a full round of 768 (three per CU) reads first, 8 interleaved
    ((2, 2, 4, 4, 4, 1), 150, 1),   # 600: some CUs hold three, all reads first
    ((2, 2, 4, 4, 4, 1), 100, 1),   # 400: at most two per CU, all interleaved
    ((2, 2, 4, 4, 4, 1), 97, 2),    # 776 split workgroups: 768 reads first, 8 interleaved, fp16 included
])
@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
def test_ring_operand_schedules(fo, tile, n_tiles, splits, a_dtype):
    """The ring kernel's two operand-read schedules (reads first on CUs holding the tile's full complement
    of blocks, interleaved elsewhere, chosen per workgroup by the launcher from the grid): grids of 512
    rows whose workgroup counts put the launch on one, the other or both, against the oracle on a row of
    every 16-row fragment (so every tile, tail rounds included)."""
    m, K = 512, 384                       # 4 row tiles, 6 stages: one period of both rings
    bn = 16 * tile[1] * tile[4]
    n = bn * n_tiles
    a = _tensor((m, K), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, n), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.5, device="cuda")
    out_dtype = a_dtype
    bias = _tensor((n,), out_dtype, seed=2)
    out = fo.scaled_mm_hip(a, bp, s, bias, out_dtype, tile=tile, splits=splits)
    rows = np.array(sorted({16 * f + (7 * f) % 16 for f in range(m // 16)} | {0, m - 1}), dtype=np.int64)
    check_against_oracle(out, a, bp, s, bias, rows=rows)


# One cell per regime of the fitted heuristic (skinny split-K with 16/32/64 columns and 4/8 slices, split
# across workgroups for long K, the 32-row streaming tile, the 64-row ring tiles for 16 < M <= 64 with a
# big weight, split or not, the 64 x 64 ring tile for mid-size grids, and the
# wave-quantization choice among 128 x 128 / 128 x 256): the auto path on the tile it picks, bf16 in and out
# with a bias, against the oracle.
HEURISTIC_CELLS = [
    (2, 2048, 16384),    # 16 x 32 streaming tile split 4 ways along K across workgroups
    (2, 4096, 16384),    # 16 x 16 streaming tile unsplit, three fetches in flight per wave
    (16, 5120, 13824),   # 16 x 64 streaming tile, 4 slices, split 3 ways
    (1, 17408, 4096),    # 16 x 32 columns: 64-column blocks would leave a small second round
    (16, 4096, 4096),    # 16 x 16 columns, 8 slices
    (16, 6144, 6144),    # 16 x 32 columns
    (32, 25600, 2048),   # 32-row streaming tile
    (20, 14336, 4096),   # 32-row streaming tile, one round of 224 blocks
    (32, 5120, 25600),   # 64 x 64 ring tile at 32 rows, split 6 ways along K (deep ring)
    (64, 16384, 4096),   # 64 x 64 ring tile at 64 rows (deep ring), split 2 ways along K
    (52, 17408, 11264),  # 64 x 128 ring tile at 52 rows (more 64 x 64 tiles than CUs), split 3 ways
    (24, 65536, 2048),   # 64 x 128 ring tile at 24 rows (512 tiles), unsplit (bf16: split 2 ways)
    (1, 96768, 2688),    # 64 x 128 ring tile at one row, an LM-head width (756 tiles)
    (128, 1024, 5120),   # 16-row tile, 8 row blocks
    (128, 4096, 14336),  # 64 x 128 ring tile split 8 ways (56 MiB weight, 32 tiles of 128 x 128)
    (128, 5120, 5120),   # 64 x 128 ring tile split 3 ways (80 tiles -> 240 workgroups)
    (256, 12288, 4096),  # 64 x 128 ring tile split 2 ways (384 tiles: the small-grid time model)
    (448, 6144, 8192),   # 64 x 128 ring tile split 3 ways, 1008 workgroups on the shallow ring
    (256, 12288, 8192),  # 128 x 128 ring tile split 4 ways, 768 workgroups (48 MiB of partial sums)
    (1040, 1024, 5120),  # 64 x 128 ring tile split 3 ways
    (2304, 1280, 1280),  # 64 x 64 ring tile
    (1000, 1000, 2560),  # 64 x 64 ring tile split 2 ways (M > 768, 256 tiles, ragged M and N)
    (4112, 1024, 5120),  # 64 x 128 ring tile, one partial wave
    (512, 1024, 1024),   # 32-row streaming tile (fp16), 4-slice streaming tile (bf16)
    (384, 1280, 4096),   # 32-row streaming tile past 256 rows (fp16)
    (512, 2048, 1024),   # 32-row streaming tile, two rounds of 256 blocks (fp16)
    (160, 1024, 8192),   # 16 x 64, 8 slices of unroll 1 (fp16) / 4 slices of unroll 2 (bf16): deep K
    (128, 2048, 8192),   # the same deep-K streaming tiles at 128 rows
    (80, 1024, 16384),   # 4-slice streaming tile split 3 ways (few ring tiles: not a ring split)
    (4096, 3072, 3072),  # 256 x 192 wide tile, one round of 256 (bf16 activations: widened first)
    (9216, 2048, 2048),  # 128 x 128 (one full wave of blocks)
    (2320, 6144, 6144),  # 128 x 256 (bf16 activations: widened first, then 128 x 64 waves)
    (2048, 8192, 2048),  # 128 x 256 (bf16 activations: widened first, then 128 x 64 waves)
]


@pytest.mark.parametrize("a_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", HEURISTIC_CELLS)
def test_heuristic_regimes(fo, m, n, k, a_dtype):
    """The picks depend on the activation dtype (bf16 ones take the small-grid ring tiles later), so each
    cell runs the auto path with both."""
    from feather_ops.scaled_mm import _auto_choice

    a = _tensor((m, k), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    scale = torch.tensor(0.75, device="cuda", dtype=torch.float32)
    bias = _tensor((n,), torch.bfloat16, seed=2)
    out = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16)
    tile, splits, widen = _auto_choice(m, n, k, a_dtype)
    rows = None if m * n * k <= (1 << 28) else sample_rows(m, n_random=16)
    res = check_against_oracle(out, a, bp, scale, bias, rows=rows)
    print(f"{m}x{n}x{k} tile {tile}/{splits}{' widened first' if widen else ''}: max_abs={res['max_abs']:.4g} "
          f"bound={res['bound']:.4g}")


def test_bf16_widened_first_replays_in_a_graph(fo):
    """The widen-first auto path captured in a HIP graph (the fp16 copy comes from the graph's pool) replays the
    eager result, re-reading the activations each replay: they change between replays, with eager work and
    synchronizations in between."""
    from feather_ops.scaled_mm import _auto_choice

    m, n, k = 2048, 8192, 2048
    assert _auto_choice(m, n, k, torch.bfloat16)[2]
    a = _tensor((m, k), torch.bfloat16)
    inputs = [_tensor((m, k), torch.bfloat16, seed=s) for s in (3, 4, 5)]
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.5, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16)
    for x in inputs + inputs[:1]:
        a.copy_(x)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        want = fo.scaled_mm_hip(x, bp, s, None, torch.bfloat16)  # eager work in between
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(2048, 8192, 2048), (2320, 6144, 6144), (4096, 12288, 3072), (32, 11264, 11264),
                                   (32, 5120, 25600)])
def test_bf16_widened_first_is_bit_identical(fo, m, n, k):
    """Where the auto path widens bf16 activations first and runs the fp16-activation kernel, its output is the
    bits of the in-place widening on the same tile and split count (the C ABI's only bf16 form), bias and
    per-column scale included: the 128 x 256 block and, at 32 rows, the 64 x 64 deep ring split 4 and 6
    ways."""
    from feather_ops.scaled_mm import _auto_choice

    tile, splits, widen = _auto_choice(m, n, k, torch.bfloat16)
    assert widen
    a = _tensor((m, k), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    bias = _tensor((n,), torch.bfloat16, seed=2)
    for scale in (torch.tensor(0.75, device="cuda"), torch.rand(n, device="cuda") + 0.5):
        auto = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16)
        in_place = fo.scaled_mm_hip(a, bp, scale, bias, torch.bfloat16, tile=tile, splits=splits)
        assert torch.equal(auto.view(torch.int16), in_place.view(torch.int16))


def _random_cases(count: int = 16, seed: int = 11, rows=(1, 7, 16, 40, 77, 300, 1000, 2048, 4097, 9000)):
    """Seeded shapes across the heuristic's regimes (M 1-9000, N and K multiples of 8 and 16 up to 14336), each
    with its activation dtype, weight format, output dtype, bias and scale form."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        m = int(rng.choice(rows))
        n = int(rng.integers(1, 14336 // 8 + 1)) * 8
        k = int(rng.integers(1, 14336 // 16 + 1)) * 16
        if m * n * k > (1 << 37) or m * k > (1 << 25):
            continue
        cases.append((m, n, k, bool(rng.integers(2)), bool(rng.integers(2)), bool(rng.integers(2)),
                      bool(rng.integers(2)), int(rng.integers(3))))
    return cases


# the second batch: M 65-512, where the streaming tiles (32-row, deep-K, split) and the split ring tiles meet
@pytest.mark.parametrize("m,n,k,a_bf16,e5m2,out_bf16,has_bias,scale_mode",
                         _random_cases() + _random_cases(12, 23, (80, 96, 128, 160, 200, 256, 320, 384, 448, 512)))
def test_random_shapes_auto_path(fo, m, n, k, a_bf16, e5m2, out_bf16, has_bias, scale_mode):
    """The whole auto path (tile, split count and, for bf16 activations, the widening pass) on seeded random
    shapes and argument forms, against the oracle on sampled rows."""
    from feather_ops.scaled_mm import _auto_choice

    a_dtype = torch.bfloat16 if a_bf16 else torch.float16
    out_dtype = torch.bfloat16 if out_bf16 else torch.float16
    a = _tensor((m, k), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2 if e5m2 else torch.float8_e4m3fn, seed=1))
    bias = _tensor((n,), out_dtype, seed=2) if has_bias else None
    scale = [None, torch.tensor(0.75, device="cuda"), torch.rand(n, device="cuda") + 0.25][scale_mode]
    out = fo.scaled_mm_hip(a, bp, scale, bias, out_dtype)
    res = check_against_oracle(out, a, bp, scale, bias, rows=sample_rows(m, n_random=8))
    tile, splits, widen = _auto_choice(m, n, k, a_dtype)
    print(f"{m}x{n}x{k} {tile}/{splits}{' widened' if widen else ''}: max_abs={res['max_abs']:.4g} "
          f"bound={res['bound']:.4g}")


# ---- BASELINE configurations (north-star recipe) -----------------------------------------------------------

CONFIGS = {
    "C1": (256, 1024, 1024, oracle.F16, False),
    "C2": (4096, 3072, 3072, oracle.BF16, False),
    "C3": (4096, 3072, 12288, oracle.F16, False),
    "C4": (16, 4096, 14336, oracle.F16, False),
    "C5_1_1000": (1, 2560, 1000, oracle.BF16, True),
    "C5_1_5120": (1, 2560, 5120, oracle.BF16, True),
    "C5_77_1000": (77, 2560, 1000, oracle.BF16, True),
    "C5_77_5120": (77, 2560, 5120, oracle.BF16, True),
    "C5_1000_1000": (1000, 2560, 1000, oracle.BF16, True),
    "C5_1000_5120": (1000, 2560, 5120, oracle.BF16, True),
    "C5_4097_1000": (4097, 2560, 1000, oracle.BF16, True),
    "C5_4097_5120": (4097, 2560, 5120, oracle.BF16, True),
}


def _log_parity(record: dict) -> None:
    """Append one configuration's strict north-star outcome to $FEATHER_PARITY_LOG (JSON lines), if set."""
    import json
    import os

    path = os.environ.get("FEATHER_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(record) + "\n")


@pytest.mark.parametrize("name", list(CONFIGS))
def test_baseline_config(fo, name):
    """Every output of the configuration against the oracle (the C oracle takes a few seconds on the host's
    cores even at C3), with the strict north-star result recorded: max|out - ref|, the bound, how many
    elements are over it and how many of those are one output ulp from the oracle."""
    m, k, n, a_fmt, outliers = CONFIGS[name]
    a_bits, packed, scale, _ = oracle.make_inputs(m, k, n, a_fmt, seed=0, outliers=outliers)
    a = to_dev_bits(a_bits, torch.bfloat16 if a_fmt == oracle.BF16 else torch.float16, "cuda")
    bp = to_dev_bits(packed, torch.float8_e5m2, "cuda")
    s = torch.tensor(scale, dtype=torch.float32, device="cuda")
    out_dtype = torch.bfloat16 if a_fmt == oracle.BF16 else torch.float16
    out = fo.scaled_mm_hip(a, bp, s, None, out_dtype)
    from feather_ops.scaled_mm import _auto_choice

    # the launch the auto path made: with widen first, the tile is the fp16-activation pick it ran
    tile, splits, widen = _auto_choice(m, n, k, a.dtype)
    res = check_against_oracle(out, a, bp, s, None, rows=None)
    _log_parity({"config": name, "M": m, "K": k, "N": n, "a": a_fmt, "out": str(out_dtype).split(".")[-1],
                 "outliers": outliers, "tile": list(tile), "splits": splits, "widened_first": widen,
                 "rows_checked": m,
                 "max_abs": res["max_abs"], "rms": res["rms"], "bound": res["bound"], "strict_ok": res["strict_ok"],
                 "n_over": res["n_over"], "n_over_one_ulp": res["n_over_one_ulp"],
                 "n_band_flips": res.get("n_band_flips", 0), "n": res["n"]})
    print(f"{name}: max_abs={res['max_abs']:.4g} bound={res['bound']:.4g} over={res['n_over']} of {res['n']}")
    # every output, against a torch fp32 reference of the same op on the GPU (upcast, fp32 matmul, scale)
    b_dec = bp.permute(0, 2, 1).reshape(-1, n)[:k].to(torch.float32)
    ref = ((a.to(torch.float16).float() @ b_dec) * s).to(out_dtype)
    full = oracle.compare(bits_of(out), bits_of(ref), oracle.BF16 if out_dtype == torch.bfloat16 else oracle.F16, k)
    assert full["nan_ok"] and full["inf_ok"]
    assert full["n_over"] == full["n_over_one_ulp"] and full["n_over"] <= max(2, 1e-3 * full["n"]), full


# ---- edge cases --------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fp8,specials", [(torch.float8_e5m2, (0x7C, 0x7E)),      # +inf, NaN
                                          (torch.float8_e4m3fn, (0x7F, 0xFF))])   # the two NaN codes
@pytest.mark.parametrize("tile", [None, (2, 2, 4, 4, 4, 1), (8, 1, 4, 1, 4, 0)])
def test_specials_propagate_like_the_oracle(fo, fp8, specials, tile):
    g = torch.Generator("cpu").manual_seed(9)
    a = torch.randn(20, 64, generator=g).to(torch.float16)
    a[3, 5] = float("inf")
    a[7, 9] = float("nan")
    codes = torch.randn(64, 24, generator=g).to(fp8).view(torch.uint8)
    codes[11, 4] = specials[0]
    codes[13, 17] = specials[1]
    bp = fo.prepack_b_for_scaled_mm(codes.view(fp8).cuda())
    for out_dtype in (torch.float16, torch.bfloat16):
        out = fo.scaled_mm_hip(a.cuda(), bp, torch.tensor(0.5, device="cuda"), None, out_dtype, tile=tile)
        check_against_oracle(out, a.cuda(), bp, torch.tensor(0.5), None)
        assert torch.isnan(out[:, 17]).all()


def test_bf16_activation_past_fp16_range_becomes_inf_like_naive(fo):
    g = torch.Generator("cpu").manual_seed(10)
    a = torch.randn(16, 32, generator=g).to(torch.bfloat16)
    a[2, 0] = 70000.0  # fp16(70000) = inf under naive.py:21
    bp = fo.prepack_b_for_scaled_mm(torch.randn(32, 16, generator=g).to(torch.float8_e5m2).cuda())
    out = fo.scaled_mm_hip(a.cuda(), bp, None, None, torch.bfloat16)
    assert not torch.isfinite(out[2]).any()
    check_against_oracle(out, a.cuda(), bp, None, None)


def test_subnormal_weights_and_activations(fo):
    g = torch.Generator("cpu").manual_seed(11)
    a = (torch.randn(32, 64, generator=g) * 1e-6).to(torch.float16)
    codes = torch.randint(0, 4, (64, 32), generator=g, dtype=torch.uint8) | (
        torch.randint(0, 2, (64, 32), generator=g, dtype=torch.uint8) << 7)
    bp = fo.prepack_b_for_scaled_mm(codes.view(torch.float8_e5m2).cuda())
    s = torch.tensor(2.0**20, device="cuda")
    out = fo.scaled_mm_hip(a.cuda(), bp, s, None, torch.float16)
    check_against_oracle(out, a.cuda(), bp, s.cpu(), None)


@pytest.mark.parametrize("tile", [None, (2, 2, 4, 4, 4, 1), (8, 1, 4, 1, 4, 0)])
def test_bf16_output_subnormals_and_rounding(fo, tile):
    """bf16 outputs round to nearest even through the whole fp32 range: a scale of 2^-130 puts the results
    among bf16's subnormals, where a flush to zero or a truncation would show."""
    g = torch.Generator("cpu").manual_seed(12)
    a = torch.randn(40, 256, generator=g).to(torch.float16)
    bp = fo.prepack_b_for_scaled_mm(torch.randn(256, 72, generator=g).to(torch.float8_e5m2).cuda())
    for s in (2.0**-130, 2.0**-120, 0.37):
        scale = torch.tensor(s, device="cuda")
        out = fo.scaled_mm_hip(a.cuda(), bp, scale, None, torch.bfloat16, tile=tile)
        check_against_oracle(out, a.cuda(), bp, scale, None)
        if s == 2.0**-130:
            assert (out != 0).float().mean().item() > 0.9  # not flushed


def test_e4m3fn_all_codes(fo):
    k = 256
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(k, 1).repeat(1, 16)
    codes[codes & 0x7F == 0x7F] = 0x38  # NaN codes checked in test_specials; keep the sums finite here
    a = torch.eye(k, dtype=torch.float16)
    bp = fo.prepack_b_for_scaled_mm(codes.view(torch.float8_e4m3fn).cuda())
    out = fo.scaled_mm_hip(a.cuda(), bp, None, None, torch.float16)
    check_against_oracle(out, a.cuda(), bp, None, None)


@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("tile", [(2, 2, 4, 4, 4, 1), (2, 2, 4, 2, 2, 1), (8, 1, 4, 1, 4, 0), (4, 1, 4, 1, 1, 0)])
def test_decode_is_exact_on_every_finite_code(fo, fp8, tile):
    """An identity activation copies the decoded weight to the output (one product per element, exact in
    fp32 and in the fp16 output), so the output must equal torch's fp8 -> fp16 cast for every finite code,
    in the ring and the streaming kernel alike: the same fp16 value (so the same bits, except that the
    -0 code sums to +0 with the other rows' zero products)."""
    k = 256
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(k, 1).repeat(1, 16)
    special = 0x7F if fp8 == torch.float8_e4m3fn else 0x7C
    codes[codes & special == special] = 0x38  # inf / NaN codes would poison every row through 0 * x
    w = codes.view(fp8)
    a = torch.eye(k, dtype=torch.float16).cuda()
    out = fo.scaled_mm_hip(a, fo.prepack_b_for_scaled_mm(w.cuda()), None, None, torch.float16, tile=tile)
    want = w.to(torch.float16)
    assert torch.equal(out.cpu(), want)
    nonzero = want != 0
    assert torch.equal(out.cpu().view(torch.int16)[nonzero], want.view(torch.int16)[nonzero])


@pytest.mark.parametrize("tile,m,n,k,splits", [
    ((4, 1, 4, 1, 4, 0), 16, 2048, 2048, 1),     # streaming tile, one tile row
    ((8, 1, 4, 1, 2, 0), 2, 1024, 8192, 2),      # streaming tile split across workgroups
    ((2, 2, 4, 2, 2, 0), 32, 1024, 1040, 1),     # 32-row streaming tile
    ((2, 2, 4, 2, 2, 1), 48, 3000, 1040, 1),     # 64-row ring tile, deep ring
    ((1, 4, 4, 4, 2, 1), 64, 3000, 2048, 4),     # 64 x 128 ring tile, deep ring, split 4 ways
    ((2, 2, 4, 2, 2, 1), 40, 70400, 1040, 1),    # 1100 tiles: the shallow ring
    ((2, 2, 4, 4, 4, 1), 100, 2048, 1040, 1),    # 128-row tile: no non-temporal variant
    ((4, 1, 4, 1, 4, 0), 40, 2048, 1040, 1),     # three tile rows: the default loads
])
@pytest.mark.parametrize("a_dtype", [torch.float16, torch.bfloat16])
def test_weight_streaming_modes_are_bit_identical(fo, tile, m, n, k, splits, a_dtype):
    """Non-temporal weight loads are a cache hint: every mode returns the same bits, on every kernel that has
    the variant (streaming and 64-row ring tiles, split or not, deep or shallow ring) and on launches that
    keep the default loads; the "on" output also against the oracle."""
    a = _tensor((m, k), a_dtype)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.25, device="cuda")
    bias = _tensor((n,), a_dtype, seed=2)
    previous = fo.set_weight_streaming("on")
    try:
        on = fo.scaled_mm_hip(a, bp, s, bias, a_dtype, tile=tile, splits=splits)
        fo.set_weight_streaming("off")
        off = fo.scaled_mm_hip(a, bp, s, bias, a_dtype, tile=tile, splits=splits)
        fo.set_weight_streaming("auto")
        auto = fo.scaled_mm_hip(a, bp, s, bias, a_dtype, tile=tile, splits=splits)
    finally:
        fo.set_weight_streaming(previous)
    assert torch.equal(on.view(torch.int16), off.view(torch.int16))
    assert torch.equal(auto.view(torch.int16), off.view(torch.int16))
    check_against_oracle(on, a, bp, s, bias, rows=None if m * n <= (1 << 20) else sample_rows(m, n_random=16))


def test_deterministic(fo):
    a = _tensor((300, 512), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((512, 1000), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.01, device="cuda")
    first = fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16)
    for tile in [None, (4, 1, 4, 1, 4, 0)]:
        x = fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16, tile=tile)
        y = fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16, tile=tile)
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert torch.equal(first.view(torch.int16), fo.scaled_mm_hip(a, bp, s, None, torch.bfloat16).view(torch.int16))


def test_c_abi_direct(fo):
    """launch_scaled_mm through ctypes on torch-owned device memory matches the torch op bit for bit."""
    from feather_ops import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    lib.launch_scaled_mm.restype = ctypes.c_bool
    lib.launch_scaled_mm.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_void_p]
    M, N, K = 100, 256, 320
    a = _tensor((M, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.3, device="cuda")
    bias = _tensor((N,), torch.float16, seed=2)
    want = fo.scaled_mm_hip(a, bp, s, bias, torch.float16, tile=(2, 2, 4, 4, 4, 1))
    c = torch.empty_like(want)
    ok = lib.launch_scaled_mm(a.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(), M, N, K, 1, 1,
                              True, True, False, 2, 2, 4, 4, 4, True, torch.cuda.current_stream().cuda_stream)
    assert ok
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), want.view(torch.int16))
    # an uninstantiated tile is refused and enqueues nothing
    assert not lib.launch_scaled_mm(a.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(), M, N, K,
                                    1, 1, True, True, False, 3, 3, 3, 3, 3, True,
                                    torch.cuda.current_stream().cuda_stream)


def test_op_rejects_bad_inputs(fo):
    a = _tensor((16, 64), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((64, 32), torch.float8_e5m2, seed=1))
    with pytest.raises(RuntimeError, match="Unsupported config"):
        fo.scaled_mm_hip(a, bp, None, None, torch.float16, tile=(3, 3, 3, 3, 3, 1))
    with pytest.raises(RuntimeError, match="K must be divisible by 16"):
        fo.scaled_mm_hip(a[:, :40], bp, None, None, torch.float16)
    with pytest.raises(RuntimeError, match="scale must be float32"):
        fo.scaled_mm_hip(a, bp, torch.tensor(1.0, device="cuda", dtype=torch.float16), None, torch.float16)
    with pytest.raises(RuntimeError, match="bias must have the same dtype as c"):
        fo.scaled_mm_hip(a, bp, None, torch.zeros(32, device="cuda", dtype=torch.bfloat16), torch.float16)


# The reference's compile shapes (tests/test_scaled_mm_hip_compile.py:7), plus one the heuristic splits K on
# (512 x 5376 x 5120: 128 x 128 tiles, 3 ways) and one whose bf16 activations the auto path widens first
# (2048 x 8192 x 2048: the pass inside the custom op, then the 128 x 64-wave tile).
@pytest.mark.parametrize("m,n,k", [(4112, 1152, 1152), (512, 1024, 5120), (512, 5376, 5120), (2048, 8192, 2048)])
def test_compile_matches_eager(fo, m, n, k):
    """Reference tests/test_scaled_mm_hip_compile.py: one opaque node, eager == compiled."""
    for dynamic in (False, True):
        a = _tensor((m, k), torch.bfloat16)
        bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=1))
        s = torch.tensor(2.34, device="cuda")
        bias = _tensor((n,), torch.bfloat16, seed=2)

        def run(a, bp, s, bias):
            return fo.scaled_mm_hip(a, bp, s, bias, torch.bfloat16)

        eager = run(a, bp, s, bias)
        compiled = torch.compile(run, fullgraph=True, dynamic=dynamic)(a, bp, s, bias)
        assert torch.equal(compiled.view(torch.int16), eager.view(torch.int16))


def test_compiled_graph_holds_the_opaque_auto_op(fo):
    """Under torch.compile the auto path is the custom op `feather_ops::scaled_mm_auto` (one node, the
    heuristic not traced into the graph), while eager calls skip the op's Python dispatch."""
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    a = _tensor((64, 256), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((256, 128), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.5, device="cuda")
    torch._dynamo.reset()
    out = torch.compile(lambda a, bp, s: fo.scaled_mm_hip(a, bp, s, None, torch.float16), backend=backend,
                        fullgraph=True)(a, bp, s)
    targets = [node.target for gm in graphs for node in gm.graph.nodes if node.op == "call_function"]
    assert torch.ops.feather_ops.scaled_mm_auto.default in targets, targets
    assert not any("scaled_mm.default" in str(t) and "auto" not in str(t) for t in targets)
    assert torch.equal(out.view(torch.int16), fo.scaled_mm_hip(a, bp, s, None, torch.float16).view(torch.int16))


# ---- empty and maximum sizes ----------------------------------------------------------------------------------

def test_empty_m_returns_an_empty_output(fo):
    """M = 0 (an empty batch): every entry point returns a [0, N] output and launches nothing."""
    bp = fo.prepack_b_for_scaled_mm(_tensor((256, 128), torch.float8_e5m2, seed=1))
    a = torch.empty((0, 256), dtype=torch.float16, device="cuda")
    for kwargs in ({}, {"tile": (2, 2, 4, 4, 4, 1)}, {"tile": (8, 1, 4, 1, 4, 0)},
                   {"tile": (2, 2, 4, 4, 4, 1), "splits": 2}):
        out = fo.scaled_mm_hip(a, bp, torch.tensor(1.0, device="cuda"), None, torch.bfloat16, **kwargs)
        assert out.shape == (0, 128) and out.dtype == torch.bfloat16
    torch.cuda.synchronize()


def test_output_just_under_2_gib(fo):
    """The largest output the 31-bit buffer offsets allow: 65528 x 16384 fp16 (2,147,221,504 bytes), checked
    on its first, last and sampled rows; one more row block is refused with the reference's message."""
    M, N, K = 65528, 16384, 256
    a = _tensor((M, K), torch.float16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.05, device="cuda")
    out = fo.scaled_mm_hip(a, bp, s, None, torch.float16)
    check_against_oracle(out, a, bp, s, None, rows=sample_rows(M, n_random=16))
    del out
    torch.cuda.empty_cache()
    a2 = _tensor((M + 8, K), torch.float16)
    with pytest.raises(RuntimeError, match="smaller than 2 GiB"):
        fo.scaled_mm_hip(a2, bp, s, None, torch.float16)


def test_long_k(fo):
    """K = 262144 (4096 stages of 64, a 256 MiB prepacked weight) through the ring and streaming kernels."""
    K, N = 262144, 1024
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    s = torch.tensor(0.02, device="cuda")
    for m, tile in ((200, (2, 2, 4, 4, 4, 1)), (16, (8, 1, 4, 1, 4, 0))):
        a = _tensor((m, K), torch.float16)
        out = fo.scaled_mm_hip(a, bp, s, None, torch.float16, tile=tile)
        check_against_oracle(out, a, bp, s, None, rows=sample_rows(m, n_random=8))


def test_split_k_at_the_maximum_split_count(fo):
    M, N, K = 130, 264, 2048  # 32 stages of 64: 32 splits of one stage each
    a = _tensor((M, K), torch.bfloat16)
    bp = fo.prepack_b_for_scaled_mm(_tensor((K, N), torch.float8_e5m2, seed=1))
    bias = _tensor((N,), torch.bfloat16, seed=2)
    out = fo.scaled_mm_hip(a, bp, None, bias, torch.bfloat16, tile=(2, 2, 4, 4, 4, 1), splits=32)
    check_against_oracle(out, a, bp, None, bias)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tile,m", [
    ((4, 1, 4, 1, 4, 0), 16),     # streaming, 64 columns: the row-piece join
    ((2, 2, 4, 4, 2, 0), 64),     # streaming, 64 rows: the row-piece join
    ((8, 1, 4, 1, 1, 0), 16),     # streaming, 16 columns: the per-fragment join
    ((1, 4, 4, 8, 4, 1), 300),    # ring
    ((2, 2, 4, 8, 8, 1), 300),    # wide 256 x 256
    ((2, 2, 4, 8, 6, 1), 300),    # wide 256 x 192
])
def test_bias_at_an_8_byte_offset(fo, tile, m, out_dtype):
    """The contract asks only 8-byte alignment of the bias: a bias view starting 8 bytes into its buffer (not 16-byte
    aligned) gives the same bits as an aligned copy, on every epilogue form."""
    n, k = 776, 512
    a = _tensor((m, k), torch.float16, seed=3)
    bp = fo.prepack_b_for_scaled_mm(_tensor((k, n), torch.float8_e5m2, seed=4))
    s = torch.tensor(0.5, device="cuda")
    buf = _tensor((n + 4,), out_dtype, seed=5)
    bias = buf[4:]
    assert bias.data_ptr() % 16 == 8
    shifted = fo.scaled_mm_hip(a, bp, s, bias, out_dtype, tile=tile)
    aligned = fo.scaled_mm_hip(a, bp, s, bias.clone(), out_dtype, tile=tile)
    assert torch.equal(shifted.view(torch.int16), aligned.view(torch.int16))
    check_against_oracle(aligned, a, bp, s, bias.clone())
