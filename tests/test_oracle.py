"""Pins the CPU oracle (oracle/) before anything is checked against it. CPU only.

Each oracle function is checked against something that does not share its code: torch's casts (the
library routines the reference's naive path calls), the reference's known-answer list, brute-force loops,
closed forms, and golden fixtures computed from torch casts plus float64 numpy matmul
(tests/golden/make_golden.py). The last tests plant mistakes in the oracle's inputs and check that the
goldens catch them.
"""

import hashlib
import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import naive as oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _golden():
    data = np.load(GOLDEN / "golden.npz", allow_pickle=False)
    cases = {}
    for key in data.files:
        case, field = key.split("/")
        cases.setdefault(case, {})[field] = data[key]
    return cases


CASES = _golden()


def _same_bits(x_f32: np.ndarray, y_f32: np.ndarray) -> bool:
    """Equal values, NaN matching NaN."""
    x = np.asarray(x_f32, dtype=np.float32)
    y = np.asarray(y_f32, dtype=np.float32)
    nan = np.isnan(x)
    return bool(np.array_equal(nan, np.isnan(y)) and np.array_equal(x[~nan], y[~nan]))


# ---- element casts ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,dtype", [(oracle.E5M2, torch.float8_e5m2), (oracle.E4M3FN, torch.float8_e4m3fn)])
def test_fp8_decode_all_codes_match_torch(fmt, dtype):
    codes = np.arange(256, dtype=np.uint8)
    mine = oracle.decode_fp8(codes, fmt)
    theirs = torch.from_numpy(codes).view(dtype).to(torch.float32).numpy()
    assert _same_bits(mine, theirs)
    # signs of zero survive too
    assert np.signbit(mine[0x80]) and not np.signbit(mine[0x00])


def test_e5m2_decode_matches_reference_known_answers():
    kat = json.loads((GOLDEN / "e5m2_kat.json").read_text())
    for code, value in kat.items():
        assert oracle.decode_fp8(np.array([int(code, 16)], np.uint8))[0] == value


def test_e5m2_decode_is_the_high_byte_of_fp16():
    """The byte move the kernel uses (csrc/hip_kernel.cu:95-102 in the reference) gives the same value."""
    codes = np.arange(256, dtype=np.uint16)
    as_f16 = (codes << 8).astype(np.uint16).view(np.float16).astype(np.float32)
    assert _same_bits(oracle.decode_fp8(codes.astype(np.uint8)), as_f16)


def test_e4m3fn_special_values():
    d = oracle.decode_fp8(np.array([0x7F, 0xFF, 0x7E, 0x01, 0x08, 0x00], np.uint8), oracle.E4M3FN)
    assert np.isnan(d[0]) and np.isnan(d[1])
    assert d[2] == 448.0 and d[3] == 2.0**-9 and d[4] == 2.0**-6 and d[5] == 0.0


def test_bf16_widening_all_codes_match_torch():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mine = oracle.widen_bf16_to_f16(codes)
    theirs = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).to(torch.float16).view(torch.int16).numpy()
    mine_f = mine.view(np.float16).astype(np.float32)
    theirs_f = theirs.view(np.uint16).view(np.float16).astype(np.float32)
    assert _same_bits(mine_f, theirs_f)
    finite = np.isfinite(mine_f)
    assert np.array_equal(mine[finite], theirs.view(np.uint16)[finite])  # bit-exact incl. signed zeros


def test_bf16_to_f16_rtz_all_codes():
    """The reference's bf16_to_fp16 (round toward zero, convert.py:6-21) on every bf16 code, split by what
    pins each region: torch's cast where fp16 holds the value exactly (every rounding mode agrees there),
    saturation to +-65504 past fp16's range, inf/NaN passed through, and the truncation closed form in
    fp16's subnormal range."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mine = oracle.bf16_to_f16_rtz(codes)
    with np.errstate(invalid="ignore"):  # signalling-NaN codes
        x = (codes.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    mine_f = mine.view(np.float16).astype(np.float64)
    sign = np.signbit(x)
    assert np.array_equal(np.signbit(mine_f), sign)  # the sign survives everywhere, zeros and NaNs included

    nan = np.isnan(x)
    assert np.array_equal(np.isnan(mine_f), nan)
    inf = np.isinf(x)
    assert np.array_equal(np.isinf(mine_f), inf)

    finite = ~nan & ~inf
    big = finite & (np.abs(x) > 65504.0)
    assert big.sum() > 0 and np.all(np.abs(mine_f[big]) == 65504.0)

    normal = finite & (np.abs(x) >= 2.0**-14) & (np.abs(x) <= 65504.0)
    torch_f16 = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).to(torch.float16)
    theirs = torch_f16.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine[normal], theirs[normal])
    assert np.array_equal(mine_f[normal], x[normal])  # exact: bf16's 8-bit significand fits fp16's 11

    small = finite & (np.abs(x) < 2.0**-14)
    want = np.trunc(np.abs(x[small]) * 2.0**24) * 2.0**-24  # multiples of the subnormal quantum, toward 0
    assert np.array_equal(np.abs(mine_f[small]), want)
    # the region is not trivial: some codes truncate to a non-zero subnormal, some round down a step that RNE
    # would round up, and everything under 2^-24 becomes zero
    assert (want > 0).sum() > 100
    rne = torch_f16.numpy().astype(np.float64)
    assert (np.abs(rne[small]) > want).sum() > 50
    assert np.all(mine_f[finite & (np.abs(x) < 2.0**-24)] == 0.0)
    assert normal.sum() + small.sum() + big.sum() + nan.sum() + inf.sum() == 65536


def test_bf16_to_f16_rtz_catches_a_rounding_mistake():
    """A planted mistake (round to nearest instead of toward zero) fails the subnormal closed form."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):  # signalling-NaN codes
        x = (codes.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    small = np.isfinite(x) & (np.abs(x) < 2.0**-14)
    wrong = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).to(torch.float16).numpy()
    want = np.trunc(np.abs(x[small]) * 2.0**24) * 2.0**-24
    assert not np.array_equal(np.abs(wrong.astype(np.float64)[small]), want)


def _cast_sweep():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.normal(size=20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65519.99, 65520.0, -65520.0, 1e30, np.inf, -np.inf, np.nan,
                  2.0**-24, 2.0**-25, 3 * 2.0**-26, 2.0**-14, 2.0**-14 - 2.0**-25, 1.0 + 2.0**-11,
                  1.0 + 3 * 2.0**-11, 1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 3.4e38, 1e-40], dtype=np.float32),
    ])
    # exact ties for both formats
    m = rng.integers(1024, 2048, 500)
    x = np.concatenate([x, ((m * 2 + 1) * 2.0 ** rng.integers(-20, 4, 500) / 2048).astype(np.float32)])
    return x.astype(np.float32)


def test_f32_to_f16_rne_matches_torch():
    x = _cast_sweep()
    mine = oracle.f32_to_f16(x).view(np.float16).astype(np.float32)
    theirs = torch.from_numpy(x).to(torch.float16).to(torch.float32).numpy()
    assert _same_bits(mine, theirs)


def test_f32_to_bf16_rne_matches_torch():
    x = _cast_sweep()
    mine = oracle.bits_to_f32(oracle.f32_to_bf16(x), oracle.BF16)
    theirs = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert _same_bits(mine, theirs)


# ---- layout ----------------------------------------------------------------------------------------------

@pytest.mark.parametrize("k,n", [(16, 8), (20 * 16, 3), (128, 24), (130 * 16, 5)])
def test_prepack_brute_force(k, n):
    rng = np.random.default_rng(k * 31 + n)
    b = rng.integers(0, 256, size=(k, n), dtype=np.uint8)
    p = oracle.prepack(b)
    k_pad = -(-k // 128) * 128
    assert p.shape == (k_pad // 16, n, 16)
    for kk in range(k_pad):
        for nn in range(n):
            assert p[kk // 16, nn, kk % 16] == (b[kk, nn] if kk < k else 0)
    assert np.array_equal(oracle.unpack(p, k), b)


def test_prepack_matches_golden_loops():
    for case in CASES.values():
        if "packed" in case:
            assert np.array_equal(oracle.prepack(case["b_codes"]), case["packed"])


def test_product_prepack_matches_oracle_on_cpu():
    """feather_ops.prepack_b_for_scaled_mm is device-agnostic torch code; check it on CPU tensors."""
    from feather_ops.scaled_mm import prepack_b_for_scaled_mm

    rng = np.random.default_rng(3)
    for k, n in [(16, 8), (272, 304), (1024, 40)]:
        b = rng.integers(0, 256, size=(k, n), dtype=np.uint8)
        got = prepack_b_for_scaled_mm(torch.from_numpy(b).view(torch.float8_e5m2)).view(torch.uint8).numpy()
        assert np.array_equal(got, oracle.prepack(b))


# ---- the matmul: closed forms ----------------------------------------------------------------------------

def _f16(x):
    return torch.tensor(np.asarray(x, np.float32)).to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def test_identity_weight_returns_scaled_activations():
    k = 64
    rng = np.random.default_rng(0)
    a = _f16(rng.normal(size=(3, k)))
    b = np.zeros((k, k), np.uint8)
    b[np.arange(k), np.arange(k)] = 0x3C  # e5m2 1.0
    out = oracle.scaled_mm(a, oracle.F16, oracle.prepack(b), oracle.E5M2, 0.25, None, oracle.F16)
    want = (a.view(np.float16).astype(np.float32) * np.float32(0.25)).astype(np.float16).view(np.uint16)
    assert np.array_equal(out, want)


def test_single_nonzero_picks_one_product():
    k, n = 48, 24
    rng = np.random.default_rng(1)
    a = _f16(rng.normal(size=(5, k)))
    b = np.zeros((k, n), np.uint8)
    b[17, 11] = 0xBA  # -0.75
    out = oracle.scaled_mm(a, oracle.F16, oracle.prepack(b), oracle.E5M2, None, None, oracle.F16)
    af = a.view(np.float16).astype(np.float32)
    want = np.zeros((5, n), np.float32)
    want[:, 11] = af[:, 17] * np.float32(-0.75)
    assert np.array_equal(out.view(np.float16).astype(np.float32), want.astype(np.float16).astype(np.float32))


def test_zero_activations_give_bias():
    k, n = 32, 16
    b = np.random.default_rng(2).integers(0, 0x7B, size=(k, n), dtype=np.uint8)
    bias = _f16(np.linspace(-3, 3, n))
    out = oracle.scaled_mm(np.zeros((4, k), np.uint16), oracle.F16, oracle.prepack(b), oracle.E5M2, 3.0, bias,
                           oracle.F16)
    assert np.array_equal(out, np.broadcast_to(bias, (4, n)))


def test_power_of_two_scale_is_exact_and_linear():
    rng = np.random.default_rng(4)
    a = _f16(rng.normal(size=(6, 96)))
    b = torch.tensor(rng.normal(size=(96, 40)), dtype=torch.float32).to(torch.float8_e5m2).view(torch.uint8).numpy()
    p = oracle.prepack(b)
    y1 = oracle.scaled_mm_f32(a, oracle.F16, p, oracle.E5M2, 1.0)
    y8 = oracle.scaled_mm_f32(a, oracle.F16, p, oracle.E5M2, 8.0)
    assert np.array_equal(y1 * 8, y8)


def test_per_column_power_of_two_scales_scale_each_column():
    """Distinct power-of-two scales per output column (`naive.py:29-33`, bias_dim = 1): column n is
    exactly the unscaled column times scale[n]; a row/column mix-up would scale rows instead."""
    rng = np.random.default_rng(14)
    m, k, n = 7, 80, 24
    a = _f16(rng.normal(size=(m, k)))
    b = torch.tensor(rng.normal(size=(k, n)), dtype=torch.float32).to(torch.float8_e5m2).view(torch.uint8).numpy()
    p = oracle.prepack(b)
    col = np.exp2(rng.integers(-6, 7, size=n)).astype(np.float32)
    assert len(set(col.tolist())) > 4
    y1 = oracle.scaled_mm_f32(a, oracle.F16, p, oracle.E5M2, None)
    yc = oracle.scaled_mm_f32(a, oracle.F16, p, oracle.E5M2, col)
    assert np.array_equal(y1 * col[None, :], yc)
    assert not np.array_equal(yc, y1 * col[:m, None])  # the row-wise (bias_dim = 0) reading


def test_constant_column_scales_equal_the_per_tensor_scale():
    rng = np.random.default_rng(15)
    a_bits, packed, scale, _ = oracle.make_inputs(9, 144, 40, oracle.BF16, seed=3)
    bias = oracle.f32_to_bf16(rng.normal(size=40).astype(np.float32))
    one = oracle.scaled_mm(a_bits, oracle.BF16, packed, oracle.E5M2, scale, bias, oracle.BF16)
    vec = oracle.scaled_mm(a_bits, oracle.BF16, packed, oracle.E5M2, np.full(40, scale, np.float32), bias,
                           oracle.BF16)
    assert np.array_equal(one, vec)


def test_per_column_scale_brute_force_tiny():
    rng = np.random.default_rng(16)
    m, k, n = 2, 32, 8
    a = _f16(rng.normal(size=(m, k)))
    codes = rng.integers(0, 0x7B, size=(k, n), dtype=np.uint8)
    col = rng.uniform(0.01, 3.0, size=n).astype(np.float32)
    bias = _f16(rng.normal(size=n))
    out = oracle.scaled_mm(a, oracle.F16, oracle.prepack(codes), oracle.E5M2, col, bias, oracle.F16)
    af = a.view(np.float16).astype(np.float64)
    bf = (codes.astype(np.uint16) << 8).view(np.float16).astype(np.float64)
    for i in range(m):
        for j in range(n):
            s = sum(af[i, kk] * bf[kk, j] for kk in range(k))
            y = np.float16(np.float32(s) * col[j])
            y = np.float16(np.float32(y) + np.float32(bias.view(np.float16)[j]))
            assert out[i, j] == np.array([y]).view(np.uint16)[0]


def test_scale_of_the_wrong_length_is_refused():
    a = np.zeros((2, 16), np.uint16)
    p = oracle.prepack(np.zeros((16, 8), np.uint8))
    with pytest.raises(AssertionError):
        oracle.scaled_mm(a, oracle.F16, p, oracle.E5M2, np.ones(7, np.float32), None, oracle.F16)


def test_brute_force_float64_loops_tiny():
    rng = np.random.default_rng(5)
    m, k, n = 3, 32, 8
    a = _f16(rng.normal(size=(m, k)))
    codes = rng.integers(0, 0x7B, size=(k, n), dtype=np.uint8) | (rng.integers(0, 2, size=(k, n)) << 7).astype(np.uint8)
    bias = _f16(rng.normal(size=n))
    out = oracle.scaled_mm(a, oracle.F16, oracle.prepack(codes), oracle.E5M2, 0.1, bias, oracle.F16)
    af = a.view(np.float16).astype(np.float64)
    bf = codes.astype(np.uint16) << 8
    bf = bf.view(np.float16).astype(np.float64)
    for i in range(m):
        for j in range(n):
            s = 0.0
            for kk in range(k):
                s += af[i, kk] * bf[kk, j]
            y = np.float16(np.float32(s) * np.float32(0.1))
            y = np.float16(np.float32(y) + np.float32(bias.view(np.float16)[j]))
            assert out[i, j] == np.array([y]).view(np.uint16)[0]


def test_literal_fp16_accumulation_overflows_at_baseline_quantization():
    """Why the oracle accumulates in fp32: naive.py:20-23's fp16 matmul overflows on C1's recipe."""
    a_bits, packed, scale, b_codes = oracle.make_inputs(64, 1024, 256, oracle.F16, seed=0)
    a16 = a_bits.view(np.float16)
    b16 = (b_codes.astype(np.uint16) << 8).view(np.float16)
    literal = oracle.literal_fp16_scaled_mm(a16, b16, scale)
    assert np.isinf(literal).mean() > 0.5
    fp32 = oracle.scaled_mm_f32(a_bits, oracle.F16, packed, oracle.E5M2, scale)
    assert np.isfinite(fp32).all()


def _torch_bits(x):
    return x.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("out_fmt", [oracle.F16, oracle.BF16])
def test_torch_restatement_matches_the_oracle_on_c1(out_fmt):
    """The timed CPU baseline (torch CPU calls, fp32 accumulation in torch's matmul order) agrees with the
    exact-sum oracle on C1's recipe within the north-star bound (bf16: off by one ulp at most, where the bar
    is below an ulp), with a bias."""
    a_bits, packed, scale, _ = oracle.make_inputs(256, 1024, 1024, oracle.F16, seed=0)
    out_dt = torch.bfloat16 if out_fmt == oracle.BF16 else torch.float16
    bias = torch.randn(1024, generator=torch.Generator().manual_seed(3)).to(out_dt)
    a = torch.from_numpy(a_bits.view(np.int16)).view(torch.float16)
    bp = torch.from_numpy(packed).view(torch.float8_e5m2)
    got = oracle.scaled_mm_torch(a, bp, torch.tensor(scale), bias, out_dt)
    assert got.dtype == out_dt and got.shape == (256, 1024)
    ref = oracle.scaled_mm(a_bits, oracle.F16, packed, oracle.E5M2, scale, _torch_bits(bias), out_fmt)
    res = oracle.compare(_torch_bits(got), ref, out_fmt, 1024)
    if out_fmt == oracle.F16:
        assert res["strict_ok"], res
    else:
        assert res["nan_ok"] and res["inf_ok"] and res["n_over"] == res["n_over_one_ulp"], res


def test_torch_restatement_closed_form():
    """Small-integer activations and weights (0, +-1, +-2, +-4 as e5m2 codes) and a power-of-two scale: every
    partial sum is an integer under 2^11, exact in fp32 and in the fp16 output whatever the summation order,
    so the restatement must give the oracle's bits exactly; a transposed or mis-unpacked weight fails."""
    k, n, m = 160, 24, 8
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float16)
    values = np.array([0x00, 0x3C, 0x40, 0x44, 0xBC, 0xC0, 0xC4], np.uint8)  # 0, 1, 2, 4, -1, -2, -4
    codes = values[rng.integers(0, len(values), size=(k, n))]
    packed = oracle.prepack(codes)
    got = oracle.scaled_mm_torch(torch.from_numpy(a), torch.from_numpy(packed).view(torch.float8_e5m2),
                                 torch.tensor(0.5), None, torch.float16)
    ref = oracle.scaled_mm(a.view(np.uint16), oracle.F16, packed, oracle.E5M2, 0.5, None, oracle.F16)
    assert np.array_equal(_torch_bits(got), ref)
    assert np.count_nonzero(ref) > m * n // 2
    wrong = torch.from_numpy(oracle.prepack(np.ascontiguousarray(codes[::-1])))  # k order reversed
    bad = oracle.scaled_mm_torch(torch.from_numpy(a), wrong.view(torch.float8_e5m2), torch.tensor(0.5), None,
                                 torch.float16)
    assert not np.array_equal(_torch_bits(bad), ref)


# ---- the matmul: golden fixtures -------------------------------------------------------------------------

SMALL = [name for name, c in CASES.items() if "a_bits" in c]


def _run_case(case, a_bits=None, packed=None):
    meta = json.loads(str(case["meta"]))
    return oracle.scaled_mm(
        case["a_bits"] if a_bits is None else a_bits, meta["a_fmt"],
        case["packed"] if packed is None else packed, meta["b_fmt"], meta["scale"],
        case.get("bias"), meta["out_fmt"],
    ), meta


@pytest.mark.parametrize("name", SMALL)
def test_golden_small_cases_bit_exact(name):
    case = CASES[name]
    out, meta = _run_case(case)
    want = case["out"]
    got_f = oracle.bits_to_f32(out, meta["out_fmt"])
    want_f = oracle.bits_to_f32(want, meta["out_fmt"])
    assert _same_bits(got_f, want_f), name
    finite = np.isfinite(want_f)
    assert np.array_equal(out[finite], want[finite])


def test_golden_specials_have_nan_and_inf():
    out, meta = _run_case(CASES["specials_f16"])
    f = oracle.bits_to_f32(out, meta["out_fmt"])
    assert np.isnan(f).any() and np.isinf(f).any() and np.isfinite(f).any()
    out, meta = _run_case(CASES["bf16_overflow"])
    f = oracle.bits_to_f32(out, meta["out_fmt"])
    assert not np.isfinite(f[0]).any() and np.isfinite(f[1:]).all()


@pytest.mark.parametrize("name,outliers", [("c1_rows", False), ("c5_rows", True)])
def test_golden_baseline_rows(name, outliers):
    case = CASES[name]
    meta = json.loads(str(case["meta"]))
    a_bits, packed, scale, _ = oracle.make_inputs(meta["m"], meta["k"], meta["n"], meta["a_fmt"], seed=meta["seed"],
                                                  outliers=outliers)
    assert hashlib.sha256(a_bits.tobytes()).hexdigest() == meta["a_sha256"], "input recipe drifted"
    assert hashlib.sha256(packed.tobytes()).hexdigest() == meta["packed_sha256"], "input recipe drifted"
    assert math.isclose(scale, meta["scale"], rel_tol=0, abs_tol=0)
    out = oracle.scaled_mm(a_bits, meta["a_fmt"], packed, oracle.E5M2, scale, None, meta["out_fmt"],
                           rows=case["rows"], threads=4)
    assert np.array_equal(out, case["out"])


# ---- planted mistakes: the goldens must catch them ----------------------------------------------------------

def test_golden_catches_a_transposed_weight():
    case = CASES["tiny_f16"]
    codes = case["b_codes"]  # [48, 24]: swap the column order as a transposition would scramble it
    wrong = oracle.prepack(np.ascontiguousarray(codes[:, ::-1]))
    out, _ = _run_case(case, packed=wrong)
    assert not np.array_equal(out, case["out"])


def test_golden_catches_a_dropped_k_term():
    case = CASES["tiny_bf16_bf16out"]
    a = case["a_bits"].copy()
    a[:, 63] = 0  # drop the last k term
    out, _ = _run_case(case, a_bits=a)
    assert not np.array_equal(out, case["out"])


def test_golden_catches_a_wrong_chunk_order():
    case = CASES["noscale_k80"]
    p = case["packed"].copy()
    p[[0, 1]] = p[[1, 0]]  # swap two 16-deep k chunks of the prepack
    out, _ = _run_case(case, packed=p)
    assert not np.array_equal(out, case["out"])


def test_compare_metric_flags_one_ulp_and_masks():
    ref = oracle.f32_to_bf16(np.array([3.0, 1.0, 0.5, -2.5], np.float32))
    out = ref.copy()
    out[0] += 1  # one bf16 ulp at 3.0 = 2^-6
    res = oracle.compare(out, ref, oracle.BF16, k=64)
    assert res["n_over"] == 1 and res["n_over_one_ulp"] == 1 and not res["strict_ok"]
    out2 = ref.copy()
    out2[1] = 0x7FC0  # NaN where the reference is finite
    assert not oracle.compare(out2, ref, oracle.BF16, k=64)["nan_ok"]


def test_band_brackets_the_answer_and_collapses_at_zero():
    a_bits, packed, scale, _ = oracle.make_inputs(32, 512, 256, oracle.BF16, seed=3)
    ref = oracle.scaled_mm(a_bits, oracle.BF16, packed, oracle.E5M2, scale, None, oracle.BF16)
    lo0, hi0 = oracle.scaled_mm_band(a_bits, oracle.BF16, packed, oracle.E5M2, scale, None, oracle.BF16, 0.0)
    assert np.array_equal(lo0, ref) and np.array_equal(hi0, ref)
    lo, hi = oracle.scaled_mm_band(a_bits, oracle.BF16, packed, oracle.E5M2, scale, None, oracle.BF16, 0.05)
    f = lambda x: oracle.bits_to_f32(x, oracle.BF16)  # noqa: E731
    assert (f(lo) <= f(ref)).all() and (f(ref) <= f(hi)).all() and (f(lo) < f(hi)).any()
