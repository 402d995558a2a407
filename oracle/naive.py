"""CPU oracle for `scaled_mm_hip`. TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` import this module, and
only as the checker. The product path (`feather_ops.scaled_mm_hip` -> `feather_ops::scaled_mm` ->
`launch_scaled_mm`) never imports it and has no CPU fallback.

It restates `feather_ops/naive.py:4-41` (`scaled_mm_naive`) and `feather_ops/scaled_mm.py:137-150`
(`prepack_b_for_scaled_mm`) of the reference, with the accumulation widened to fp32 as the target
semantics require (the literal fp16 accumulation of `naive.py:20-23` overflows at a per-tensor
quantization scale). The arithmetic lives in `scaled_mm_oracle.c` (built by `oracle/Makefile`); this file
holds the layout functions, the input recipe and the comparison metric.

What pins each function (tests/test_oracle.py):
- `decode_fp8` (C `oracle_e5m2_to_f32`, `oracle_e4m3fn_to_f32`): all 256 codes against torch's
  float8 -> float32 casts (a library routine) and against the known-answer list the reference holds at
  `cpp_benchmarks/benchmark_scaled_mm_hip.cpp:129-139` (committed as `tests/golden/e5m2_kat.json`).
- `f32_to_f16` / `f32_to_bf16` / `widen_bf16_to_f16` (C RNE casts): every bf16 code and a 1M-value sweep
  against torch's `.to()` casts (RNE library routines), plus hand-picked ties and overflows.
- `prepack` / `unpack`: brute force on tiny shapes against the index formula and the golden prepack
  fixture, the round trip through `naive.py:13-16`'s unpack, and zero pad rows.
- `scaled_mm` (C `oracle_scaled_mm`): closed forms (identity weight, one non-zero, zero activations,
  power-of-two scales), brute-force float64 loops on tiny inputs, and golden fixtures computed by float64
  `numpy.matmul` on the decoded operands (`tests/golden/make_golden.py`), chosen non-square and
  non-symmetric so that a transposed operand, a dropped k term or a wrong scale/bias order fails. The
  per-output-column scale (`naive.py:29-33`) is pinned by distinct power-of-two column scales (exact:
  column n equals the unscaled column times scale[n], so a row/column mix-up fails), by a constant vector
  agreeing bit for bit with the per-tensor scale, and by float64 loops on tiny inputs.
- `bf16_to_f16_rtz` (C `oracle_bf16_to_f16_rtz`, the reference's `convert.py:6-21`): all 65,536 bf16
  codes against torch's fp16 cast where fp16 holds the value exactly (there every rounding mode agrees),
  +-65504 for every finite code past fp16's range, inf and NaN passed through, and in fp16's subnormal
  range against the closed form trunc(|x| * 2^24) * 2^-24 with x's sign, evaluated in float64.
- `scaled_mm_band`: the same core as `scaled_mm` evaluated at the fp32 value -/+ delta; pinned by the
  answer at delta = 0 (itself pinned by the goldens) and by monotonicity (lo <= answer <= hi) on a
  seeded bf16 cell.
- `scaled_mm_torch` (torch CPU calls, used only as bench.py's timed CPU baseline): against `scaled_mm` on
  C1's seeded inputs within the north-star bound, and bit for bit on a power-of-two closed form.
- `literal_fp16_scaled_mm`: the reference's fp16-accumulate form, pinned by the same closed forms; it is
  only used to show the overflow that rules it out as an oracle at BASELINE's quantization.
"""

from __future__ import annotations

import ctypes
import math
import os
import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_lib = None

E5M2 = "e5m2"
E4M3FN = "e4m3fn"
F16 = "fp16"
BF16 = "bf16"


def build(force: bool = False) -> pathlib.Path:
    """Compile the C oracle with `make` (gcc, OpenMP)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-C", str(_HERE), "-B" if force else "all"], check=True, capture_output=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        u16p = ctypes.POINTER(ctypes.c_uint16)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        i64 = ctypes.c_int64
        lib.oracle_scaled_mm.argtypes = [
            u16p, ctypes.c_int, u8p, ctypes.c_int, i64, i64, i64,
            ctypes.POINTER(ctypes.c_float), i64, u16p, ctypes.c_int, u16p,
            ctypes.POINTER(ctypes.c_int64), i64, ctypes.c_int,
        ]
        lib.oracle_scaled_mm.restype = None
        lib.oracle_scaled_mm_f32.argtypes = [
            u16p, ctypes.c_int, u8p, ctypes.c_int, i64, i64, i64,
            ctypes.POINTER(ctypes.c_float), i64, ctypes.POINTER(ctypes.c_float),
            ctypes.POINTER(ctypes.c_int64), i64, ctypes.c_int,
        ]
        lib.oracle_scaled_mm_f32.restype = None
        lib.oracle_scaled_mm_band.argtypes = [
            u16p, ctypes.c_int, u8p, ctypes.c_int, i64, i64, i64,
            ctypes.POINTER(ctypes.c_float), i64, u16p, ctypes.c_int, ctypes.c_float, u16p, u16p,
            ctypes.POINTER(ctypes.c_int64), i64, ctypes.c_int,
        ]
        lib.oracle_scaled_mm_band.restype = None
        lib.oracle_prepack.argtypes = [u8p, i64, i64, u8p]
        lib.oracle_prepack.restype = None
        for name in ("oracle_e5m2_to_f32", "oracle_e4m3fn_to_f32"):
            getattr(lib, name).argtypes = [ctypes.c_uint8]
            getattr(lib, name).restype = ctypes.c_float
        for name in ("oracle_f16_to_f32", "oracle_bf16_to_f32"):
            getattr(lib, name).argtypes = [ctypes.c_uint16]
            getattr(lib, name).restype = ctypes.c_float
        for name in ("oracle_f32_to_f16_rne", "oracle_f32_to_bf16_rne"):
            getattr(lib, name).argtypes = [ctypes.c_float]
            getattr(lib, name).restype = ctypes.c_uint16
        lib.oracle_bf16_to_f16_rtz.argtypes = [ctypes.c_uint16]
        lib.oracle_bf16_to_f16_rtz.restype = ctypes.c_uint16
        _lib = lib
    return _lib


def _ptr(arr: np.ndarray, ctype):
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


# ---- element casts (scalar C functions, vectorised here) -------------------------------------------------

def decode_fp8(codes: np.ndarray, fmt: str = E5M2) -> np.ndarray:
    """fp8 codes (uint8) -> float32 values."""
    lib = _load()
    fn = lib.oracle_e5m2_to_f32 if fmt == E5M2 else lib.oracle_e4m3fn_to_f32
    table = np.array([fn(c) for c in range(256)], dtype=np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    lib = _load()
    flat = np.asarray(bits, dtype=np.uint16).ravel()
    return np.array([lib.oracle_f16_to_f32(int(b)) for b in flat], dtype=np.float32).reshape(np.shape(bits))


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> fp16 bits, RNE."""
    lib = _load()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.oracle_f32_to_f16_rne(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, RNE."""
    lib = _load()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.oracle_f32_to_bf16_rne(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


def widen_bf16_to_f16(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp16 bits with RNE (`naive.py:21` `a.to(torch.float16)`)."""
    lib = _load()
    flat = np.asarray(bits, dtype=np.uint16).ravel()
    out = [lib.oracle_f32_to_f16_rne(lib.oracle_bf16_to_f32(int(b))) for b in flat]
    return np.array(out, dtype=np.uint16).reshape(np.shape(bits))


def bf16_to_f16_rtz(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp16 bits with round-toward-zero (`convert.py:6-21`, `bf16_to_fp16`): C
    `oracle_bf16_to_f16_rtz`, evaluated once per distinct code."""
    lib = _load()
    table = np.array([lib.oracle_bf16_to_f16_rtz(c) for c in range(65536)], dtype=np.uint16)
    return table[np.asarray(bits, dtype=np.uint16)]


# ---- layout ----------------------------------------------------------------------------------------------

def k_padded(k: int) -> int:
    """K rounded up to a multiple of 128 (`scaled_mm.py:145`)."""
    return -(-k // 128) * 128


def prepack(b: np.ndarray) -> np.ndarray:
    """[K, N] fp8 codes -> [K_pad/16, N, 16] (`scaled_mm.py:137-150`), via the C index formula."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    k, n = b.shape
    out = np.empty((k_padded(k) // 16, n, 16), dtype=np.uint8)
    _load().oracle_prepack(_ptr(b, ctypes.c_uint8), k, n, _ptr(out, ctypes.c_uint8))
    return out


def unpack(packed: np.ndarray, k: int) -> np.ndarray:
    """[K_pad/16, N, 16] -> [K, N] (`naive.py:13-16`: permute(0, 2, 1).reshape(k * 16, N)[:K])."""
    kb, n, sixteen = packed.shape
    assert sixteen == 16
    return np.ascontiguousarray(packed.transpose(0, 2, 1).reshape(kb * 16, n)[:k])


# ---- the matmul ------------------------------------------------------------------------------------------

def _scales(scale, n: int) -> np.ndarray | None:
    """None, a python float (one per-tensor fp32 value) or N per-output-column values -> fp32 array."""
    if scale is None:
        return None
    sc = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)).ravel())
    assert sc.shape in ((1,), (n,)), f"scale must hold 1 or N={n} values, got {sc.shape}"
    return sc


def scaled_mm(a_bits: np.ndarray, a_fmt: str, packed: np.ndarray, b_fmt: str, scale,
              bias_bits: np.ndarray | None, out_fmt: str, rows: np.ndarray | None = None,
              threads: int = 0) -> np.ndarray:
    """`naive.py` semantics with fp32 accumulation; returns out-dtype bits [M or len(rows), N].

    a_bits: [M, K] uint16 (fp16 or bf16 bits). packed: [K_pad/16, N, 16] uint8 codes.
    scale: python float (rounded to fp32), N per-output-column values (`naive.py:29-33`, bias_dim = 1) or
    None. bias_bits: [N] uint16 in the output format or None.
    rows: optional row subset (int64) to evaluate, for full-size spot checks.
    """
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    m, k = a_bits.shape
    kb, n, _ = packed.shape
    assert kb * 16 >= k
    sc = _scales(scale, n)
    bias = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    if bias is not None:
        assert bias.shape == (n,)
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    r = m if rws is None else len(rws)
    out = np.empty((r, n), dtype=np.uint16)
    _load().oracle_scaled_mm(
        _ptr(a_bits, ctypes.c_uint16), int(a_fmt == BF16), _ptr(packed, ctypes.c_uint8), int(b_fmt == E5M2),
        m, n, k, None if sc is None else _ptr(sc, ctypes.c_float), 0 if sc is None else sc.size,
        None if bias is None else _ptr(bias, ctypes.c_uint16), int(out_fmt == BF16), _ptr(out, ctypes.c_uint16),
        None if rws is None else _ptr(rws, ctypes.c_int64), 0 if rws is None else len(rws), int(threads),
    )
    return out


def scaled_mm_f32(a_bits: np.ndarray, a_fmt: str, packed: np.ndarray, b_fmt: str, scale,
                  rows: np.ndarray | None = None, threads: int = 0) -> np.ndarray:
    """The fp32 value before the output rounding (diagnostics for rounding-neighbour flips)."""
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    m, k = a_bits.shape
    _, n, _ = packed.shape
    sc = _scales(scale, n)
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    r = m if rws is None else len(rws)
    out = np.empty((r, n), dtype=np.float32)
    _load().oracle_scaled_mm_f32(
        _ptr(a_bits, ctypes.c_uint16), int(a_fmt == BF16), _ptr(packed, ctypes.c_uint8), int(b_fmt == E5M2),
        m, n, k, None if sc is None else _ptr(sc, ctypes.c_float), 0 if sc is None else sc.size,
        _ptr(out, ctypes.c_float),
        None if rws is None else _ptr(rws, ctypes.c_int64), 0 if rws is None else len(rws), int(threads),
    )
    return out


def scaled_mm_band(a_bits: np.ndarray, a_fmt: str, packed: np.ndarray, b_fmt: str, scale,
                   bias_bits: np.ndarray | None, out_fmt: str, delta: float, rows: np.ndarray | None = None,
                   threads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """The oracle's answers had the fp32 pre-rounding value been `delta` lower / higher (output units).

    An implementation whose fp32 sum differs from the exact one only in summation order produces, for
    every element, the oracle's answer at some value within a small band around the exact one; an output
    that equals neither the answer nor the band's ends is an error, not a rounding-neighbour flip.
    """
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    m, k = a_bits.shape
    _, n, _ = packed.shape
    sc = _scales(scale, n)
    bias = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    r = m if rws is None else len(rws)
    lo = np.empty((r, n), dtype=np.uint16)
    hi = np.empty((r, n), dtype=np.uint16)
    _load().oracle_scaled_mm_band(
        _ptr(a_bits, ctypes.c_uint16), int(a_fmt == BF16), _ptr(packed, ctypes.c_uint8), int(b_fmt == E5M2),
        m, n, k, None if sc is None else _ptr(sc, ctypes.c_float), 0 if sc is None else sc.size,
        None if bias is None else _ptr(bias, ctypes.c_uint16), int(out_fmt == BF16), float(delta),
        _ptr(lo, ctypes.c_uint16), _ptr(hi, ctypes.c_uint16),
        None if rws is None else _ptr(rws, ctypes.c_int64), 0 if rws is None else len(rws), int(threads),
    )
    return lo, hi


def scaled_mm_torch(a, b_prepacked, scale, bias, out_dtype):
    """`naive.py:4-41` as torch CPU calls with fp32 accumulation: the reference's CPU path, as timed by
    bench.py's `cpu_baseline` leg (torch's multi-threaded CPU matmul, not the exact double sum of the C
    oracle). Takes and returns torch CPU tensors:
      unpack `permute(0, 2, 1).reshape(kb * 16, N)[:K]` (naive.py:13-16), a.to(fp16), b.to(fp16)
      (naive.py:20-22), the product in fp32 (naive.py:23, widened), `* scale` in fp32 (naive.py:24-33),
      `.to(out_dtype)` (naive.py:34), `+ bias` in the output dtype (naive.py:35-40).
    """
    import torch

    k = a.shape[1]
    kb, n, _ = b_prepacked.shape
    b = b_prepacked.permute(0, 2, 1).reshape(kb * 16, n)[:k]
    c = a.to(torch.float16).to(torch.float32) @ b.to(torch.float16).to(torch.float32)
    if scale is not None:
        c = c * scale.to(torch.float32)
    c = c.to(out_dtype)
    if bias is not None:
        c = c + bias
    return c


def literal_fp16_scaled_mm(a_f16: np.ndarray, b_f16: np.ndarray, scale: float | None) -> np.ndarray:
    """The reference's literal order (`naive.py:20-33`): fp16 matmul result, then the fp32 scale.

    Accumulates in float64 and rounds the product matrix to fp16, which is the best case of an fp16
    matmul; values past 65504 become inf, which is the overflow that rules this form out as the oracle.
    Returns float32.
    """
    c = (a_f16.astype(np.float64) @ b_f16.astype(np.float64)).astype(np.float16).astype(np.float32)
    if scale is not None:
        c = c * np.float32(scale)
    return c


# ---- the comparison metric -------------------------------------------------------------------------------

def tolerance(k: int) -> float:
    """North-star bound, relative to the reference output's RMS: 1e-2 * sqrt(K) / 64."""
    return 1e-2 * math.sqrt(k) / 64.0


def bits_to_f32(bits: np.ndarray, fmt: str) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    if fmt == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def ulp(values: np.ndarray, fmt: str) -> np.ndarray:
    """Spacing of the output format at |values| (normal range), as float32."""
    mant_bits = 7 if fmt == BF16 else 10
    min_exp = -126 if fmt == BF16 else -14
    a = np.abs(values.astype(np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, min_exp)
    return np.exp2(e - mant_bits).astype(np.float32)


def compare(out_bits: np.ndarray, ref_bits: np.ndarray, fmt: str, k: int) -> dict:
    """North-star metric plus rounding diagnostics.

    Returns max_abs / rms / bound (strict: max|out - ref| <= tolerance(K) * RMS(ref)), whether the
    NaN and Inf masks agree, and for the elements over the bound how many are exactly one output-ulp
    rounding neighbours of the reference (an fp32 accumulation-order flip at a rounding midpoint).
    """
    out = bits_to_f32(out_bits, fmt).astype(np.float64)
    ref = bits_to_f32(ref_bits, fmt).astype(np.float64)
    nan_ok = bool(np.array_equal(np.isnan(out), np.isnan(ref)))
    inf_ok = bool(np.array_equal(np.isinf(out), np.isinf(ref)) and
                  np.array_equal(np.signbit(out[np.isinf(out)]), np.signbit(ref[np.isinf(ref)])))
    finite = np.isfinite(ref) & np.isfinite(out)
    rms = float(np.sqrt(np.mean(ref[finite] ** 2))) if finite.any() else 0.0
    bound = tolerance(k) * rms
    diff = np.abs(out - ref)
    diff[~finite] = 0.0
    max_abs = float(diff.max()) if diff.size else 0.0
    over = diff > bound
    ref_u = ulp(ref[over], fmt).astype(np.float64)
    neighbour = np.abs(diff[over] - ref_u) <= 0.0
    return {
        "max_abs": max_abs,
        "rms": rms,
        "bound": bound,
        "strict_ok": bool(max_abs <= bound) and nan_ok and inf_ok,
        "nan_ok": nan_ok,
        "inf_ok": inf_ok,
        "n_over": int(over.sum()),
        "n_over_one_ulp": int(neighbour.sum()),
        "n": int(out.size),
    }


# ---- the input recipe ------------------------------------------------------------------------------------

def make_inputs(m: int, k: int, n: int, a_fmt: str = F16, seed: int = 0, outliers: bool = False):
    """The seeded workload recipe shared by tests and bench.

    A ~ N(0, 1) [M, K] (1% of entries x50 when `outliers`), W ~ N(0, 0.02) [N, K], per-tensor
    scale = max|W| / 57344, Wq = e5m2(W / scale) (RNE), B = Wq^T [K, N], P = prepack(B).
    Drawn with torch's CPU generator (A first, then W); returns numpy arrays:
    (a_bits [M, K] uint16, packed [K_pad/16, N, 16] uint8, scale float, b_codes [K, N] uint8).
    """
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    a = torch.randn(m, k, generator=g)
    if outliers:
        a[torch.rand(m, k, generator=g) < 0.01] *= 50
    a = a.to(torch.bfloat16 if a_fmt == BF16 else torch.float16)
    w = torch.randn(n, k, generator=g) * 0.02
    scale = (w.abs().max() / 57344).to(torch.float32)
    wq = (w / scale).to(torch.float8_e5m2)
    b_codes = wq.t().contiguous().view(torch.uint8).numpy()
    a_bits = a.view(torch.int16).numpy().view(np.uint16)
    return a_bits, prepack(b_codes), float(scale.item()), b_codes


def cpu_count() -> int:
    return len(os.sched_getaffinity(0))
