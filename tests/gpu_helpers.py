"""Shared helpers of the GPU parity tests: move oracle-format arrays to the device and compare results."""

import numpy as np
import torch

from oracle import naive as oracle

A_DT = {oracle.F16: torch.float16, oracle.BF16: torch.bfloat16}
B_DT = {oracle.E5M2: torch.float8_e5m2, oracle.E4M3FN: torch.float8_e4m3fn}
FMT_OF = {torch.float16: oracle.F16, torch.bfloat16: oracle.BF16,
          torch.float8_e5m2: oracle.E5M2, torch.float8_e4m3fn: oracle.E4M3FN}


def to_dev_bits(bits: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    if dtype in (torch.float8_e5m2, torch.float8_e4m3fn):
        return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint8)).view(dtype).to(device)
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(dtype).to(device)


def bits_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float8_e5m2, torch.float8_e4m3fn):
        return t.view(torch.uint8).numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def sample_rows(m: int, n_random: int = 32, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    rows = set(range(min(m, 16))) | set(range(max(0, m - 16), m))
    rows |= set(rng.integers(0, m, size=min(m, n_random)).tolist())
    return np.array(sorted(rows), dtype=np.int64)


def scale_arg(scale):
    """A device scale tensor as the oracle takes it: None, one float, or N per-column fp32 values."""
    if scale is None:
        return None
    if scale.numel() == 1:
        return float(scale.item())
    return scale.detach().float().cpu().numpy()


def oracle_ref(a: torch.Tensor, b_prepacked: torch.Tensor, scale, bias, out_dtype, rows=None) -> np.ndarray:
    """Oracle output bits for device inputs (all rows, or the given subset)."""
    return oracle.scaled_mm(
        bits_of(a), FMT_OF[a.dtype], bits_of(b_prepacked), FMT_OF[b_prepacked.dtype], scale_arg(scale),
        None if bias is None else bits_of(bias), FMT_OF[out_dtype], rows=rows, threads=16,
    )


BAND_REL = 1e-4  # half-width of the accepted band around the exact sum, relative to RMS(reference)


def check_against_oracle(out: torch.Tensor, a, b_prepacked, scale, bias, rows=None, max_flip_frac=1e-3):
    """North-star comparison with the oracle.

    Strict (max|out - ref| <= 1e-2 sqrt(K)/64 RMS, identical NaN/Inf masks) for fp16 output. For bf16
    output the bound is below one bf16 ulp at |y| >= 2 RMS, so an element over it is accepted only when
    it is exactly the oracle's answer for a pre-rounding value within BAND_REL * RMS of the exact sum
    (an fp32 summation-order flip at a rounding midpoint, possibly carried through the bias add), and such
    elements must be at most `max_flip_frac` of the outputs. Returns the comparison dict.
    """
    fmt = FMT_OF[out.dtype]
    ref = oracle_ref(a, b_prepacked, scale, bias, out.dtype, rows=rows)
    got = bits_of(out)
    if rows is not None:
        got = got[rows]
    res = oracle.compare(got, ref, fmt, a.shape[1])
    assert res["nan_ok"] and res["inf_ok"], res
    if fmt == oracle.F16 or res["strict_ok"]:
        assert res["strict_ok"], res
        return res
    lo, hi = oracle.scaled_mm_band(
        bits_of(a), FMT_OF[a.dtype], bits_of(b_prepacked), FMT_OF[b_prepacked.dtype],
        scale_arg(scale), None if bias is None else bits_of(bias), fmt,
        BAND_REL * res["rms"], rows=rows, threads=16)
    got_f = oracle.bits_to_f32(got, fmt).astype(np.float64)
    ref_f = oracle.bits_to_f32(ref, fmt).astype(np.float64)
    over = np.abs(got_f - ref_f) > res["bound"]
    over &= np.isfinite(got_f) & np.isfinite(ref_f)
    in_band = (got == lo) | (got == hi)
    bad = over & ~in_band
    assert not bad.any(), {**res, "n_outside_band": int(bad.sum())}
    assert over.sum() <= max(2, max_flip_frac * res["n"]), res
    res["n_band_flips"] = int(over.sum())
    return res
