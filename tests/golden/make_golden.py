"""Writes the golden fixtures under tests/golden/ (committed; re-run only to regenerate them).

The expected outputs are computed WITHOUT the oracle's C code, from the same library routines the
reference's naive path calls (feather_ops/naive.py): torch's float8 -> float cast for the weight
(`b.to(fp16)`, naive.py:22), torch's bf16 -> fp16 cast for bf16 activations (naive.py:21), torch's RNE
`.to(out_dtype)` (naive.py:34) and torch's output-precision bias add (naive.py:35-40). Only the matmul
differs from the literal reference: it is float64 `numpy.matmul` (exact to far below fp32's rounding),
rounded once to fp32, then scaled in fp32, which is the fp32-accumulation semantics the oracle restates.
The layout is the reference's `prepack_b_for_scaled_mm` (scaled_mm.py:144-150) restated with explicit
index loops here, independent of both the oracle's C index formula and the product's torch view.

e5m2_kat.json is the literal known-answer list the reference holds for the e5m2 decode
(cpp_benchmarks/benchmark_scaled_mm_hip.cpp:129-139).

    python tests/golden/make_golden.py
"""

import hashlib
import json
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.naive import make_inputs  # noqa: E402  (the seeded recipe only; no oracle arithmetic)

E5M2_KAT = {  # code -> value, from cpp_benchmarks/benchmark_scaled_mm_hip.cpp:129-139
    "0xbc": -1.0, "0xba": -0.75, "0xb8": -0.5, "0xb4": -0.25, "0x00": 0.0,
    "0x34": 0.25, "0x38": 0.5, "0x3a": 0.75, "0x3c": 1.0,
}


def prepack_loops(codes: np.ndarray) -> np.ndarray:
    k, n = codes.shape
    k_pad = -(-k // 128) * 128
    out = np.zeros((k_pad // 16, n, 16), dtype=np.uint8)
    for kk in range(k):
        for nn in range(n):
            out[kk // 16, nn, kk % 16] = codes[kk, nn]
    return out


def expected(a_bits, a_fmt, b_codes, b_fmt, scale, bias_bits, out_fmt):
    """Reference semantics with float64 accumulation, from torch casts; returns out-dtype bits."""
    a_t = torch.from_numpy(a_bits.view(np.int16))
    a_t = a_t.view(torch.bfloat16 if a_fmt == "bf16" else torch.float16).to(torch.float16)
    b_t = torch.from_numpy(b_codes).view(torch.float8_e5m2 if b_fmt == "e5m2" else torch.float8_e4m3fn)
    a64 = a_t.double().numpy()
    b64 = b_t.to(torch.float32).double().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        acc = np.float32(a64 @ b64) if a64.size else np.zeros((a64.shape[0], b64.shape[1]), np.float32)
        acc = acc.astype(np.float32)
        if scale is not None:
            acc = acc * np.float32(scale)
    out_dtype = torch.bfloat16 if out_fmt == "bf16" else torch.float16
    c = torch.from_numpy(acc).to(out_dtype)
    if bias_bits is not None:
        c = c + torch.from_numpy(bias_bits.view(np.int16)).view(out_dtype)
    return c.view(torch.int16).numpy().view(np.uint16)


def f16_bits(x):
    return torch.tensor(x, dtype=torch.float32).to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def bf16_bits(x):
    return torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main():
    rng = np.random.default_rng(20261201)
    cases = {}

    def add(name, a_bits, a_fmt, b_codes, b_fmt, scale, bias_bits, out_fmt, rows=None):
        out = expected(a_bits, a_fmt, b_codes, b_fmt, scale, bias_bits, out_fmt)
        entry = {
            "a_bits": a_bits, "b_codes": b_codes, "packed": prepack_loops(b_codes), "out": out,
            "meta": np.array(json.dumps({"a_fmt": a_fmt, "b_fmt": b_fmt, "out_fmt": out_fmt, "scale": scale,
                                         "has_bias": bias_bits is not None})),
        }
        if bias_bits is not None:
            entry["bias"] = bias_bits
        if rows is not None:
            entry["rows"] = np.asarray(rows, dtype=np.int64)
        cases[name] = entry

    # non-square, non-symmetric small cases: a transposed operand or a dropped k term changes the answer
    a = f16_bits(rng.normal(size=(5, 48)))
    b = torch.tensor(rng.normal(scale=3.0, size=(48, 24)), dtype=torch.float32).to(torch.float8_e5m2)
    add("tiny_f16", a, "fp16", b.view(torch.uint8).numpy(), "e5m2", 0.375, f16_bits(rng.normal(size=24)), "fp16")

    a = bf16_bits(rng.normal(size=(7, 64)) * 4)
    b = torch.tensor(rng.normal(scale=40.0, size=(64, 40)), dtype=torch.float32).to(torch.float8_e5m2)
    add("tiny_bf16_bf16out", a, "bf16", b.view(torch.uint8).numpy(), "e5m2", 0.0123, bf16_bits(rng.normal(size=40)),
        "bf16")

    a = f16_bits(rng.normal(size=(3, 32)))
    codes = rng.integers(0, 256, size=(32, 16), dtype=np.uint8)
    codes[codes & 0x7F == 0x7F] = 0x3A  # keep NaN codes out of this one
    codes[0, :8] = np.arange(8, dtype=np.uint8)  # e4m3fn subnormals and zero
    add("tiny_e4m3fn", a, "fp16", codes, "e4m3fn", 1.5, None, "bf16")

    # no scale step (naive.py:24 skipped), fp16 out, K not a multiple of 128 (pad rows in play)
    a = f16_bits(rng.normal(size=(4, 80)))
    b = torch.tensor(rng.normal(scale=0.5, size=(80, 8)), dtype=torch.float32).to(torch.float8_e5m2)
    add("noscale_k80", a, "fp16", b.view(torch.uint8).numpy(), "e5m2", None, None, "fp16")

    # e5m2 subnormal codes and fp16 subnormal activations
    a = f16_bits(rng.normal(size=(2, 32)) * 1e-6)
    codes = rng.integers(0, 4, size=(32, 8), dtype=np.uint8) | (rng.integers(0, 2, size=(32, 8), dtype=np.uint8) << 7)
    add("subnormals", a, "fp16", codes, "e5m2", 2.0**20, None, "fp16")

    # specials: inf / NaN in A, inf / NaN codes in B, and a bf16 activation past fp16's range
    a = f16_bits(rng.normal(size=(4, 32)))
    a[1, 3] = 0x7C00  # +inf
    a[2, 5] = 0x7E00  # NaN
    codes = torch.tensor(rng.normal(size=(32, 8)), dtype=torch.float32).to(torch.float8_e5m2).view(torch.uint8).numpy()
    codes[7, 2] = 0x7C  # +inf
    codes[9, 6] = 0x7E  # NaN
    add("specials_f16", a, "fp16", codes, "e5m2", 0.5, None, "fp16")
    a = bf16_bits(rng.normal(size=(3, 32)))
    a[0, 0] = bf16_bits(np.float32(70000.0))  # becomes fp16 inf under naive.py:21
    codes = torch.tensor(rng.normal(size=(32, 8)), dtype=torch.float32).to(torch.float8_e5m2).view(torch.uint8).numpy()
    add("bf16_overflow", a, "bf16", codes, "e5m2", 1.0, None, "bf16")

    # C1 recipe: inputs regenerate from the seed; store their hashes and some rows
    a_bits, packed, scale, b_codes = make_inputs(256, 1024, 1024, "fp16", seed=0)
    rows = [0, 1, 100, 255]
    out = expected(a_bits[rows], "fp16", b_codes, "e5m2", scale, None, "fp16")
    cases["c1_rows"] = {
        "rows": np.array(rows, dtype=np.int64), "out": out,
        "meta": np.array(json.dumps({"m": 256, "k": 1024, "n": 1024, "a_fmt": "fp16", "out_fmt": "fp16", "seed": 0,
                                     "scale": scale, "a_sha256": hashlib.sha256(a_bits.tobytes()).hexdigest(),
                                     "packed_sha256": hashlib.sha256(packed.tobytes()).hexdigest()})),
    }
    # C5 ragged cell with outliers (M=77, K=2560, N=1000, bf16)
    a_bits, packed, scale, b_codes = make_inputs(77, 2560, 1000, "bf16", seed=0, outliers=True)
    rows = [0, 38, 76]
    out = expected(a_bits[rows], "bf16", b_codes, "e5m2", scale, None, "bf16")
    cases["c5_rows"] = {
        "rows": np.array(rows, dtype=np.int64), "out": out,
        "meta": np.array(json.dumps({"m": 77, "k": 2560, "n": 1000, "a_fmt": "bf16", "out_fmt": "bf16", "seed": 0,
                                     "outliers": True, "scale": scale,
                                     "a_sha256": hashlib.sha256(a_bits.tobytes()).hexdigest(),
                                     "packed_sha256": hashlib.sha256(packed.tobytes()).hexdigest()})),
    }

    flat = {f"{case}/{key}": val for case, entry in cases.items() for key, val in entry.items()}
    np.savez_compressed(HERE / "golden.npz", **flat)
    (HERE / "e5m2_kat.json").write_text(json.dumps(E5M2_KAT, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {HERE / 'golden.npz'}")


if __name__ == "__main__":
    main()
