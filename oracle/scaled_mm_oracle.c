/*
 * CPU oracle for the fp16/bf16 x fp8 scaled matmul. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker, never the thing measured or shipped: only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it. The product path
 * (feather_ops.scaled_mm_hip, launch_scaled_mm) never calls into it and has no CPU fallback.
 *
 * It restates the semantics of the reference's naive path, with the accumulation widened:
 *   feather_ops/naive.py:13-16  unpack the (K_pad/16, N, 16) prepack back to B[K, N]
 *   feather_ops/naive.py:20-22  a.to(fp16), b.to(fp16)        -> widen_a(), decode_b()
 *   feather_ops/naive.py:23     a @ b                          -> exact sum (double), rounded once to fp32
 *   feather_ops/naive.py:24-33  .to(fp32) * scale             -> fp32 multiply (per tensor, or per output
 *                                                                  column: bias_dim = 1's scale[None, :])
 *   feather_ops/naive.py:34     .to(out_dtype)                 -> round-to-nearest-even
 *   feather_ops/naive.py:35-40  c += bias (in out precision)   -> fp32 add of two out-dtype values, RNE
 * The literal naive.py accumulates in fp16 and overflows at the per-tensor quantization used here, so the
 * sum is taken exactly (double; the fp16 x fp16 products are exact in fp32 and the K sums stay far inside
 * double's range) and rounded to fp32 once, which is "fp32 accumulation" with no ordering error at all.
 *
 * Decode of the weight byte follows the fp8 formats' definitions (OCP 8-bit floating point):
 *   e5m2:   1 sign, 5 exponent (bias 15), 2 mantissa; exponent 31 is inf (mantissa 0) or NaN.
 *   e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa; only S.1111.111 is NaN, no infinities.
 * The reference decodes e5m2 by moving the byte into the high half of an fp16 lane
 * (csrc/hip_kernel.cu:95-102), which is the same value for every code.
 *
 * Every function here is pinned by tests/test_oracle.py against golden vectors, library routines and
 * closed forms; the header of oracle/naive.py lists which check pins which function.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* fp8 e5m2 byte -> float (exact). */
float oracle_e5m2_to_f32(uint8_t b) {
    const int sign = (b >> 7) & 1;
    const int exp = (b >> 2) & 0x1f;
    const int man = b & 0x3;
    float v;
    if (exp == 0x1f) {
        v = man == 0 ? INFINITY : NAN;
    } else if (exp == 0) {
        v = ldexpf((float)man, -16); /* subnormal: man/4 * 2^-14 */
    } else {
        v = ldexpf(1.0f + (float)man / 4.0f, exp - 15);
    }
    return sign ? -v : v;
}

/* fp8 e4m3fn byte -> float (exact). */
float oracle_e4m3fn_to_f32(uint8_t b) {
    const int sign = (b >> 7) & 1;
    const int exp = (b >> 3) & 0xf;
    const int man = b & 0x7;
    float v;
    if (exp == 0xf && man == 0x7) {
        v = NAN;
    } else if (exp == 0) {
        v = ldexpf((float)man, -9); /* subnormal: man/8 * 2^-6 */
    } else {
        v = ldexpf(1.0f + (float)man / 8.0f, exp - 7);
    }
    return sign ? -v : v;
}

/* IEEE binary16 bits -> float (exact). */
float oracle_f16_to_f32(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int exp = (h >> 10) & 0x1f;
    const int man = h & 0x3ff;
    float v;
    if (exp == 0x1f) {
        v = man == 0 ? INFINITY : NAN;
    } else if (exp == 0) {
        v = ldexpf((float)man, -24);
    } else {
        v = ldexpf(1.0f + (float)man / 1024.0f, exp - 15);
    }
    return sign ? -v : v;
}

/* bfloat16 bits -> float (exact: bf16 is the top half of binary32). */
float oracle_bf16_to_f32(uint16_t h) {
    return bits_to_f32((uint32_t)h << 16);
}

/* float -> binary16, round to nearest even, overflow to inf, NaN kept NaN. */
uint16_t oracle_f32_to_f16_rne(float f) {
    const uint32_t u = f32_to_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const float a = fabsf(f);
    if (isnan(f)) {
        return (uint16_t)(sign | 0x7e00u);
    }
    if (a >= 65520.0f) { /* half-way between 65504 and 2^16 rounds to even, i.e. up: inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a < ldexpf(1.0f, -14)) {
        /* subnormal range: quantum 2^-24; nearbyintf rounds half to even in the default mode */
        const float q = nearbyintf(ldexpf(a, 24));
        return (uint16_t)(sign | (uint16_t)q); /* q == 1024 carries into the smallest normal */
    }
    int e;
    const float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    /* 11 significant bits: scale the mantissa to [1024, 2048) and round half to even */
    float q = nearbyintf(ldexpf(m, 11));
    int exp = e - 1; /* a = (q/1024) * 2^exp */
    if (q >= 2048.0f) {
        q = 1024.0f;
        exp += 1;
    }
    if (exp > 15) {
        return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (uint16_t)((exp + 15) << 10) | (uint16_t)((int)q - 1024));
}

/* float -> bfloat16, round to nearest even, NaN kept NaN. */
uint16_t oracle_f32_to_bf16_rne(float f) {
    const uint32_t u = f32_to_bits(f);
    if (isnan(f)) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    const uint64_t wide = (uint64_t)u + 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(wide >> 16);
}

/*
 * bfloat16 bits -> binary16 bits, rounding toward zero: the semantics of the reference's bf16_to_fp16
 * (feather_ops/convert.py:6-21, which widens bf16 to fp32 and packs with v_cvt_pkrtz_f16_f32, IEEE
 * round-toward-zero). Values fp16 holds exactly stay exact; finite values past 65504 truncate to the
 * largest finite fp16, +-65504, not to inf; inf stays inf and NaN stays (a quiet) NaN; below fp16's normal
 * range the magnitude truncates to a multiple of 2^-24 (the subnormal quantum), so |x| < 2^-24 becomes a
 * zero of x's sign. The exponent/mantissa arithmetic below works on the bit fields of the bf16 code.
 */
uint16_t oracle_bf16_to_f16_rtz(uint16_t h) {
    const uint16_t sign = (uint16_t)(h & 0x8000u);
    const int exp = (h >> 7) & 0xff; /* bf16: 8-bit exponent, bias 127, 7 stored mantissa bits */
    const uint32_t man = h & 0x7fu;
    if (exp == 0xff) {
        return (uint16_t)(sign | (man ? 0x7e00u : 0x7c00u));
    }
    if (exp == 0) { /* zero or a bf16 subnormal (< 2^-126): far below fp16's quantum */
        return sign;
    }
    const int e = exp - 127; /* |x| = (1 + man / 128) * 2^e */
    if (e > 15) {
        return (uint16_t)(sign | 0x7bffu); /* 65504 */
    }
    if (e >= -14) { /* normal in fp16: 10 mantissa bits hold bf16's 7 exactly */
        return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)(man << 3));
    }
    /* fp16 subnormal: value / 2^-24 = (128 + man) * 2^(e + 24 - 7), truncated */
    const int shift = e + 24 - 7;
    const uint32_t sig = 128u + man;
    const uint32_t q = shift >= 0 ? sig << shift : (shift > -32 ? sig >> -shift : 0u);
    return (uint16_t)(sign | (uint16_t)q);
}

static uint16_t finish(float y, const uint16_t* bias, int64_t n, int out_bf16) {
    uint16_t o;
    if (out_bf16) {
        o = oracle_f32_to_bf16_rne(y);
        if (bias) {
            o = oracle_f32_to_bf16_rne(oracle_bf16_to_f32(o) + oracle_bf16_to_f32(bias[n]));
        }
    } else {
        o = oracle_f32_to_f16_rne(y);
        if (bias) {
            o = oracle_f32_to_f16_rne(oracle_f16_to_f32(o) + oracle_f16_to_f32(bias[n]));
        }
    }
    return o;
}

/*
 * The shared core: y[r, n] = fp32(exact sum_k widen(a[m, k]) * decode(B[k, n])) (* scale, in fp32), with B
 * read from the prepack: B[k, n] = packed[(k / 16) * N * 16 + n * 16 + (k % 16)] (feather_ops/scaled_mm.py:150,
 * feather_ops/naive.py:15-16). Then, per mode:
 *   out      != NULL: out[r, n]  = finish(y)                        (the oracle's answer)
 *   out_f32  != NULL: out_f32[r, n] = y                             (diagnostics)
 *   lo, hi   != NULL: lo/hi[r, n] = finish(y -/+ delta)             (the answers for a sum off by +-delta)
 * finish() rounds to the output dtype (RNE) and adds the bias in output precision (naive.py:34-40).
 *
 * a_bf16:  a holds bf16 bits, widened to fp16 with RNE first (naive.py:21 a.to(fp16)); else fp16 bits.
 * b_e5m2:  packed holds e5m2 codes; else e4m3fn codes.
 * scale:   scale_n fp32 values (1: per tensor, N: per output column, naive.py:27-33 with bias_dim = 1) or
 *          NULL (no scale step: naive.py:24 skipped).
 * bias:    N values in the output dtype or NULL.
 * rows:    optional list of n_rows row indices to compute (NULL = all M rows); outputs are [n_rows, N].
 */
static void core(const uint16_t* a, int a_bf16, const uint8_t* packed, int b_e5m2, int64_t M, int64_t N, int64_t K,
                 const float* scale, int64_t scale_n, const uint16_t* bias, int out_bf16, uint16_t* out, float* out_f32, float delta,
                 uint16_t* lo, uint16_t* hi, const int64_t* rows, int64_t n_rows, int n_threads) {
    const int64_t R = rows ? n_rows : M;
    float lut[256];
    for (int c = 0; c < 256; ++c) {
        lut[c] = b_e5m2 ? oracle_e5m2_to_f32((uint8_t)c) : oracle_e4m3fn_to_f32((uint8_t)c);
    }
    /* unpack and decode the weight once, column-major: bcol[n * K + k] = decode(B[k, n]) */
    float* bcol = (float*)malloc((size_t)N * (size_t)K * sizeof(float));
    if (!bcol) {
        return;
    }
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            bcol[n * K + k] = lut[packed[((k / 16) * N + n) * 16 + (k % 16)]];
        }
    }
#ifdef _OPENMP
    if (n_threads > 0) {
        omp_set_num_threads(n_threads);
    }
#pragma omp parallel
#endif
    {
        double* arow_f = (double*)malloc((size_t)K * sizeof(double));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t r = 0; r < R; ++r) {
            const int64_t m = rows ? rows[r] : r;
            const uint16_t* arow = a + m * K;
            for (int64_t k = 0; k < K; ++k) {
                arow_f[k] = a_bf16 ? oracle_f16_to_f32(oracle_f32_to_f16_rne(oracle_bf16_to_f32(arow[k])))
                                   : oracle_f16_to_f32(arow[k]);
            }
            for (int64_t n = 0; n < N; ++n) {
                const float* bc = bcol + n * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) {
                    acc += arow_f[k] * (double)bc[k];
                }
                float y = (float)acc;
                if (scale) {
                    y = y * scale[scale_n == 1 ? 0 : n];
                }
                if (out) {
                    out[r * N + n] = finish(y, bias, n, out_bf16);
                }
                if (out_f32) {
                    out_f32[r * N + n] = y;
                }
                if (lo) {
                    lo[r * N + n] = finish((float)((double)y - (double)delta), bias, n, out_bf16);
                }
                if (hi) {
                    hi[r * N + n] = finish((float)((double)y + (double)delta), bias, n, out_bf16);
                }
            }
        }
        free(arow_f);
    }
    free(bcol);
}

void oracle_scaled_mm(const uint16_t* a, int a_bf16, const uint8_t* packed, int b_e5m2, int64_t M, int64_t N,
                      int64_t K, const float* scale, int64_t scale_n, const uint16_t* bias, int out_bf16,
                      uint16_t* out, const int64_t* rows, int64_t n_rows, int n_threads) {
    core(a, a_bf16, packed, b_e5m2, M, N, K, scale, scale_n, bias, out_bf16, out, NULL, 0.0f, NULL, NULL, rows, n_rows,
         n_threads);
}

/* The fp32 value before the output rounding, for diagnostics: out[r, n] = fp32(sum) (* scale). */
void oracle_scaled_mm_f32(const uint16_t* a, int a_bf16, const uint8_t* packed, int b_e5m2, int64_t M, int64_t N,
                          int64_t K, const float* scale, int64_t scale_n, float* out, const int64_t* rows,
                          int64_t n_rows, int n_threads) {
    core(a, a_bf16, packed, b_e5m2, M, N, K, scale, scale_n, NULL, 0, NULL, out, 0.0f, NULL, NULL, rows, n_rows, n_threads);
}

/* The answers for a pre-rounding value off by -delta / +delta (absolute, output units). */
void oracle_scaled_mm_band(const uint16_t* a, int a_bf16, const uint8_t* packed, int b_e5m2, int64_t M, int64_t N,
                           int64_t K, const float* scale, int64_t scale_n, const uint16_t* bias, int out_bf16,
                           float delta, uint16_t* lo, uint16_t* hi, const int64_t* rows, int64_t n_rows,
                           int n_threads) {
    core(a, a_bf16, packed, b_e5m2, M, N, K, scale, scale_n, bias, out_bf16, NULL, NULL, delta, lo, hi, rows, n_rows,
         n_threads);
}

/* [K, N] fp8 codes -> (K_pad/16, N, 16) with K zero-padded to a multiple of 128 (scaled_mm.py:137-150). */
void oracle_prepack(const uint8_t* b, int64_t K, int64_t N, uint8_t* packed) {
    const int64_t k_pad = (K + 127) / 128 * 128;
    for (int64_t k = 0; k < k_pad; ++k) {
        for (int64_t n = 0; n < N; ++n) {
            packed[((k / 16) * N + n) * 16 + (k % 16)] = k < K ? b[k * N + n] : 0;
        }
    }
}
