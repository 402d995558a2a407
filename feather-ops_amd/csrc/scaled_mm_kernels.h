// fp16/bf16 activation x fp8 (e5m2 / e4m3fn) prepacked weight -> fp16/bf16, for gfx950 (CDNA4, wave64).
//
//   c[m, n] = round_out( fp32( sum_k fp16(a[m, k]) * fp16(B[k, n]) ) * scale ) (+ bias[n], in out precision)
//   B[k, n] = b_prepacked[k / 16][n][k % 16]                 (feather_ops/scaled_mm.py:137-150)
//
// Semantics follow the reference's naive path (feather_ops/naive.py:4-41) with fp32 accumulation:
// bf16 activations are widened to fp16 with round-to-nearest-even (naive.py:21), the weight byte is
// decoded exactly to fp16 (every e5m2 and e4m3fn value is an fp16 value), the products are summed by
// fp16 MFMAs into fp32 accumulators, the fp32 scale is applied in fp32, the downcast is RNE for both
// output types, and the bias is added after the downcast in the output precision (naive.py:34-40).
//
// Two kernel families share the fragment layout, the decode and the epilogue:
//  - ring_kernel   (tile field prefetch = 1): a block owns a BM x BN output tile, waves split it WM x WN,
//                  and K streams through a double-buffered LDS ring, one 16*U-deep stage at a time. The
//                  next stage's global loads are in flight while the current stage feeds the MFMAs.
//  - stream_kernel (prefetch = 0): for skinny M. No LDS staging: each wave streams its fragments
//                  straight from global memory into VGPRs (register double buffer), the block's WM
//                  waves split K, and a short LDS reduction joins their fp32 partial sums.
//
// Fragment layout (v_mfma_f32_16x16x32_f16, wave64). The MFMA's first operand (16 "rows" i) carries 16
// weight columns and its second operand (16 "columns" j) carries 16 activation rows, so each lane ends
// up holding 4 consecutive output columns of one output row: lane l owns row (l % 16) and columns
// 4 * (l / 16) + {0..3} of a 16 x 16 tile, which the epilogue writes as one 8-byte store.
// K is covered in groups of 64 = four prepack chunks of 16: lane group g = l / 16 takes chunk g of the
// group (16 bytes of the weight column, 32 bytes of the activation row), and the chunk's first 8 k values
// feed the group's first MFMA, the last 8 its second. Both operands use the same (lane group, element)
// -> k assignment, which is all a k-reduction needs.
//
// Out-of-range rows, columns and k chunks are read through buffer resources with an offset past the
// buffer's end, which returns zeros, and stores past the end are dropped, so no path branches on tails.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace feather {

using half8 = _Float16 __attribute__((ext_vector_type(8)));
using half2v = _Float16 __attribute__((ext_vector_type(2)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr int kWave = 64;
// A buffer offset at or past num_records reads zero and drops stores; every buffer here is < 2 GiB.
constexpr uint32_t kOob = 0x80000000u;
// Buffer resource word 3 for gfx9-family raw (untyped, stride 0) buffers.
constexpr int kRsrcFlags = 0x00020000;

struct Params {
    const uint16_t* a;          // [M, K] fp16 or bf16 bits, row-major
    const uint8_t* b;           // [kb_total, N, 16] fp8 codes
    const float* scale;         // 1 fp32 value, or nullptr
    const uint16_t* bias;       // [N] in the output dtype, or nullptr
    uint16_t* c;                // [M, N] output bits, row-major
    int32_t M, N, K;
    int32_t kb_total;           // b_prepacked.shape[0]
};

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kRsrcFlags);
}

__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ u32x2 buf_load8(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ void buf_store8(u32x2 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, static_cast<int>(off), 0, 0);
}

// ---- element conversions ---------------------------------------------------------------------------------

// v_perm_b32 selector: byte i of the result takes selector byte i; 0..3 pick bytes of the second
// source, 0x0c yields 0x00.
constexpr uint32_t perm_sel(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}
constexpr uint32_t kZeroByte = 0x0c;

// e5m2 and fp16 share the sign bit, the 5-bit exponent and its bias (15), and e5m2's two mantissa bits
// are fp16's top two, so an e5m2 byte placed in the high byte of a 16-bit lane is that value's fp16 bit
// pattern (subnormals, inf and NaN included). Four bytes -> two dwords of two fp16 lanes each.
__device__ __forceinline__ void e5m2x4_to_f16(uint32_t p, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(0u, p, perm_sel(kZeroByte, 0, kZeroByte, 1));
    hi = __builtin_amdgcn_perm(0u, p, perm_sel(kZeroByte, 2, kZeroByte, 3));
}

// e4m3fn -> fp16, exact. The 7 magnitude bits (eeee mmm) placed at fp16 bits 13..7 form an fp16 whose
// value is exactly |x| / 256 for every finite code: a normal code is 2^(e-7) (1 + m/8) and reads as
// 2^(e-15) (1 + m/8); a subnormal code is m 2^-9 and reads as the fp16 subnormal (m << 7) 2^-24 = m 2^-17.
// One exact fp16 multiply by 256 restores |x|, the sign is or-ed back, and the one NaN magnitude (0x7f)
// becomes an fp16 NaN.
__device__ __forceinline__ uint32_t e4m3x2_to_f16(uint32_t pair /* bytes in bits 7..0 and 23..16 */) {
    const uint32_t mag = (pair & 0x007f007fu) << 7;
    half2v h = __builtin_bit_cast(half2v, mag);
    h = h * half2v{static_cast<_Float16>(256.0f), static_cast<_Float16>(256.0f)};
    uint32_t r = __builtin_bit_cast(uint32_t, h) | ((pair & 0x00800080u) << 8);
    if ((pair & 0x7fu) == 0x7fu) r = (r & 0xffff0000u) | 0x7e00u;
    if ((pair & 0x007f0000u) == 0x007f0000u) r = (r & 0x0000ffffu) | 0x7e000000u;
    return r;
}

__device__ __forceinline__ void e4m3x4_to_f16(uint32_t p, uint32_t& lo, uint32_t& hi) {
    lo = e4m3x2_to_f16(__builtin_amdgcn_perm(0u, p, perm_sel(0, kZeroByte, 1, kZeroByte)));
    hi = e4m3x2_to_f16(__builtin_amdgcn_perm(0u, p, perm_sel(2, kZeroByte, 3, kZeroByte)));
}

// 16 weight bytes (16 consecutive k of one column) -> the two 8-wide fp16 MFMA operands.
template <bool kE5M2>
__device__ __forceinline__ void decode_chunk(const u32x4 raw, half8& first, half8& second) {
    uint32_t d[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if constexpr (kE5M2) {
            e5m2x4_to_f16(raw[w], d[2 * w], d[2 * w + 1]);
        } else {
            e4m3x4_to_f16(raw[w], d[2 * w], d[2 * w + 1]);
        }
    }
    first = __builtin_bit_cast(half8, u32x4{d[0], d[1], d[2], d[3]});
    second = __builtin_bit_cast(half8, u32x4{d[4], d[5], d[6], d[7]});
}

// Two bf16 -> two fp16 with round-to-nearest-even and overflow to inf, as a tensor cast does.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v) {
    const float lo = __builtin_bit_cast(float, v << 16);
    const float hi = __builtin_bit_cast(float, v & 0xffff0000u);
    const half2v h{static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 v) {
    return u32x4{bf16x2_to_f16x2(v[0]), bf16x2_to_f16x2(v[1]), bf16x2_to_f16x2(v[2]), bf16x2_to_f16x2(v[3])};
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // NaN stays NaN (quieted)
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <bool kOutBf16>
__device__ __forceinline__ uint32_t round_out(float x) {
    if constexpr (kOutBf16) {
        return f32_to_bf16_bits(x);
    } else {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
}

template <bool kOutBf16>
__device__ __forceinline__ float out_to_f32(uint32_t bits) {
    if constexpr (kOutBf16) {
        return __builtin_bit_cast(float, bits << 16);
    } else {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
    }
}

// acc (4 consecutive columns of one row) -> scaled, rounded, biased output bits, packed for one 8-byte store.
template <bool kOutBf16>
__device__ __forceinline__ u32x2 epilogue4(const f32x4 acc, float scale, bool has_bias, u32x2 bias_bits) {
    uint32_t o[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        uint32_t y = round_out<kOutBf16>(acc[v] * scale);
        if (has_bias) {
            const uint32_t bb = (bias_bits[v / 2] >> (16 * (v % 2))) & 0xffffu;
            y = round_out<kOutBf16>(out_to_f32<kOutBf16>(y) + out_to_f32<kOutBf16>(bb));
        }
        o[v] = y;
    }
    return u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
}

__device__ __forceinline__ f32x4 mfma16(half8 w, half8 x, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(w, x, acc, 0, 0, 0);
}

// Store one wave's RM x RN accumulator tiles. rows0/cols0: the wave's first output row and column.
template <int RM, int RN, bool kOutBf16>
__device__ __forceinline__ void store_tiles(const Params& p, const f32x4 (&acc)[RM][RN], int row0, int col0,
                                            int lane) {
    const rsrc_t c_rsrc = make_rsrc(p.c, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.N) * 2u);
    const rsrc_t bias_rsrc = make_rsrc(p.bias, p.bias ? static_cast<uint32_t>(p.N) * 2u : 0u);
    const float scale = p.scale ? *p.scale : 1.0f;
    const bool has_bias = p.bias != nullptr;
    const int r_in = lane & 15;
    const int c_in = 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        const int col = col0 + 16 * j + c_in;
        const bool col_ok = col < p.N;
        u32x2 bias_bits{0u, 0u};
        if (has_bias) bias_bits = buf_load8(bias_rsrc, col_ok ? static_cast<uint32_t>(col) * 2u : kOob);
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int row = row0 + 16 * i + r_in;
            const bool ok = col_ok && row < p.M;
            const uint32_t off = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.N) +
                                       static_cast<uint32_t>(col)) * 2u
                                    : kOob;
            buf_store8(epilogue4<kOutBf16>(acc[i][j], scale, has_bias, bias_bits), c_rsrc, off);
        }
    }
}

// ---- ring kernel: LDS double buffer ---------------------------------------------------------------------

template <int WM, int WN, int U, int RM, int RN>
struct RingShape {
    static constexpr int kThreads = kWave * WM * WN;
    static constexpr int kBM = 16 * WM * RM;
    static constexpr int kBN = 16 * WN * RN;
    static constexpr int kChunks = U;                 // 16-deep k chunks per stage
    static constexpr int kGroups = U / 4;             // 64-deep MFMA groups per stage
    static constexpr int kABytes = kBM * U * 32;      // [chunk][row][16 halves]
    static constexpr int kBBytes = kBN * U * 16;      // [chunk][col][16 bytes]
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kLdsBytes = 2 * kStageBytes;
    static constexpr int kAUnits = kBM * U * 2;       // 16-byte pieces of one A stage
    static constexpr int kBUnits = kBN * U;           // 16-byte pieces of one B stage
    static constexpr int kALoads = (kAUnits + kThreads - 1) / kThreads;
    static constexpr int kBLoads = (kBUnits + kThreads - 1) / kThreads;
    static_assert(U % 4 == 0, "a stage is a whole number of 64-deep MFMA groups");
    static_assert(kThreads <= 1024, "block size");
    static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");
};

// LDS position of the 16-byte half `s` of row `row`'s chunk: the halves of every eighth row are swapped
// so that the 16 rows one MFMA operand read touches land on distinct banks.
__device__ __forceinline__ int a_lds_offset(int chunk, int row, int s, int bm) {
    return chunk * bm * 32 + row * 32 + ((s ^ ((row >> 3) & 1)) << 4);
}

// Tile order: consecutive workgroup ids go to different XCDs, so give each XCD a contiguous run of tiles,
// and walk tiles in groups of kGroupM tile rows so that the blocks resident on one XCD share A and B panels
// in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcds = 8;
    constexpr int kGroupM = 4;
    const int xcd = bid % kXcds;
    const int q = nblocks / kXcds;
    const int r = nblocks % kXcds;
    const int t = xcd * q + (xcd < r ? xcd : r) + bid / kXcds;
    const int group = t / (kGroupM * tiles_n);
    const int first_m = group * kGroupM;
    const int gm = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
    const int in = t - group * kGroupM * tiles_n;
    tm = first_m + in % gm;
    tn = in / gm;
}

template <int WM, int WN, int U, int RM, int RN, bool kE5M2, bool kABf16, bool kOutBf16>
__global__ __launch_bounds__(kWave * WM * WN) void ring_kernel(const Params p) {
    using S = RingShape<WM, WN, U, RM, RN>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wave_m = wave / WN;
    const int wave_n = wave % WN;

    const int tiles_m = (p.M + S::kBM - 1) / S::kBM;
    const int tiles_n = (p.N + S::kBN - 1) / S::kBN;
    int tm, tn;
    tile_of_block(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * S::kBM;
    const int n0 = tn * S::kBN;

    const uint32_t a_bytes = static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.K) * 2u;
    const uint32_t b_bytes = static_cast<uint32_t>(p.kb_total) * static_cast<uint32_t>(p.N) * 16u;
    const rsrc_t a_rsrc = make_rsrc(p.a, a_bytes);
    const rsrc_t b_rsrc = make_rsrc(p.b, b_bytes);
    const int k_chunks = p.K / 16;
    const int stages = (p.K + 16 * U - 1) / (16 * U);

    // Per-thread global offsets of its share of a stage (stage 0), and where they land in LDS.
    uint32_t a_goff[S::kALoads];
    int a_loff[S::kALoads];
    int a_chunk[S::kALoads];
    bool a_valid[S::kALoads];
#pragma unroll
    for (int i = 0; i < S::kALoads; ++i) {
        const int u = tid + i * S::kThreads;
        const int row = u / (2 * U);
        const int c = u % (2 * U);
        const int chunk = c >> 1;
        const int s = c & 1;
        a_valid[i] = u < S::kAUnits;
        a_chunk[i] = chunk;
        const int grow = m0 + row;
        a_goff[i] = grow < p.M ? (static_cast<uint32_t>(grow) * static_cast<uint32_t>(p.K) +
                                  static_cast<uint32_t>(chunk * 16 + s * 8)) * 2u
                               : kOob;
        a_loff[i] = a_lds_offset(chunk, row, s, S::kBM);
    }
    uint32_t b_goff[S::kBLoads];
    int b_loff[S::kBLoads];
    int b_chunk[S::kBLoads];
    bool b_valid[S::kBLoads];
#pragma unroll
    for (int i = 0; i < S::kBLoads; ++i) {
        const int u = tid + i * S::kThreads;
        const int chunk = u / S::kBN;
        const int col = u % S::kBN;
        b_valid[i] = u < S::kBUnits;
        b_chunk[i] = chunk;
        const int gcol = n0 + col;
        b_goff[i] = gcol < p.N ? (static_cast<uint32_t>(chunk) * static_cast<uint32_t>(p.N) +
                                  static_cast<uint32_t>(gcol)) * 16u
                               : kOob;
        b_loff[i] = S::kABytes + chunk * S::kBN * 16 + col * 16;
    }

    u32x4 a_reg[S::kALoads];
    u32x4 b_reg[S::kBLoads];

    auto fetch = [&](int stage) {
        const int chunk0 = stage * U;
#pragma unroll
        for (int i = 0; i < S::kALoads; ++i) {
            const bool in_k = chunk0 + a_chunk[i] < k_chunks;
            const uint32_t off = (a_goff[i] == kOob || !in_k) ? kOob : a_goff[i] + static_cast<uint32_t>(chunk0) * 32u;
            a_reg[i] = buf_load16(a_rsrc, off);
        }
#pragma unroll
        for (int i = 0; i < S::kBLoads; ++i) {
            const bool in_k = chunk0 + b_chunk[i] < k_chunks;
            const uint32_t off = (b_goff[i] == kOob || !in_k)
                                     ? kOob
                                     : b_goff[i] + static_cast<uint32_t>(chunk0) * static_cast<uint32_t>(p.N) * 16u;
            b_reg[i] = buf_load16(b_rsrc, off);
        }
    };
    auto deposit = [&](int buf) {
        uint8_t* base = lds + buf * S::kStageBytes;
#pragma unroll
        for (int i = 0; i < S::kALoads; ++i) {
            if (S::kAUnits % S::kThreads == 0 || a_valid[i]) {
                u32x4 v = a_reg[i];
                if constexpr (kABf16) v = bf16x8_to_f16x8(v);
                *reinterpret_cast<u32x4*>(base + a_loff[i]) = v;
            }
        }
#pragma unroll
        for (int i = 0; i < S::kBLoads; ++i) {
            if (S::kBUnits % S::kThreads == 0 || b_valid[i]) {
                *reinterpret_cast<u32x4*>(base + b_loff[i]) = b_reg[i];
            }
        }
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int g = lane >> 4;       // lane group: which 16-deep chunk of a 64-deep group
    const int r16 = lane & 15;     // row (A) / column (B) within a 16-wide fragment
    const int a_row_base = wave_m * 16 * RM + r16;
    const int b_col_base = wave_n * 16 * RN + r16;

    fetch(0);
    deposit(0);
    __syncthreads();

    for (int t = 0; t < stages; ++t) {
        const bool more = t + 1 < stages;
        if (more) fetch(t + 1);
        const uint8_t* base = lds + (t & 1) * S::kStageBytes;
#pragma unroll
        for (int q = 0; q < S::kGroups; ++q) {
            const int chunk = 4 * q + g;
            half8 xa[RM][2];
#pragma unroll
            for (int i = 0; i < RM; ++i) {
                const int row = a_row_base + 16 * i;
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    xa[i][s] = *reinterpret_cast<const half8*>(base + a_lds_offset(chunk, row, s, S::kBM));
                }
            }
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                const int col = b_col_base + 16 * j;
                const u32x4 raw = *reinterpret_cast<const u32x4*>(base + S::kABytes + chunk * S::kBN * 16 + col * 16);
                half8 w0, w1;
                decode_chunk<kE5M2>(raw, w0, w1);
#pragma unroll
                for (int i = 0; i < RM; ++i) {
                    acc[i][j] = mfma16(w0, xa[i][0], acc[i][j]);
                    acc[i][j] = mfma16(w1, xa[i][1], acc[i][j]);
                }
            }
        }
        if (more) deposit((t + 1) & 1);
        __syncthreads();
    }

    store_tiles<RM, RN, kOutBf16>(p, acc, m0 + wave_m * 16 * RM, n0 + wave_n * 16 * RN, lane);
}

// ---- stream kernel: split-K, global -> VGPR ----------------------------------------------------------------

template <int KS, int WN, int U, int RM, int RN>
struct StreamShape {
    static constexpr int kThreads = kWave * KS * WN;
    static constexpr int kBM = 16 * RM;
    static constexpr int kBN = 16 * WN * RN;
    static constexpr int kGroups = U / 4;             // 64-deep groups per iteration of one wave
    static constexpr int kRedBytes = (KS > 1 ? KS - 1 : 0) * WN * RM * RN * kWave * 16;
    static_assert(U % 4 == 0, "an iteration is a whole number of 64-deep MFMA groups");
    static_assert(kThreads <= 1024, "block size");
    static_assert(kRedBytes <= 160 * 1024, "LDS budget of one CU");
};

template <int KS, int WN, int U, int RM, int RN, bool kE5M2, bool kABf16, bool kOutBf16>
__global__ __launch_bounds__(kWave * KS * WN) void stream_kernel(const Params p) {
    using S = StreamShape<KS, WN, U, RM, RN>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kRedBytes > 0 ? S::kRedBytes : 16];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int ks = wave / WN;          // which K slice this wave reduces
    const int wave_n = wave % WN;

    const int tiles_n = (p.N + S::kBN - 1) / S::kBN;
    const int tm = blockIdx.x / tiles_n;
    const int tn = blockIdx.x % tiles_n;
    const int m0 = tm * S::kBM;
    const int n0 = tn * S::kBN + wave_n * 16 * RN;

    const uint32_t a_bytes = static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.K) * 2u;
    const uint32_t b_bytes = static_cast<uint32_t>(p.kb_total) * static_cast<uint32_t>(p.N) * 16u;
    const rsrc_t a_rsrc = make_rsrc(p.a, a_bytes);
    const rsrc_t b_rsrc = make_rsrc(p.b, b_bytes);

    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int k_chunks = p.K / 16;
    const int groups_total = (k_chunks + 3) / 4;   // 64-deep groups covering K

    // Row / column base offsets (chunk 0); kOob when the row or column is past the edge.
    uint32_t a_base[RM];
#pragma unroll
    for (int i = 0; i < RM; ++i) {
        const int row = m0 + 16 * i + r16;
        a_base[i] = row < p.M ? static_cast<uint32_t>(row) * static_cast<uint32_t>(p.K) * 2u : kOob;
    }
    uint32_t b_base[RN];
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        const int col = n0 + 16 * j + r16;
        b_base[j] = col < p.N ? static_cast<uint32_t>(col) * 16u : kOob;
    }
    const uint32_t b_chunk_stride = static_cast<uint32_t>(p.N) * 16u;

    struct Frag {
        u32x4 a[S::kGroups][RM][2];
        u32x4 b[S::kGroups][RN];
    };
    auto fetch = [&](Frag& f, int it) {
#pragma unroll
        for (int q = 0; q < S::kGroups; ++q) {
            const int group = (it * S::kGroups + q) * KS + ks;   // K slices interleave group by group
            const int chunk = 4 * group + g;
            const bool in_k = chunk < k_chunks;
#pragma unroll
            for (int i = 0; i < RM; ++i) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const uint32_t off = (a_base[i] == kOob || !in_k)
                                             ? kOob
                                             : a_base[i] + static_cast<uint32_t>(chunk * 16 + 8 * s) * 2u;
                    f.a[q][i][s] = buf_load16(a_rsrc, off);
                }
            }
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                const uint32_t off = (b_base[j] == kOob || !in_k)
                                         ? kOob
                                         : b_base[j] + static_cast<uint32_t>(chunk) * b_chunk_stride;
                f.b[q][j] = buf_load16(b_rsrc, off);
            }
        }
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](const Frag& f) {
#pragma unroll
        for (int q = 0; q < S::kGroups; ++q) {
            half8 xa[RM][2];
#pragma unroll
            for (int i = 0; i < RM; ++i) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    u32x4 v = f.a[q][i][s];
                    if constexpr (kABf16) v = bf16x8_to_f16x8(v);
                    xa[i][s] = __builtin_bit_cast(half8, v);
                }
            }
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                half8 w0, w1;
                decode_chunk<kE5M2>(f.b[q][j], w0, w1);
#pragma unroll
                for (int i = 0; i < RM; ++i) {
                    acc[i][j] = mfma16(w0, xa[i][0], acc[i][j]);
                    acc[i][j] = mfma16(w1, xa[i][1], acc[i][j]);
                }
            }
        }
    };

    // Iterations of this wave: groups ks, ks + KS, ... taken kGroups at a time.
    const int per_iter = S::kGroups * KS;
    const int iters = (groups_total + per_iter - 1) / per_iter;
    Frag f0, f1;
    if (iters > 0) fetch(f0, 0);
    int it = 0;
    for (; it + 1 < iters; it += 2) {
        fetch(f1, it + 1);
        consume(f0);
        if (it + 2 < iters) fetch(f0, it + 2);
        consume(f1);
    }
    if (it < iters) consume(f0);

    if constexpr (KS > 1) {
        // Deterministic join of the K slices: slices 1..KS-1 park their sums in LDS, slice 0 adds them
        // in slice order and runs the epilogue.
        f32x4* red = reinterpret_cast<f32x4*>(lds);
        if (ks > 0) {
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int j = 0; j < RN; ++j)
                    red[(((ks - 1) * WN + wave_n) * RM * RN + i * RN + j) * kWave + lane] = acc[i][j];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int k2 = 1; k2 < KS; ++k2)
#pragma unroll
                for (int i = 0; i < RM; ++i)
#pragma unroll
                    for (int j = 0; j < RN; ++j)
                        acc[i][j] += red[(((k2 - 1) * WN + wave_n) * RM * RN + i * RN + j) * kWave + lane];
            store_tiles<RM, RN, kOutBf16>(p, acc, m0, n0, lane);
        }
    } else {
        store_tiles<RM, RN, kOutBf16>(p, acc, m0, n0, lane);
    }
}

}  // namespace feather
