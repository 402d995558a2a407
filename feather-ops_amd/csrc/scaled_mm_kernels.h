// fp16/bf16 activation x fp8 (e5m2 / e4m3fn) prepacked weight -> fp16/bf16, for gfx950 (CDNA4, wave64).
//
//   c[m, n] = round_out( fp32( sum_k fp16(a[m, k]) * fp16(B[k, n]) ) * scale ) (+ bias[n], in out precision)
//   B[k, n] = b_prepacked[k / 16][n][k % 16]                 (feather_ops/scaled_mm.py:137-150)
// with `scale` one value per tensor or one per output column n (naive.py:29-33).
//
// Semantics follow the reference's naive path (feather_ops/naive.py:4-41) with fp32 accumulation:
// bf16 activations are widened to fp16 with round-to-nearest-even (naive.py:21), the weight byte is
// decoded exactly to fp16 (every e5m2 and e4m3fn value is an fp16 value), the products are summed by
// fp16 MFMAs into fp32 accumulators, the fp32 scale is applied in fp32, the downcast is RNE for both
// output types, and the bias is added after the downcast in the output precision (naive.py:34-40).
//
// Two kernel families share the fragment layout, the decode and the epilogue:
//  - ring_dma_kernel (tile field prefetch = 1): a block owns a BM x BN output tile, waves split it WM x WN,
//                  and K streams through separate activation and weight LDS rings of 16*U-deep stages.
//                  The tiles go from HBM straight into LDS with buffer loads that write LDS; the next
//                  stages are in flight while the current one feeds the MFMAs. bf16 activations are
//                  staged through registers and widened to fp16 once per block in 4-wave blocks, per
//                  fragment after the LDS read in 8-wave blocks. A separate instantiation splits each
//                  tile's K range over several workgroups whose partial sums meet in a workspace.
//  - stream_kernel (prefetch = 0): for skinny M. Weights stream from HBM straight into VGPRs (register
//                  double buffer), activations through a small per-wave LDS double buffer; the block's WM
//                  waves split K, and a short LDS reduction joins their fp32 partial sums. A separate
//                  instantiation also splits each tile's K range over workgroups, joined per fragment.
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
    const float* scale;         // 1 fp32 value (col_scale == 0) or N (col_scale != 0), or nullptr
    const uint16_t* bias;       // [N] in the output dtype, or nullptr
    uint16_t* c;                // [M, N] output bits, row-major
    int32_t M, N, K;
    int32_t kb_total;           // b_prepacked.shape[0]
    int32_t col_scale;          // scale holds one value per output column (16-byte aligned)
    // Split-K (ring kernel only): each output tile's 64-deep stages are cut into `splits` contiguous
    // ranges, one workgroup per range. 1 = no split; then the two pointers are unused.
    int32_t splits;
    uint32_t* split_ctr;        // [tiles * waves] arrival counters: zero before a launch, zero after it
    uint8_t* split_part;        // [tiles][splits][waves][RM * RN][64 lanes] fp32x4 partial sums
    // Ring kernel: workgroups [0, reads_first_blocks) take the reads-first operand schedule, the rest the
    // interleaved one (0: all interleaved). The launcher picks it from the grid's CU occupancy.
    int32_t reads_first_blocks;
    // The weight may be loaded non-temporally (set by the C ABI from the weight's size and the process-wide
    // mode): the launcher does so for tiles whose launch reads each weight byte once (M within one tile row).
    int32_t stream_weight;
};

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kRsrcFlags);
}

// Cache-policy operand of a buffer load: 0 (the default), or kCpolNt, the non-temporal hint. A weight read
// once per launch and streamed from HBM loads faster with it (the caches do not keep its lines); data that a
// later launch would find in the 256 MB MALL loads slower, since nt lines are not kept there.
constexpr int kCpolNt = 2;

template <int kCpol = 0>
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off, uint32_t soff = 0) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), static_cast<int>(soff), kCpol);
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

// e4m3fn -> fp16, exact: every e4m3fn value (normals 2^-6 .. 448, subnormals m 2^-9) is an fp16 normal,
// so gfx950's fp8 -> fp16 conversion at scale 1 (v_cvt_scalef32_pk_f16_fp8: the two codes of one 16-bit
// word per instruction) is exact, and the NaN codes 0x7f / 0xff convert to fp16 NaNs. One instruction per
// two codes, against ten bit operations and an fp16 multiply for the same exact result by hand.
__device__ __forceinline__ void e4m3x4_to_f16(uint32_t p, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(p, 1.0f, false));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(p, 1.0f, true));
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

// Two fp32 values -> a packed pair of the output type, each rounded to nearest even, subnormals kept, NaN staying
// NaN (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32).
template <bool kOutBf16>
__device__ __forceinline__ uint32_t pack_out(float x, float y) {
    if constexpr (kOutBf16) {
        using bf16x2v = __bf16 __attribute__((ext_vector_type(2)));
        using f32x2 = float __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x, y}), bf16x2v));
    } else {
        return __builtin_bit_cast(uint32_t, (half2v{static_cast<_Float16>(x), static_cast<_Float16>(y)}));
    }
}

// The epilogue's arithmetic for 4 consecutive columns of one row (naive.py:29-40): the fp32 product with the
// scale, rounded to the output type, then the bias added in the output precision (the fp32 sum of two fp16 or
// bf16 values rounded once, as a packed fp16 add rounds it), with packed conversions: 4 multiplies and 2
// conversions for 4 outputs, plus 2 packed adds with a bias (fp16). The product is rounded to fp32 first, as
// the reference computes it: a multiply whose result goes straight to an fp16 conversion compiles to
// v_fma_mixlo_f16, one rounding of the exact product, which differs from that by one fp16 ulp now and then;
// the packed conversion keeps the two roundings.
template <bool kOutBf16, bool kBias>
__device__ __forceinline__ u32x2 out4(const f32x4 acc, const f32x4 sc, const u32x2 bias_bits) {
    uint32_t d[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        d[h] = pack_out<kOutBf16>(acc[2 * h] * sc[2 * h], acc[2 * h + 1] * sc[2 * h + 1]);
        if constexpr (kBias) {
            if constexpr (kOutBf16) {
                const float y0 = __builtin_bit_cast(float, d[h] << 16) + __builtin_bit_cast(float, bias_bits[h] << 16);
                const float y1 = __builtin_bit_cast(float, d[h] & 0xffff0000u) +
                                 __builtin_bit_cast(float, bias_bits[h] & 0xffff0000u);
                d[h] = pack_out<true>(y0, y1);
            } else {
                // The element goes through a scalar first: this hipcc's __builtin_bit_cast of an ext-vector
                // element lvalue (bias_bits[h] itself) reads element 0 whatever h is.
                const uint32_t bias_pair = bias_bits[h];
                d[h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, d[h]) + __builtin_bit_cast(half2v, bias_pair));
            }
        }
    }
    return u32x2{d[0], d[1]};
}

// acc (4 consecutive columns of one row) -> scaled, rounded, biased output bits, packed for one 8-byte store.
// scale: the 4 columns' scales (all equal for a per-tensor scale).
template <bool kOutBf16>
__device__ __forceinline__ u32x2 epilogue4(const f32x4 acc, f32x4 scale, bool has_bias, u32x2 bias_bits) {
    return has_bias ? out4<kOutBf16, true>(acc, scale, bias_bits) : out4<kOutBf16, false>(acc, scale, bias_bits);
}

__device__ __forceinline__ f32x4 mfma16(half8 w, half8 x, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(w, x, acc, 0, 0, 0);
}

// The per-tensor weight scale, read once at kernel start so that its latency hides under the main loop
// (1 when there is none or the scales are per column).
__device__ __forceinline__ float load_scale(const Params& p) {
    return p.scale && !p.col_scale ? *p.scale : 1.0f;
}

// Per-column scales of the 4 columns each lane stores in each of a wave's RN column tiles (16-byte loads:
// the 4 columns start at a multiple of 4), issued together. Columns past N read 0; they are not stored.
template <int RN>
__device__ __forceinline__ void load_col_scales(const Params& p, int col0, int lane, f32x4 (&scales)[RN]) {
    const int c_in = 4 * (lane >> 4);
    const rsrc_t scale_rsrc = make_rsrc(p.scale, static_cast<uint32_t>(p.N) * 4u);
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        const int col = col0 + 16 * j + c_in;
        const uint32_t off = col < p.N ? static_cast<uint32_t>(col) * 4u : kOob;
        scales[j] = __builtin_bit_cast(f32x4, buf_load16(scale_rsrc, off));
    }
}

// The scale operand of store_tiles: one per-tensor value, or RN vectors of per-column values.
__device__ __forceinline__ f32x4 tile_scale(float scale, int) {
    return f32x4{scale, scale, scale, scale};
}

template <int RN>
__device__ __forceinline__ f32x4 tile_scale(const f32x4 (&scales)[RN], int j) {
    return scales[j];
}

// Bias bits of the 4 columns each lane stores in each of a wave's RN column tiles, all loads issued
// together (one round trip for the wave). Zero when there is no bias.
template <int RN>
__device__ __forceinline__ void load_bias(const Params& p, int col0, int lane, u32x2 (&bias_bits)[RN]) {
    const int c_in = 4 * (lane >> 4);
    if (p.bias) {
        const rsrc_t bias_rsrc = make_rsrc(p.bias, static_cast<uint32_t>(p.N) * 2u);
#pragma unroll
        for (int j = 0; j < RN; ++j) {
            const int col = col0 + 16 * j + c_in;
            bias_bits[j] = buf_load8(bias_rsrc, col < p.N ? static_cast<uint32_t>(col) * 2u : kOob);
        }
    } else {
#pragma unroll
        for (int j = 0; j < RN; ++j) bias_bits[j] = u32x2{0u, 0u};
    }
}

// Store one wave's RM x RN accumulator tiles. rows0/cols0: the wave's first output row and column.
// scale: a float (per tensor) or f32x4[RN] (per column, from load_col_scales).
template <int RM, int RN, bool kOutBf16, typename Scale>
__device__ __forceinline__ void store_tiles(const Params& p, const f32x4 (&acc)[RM][RN], int row0, int col0,
                                            int lane, const Scale& scale, const u32x2 (&bias_bits)[RN]) {
    const rsrc_t c_rsrc = make_rsrc(p.c, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.N) * 2u);
    const bool has_bias = p.bias != nullptr;
    const int r_in = lane & 15;
    const int c_in = 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        const int col = col0 + 16 * j + c_in;
        const bool col_ok = col < p.N;
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int row = row0 + 16 * i + r_in;
            const bool ok = col_ok && row < p.M;
            const uint32_t off = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.N) +
                                       static_cast<uint32_t>(col)) * 2u
                                    : kOob;
            buf_store8(epilogue4<kOutBf16>(acc[i][j], tile_scale(scale, j), has_bias, bias_bits[j]), c_rsrc, off);
        }
    }
}

// A wave's whole epilogue: bias (and per-column scale) loads for its RN column tiles, all in flight
// together, then the RM x RN stores. The scale mode is uniform, so each branch is a straight-line store
// sequence and the per-tensor one holds no scale vectors.
template <int RM, int RN, bool kOutBf16>
__device__ __forceinline__ void store_wave_tiles(const Params& p, const f32x4 (&acc)[RM][RN], int row0, int col0,
                                                 int lane, float scale) {
    u32x2 bias_bits[RN];
    load_bias<RN>(p, col0, lane, bias_bits);
    if (p.col_scale) {
        f32x4 col_scales[RN];
        load_col_scales<RN>(p, col0, lane, col_scales);
        store_tiles<RM, RN, kOutBf16>(p, acc, row0, col0, lane, col_scales, bias_bits);
    } else {
        store_tiles<RM, RN, kOutBf16>(p, acc, row0, col0, lane, scale, bias_bits);
    }
}

// ---- block -> tile mapping -------------------------------------------------------------------------------

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

// ---- split-K join ------------------------------------------------------------------------------------------

// Buffer instruction cache-policy bit that makes a load or store coherent at device (agent) scope on gfx950:
// stores write through to the point shared by all XCDs, loads never return a stale cached line. (It is the
// bit the compiler itself sets for relaxed agent-scope atomic loads and stores.)
constexpr int kDeviceScope = 16;

// One wave's side of the split-K join, after its K range is accumulated. A tile joins in kSlots independent
// parts (the ring kernel: one per wave's sub-tile; the streaming kernel: one per 16 x 16 fragment), and the
// wave holds part `slot`. It parks its partial sums in that part's place in the workspace with
// device-coherent stores, waits until they are written, and counts itself in at the (tile, slot) counter.
// The last of the part's `splits` waves to arrive reads every partial back,
// adds them in split order 0, 1, ..., splits - 1 (the same order whichever arrives last, so results are
// deterministic), resets the counter to zero for the next launch and returns true: it then stores the tile.
// The others return false and end. No wave ever waits for another workgroup, so the join cannot stall
// whatever the dispatch order. Agent-scope fences would do instead of the coherent accesses, but they write
// back and invalidate the whole L2 of the XCD under every co-resident workgroup (measured 1.5-2x slower).
template <int kSlots, int RM, int RN>
__device__ __forceinline__ bool join_split(const Params& p, f32x4 (&acc)[RM][RN], int tile_id, int split, int slot_id,
                                           int lane) {
    constexpr uint32_t kSlotBytes = RM * RN * kWave * 16;
    const rsrc_t part = make_rsrc(p.split_part, 0x7fffffffu);
    const auto slot = [&](int s) {
        return (static_cast<uint32_t>(tile_id * p.splits + s) * kSlots + static_cast<uint32_t>(slot_id)) * kSlotBytes +
               static_cast<uint32_t>(lane) * 16u;
    };
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), part,
                                                   slot(split) + (i * RN + j) * kWave * 16u, 0, kDeviceScope);
    // The stores must be complete (visible at device scope) before the counter says so; the memory clobber
    // keeps the compiler from moving the atomic above them.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint32_t* ctr = p.split_ctr + tile_id * kSlots + slot_id;
    uint32_t arrived = 0;
    if (lane == 0) arrived = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    arrived = __builtin_amdgcn_readfirstlane(arrived);
    asm volatile("" ::: "memory");  // the partial reads below stay after the atomic
    if (arrived != static_cast<uint32_t>(p.splits - 1)) return false;
    for (int s = 0; s < p.splits; ++s) {
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                const f32x4 v = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(part, slot(s) + (i * RN + j) * kWave * 16u, 0,
                                                                 kDeviceScope));
                acc[i][j] = s == 0 ? v : acc[i][j] + v;
            }
    }
    if (lane == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// ---- ring kernel: direct-to-LDS loads, LDS ring of 64-deep stages -----------------------------------------

// s_waitcnt immediate that waits until at most n vector-memory operations of this wave are outstanding
// and leaves the other counters alone (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
constexpr int vmcnt_imm(int n) {
    return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8);
}

// s_waitcnt immediate that waits for every outstanding LDS operation of this wave (vmcnt left alone).
constexpr int kLgkm0Imm = 0xf | (0x3 << 14) | (0x7 << 4);

// Workgroup barrier that does not wait for outstanding loads (unlike __syncthreads, whose fence waits
// for every in-flight load, including the ones filling later ring stages). The memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier_only() {
    asm volatile("s_barrier" ::: "memory");
}

// Ring schedule shared by the host-side tile checks and the kernel: A stage t lands in A slot t % SA and is
// issued LA = SA - 1 stages ahead, B stage t in B slot t % SB, LB = SB - 1 ahead (LB >= LA). Iteration u
// issues A(u + LA) and then B(u + LB); the prologue runs the same pattern for u = -LB .. -1. Returns how
// many of this wave's loads were issued after both A(t) and B(t), up to the end of iteration t - 1, when r
// stages follow t: the vmcnt that waits for stage t and nothing newer (loads retire in issue order).
constexpr int ring_loads_after(int LA, int LB, int nA, int nB, int r) {
    int count = 0;
    if (LB > LA && LB - LA <= r) count += nB;  // B(t - LA + LB), issued right after A(t)
    for (int d = 1; d < LA; ++d) {             // iteration t - LA + d: A(t + d), B(t + d + LB - LA)
        if (d <= r) count += nA;
        if (d + LB - LA <= r) count += nB;
    }
    return count;
}

// s_waitcnt for stage t given r = stages - 1 - t (an immediate per case; r >= R covers every larger r).
template <int LA, int LB, int nA, int nB, int R = LB>
__device__ __forceinline__ void wait_ring_stage(int r) {
    if constexpr (R > 0) {
        if (r >= R) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(ring_loads_after(LA, LB, nA, nB, R)));
            return;
        }
        wait_ring_stage<LA, LB, nA, nB, R - 1>(r);
    } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
}

// 16 bytes per lane from buffer offset voff + soff straight into LDS at lds_dst + 16 * lane (lds_dst is
// wave-uniform). soff is a scalar (SGPR) offset, so a per-lane offset computed once can walk K.
template <int kCpol = 0>
__device__ __forceinline__ void dma16(rsrc_t r, const uint8_t* lds_dst, uint32_t voff, uint32_t soff = 0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(reinterpret_cast<uintptr_t>(lds_dst)), 16,
        static_cast<int>(voff), static_cast<int>(soff), 0, kCpol);
}

constexpr int gcd(int a, int b) {
    return b == 0 ? a : gcd(b, a % b);
}

constexpr int lcm(int a, int b) {
    return a / gcd(a, b) * b;
}

// A compile-time choice passed to generic lambdas.
template <bool B>
struct Flag {
    static constexpr bool value = B;
};

template <int WM, int WN, int U, int RM, int RN, bool kDeep = false>
struct DmaShape {
    static constexpr int kWaves = WM * WN;
    static constexpr int kThreads = kWave * kWaves;
    static constexpr int kBM = 16 * WM * RM;
    static constexpr int kBN = 16 * WN * RN;
    static constexpr int kUnitsPerRow = 2 * U;            // 16-byte units in one A row of a stage
    static constexpr int kABytes = kBM * U * 32;          // A: [row][2U units], units XOR-swizzled per row
    static constexpr int kBBytes = kBN * U * 16;          // B: [chunk][col][16 bytes]
    static constexpr int kStageBytes = kABytes + kBBytes;
    // Ring slots. Blocks of up to 4 waves keep 2 A slots within 80 KiB so that two or three blocks share a CU
    // (one block's MFMAs run while another waits at its barrier); bigger blocks keep 3 A slots in 160 KiB.
    // The weight ring gets one slot more (one more stage in flight) when that fits the budget and the tile
    // is already limited to that many blocks per CU: weight tiles are shared by fewer co-resident blocks
    // than activation tiles, so their loads miss L2 more often and need the longer lead.
    // The deep variant (64-row tiles only, launched when all of a small grid's blocks fit on the CUs at
    // once) keeps 3 A and 4 B slots: with one or two blocks per CU and stages of 8-16 KiB, the shallow ring
    // has a single stage in flight and the block waits out the memory latency at every stage.
    static constexpr int kSlotsA0 = kWaves <= 4 ? 2 : 3;
    static constexpr int kBudget = (kWaves <= 4 ? 80 : 160) * 1024;
    static constexpr bool kDeepB = kSlotsA0 * kABytes + (kSlotsA0 + 1) * kBBytes <= kBudget &&
                                   (kWaves > 4 || 2 * kStageBytes > 160 * 1024 / 3);
    static constexpr int kSlotsA = kDeep ? 3 : kSlotsA0;
    static constexpr int kSlotsB = kDeep ? 4 : kSlotsA0 + (kDeepB ? 1 : 0);
    static constexpr int kLeadA = kSlotsA - 1;
    static constexpr int kLeadB = kSlotsB - 1;
    static constexpr int kPeriod = lcm(kSlotsA, kSlotsB);  // one period of both rings: compile-time slots
    static constexpr int kBRing = kSlotsA * kABytes;  // LDS offset of the B ring
    static constexpr int kLdsBytes = kSlotsA * kABytes + kSlotsB * kBBytes;
    // Blocks per CU the LDS allows (the register budgets of the tiles allow as many).
    static constexpr int kBlocksPerCu = 160 * 1024 / kLdsBytes;
    // Waves per SIMD the register budget must allow: two co-resident 4-wave blocks need two, three need
    // three (at most 168 VGPRs). Tiles that share a CU more ways stay far below their budget and keep the
    // two-wave bound, which leaves the compiler's schedule for them as it is.
    static constexpr int kWavesPerEu = kWaves <= 4 ? (kBlocksPerCu == 3 ? 3 : 2) : (kWaves + 3) / 4;
    static constexpr int kAInstr = kBM * kUnitsPerRow / kWave / kWaves;   // 1 KiB direct loads per wave
    static constexpr int kBInstr = U * kBN / kWave / kWaves;
    static_assert(U % 4 == 0, "a stage is a whole number of 64-deep MFMA groups");
    static_assert(!kDeep || kBM <= 64, "the deep ring is for 64-row tiles");
    static_assert(kLeadB >= kLeadA, "the weight ring leads at least as far as the activation ring");
    static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");
    static_assert(kBM * kUnitsPerRow % (kWave * kWaves) == 0, "A stage splits into whole wave loads");
    static_assert(kBN % kWave == 0 && (U * kBN / kWave) % kWaves == 0, "B stage splits into whole wave loads");
    static_assert(ring_loads_after(kLeadA, kLeadB, kAInstr, kBInstr, kLeadB) < 64, "vmcnt range");
};

// Physical 16-byte unit of logical unit u in A row `row`. The XOR key depends on row mod 16 only, so it is
// the same for every 16-row fragment a lane reads and folds into one per-lane base address. The keys give
// the 16 rows one fragment read touches 16 distinct bank groups whether the LDS serves 8 or 16 lanes of a
// 16-byte read per cycle: with 8 units per row (128-byte rows) (r ^ (r >> 3)) & 7, wider rows r itself.
template <int kUnits>
__device__ __forceinline__ int a_swizzle_key(int row) {
    const int r = row & 15;
    if constexpr (kUnits == 8) {
        return (r ^ (r >> 3)) & 7;
    } else {
        return r & (kUnits - 1);
    }
}

template <int kUnits>
__device__ __forceinline__ int a_unit_phys(int row, int u) {
    return u ^ a_swizzle_key<kUnits>(row);
}

// A wave's epilogue staged through LDS, for kernels whose waves all reach it (a block barrier comes first):
// the wave writes its rounded, biased 16 RM x 16 RN output tile into its own LDS area (`area`, rows
// 16 RN * 2 + 16 bytes apart, so the 8-byte writes of a fragment's 16 rows fall in distinct banks), then stores
// it as 16-byte pieces, consecutive lanes covering whole row segments (2 RN lanes per row, 32 / RN rows per
// instruction). Against the 8-byte stores of 16 rows x 32 bytes that store_wave_tiles issues: half the store
// instructions, and every row segment written whole (measured 4.8% faster on a 128 x 256 tile).
template <int RM, int RN, bool kOutBf16>
__device__ __forceinline__ void store_wave_tiles_via_lds(const Params& p, const f32x4 (&acc)[RM][RN], uint8_t* area,
                                                         int row0, int col0, int lane, float scale) {
    constexpr int kRowBytes = 16 * RN * 2;
    constexpr int kPitch = kRowBytes + 16;
    constexpr int kRows = 16 * RM;
    constexpr int kLanesPerRow = kRowBytes / 16;
    constexpr int kRowsPerInstr = kWave / kLanesPerRow;
    static_assert(kWave % kLanesPerRow == 0 && kRows % kRowsPerInstr == 0, "whole rows per store instruction");
    u32x2 bias_bits[RN];
    load_bias<RN>(p, col0, lane, bias_bits);
    f32x4 col_scales[RN];
    if (p.col_scale) load_col_scales<RN>(p, col0, lane, col_scales);
    const bool has_bias = p.bias != nullptr;
    const int r_in = lane & 15;
    const int c_in = 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) {
            const f32x4 sc = p.col_scale ? col_scales[j] : f32x4{scale, scale, scale, scale};
            *reinterpret_cast<u32x2*>(area + (16 * i + r_in) * kPitch + (16 * j + c_in) * 2) =
                epilogue4<kOutBf16>(acc[i][j], sc, has_bias, bias_bits[j]);
        }
    __builtin_amdgcn_s_waitcnt(kLgkm0Imm);  // the wave reads back only what it wrote itself
    const rsrc_t c_rsrc = make_rsrc(p.c, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.N) * 2u);
    // N % 8 == 0, so a piece of 8 columns lies wholly inside N or wholly outside
    const int col = col0 + (lane % kLanesPerRow) * 8;
#pragma unroll
    for (int q = 0; q < kRows / kRowsPerInstr; ++q) {
        const int r = kRowsPerInstr * q + lane / kLanesPerRow;
        const u32x4 v = *reinterpret_cast<const u32x4*>(area + r * kPitch + (lane % kLanesPerRow) * 16);
        const int row = row0 + r;
        const uint32_t off = col < p.N && row < p.M ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.N) +
                                                       static_cast<uint32_t>(col)) * 2u
                                                    : kOob;
        __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, static_cast<int>(off), 0, 0);
    }
}

// LDS bytes store_wave_tiles_via_lds stages per wave.
template <int RM, int RN>
constexpr int lds_epilogue_bytes() {
    return 16 * RM * (16 * RN * 2 + 16);
}

// kSplitK: this launch splits K (p.splits > 1). A separate instantiation, so the unsplit kernel carries no
// join code (its partial reads raise register pressure: measured 3% slower on a 128 x 256 tile).
// kDeep: the deep-ring variant of a 64-row tile (DmaShape), chosen by the launcher for small grids.
// kNtWeight: the weight's direct loads carry the non-temporal hint (launches that read the weight once).
template <int WM, int WN, int U, int RM, int RN, bool kE5M2, bool kABf16, bool kOutBf16, bool kSplitK, bool kDeep,
          bool kNtWeight = false>
__global__ __launch_bounds__(kWave * WM * WN)
__attribute__((amdgpu_waves_per_eu(DmaShape<WM, WN, U, RM, RN, kDeep>::kWavesPerEu))) void ring_dma_kernel(
    const Params p) {
    using S = DmaShape<WM, WN, U, RM, RN, kDeep>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform: scalar LDS addresses
    const int wave_m = wave / WN;
    const int wave_n = wave % WN;

    const int tiles_m = (p.M + S::kBM - 1) / S::kBM;
    const int tiles_n = (p.N + S::kBN - 1) / S::kBN;
    // Workgroup -> (K range, tile): split-major, so the workgroups of one K range walk the tiles in the
    // XCD-aware order and share operand panels as the unsplit grid does.
    const int n_tiles = tiles_m * tiles_n;
    const int splits = kSplitK ? p.splits : 1;
    const int split = kSplitK ? static_cast<int>(blockIdx.x) / n_tiles : 0;
    const int tile_id = static_cast<int>(blockIdx.x) - split * n_tiles;
    int tm, tn;
    tile_of_block(tile_id, n_tiles, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * S::kBM;
    const int n0 = tn * S::kBN;

    const rsrc_t a_rsrc = make_rsrc(p.a, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.K) * 2u);
    const rsrc_t b_rsrc = make_rsrc(p.b, static_cast<uint32_t>(p.kb_total) * static_cast<uint32_t>(p.N) * 16u);
    const int k_chunks = p.K / 16;
    // This workgroup's stages: global stages [stage0, stage0 + stages). Loads address global stages; the
    // ring slots and the wait schedule count local ones.
    const int stages_total = (p.K + 16 * U - 1) / (16 * U);
    const int stage0 = split * stages_total / splits;
    const int stages = (split + 1) * stages_total / splits - stage0;
    const float scale = load_scale(p);
    const int full_stages = k_chunks / U;  // stages with every chunk inside K

    // Direct loads: instruction i of this wave fills 1 KiB of LDS, lane l the l-th 16 bytes of it. The
    // per-lane offsets are for stage 0; a stage adds a scalar offset. Out-of-range rows and columns carry
    // kOob, which stays past the buffer's end whatever is added.
    uint32_t a_off[S::kAInstr];
    int a_chunk[S::kAInstr];
#pragma unroll
    for (int i = 0; i < S::kAInstr; ++i) {
        const int unit = (wave + i * S::kWaves) * kWave + lane;
        const int row = unit / S::kUnitsPerRow;
        const int u = a_unit_phys<S::kUnitsPerRow>(row, unit % S::kUnitsPerRow);  // XOR is its own inverse
        a_chunk[i] = u >> 1;
        const int grow = m0 + row;
        a_off[i] = grow < p.M ? (static_cast<uint32_t>(grow) * static_cast<uint32_t>(p.K) +
                                 static_cast<uint32_t>(u * 8)) * 2u
                              : kOob;
    }
    uint32_t b_off[S::kBInstr];
    int b_chunk[S::kBInstr];
#pragma unroll
    for (int i = 0; i < S::kBInstr; ++i) {
        const int unit = (wave + i * S::kWaves) * kWave + lane;
        const int chunk = unit / S::kBN;
        const int gcol = n0 + unit % S::kBN;
        b_chunk[i] = chunk;
        b_off[i] = gcol < p.N ? (static_cast<uint32_t>(chunk) * static_cast<uint32_t>(p.N) +
                                 static_cast<uint32_t>(gcol)) * 16u
                              : kOob;
    }
    const uint32_t b_stage_stride = static_cast<uint32_t>(U) * static_cast<uint32_t>(p.N) * 16u;

    // Stages at or past full_stages are the ragged last one: chunks past K read zeros.
    // fp16 activations go straight to LDS (issue_a). bf16 activations in 4-wave blocks are staged through
    // registers (load_a) and widened to fp16 once per block when written to LDS (commit_a), so the operand
    // reads need no conversion and no element is widened twice (measured ~9% faster on 4096x3072x3072).
    // 8-wave blocks keep the deeper direct-load ring for bf16 too and widen per fragment (register staging
    // shortens their activation lead from two stages to one and measured 11% slower), and so does the deep
    // ring (launched for bf16 only at M <= 64 on tiles of at most two column waves): its small grids are
    // latency-bound, and a one-stage activation lead undid the deep ring (32x5120x25600 on the 64 x 64
    // tile: 106 TFLOP/s staged, 235 widened per fragment).
    constexpr bool kStageA = kABf16 && S::kWaves <= 4 && !kDeep;
    u32x4 a_regs[S::kAInstr];
    auto load_a = [&](int local_stage) {
        const int stage = stage0 + local_stage;
        const uint32_t soff = static_cast<uint32_t>(stage) * static_cast<uint32_t>(U) * 32u;
        if (stage < full_stages) {
#pragma unroll
            for (int i = 0; i < S::kAInstr; ++i) a_regs[i] = buf_load16(a_rsrc, a_off[i], soff);
        } else {
#pragma unroll
            for (int i = 0; i < S::kAInstr; ++i) {
                const bool ok = stage * U + a_chunk[i] < k_chunks;
                a_regs[i] = buf_load16(a_rsrc, ok ? a_off[i] : kOob, soff);
            }
        }
    };
    auto commit_a = [&](int slot) {
        uint8_t* base = lds + slot * S::kABytes + lane * 16;
#pragma unroll
        for (int i = 0; i < S::kAInstr; ++i) {
            *reinterpret_cast<u32x4*>(base + (wave + i * S::kWaves) * 1024) = bf16x8_to_f16x8(a_regs[i]);
        }
    };
    auto issue_a = [&](int local_stage) {
        uint8_t* base = lds + (local_stage % S::kSlotsA) * S::kABytes;
        const int stage = stage0 + local_stage;
        const uint32_t soff = static_cast<uint32_t>(stage) * static_cast<uint32_t>(U) * 32u;
        if (stage < full_stages) {
#pragma unroll
            for (int i = 0; i < S::kAInstr; ++i) dma16(a_rsrc, base + (wave + i * S::kWaves) * 1024, a_off[i], soff);
        } else {
#pragma unroll
            for (int i = 0; i < S::kAInstr; ++i) {
                const bool ok = stage * U + a_chunk[i] < k_chunks;
                dma16(a_rsrc, base + (wave + i * S::kWaves) * 1024, ok ? a_off[i] : kOob, soff);
            }
        }
    };
    auto issue_b = [&](int local_stage) {
        uint8_t* base = lds + S::kBRing + (local_stage % S::kSlotsB) * S::kBBytes;
        const int stage = stage0 + local_stage;
        const uint32_t soff = static_cast<uint32_t>(stage) * b_stage_stride;
        if (stage < full_stages) {
#pragma unroll
            for (int i = 0; i < S::kBInstr; ++i) {
                dma16<kNtWeight ? kCpolNt : 0>(b_rsrc, base + (wave + i * S::kWaves) * 1024, b_off[i], soff);
            }
        } else {
#pragma unroll
            for (int i = 0; i < S::kBInstr; ++i) {
                const bool ok = stage * U + b_chunk[i] < k_chunks;
                dma16<kNtWeight ? kCpolNt : 0>(b_rsrc, base + (wave + i * S::kWaves) * 1024, ok ? b_off[i] : kOob,
                                               soff);
            }
        }
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int a_row_base = wave_m * 16 * RM + r16;
    const int b_col_base = wave_n * 16 * RN + r16;

    // Per-lane LDS byte offsets within a stage; everything else is a compile-time immediate. Lane group g
    // reads chunk 4q + g of the stage, whose two 16-byte halves (s = 0, 1) feed the group's two MFMAs and
    // sit at units (8q + 2g + s) ^ key of the row; the key depends on the lane only (row mod 16), so each
    // (q, s) needs one base register.
    const int key = a_swizzle_key<S::kUnitsPerRow>(a_row_base);
    constexpr int kGroups = U / 4;
    int a_lane[kGroups][2];
#pragma unroll
    for (int q = 0; q < kGroups; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
            a_lane[q][s2] = a_row_base * (S::kUnitsPerRow * 16) + (((8 * q + 2 * g + s2) ^ key) << 4);
    const int b_lane = g * S::kBN * 16 + b_col_base * 16;

    // Two schedules of a stage's LDS reads. Reads first: right after the stage's barrier the wave issues all
    // of the stage's LDS reads (RN weight and 2 RM activation fragments; a scheduling barrier keeps the
    // compiler from spreading them out), then the stage's refills, then waits once, decodes every weight
    // fragment and issues the stage's MFMAs as one uninterrupted run. The waves of a SIMD belong to
    // different blocks, so one wave's reads, refills and decode run under the others' MFMA runs: on a CU
    // holding the tile's full complement of blocks that is 3-5% faster than the interleaved schedule (C3,
    // and C2 with the refills after the reads). Where CUs hold fewer blocks it measured slower when first
    // built (a 128 x 256 block alone on its CU: ~18%; 128 x 128 tiles two per CU: 2-6%) and still is with
    // bf16 activations and in split launches, hence the launcher's per-workgroup choice (reads_first_blocks);
    // unsplit fp16 launches of the current kernel gain 1-4% from it there too and take it everywhere.
    // Interleaved: the refills go out first, then each k half's reads issue as its
    // MFMAs need them. Reads first holds all of a stage's operands at once, up to 8 (RM + RN) more VGPRs:
    // the bf16-activation variants of the larger wave tiles cannot spare them (they would spill), tiles
    // sharing a CU four or more ways would lose a block per CU to them, and 8-wave blocks pair a SIMD's
    // waves inside one block, in step.
    constexpr bool kReadsFirst = kGroups == 1 && S::kWaves <= 4 && S::kBlocksPerCu >= 2 && S::kBlocksPerCu <= 3 &&
                                 (!kABf16 || (RM <= 4 && RN <= 4));
    if constexpr (kReadsFirst) {
        struct StageOperands {
            u32x4 b[RN];
            u32x4 a[2][RM];
        };
        auto read_stage = [&](const uint8_t* a_stage, const uint8_t* b_stage, StageOperands& op) {
#pragma unroll
            for (int j = 0; j < RN; ++j) op.b[j] = *reinterpret_cast<const u32x4*>(b_stage + b_lane + 16 * j * 16);
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int i = 0; i < RM; ++i)
                    op.a[s2][i] =
                        *reinterpret_cast<const u32x4*>(a_stage + a_lane[0][s2] + i * 16 * S::kUnitsPerRow * 16);
        };
        auto multiply_stage = [&](const StageOperands& op) {
            half8 w[2][RN];
#pragma unroll
            for (int j = 0; j < RN; ++j) decode_chunk<kE5M2>(op.b[j], w[0][j], w[1][j]);
            // Each activation fragment feeds its RN MFMAs back to back, the weight fragment changing each time;
            // odd fragments take the weights in reverse, so one weight operand carries across the boundary
            // (~1% faster than restarting at j = 0; holding a weight fragment for RM MFMAs instead, or
            // swapping the operands' places, measured 2-10% slower).
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int i = 0; i < RM; ++i) {
                    const half8 x =
                        __builtin_bit_cast(half8, (kABf16 && !kStageA) ? bf16x8_to_f16x8(op.a[s2][i]) : op.a[s2][i]);
#pragma unroll
                    for (int jj = 0; jj < RN; ++jj) {
                        const int j = (i & 1) ? RN - 1 - jj : jj;
                        acc[i][j] = mfma16(w[s2][j], x, acc[i][j]);
                    }
                }
        };
        // One stage of the ring loop after its barrier: `refill` issues the stage's refills.
        auto run_stage = [&](auto reads_first, const uint8_t* a_stage, const uint8_t* b_stage, auto refill) {
            if constexpr (decltype(reads_first)::value) {
                StageOperands op;
                read_stage(a_stage, b_stage, op);
                refill();
                __builtin_amdgcn_sched_barrier(0);
                multiply_stage(op);
            } else {
                refill();
#pragma unroll
                for (int q = 0; q < kGroups; ++q) {
                    u32x4 braw[RN];
#pragma unroll
                    for (int j = 0; j < RN; ++j) {
                        braw[j] = *reinterpret_cast<const u32x4*>(b_stage + b_lane + (4 * q * S::kBN + 16 * j) * 16);
                    }
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        half8 w[RN];
#pragma unroll
                        for (int j = 0; j < RN; ++j) {
                            half8 w0, w1;
                            decode_chunk<kE5M2>(braw[j], w0, w1);
                            w[j] = s2 == 0 ? w0 : w1;
                        }
#pragma unroll
                        for (int i = 0; i < RM; ++i) {
                            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                                a_stage + a_lane[q][s2] + i * 16 * S::kUnitsPerRow * 16);
                            const half8 x =
                                __builtin_bit_cast(half8, (kABf16 && !kStageA) ? bf16x8_to_f16x8(raw) : raw);
#pragma unroll
                            for (int j = 0; j < RN; ++j) acc[i][j] = mfma16(w[j], x, acc[i][j]);
                        }
                    }
                }
            }
        };
        // Runs `loop` with the schedule this workgroup takes; one copy of the loop per schedule.
        const bool reads_first = static_cast<int>(blockIdx.x) < p.reads_first_blocks;
        auto with_schedule = [&](auto loop) {
            if constexpr (kReadsFirst) {
                if (reads_first) {
                    loop(Flag<true>{});
                    return;
                }
            }
            loop(Flag<false>{});
        };

        if constexpr (kStageA) {
            // Iteration u loads A(u + 1) into registers and issues B(u + LB); the prologue runs the same pattern
            // for u = -LB .. -1, then commits A(0). With LB >= 2 every B(t) is issued before A(t), so the wait for
            // A(t)'s registers in commit_a (placed by the compiler; loads retire in issue order) also retires
            // B(t); with LB == 1, B(t) follows A(t) and the iteration waits for it explicitly.
#pragma unroll
            for (int u = -S::kLeadB; u < 0; ++u) {
                if (u == -1) load_a(0);
                if (u + S::kLeadB < stages) issue_b(u + S::kLeadB);
            }
            commit_a(0);
            with_schedule([&](auto reads_first) {
                for (int t0 = 0; t0 < stages; t0 += S::kPeriod) {
#pragma unroll
                    for (int b = 0; b < S::kPeriod; ++b) {
                        const int t = t0 + b;
                        if (t < stages) {
                            if constexpr (S::kLeadB == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                            // This wave's LDS writes of A(t) are done; the barrier publishes every wave's and
                            // retires all reads of the slots refilled next (they held stage t - 1).
                            __builtin_amdgcn_s_waitcnt(kLgkm0Imm);
                            barrier_only();
                            run_stage(reads_first, lds + (b % S::kSlotsA) * S::kABytes,
                                      lds + S::kBRing + (b % S::kSlotsB) * S::kBBytes, [&] {
                                          __builtin_amdgcn_s_setprio(1);  // see the unstaged loop below
                                          if (t + 1 < stages) load_a(t + 1);
                                          if (t + S::kLeadB < stages) issue_b(t + S::kLeadB);
                                          __builtin_amdgcn_s_setprio(0);
                                      });
                            // The widening and LDS writes of the next stage's activations run at raised priority
                            // too: they gate this block's next barrier (measured +5% on a bf16 128 x 256 tile).
                            __builtin_amdgcn_s_setprio(1);
                            if (t + 1 < stages) commit_a((b + 1) % S::kSlotsA);
                            __builtin_amdgcn_s_setprio(0);
                        }
                    }
                }
            });
        } else {
            // Prologue: iterations -LB .. -1 of the issue pattern.
#pragma unroll
            for (int u = -S::kLeadB; u < 0; ++u) {
                if (u + S::kLeadA >= 0 && u + S::kLeadA < stages) issue_a(u + S::kLeadA);
                if (u + S::kLeadB < stages) issue_b(u + S::kLeadB);
            }

            // One period of both rings per outer iteration, so every slot is a compile-time offset.
            with_schedule([&](auto reads_first) {
                for (int t0 = 0; t0 < stages; t0 += S::kPeriod) {
#pragma unroll
                    for (int b = 0; b < S::kPeriod; ++b) {
                        const int t = t0 + b;
                        if (t < stages) {
                            // Stage t's loads are complete for this wave; the barrier then makes every wave's share
                            // visible and retires all reads of the slots the next issues reuse (they held stage t - 1).
                            wait_ring_stage<S::kLeadA, S::kLeadB, S::kAInstr, S::kBInstr>(stages - 1 - t);
                            barrier_only();
                            // The refills go out at raised wave priority, so a wave issues them ahead of the
                            // co-resident blocks' MFMAs (measured +1.6% on a 128 x 256 tile; raising it for the
                            // MFMAs instead lost).
                            run_stage(reads_first, lds + (b % S::kSlotsA) * S::kABytes,
                                      lds + S::kBRing + (b % S::kSlotsB) * S::kBBytes, [&] {
                                          __builtin_amdgcn_s_setprio(1);
                                          if (t + S::kLeadA < stages) issue_a(t + S::kLeadA);
                                          if (t + S::kLeadB < stages) issue_b(t + S::kLeadB);
                                          __builtin_amdgcn_s_setprio(0);
                                      });
                        }
                    }
                }
            });
        }
    } else {
        // Tiles without the reads-first schedule keep this form of the loop (the same interleaved
        // schedule as run_stage's): the compiler's code for it, and the measured speed of those tiles
        // (bf16 activations on 128 x 256: 1-3%), depend on it.
        auto compute = [&](const uint8_t* a_stage, const uint8_t* b_stage) {
#pragma unroll
            for (int q = 0; q < kGroups; ++q) {
                u32x4 braw[RN];
#pragma unroll
                for (int j = 0; j < RN; ++j) {
                    braw[j] = *reinterpret_cast<const u32x4*>(b_stage + b_lane + (4 * q * S::kBN + 16 * j) * 16);
                }
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    half8 w[RN];
#pragma unroll
                    for (int j = 0; j < RN; ++j) {
                        half8 w0, w1;
                        decode_chunk<kE5M2>(braw[j], w0, w1);
                        w[j] = s2 == 0 ? w0 : w1;
                    }
#pragma unroll
                    for (int i = 0; i < RM; ++i) {
                        const u32x4 raw = *reinterpret_cast<const u32x4*>(
                            a_stage + a_lane[q][s2] + i * 16 * S::kUnitsPerRow * 16);
                        const half8 x = __builtin_bit_cast(half8, (kABf16 && !kStageA) ? bf16x8_to_f16x8(raw) : raw);
#pragma unroll
                        for (int j = 0; j < RN; ++j) acc[i][j] = mfma16(w[j], x, acc[i][j]);
                    }
                }
            }
        };

        if constexpr (kStageA) {
            // Iteration u loads A(u + 1) into registers and issues B(u + LB); the prologue runs the same pattern
            // for u = -LB .. -1, then commits A(0). With LB >= 2 every B(t) is issued before A(t), so the wait for
            // A(t)'s registers in commit_a (placed by the compiler; loads retire in issue order) also retires
            // B(t); with LB == 1, B(t) follows A(t) and the iteration waits for it explicitly.
#pragma unroll
            for (int u = -S::kLeadB; u < 0; ++u) {
                if (u == -1) load_a(0);
                if (u + S::kLeadB < stages) issue_b(u + S::kLeadB);
            }
            commit_a(0);
            for (int t0 = 0; t0 < stages; t0 += S::kPeriod) {
#pragma unroll
                for (int b = 0; b < S::kPeriod; ++b) {
                    const int t = t0 + b;
                    if (t < stages) {
                        if constexpr (S::kLeadB == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                        // This wave's LDS writes of A(t) are done; the barrier publishes every wave's and
                        // retires all reads of the slots refilled next (they held stage t - 1).
                        __builtin_amdgcn_s_waitcnt(kLgkm0Imm);
                        barrier_only();
                        __builtin_amdgcn_s_setprio(1);  // see the unstaged loop below
                        if (t + 1 < stages) load_a(t + 1);
                        if (t + S::kLeadB < stages) issue_b(t + S::kLeadB);
                        __builtin_amdgcn_s_setprio(0);
                        compute(lds + (b % S::kSlotsA) * S::kABytes, lds + S::kBRing + (b % S::kSlotsB) * S::kBBytes);
                        // The widening and LDS writes of the next stage's activations run at raised priority
                        // too: they gate this block's next barrier (measured +5% on a bf16 128 x 256 tile).
                        __builtin_amdgcn_s_setprio(1);
                        if (t + 1 < stages) commit_a((b + 1) % S::kSlotsA);
                        __builtin_amdgcn_s_setprio(0);
                    }
                }
            }
        } else {
            // Prologue: iterations -LB .. -1 of the issue pattern.
#pragma unroll
            for (int u = -S::kLeadB; u < 0; ++u) {
                if (u + S::kLeadA >= 0 && u + S::kLeadA < stages) issue_a(u + S::kLeadA);
                if (u + S::kLeadB < stages) issue_b(u + S::kLeadB);
            }

            // One period of both rings per outer iteration, so every slot is a compile-time offset.
            for (int t0 = 0; t0 < stages; t0 += S::kPeriod) {
#pragma unroll
                for (int b = 0; b < S::kPeriod; ++b) {
                    const int t = t0 + b;
                    if (t < stages) {
                        // Stage t's loads are complete for this wave; the barrier then makes every wave's share
                        // visible and retires all reads of the slots the next issues reuse (they held stage t - 1).
                        wait_ring_stage<S::kLeadA, S::kLeadB, S::kAInstr, S::kBInstr>(stages - 1 - t);
                        barrier_only();
                        // The refills go out at raised wave priority, so a wave that just passed its barrier
                        // issues them ahead of the co-resident block's MFMAs (measured +1.6% on a 128 x 256 tile;
                        // raising it for the MFMAs instead lost).
                        __builtin_amdgcn_s_setprio(1);
                        if (t + S::kLeadA < stages) issue_a(t + S::kLeadA);
                        if (t + S::kLeadB < stages) issue_b(t + S::kLeadB);
                        __builtin_amdgcn_s_setprio(0);
                        compute(lds + (b % S::kSlotsA) * S::kABytes, lds + S::kBRing + (b % S::kSlotsB) * S::kBBytes);
                    }
                }
            }
        }
    }

    if constexpr (kSplitK) {
        // waves leave after the join unless they are their tile's last: no block barrier, per-wave stores
        if (!join_split<S::kWaves, RM, RN>(p, acc, tile_id, split, wave, lane)) return;
        store_wave_tiles<RM, RN, kOutBf16>(p, acc, m0 + wave_m * 16 * RM, n0 + wave_n * 16 * RN, lane, scale);
    } else {
        // the ring is free once every wave has read the last stage: stage the output through it
        static_assert(S::kWaves * lds_epilogue_bytes<RM, RN>() <= S::kLdsBytes, "epilogue staging fits the ring");
        __syncthreads();
        store_wave_tiles_via_lds<RM, RN, kOutBf16>(p, acc, lds + wave * lds_epilogue_bytes<RM, RN>(),
                                                   m0 + wave_m * 16 * RM, n0 + wave_n * 16 * RN, lane, scale);
    }
}

// ---- stream kernel: split-K, global -> VGPR ----------------------------------------------------------------

template <int KS, int WN, int U, int RM, int RN>
struct StreamShape {
    static constexpr int kThreads = kWave * KS * WN;
    static constexpr int kBM = 16 * RM;
    static constexpr int kBN = 16 * WN * RN;
    static constexpr int kGroups = U / 4;             // 64-deep groups per iteration of one wave
    static constexpr int kFrags = WN * RM * RN;       // 16 x 16 output fragments of the block
    static constexpr int kRedBytes = (KS > 1 ? KS : 0) * kFrags * kWave * 16;
    // Fetches a wave keeps in flight. One fetch of the whole block carries KS * WN * RN * kGroups KiB of weight
    // (1 KiB per wave, 16-column fragment and 64-deep group); blocks whose fetch carries at most 8 KiB go
    // three deep, so that 12-24 KiB of weight stay in flight per block, and wider ones two (16-64 KiB), where a
    // third fetch measured slower. Blocks of 4 fragment rows (RM = 4) move 4x the activations per fetch and
    // keep two.
    static constexpr int kDepth = (KS * WN * RN * kGroups <= 8 && RM <= 2) ? 3 : 2;
    // Activations: per wave, one buffer per fetch in flight of one iteration's fragments (16 rows x 64 k x
    // 2 bytes each).
    static constexpr int kAFragBytes = 2048;
    static constexpr int kABufBytes = kGroups * RM * kAFragBytes;
    static constexpr int kAWaveBytes = kDepth * kABufBytes;
    static constexpr int kALdsBytes = KS * WN * kAWaveBytes;
    static constexpr int kLdsBytes = kALdsBytes + kRedBytes;
    static constexpr int kLoadsPerFetch = kGroups * (2 * RM + RN);  // vector-memory ops of one fetch
    static_assert(U % 4 == 0, "an iteration is a whole number of 64-deep MFMA groups");
    static_assert(kThreads <= 1024, "block size");
    static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");
    static_assert((kDepth - 1) * kLoadsPerFetch < 64, "vmcnt range");
};

// kNtWeight: the weight loads carry the non-temporal hint (launches that read the weight once).
template <int KS, int WN, int U, int RM, int RN, bool kE5M2, bool kABf16, bool kOutBf16, bool kSplitK,
          bool kNtWeight = false>
__global__ __launch_bounds__(kWave * KS * WN) void stream_kernel(const Params p) {
    using S = StreamShape<KS, WN, U, RM, RN>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int ks = wave / WN;          // which K slice this wave reduces
    const int wave_n = wave % WN;

    const float scale = load_scale(p);
    const int tiles_n = (p.N + S::kBN - 1) / S::kBN;
    // A split launch runs `splits` workgroups per tile, split-major (as the ring kernel's split launch).
    const int n_tiles = ((p.M + S::kBM - 1) / S::kBM) * tiles_n;
    const int split = kSplitK ? static_cast<int>(blockIdx.x) / n_tiles : 0;
    const int tile_id = static_cast<int>(blockIdx.x) - split * n_tiles;
    const int tm = tile_id / tiles_n;
    const int tn = tile_id % tiles_n;
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
    // This workgroup's groups [group0, group_end): all of them, or its split's share. Chunks from chunk_end
    // on read as zeros (the end of K, or the next split's range).
    const int splits = kSplitK ? p.splits : 1;
    const int group0 = split * groups_total / splits;
    const int group_end = (split + 1) * groups_total / splits;
    const int chunk_end = kSplitK ? min(k_chunks, 4 * group_end) : k_chunks;

    // Activation fragments reach this wave's LDS buffer by direct loads of whole 128-byte row segments
    // (one instruction: 8 rows x 8 units of 16 bytes, unit = 8 consecutive k), so every cache line an
    // instruction touches is used in full. Unit u of fragment row r sits at slot u ^ key(r), the key of the
    // ring kernel's A tiles, so the operand reads below are free of bank conflicts. Lane l of half h fills
    // slot l % 8 of row 8h + l / 8; a_dma[i][h] is its row's offset plus the unit's, kOob past M.
    uint8_t* const a_lds = lds + wave * S::kAWaveBytes;
    uint32_t a_dma[RM][2];
    int a_dma_chunk[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row_in = 8 * h + (lane >> 3);
        const int unit = (lane & 7) ^ a_swizzle_key<8>(row_in);
        a_dma_chunk[h] = unit >> 1;
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int row = m0 + 16 * i + row_in;
            a_dma[i][h] = row < p.M ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.K) +
                                       static_cast<uint32_t>(unit * 8)) * 2u
                                    : kOob;
        }
    }
    // Operand reads: lane (g, r16) takes units 2g (s = 0) and 2g + 1 (s = 1) of row r16.
    int a_rd[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) a_rd[s] = r16 * 128 + (((2 * g + s) ^ a_swizzle_key<8>(r16)) << 4);

    uint32_t b_base[RN];
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        const int col = n0 + 16 * j + r16;
        b_base[j] = col < p.N ? static_cast<uint32_t>(col) * 16u : kOob;
    }
    const uint32_t b_chunk_stride = static_cast<uint32_t>(p.N) * 16u;

    struct Frag {
        u32x4 b[S::kGroups][RN];
    };
    // One iteration's operands: activations into LDS buffer `buf`, weights into registers. The LDS wait
    // first retires this wave's reads of the buffer being refilled. Branch-free (chunks past the range take
    // the out-of-range offset, also for whole iterations past the end, which then load zeros and move no
    // data): every path through the main loop then has the same loads in flight, so the compiler's own
    // register waits agree with the explicit ones below. (With a branch here and a conditional last fetch,
    // the merged paths made it wait for the fetch just issued, one iteration of lead instead of two.)
    auto fetch = [&](Frag& f, int buf, int it) {
        __builtin_amdgcn_s_waitcnt(kLgkm0Imm);
#pragma unroll
        for (int q = 0; q < S::kGroups; ++q) {
            const int group = group0 + (it * S::kGroups + q) * KS + ks;   // K slices interleave group by group
            const uint32_t a_soff = static_cast<uint32_t>(group) * 128u;
            uint8_t* const dst = a_lds + buf * S::kABufBytes + q * RM * S::kAFragBytes;
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bool ok = 4 * group + a_dma_chunk[h] < chunk_end;
                    dma16(a_rsrc, dst + i * S::kAFragBytes + h * 1024, ok ? a_dma[i][h] : kOob, a_soff);
                }
            const int chunk = 4 * group + g;
            const bool in_k = chunk < chunk_end;
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                const uint32_t off = (b_base[j] == kOob || !in_k)
                                         ? kOob
                                         : b_base[j] + static_cast<uint32_t>(chunk) * b_chunk_stride;
                f.b[q][j] = buf_load16<kNtWeight ? kCpolNt : 0>(b_rsrc, off);
            }
        }
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](const Frag& f, int buf) {
#pragma unroll
        for (int q = 0; q < S::kGroups; ++q) {
            half8 xa[RM][2];
#pragma unroll
            for (int i = 0; i < RM; ++i) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    u32x4 v = *reinterpret_cast<const u32x4*>(
                        a_lds + buf * S::kABufBytes + (q * RM + i) * S::kAFragBytes + a_rd[s]);
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

    // Iterations of this wave: groups ks, ks + KS, ... taken kGroups at a time; fetches it + 1 .. it + kDepth - 1
    // are in flight while iteration it computes, in buffers (it + d) % kDepth. Before a consume, this wave's
    // loads of that iteration have landed (vector-memory operations retire in issue order, so only the
    // kDepth - 1 newer fetches may stay outstanding). The loop body is straight-line: its fetches go out even
    // in the last round of iterations, where they load zeros that are never consumed.
    // Scheduling barriers keep each fetch ahead of the decode of the iteration before it (left alone, the
    // compiler hoists that decode above the fetch, and its register wait then retires the older fetch before
    // the newer one is issued).
    constexpr int D = S::kDepth;
    const int per_iter = S::kGroups * KS;
    const int iters = (group_end - group0 + per_iter - 1) / per_iter;
    Frag f[D];
#pragma unroll
    for (int d = 0; d + 1 < D; ++d) {
        __builtin_amdgcn_sched_barrier(0);
        fetch(f[d], d, d);
    }
    int it = 0;
    for (; it + D - 1 < iters; it += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(f[(d + D - 1) % D], (d + D - 1) % D, it + d + D - 1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((D - 1) * S::kLoadsPerFetch));
            consume(f[d], d);
        }
    }
    // The last iterations (fewer than D): fetches it .. it + D - 2 are in flight, in buffers 0 .. D - 2.
    static_assert(D == 2 || D == 3, "the tail below is written out for these depths");
    if (it < iters) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((D - 2) * S::kLoadsPerFetch));
        consume(f[0], 0);
    }
    if constexpr (D == 3) {
        if (it + 1 < iters) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            consume(f[1], 1);
        }
    }

    if constexpr (KS > 1 && !kSplitK && S::kBN >= 64) {
        // Deterministic join of the K slices: every wave parks its sums in LDS, then the block's threads share
        // the output tile in pieces of 8 columns of one row, consecutive threads taking a row's consecutive
        // pieces, so that 8 neighbouring lanes store a 128-byte row segment whole (16 bytes each, with the
        // non-temporal hint: nothing reads the output back in this launch). A piece is two 4-column groups of
        // one fragment row, each the sum of its slices in slice order (0, 1, ..., KS - 1). Against each wave
        // storing whole fragments (8-byte stores, a row segment written by several waves), same-box graph
        // replays, bit-identical: C4 0.6% faster, the 32- and 64-row tiles 2-4%. Blocks narrower than 64 columns
        // (row segments of 32 or 64 bytes) keep the per-fragment join below, which measured 0.3-5.7% faster
        // there.
        f32x4* red = reinterpret_cast<f32x4*>(lds + S::kALdsBytes);
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int j = 0; j < RN; ++j)
                red[(ks * S::kFrags + (wave_n * RM + i) * RN + j) * kWave + lane] = acc[i][j];
        __syncthreads();
        constexpr int kPiecesPerRow = S::kBN / 8;
        constexpr int kPieces = S::kBM * kPiecesPerRow;
        const rsrc_t c_rsrc = make_rsrc(p.c, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.N) * 2u);
        const rsrc_t bias_rsrc = make_rsrc(p.bias, static_cast<uint32_t>(p.N) * 2u);
        const rsrc_t scale_rsrc = make_rsrc(p.scale, static_cast<uint32_t>(p.N) * 4u);
        const bool has_bias = p.bias != nullptr;
        for (int piece = tid; piece < kPieces; piece += S::kThreads) {
            const int r = piece / kPiecesPerRow;            // row within the tile
            const int cb = 8 * (piece % kPiecesPerRow);     // first column within the tile
            const int f = ((cb / (16 * RN)) * RM + r / 16) * RN + (cb % (16 * RN)) / 16;
            const int slot = (cb % 16) / 4 * 16 + r % 16;   // lane of the first 4-column group
            f32x4 lo = red[f * kWave + slot];
            f32x4 hi = red[f * kWave + slot + 16];
#pragma unroll
            for (int k2 = 1; k2 < KS; ++k2) {
                lo += red[(k2 * S::kFrags + f) * kWave + slot];
                hi += red[(k2 * S::kFrags + f) * kWave + slot + 16];
            }
            const int row = m0 + r;
            const int col = tn * S::kBN + cb;
            // N % 8 == 0, so a piece lies wholly inside N or wholly outside
            const bool ok = row < p.M && col < p.N;
            // two 8-byte loads: the bias is only 8-byte aligned (the C ABI's contract)
            const u32x2 bias_lo = has_bias ? buf_load8(bias_rsrc, ok ? static_cast<uint32_t>(col) * 2u : kOob)
                                           : u32x2{0u, 0u};
            const u32x2 bias_hi = has_bias ? buf_load8(bias_rsrc, ok ? static_cast<uint32_t>(col + 4) * 2u : kOob)
                                           : u32x2{0u, 0u};
            f32x4 sc_lo = f32x4{scale, scale, scale, scale};
            f32x4 sc_hi = sc_lo;
            if (p.col_scale) {
                sc_lo = __builtin_bit_cast(f32x4, buf_load16(scale_rsrc, ok ? static_cast<uint32_t>(col) * 4u : kOob));
                sc_hi = __builtin_bit_cast(f32x4, buf_load16(scale_rsrc, ok ? static_cast<uint32_t>(col + 4) * 4u : kOob));
            }
            const u32x2 y_lo = epilogue4<kOutBf16>(lo, sc_lo, has_bias, bias_lo);
            const u32x2 y_hi = epilogue4<kOutBf16>(hi, sc_hi, has_bias, bias_hi);
            const uint32_t off = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.N) +
                                       static_cast<uint32_t>(col)) * 2u
                                    : kOob;
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{y_lo[0], y_lo[1], y_hi[0], y_hi[1]}, c_rsrc,
                                                   static_cast<int>(off), 0, kCpolNt);
        }
    } else if constexpr (KS > 1) {
        // Narrow blocks and split launches: the same parking, then the block's waves share the output
        // fragments, each adding a fragment's slices in slice order (and, split, joining it across workgroups)
        // and storing it; the fragment's bias loads are in flight during its join.
        f32x4* red = reinterpret_cast<f32x4*>(lds + S::kALdsBytes);
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int j = 0; j < RN; ++j)
                red[(ks * S::kFrags + (wave_n * RM + i) * RN + j) * kWave + lane] = acc[i][j];
        __syncthreads();
        for (int f = wave; f < S::kFrags; f += KS * WN) {
            const int i = (f / RN) % RM;
            const int j = f % RN;
            const int col0 = tn * S::kBN + (f / (RM * RN)) * 16 * RN + 16 * j;
            u32x2 bias_bits[1];
            load_bias<1>(p, col0, lane, bias_bits);
            f32x4 col_scales[1];
            if (p.col_scale) load_col_scales<1>(p, col0, lane, col_scales);
            f32x4 sum[1][1] = {{red[f * kWave + lane]}};
#pragma unroll
            for (int k2 = 1; k2 < KS; ++k2) sum[0][0] += red[(k2 * S::kFrags + f) * kWave + lane];
            if constexpr (kSplitK) {
                // Across workgroups, the fragment is the unit: its last split sums and stores it.
                if (!join_split<S::kFrags, 1, 1>(p, sum, tile_id, split, f, lane)) continue;
            }
            if (p.col_scale) {
                store_tiles<1, 1, kOutBf16>(p, sum, m0 + 16 * i, col0, lane, col_scales, bias_bits);
            } else {
                store_tiles<1, 1, kOutBf16>(p, sum, m0 + 16 * i, col0, lane, scale, bias_bits);
            }
        }
    } else {
        if constexpr (kSplitK) {
            if (!join_split<WN, RM, RN>(p, acc, tile_id, split, wave_n, lane)) return;
        }
        store_wave_tiles<RM, RN, kOutBf16>(p, acc, m0, n0, lane, scale);
    }
}

}  // namespace feather
