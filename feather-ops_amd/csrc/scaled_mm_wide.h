// The wide kernel: 256 x 256 output tiles, 4 waves of 128 x 128 per workgroup, one workgroup per CU, so each
// SIMD runs a single wave with 512 registers (the 8 x 8 fp32 accumulator fragments in AGPRs). With one wave per
// SIMD nothing hides a wave's memory and LDS traffic behind another wave's MFMAs, so the wave does it itself:
// its stage loop is software-pipelined by hand, every LDS read, weight decode and direct-to-LDS load placed
// between two of its own MFMAs, in an order pinned by scheduling barriers.
//
// Per 64-deep stage a wave issues 128 MFMAs (v_mfma_f32_16x16x32_f16, 2 k halves x 8 x 8 fragments), 24 LDS
// reads (8 weight chunks and 2 x 8 activation halves), 12 direct loads (its quarter of a stage's 48 KiB) and 64
// byte-moves of weight decode. Against the ring kernel's 128 x 256 tile, two workgroups per CU: the same MFMAs
// read 33% less LDS (a 128 x 128 wave tile against 128 x 64) and the CU loads 25% fewer operand bytes per
// stage (a 256 x 256 tile against two 128 x 256).
//
// A workgroup computes one tile (or one K range of a tile in a split launch). Its stages stream through a 3-slot
// LDS ring (each slot 32 KiB of activations + 16 KiB of weights); stage t uses slot t % 3:
//   first k half:   MFMAs acc[i][j] += w0[j] * x0[i]. Between them: the LDS reads of the second half's
//                   activations x1 (slot t % 3), the decode of the second half's weights w1, and 4 of the 12
//                   direct loads of stage t + 2 (into slot (t + 2) % 3).
//   second k half:  MFMAs acc[i][j] += w1[j] * x1[i]. After its first 8: the wave's LDS reads are complete,
//                   its loads of stage t + 1 have landed (vmcnt), and the workgroup barrier makes every wave's
//                   share of stage t + 1 visible and retires every read of slot t % 3. Then, between the remaining
//                   MFMAs: the LDS reads of stage t + 1's weights and first-half activations, 8 of the direct
//                   loads of stage t + 3 into slot t % 3, and the decode of stage t + 1's first-half weights w0.
// A stage's loads thus have about two stages of MFMAs to land. Issued in a burst, the CU's 48 loads of a stage
// cost the MFMAs of all 4 waves about 40 clocks each (measured); spread one per 5-14 MFMAs, most of their issue
// hides under the MFMAs. Stages past the end load through a resource of size 0 (zeros into a slot nobody reads),
// so every iteration waits for the same count.
//
// The outputs go straight from registers to memory: each lane's 4 consecutive output columns of two neighbouring
// 16 x 16 fragments are exchanged across lane rows (v_permlane16_swap) so that every lane holds 8 consecutive
// columns, one 16-byte store per fragment pair.
//
// MFMA order within a k half is the ring kernel's (each activation fragment feeds its 8 MFMAs back to back, the
// weight fragment changing; odd fragments take the weights in reverse), and each accumulator sums a stage's two
// k halves in order, so the outputs are bit-identical to the ring kernel's for the same K range.
#pragma once

#include "scaled_mm_kernels.h"

namespace feather {

// RN_: 16-column weight fragments per wave, 8 (256 x 256 tiles) or 6 (256 x 192 tiles: 4 waves of 128 x 96, a
// 132 KiB ring; e.g. one tile per CU on a 4096 x 3072 output).
template <int RN_>
struct WideShape {
    static constexpr int kWaves = 4;
    static constexpr int kThreads = kWave * kWaves;
    static constexpr int RM = 8;                           // 16-row activation fragments per wave
    static constexpr int RN = RN_;                         // 16-column weight fragments per wave
    static constexpr int kBM = 2 * 16 * RM;                // 256
    static constexpr int kBN = 2 * 16 * RN;                // 256 or 192
    static constexpr int kUnitsPerRow = 8;                 // a stage's activation row: 64 k x 2 bytes = 8 x 16 B
    static constexpr int kABytes = kBM * kUnitsPerRow * 16;   // 32 KiB, [row][8 units], units XOR-swizzled
    static constexpr int kBBytes = 4 * kBN * 16;              // 16 or 12 KiB, [chunk][col][16 bytes]
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kSlots = 3;
    static constexpr int kLdsBytes = kSlots * kStageBytes;    // 144 or 132 KiB: one workgroup per CU
    static constexpr int kAInstr = kABytes / 1024 / kWaves;   // 8 direct loads of 1 KiB per wave and stage
    static constexpr int kBInstr = kBBytes / 1024 / kWaves;   // 4 or 3
    static constexpr int kLoadsPerStage = kAInstr + kBInstr;
    static constexpr int kMfmas = RM * RN;                    // MFMAs of one k half
    // Direct loads of stage t + 3 issued in the second half of stage t (every kEarlyStep MFMAs from kEarlyAt); the
    // rest of them in the first half of stage t + 1 (every kLateStep MFMAs from kLateAt). Of the placements
    // measured (bursts, and spreads over one half or both), these took the fewest clocks per stage. For the
    // 256 x 192 tile the spreads over both halves measured within 1% of each other on 4096 x 3072 x 3072 and
    // 4096 x 3072 x 12288 (5 early from MFMA 24 and 6 late from MFMA 4 the fastest); all 11 in one half, 30% slower.
    static constexpr int kLoadsEarly = RN == 8 ? 8 : 5;
    static constexpr int kEarlyAt = 24;
    static constexpr int kEarlyStep = 5;
    static constexpr int kLateAt = RN == 8 ? 5 : 4;
    static constexpr int kLateStep = RN == 8 ? 14 : 8;
    // Second k half: the weights of stage t + 1 are read at MFMAs [8, 8 + RN), its first-half activations at
    // [8 + RN, 8 + RN + RM), and its first-half weights decoded two dwords per MFMA from kDecode0; the first half
    // decodes the second-half weights one dword per MFMA from kDecode1.
    static constexpr int kDecode0 = kMfmas - 2 * RN;
    static constexpr int kDecode1 = kMfmas - 4 * RN;
    static_assert(RN == 8 || RN == 6, "the two wide tiles");
    static_assert(kEarlyAt >= 8 && kEarlyAt + kEarlyStep * (kLoadsEarly - 1) < kMfmas, "early loads fit");
    static_assert(kLateAt + kLateStep * (kLoadsPerStage - kLoadsEarly - 1) < kMfmas, "late loads fit");
    static_assert(8 + RN + RM <= kDecode0, "operand reads precede the decode they feed");
    static_assert(2 * kLoadsPerStage < 64, "vmcnt range");
};

// The tiles the launcher runs on the wide kernel: (warps_m, warps_n, unroll_k, repeat_m, repeat_n) = (2, 2, 4, 8, 8)
// and (2, 2, 4, 8, 6).
template <int WM, int WN, int U, int RM, int RN>
constexpr bool is_wide_tile() {
    return WM == 2 && WN == 2 && U == 4 && RM == 8 && (RN == 8 || RN == 6);
}

// One fp16 dword (two k values) of a weight fragment from one dword of 4 codes: its low (kHi = false) or high two
// codes. decode_chunk's dword d of a 16-code chunk is decode_word(raw[d / 2], d % 2).
template <bool kE5M2, bool kHi>
__device__ __forceinline__ uint32_t decode_word_(uint32_t w) {
    if constexpr (kE5M2) {
        return __builtin_amdgcn_perm(0u, w, kHi ? perm_sel(kZeroByte, 2, kZeroByte, 3) : perm_sel(kZeroByte, 0, kZeroByte, 1));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, kHi));
    }
}

template <bool kE5M2>
__device__ __forceinline__ uint32_t decode_word(uint32_t w, bool hi) {
    return hi ? decode_word_<kE5M2, true>(w) : decode_word_<kE5M2, false>(w);
}

// A wave's 128 x 128 outputs from its accumulators straight to memory. Lane (g, r) = (lane / 16, lane % 16) holds
// columns 4g .. 4g + 3 of row r of each 16 x 16 fragment; for fragments j and j + 1, exchanging lane rows 1 and 3
// of j's values with rows 0 and 2 of j + 1's (v_permlane16_swap, once per dword) leaves lane (g, r) with columns
// 16 (g & 1) + 8 (g >> 1) .. + 7 of the pair's 32: one 16-byte store. The lane's offset is computed once; a
// fragment row's goes in the scalar offset and a pair's in the instruction's. kRagged: rows past M and columns
// past N (N % 8 == 0, so a piece of 8 columns is wholly in or out) take an out-of-range offset, dropped by the
// buffer's range check. Scheduling barriers keep the pairs in order, so that only one pair's values are held in
// VGPRs at a time. The stores write through at device scope: the output's lines leave L2 as they are written
// instead of staying dirty there until the end of the launch (measured on copies of the kernel, interleaved
// runs: C3 0.5% faster, C2's shape, one round of 256 x 192 tiles, 2.6%; the non-temporal hint instead, 2%
// slower).
template <int RM, int RN, bool kOutBf16, bool kBias, bool kColScale, bool kRagged>
__device__ __forceinline__ void store_wave_tiles_swap(const Params& p, const f32x4 (&acc)[RM][RN], int row0, int col0,
                                                      int lane, float scale) {
    static_assert(RN % 2 == 0, "fragment pairs");
    const int g = lane >> 4;
    const int r16 = lane & 15;
    u32x2 bias_bits[RN];
    if constexpr (kBias) {
        load_bias<RN>(p, col0, lane, bias_bits);
    } else {
#pragma unroll
        for (int j = 0; j < RN; ++j) bias_bits[j] = u32x2{0u, 0u};
    }
    f32x4 col_scales[RN];
    if constexpr (kColScale) load_col_scales<RN>(p, col0, lane, col_scales);
    const rsrc_t c_rsrc = make_rsrc(p.c, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.N) * 2u);
    const int col = col0 + 16 * (g & 1) + 8 * (g >> 1);
    const uint32_t pitch = static_cast<uint32_t>(p.N) * 2u;
    const uint32_t base = static_cast<uint32_t>(row0 + r16) * pitch + static_cast<uint32_t>(col) * 2u;
#pragma unroll
    for (int i = 0; i < RM; ++i) {
#pragma unroll
        for (int jp = 0; jp < RN / 2; ++jp) {
            u32x2 y[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = 2 * jp + h;
                f32x4 sc = f32x4{scale, scale, scale, scale};
                if constexpr (kColScale) sc = col_scales[j];
                y[h] = out4<kOutBf16, kBias>(acc[i][j], sc, bias_bits[j]);
            }
            const auto s0 = __builtin_amdgcn_permlane16_swap(y[0][0], y[1][0], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(y[0][1], y[1][1], false, false);
            const u32x4 v{s0[0], s1[0], s0[1], s1[1]};
            if constexpr (kRagged) {
                const bool ok = row0 + 16 * i + r16 < p.M && col + 32 * jp < p.N;
                const uint32_t off = ok ? base + static_cast<uint32_t>(16 * i) * pitch + 64u * jp : kOob;
                __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, static_cast<int>(off), 0, kDeviceScope);
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, static_cast<int>(base + 64u * jp),
                                                       static_cast<int>(static_cast<uint32_t>(16 * i) * pitch),
                                                       kDeviceScope);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// kRagged: M % 256, N % kBN or K % 64 is not zero. Then every direct load masks its lanes (rows past M, columns
// past N and chunks past K read zeros). Otherwise every load is whole and in range: the per-lane offsets are fixed
// and the tile and stage go in the scalar offset.
template <int RN_, bool kE5M2, bool kABf16, bool kOutBf16, bool kSplitK, bool kRagged>
__global__ __launch_bounds__(WideShape<RN_>::kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void wide_kernel(
    const Params p) {
    using S = WideShape<RN_>;
    constexpr int RM = S::RM;
    constexpr int RN = S::RN;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wave_m = wave >> 1;
    const int wave_n = wave & 1;

    // Workgroup -> (K range, tile), split-major as in the ring kernel.
    const int tiles_m = (p.M + S::kBM - 1) / S::kBM;
    const int tiles_n = (p.N + S::kBN - 1) / S::kBN;
    const int n_tiles = tiles_m * tiles_n;
    const int splits = kSplitK ? p.splits : 1;
    const int split = kSplitK ? static_cast<int>(blockIdx.x) / n_tiles : 0;
    const int tile_id = static_cast<int>(blockIdx.x) - split * n_tiles;
    int tm, tn;
    tile_of_block(tile_id, n_tiles, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * S::kBM;
    const int n0 = tn * S::kBN;
    const int stages_total = (p.K + 63) / 64;
    const int stage0 = split * stages_total / splits;
    const int stages = (split + 1) * stages_total / splits - stage0;
    const int k_chunks = p.K / 16;

    const rsrc_t a_rsrc = make_rsrc(p.a, static_cast<uint32_t>(p.M) * static_cast<uint32_t>(p.K) * 2u);
    const rsrc_t b_rsrc = make_rsrc(p.b, static_cast<uint32_t>(p.kb_total) * static_cast<uint32_t>(p.N) * 16u);
    const rsrc_t null_rsrc = make_rsrc(p.a, 0u);
    const float scale = load_scale(p);

    // Direct loads (the ring kernel's layout): load d < 8 of this wave fills 1 KiB of a slot's activations (8 rows
    // of 8 units: row (wave + 4d) * 8 + lane / 8 of the tile, physical unit lane % 8), load 8 + i fills the slot's
    // weight pieces e * 64 + lane, e = wave + 4i, of its [4 chunks][kBN columns] (kBN a multiple of 64, so one
    // load covers 64 columns of one chunk). Per-lane offsets within the tile and stage; the unit's k chunk (the
    // same for every d: the swizzle key depends on the row mod 16 only).
    uint32_t a_lane_off[S::kAInstr];
    int a_chunk = 0;
#pragma unroll
    for (int d = 0; d < S::kAInstr; ++d) {
        const int unit = (wave + d * S::kWaves) * kWave + lane;
        const int row = unit / S::kUnitsPerRow;
        const int u = a_unit_phys<S::kUnitsPerRow>(row, unit % S::kUnitsPerRow);
        a_chunk = u >> 1;
        a_lane_off[d] = (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.K) + static_cast<uint32_t>(u * 8)) * 2u;
    }
    const int a_row_in = lane / S::kUnitsPerRow + wave * S::kUnitsPerRow;   // + 32 d: the row of load d
    static_assert(S::kBN % kWave == 0, "a weight load covers one chunk");
    int b_col_in[S::kBInstr], b_chunk[S::kBInstr];
    uint32_t b_lane_off[S::kBInstr];
#pragma unroll
    for (int i = 0; i < S::kBInstr; ++i) {
        if constexpr (S::kBN == S::kWaves * kWave) {
            b_chunk[i] = i;   // load i: chunk i, column wave * 64 + lane
            b_col_in[i] = wave * kWave + lane;
        } else {
            const int e = wave + i * S::kWaves;
            b_chunk[i] = e * kWave / S::kBN;
            b_col_in[i] = e * kWave % S::kBN + lane;
        }
        b_lane_off[i] = (static_cast<uint32_t>(b_chunk[i]) * static_cast<uint32_t>(p.N) +
                         static_cast<uint32_t>(b_col_in[i])) * 16u;
    }
    const uint32_t a_tile_off = static_cast<uint32_t>(m0) * static_cast<uint32_t>(p.K) * 2u;
    const uint32_t b_tile_off = static_cast<uint32_t>(n0) * 16u;
    const uint32_t b_stage_stride = 4u * static_cast<uint32_t>(p.N) * 16u;

    // Direct load d of local stage lt into the slot at byte `slot`. Stages past this workgroup's range load zeros
    // through the size-0 resource.
    auto dma = [&](int d, int lt, uint32_t slot) {
        const bool live = lt < stages;
        const int stage = stage0 + lt;
        if (d < S::kAInstr) {
            uint8_t* dst = lds + slot + (wave + d * S::kWaves) * 1024;
            if constexpr (kRagged) {
                const bool ok = m0 + a_row_in + 32 * d < p.M && a_chunk < k_chunks - 4 * stage;
                dma16(live ? a_rsrc : null_rsrc, dst, ok ? a_tile_off + a_lane_off[d] : kOob,
                      live ? static_cast<uint32_t>(stage) * 128u : 0u);
            } else {
                dma16(live ? a_rsrc : null_rsrc, dst, a_lane_off[d],
                      live ? a_tile_off + static_cast<uint32_t>(stage) * 128u : 0u);
            }
        } else {
            const int i = d - S::kAInstr;
            uint8_t* dst = lds + slot + S::kABytes + (wave + i * S::kWaves) * 1024;
            if constexpr (kRagged) {
                const bool ok = n0 + b_col_in[i] < p.N && b_chunk[i] < k_chunks - 4 * stage;
                dma16(live ? b_rsrc : null_rsrc, dst, ok ? b_tile_off + b_lane_off[i] : kOob,
                      live ? static_cast<uint32_t>(stage) * b_stage_stride : 0u);
            } else {
                dma16(live ? b_rsrc : null_rsrc, dst, b_lane_off[i],
                      live ? b_tile_off + static_cast<uint32_t>(stage) * b_stage_stride : 0u);
            }
        }
    };

    // LDS operand reads (the ring kernel's fragment layout): lane group g = lane / 16 reads chunk g of the
    // stage; activation half s of fragment i is unit (2g + s) ^ key of row 128 wave_m + 16 i + lane % 16.
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int a_row = wave_m * 16 * RM + r16;
    const int key = a_swizzle_key<S::kUnitsPerRow>(a_row);
    const uint32_t a_rd0 = static_cast<uint32_t>(a_row * S::kUnitsPerRow * 16 + (((2 * g) ^ key) << 4));
    const uint32_t a_rd1 = static_cast<uint32_t>(a_row * S::kUnitsPerRow * 16 + (((2 * g + 1) ^ key) << 4));
    const uint32_t b_rd = static_cast<uint32_t>(S::kABytes + g * S::kBN * 16 + (wave_n * 16 * RN + r16) * 16);
    auto read16 = [&](uint32_t off) { return *reinterpret_cast<const u32x4*>(lds + off); };
    auto as_f16 = [](u32x4 v) { return __builtin_bit_cast(half8, kABf16 ? bf16x8_to_f16x8(v) : v); };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 x0[RM], x1[RM], braw[RN];
    uint32_t w0[RN][4], w1[RN][4];

    // Prologue: stages 0 and 1 and the early loads of stage 2 in flight; wait for stage 0; read its weights and
    // first-half activations and decode the first-half weights.
#pragma unroll
    for (int lt = 0; lt < 2; ++lt)
#pragma unroll
        for (int d = 0; d < S::kLoadsPerStage; ++d) dma(d, lt, static_cast<uint32_t>(lt * S::kStageBytes));
#pragma unroll
    for (int d = 0; d < S::kLoadsEarly; ++d) dma(d, 2, 2u * S::kStageBytes);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(S::kLoadsPerStage + S::kLoadsEarly));
    barrier_only();
#pragma unroll
    for (int j = 0; j < RN; ++j) braw[j] = read16(b_rd + j * 256);
#pragma unroll
    for (int i = 0; i < RM; ++i) x0[i] = read16(a_rd0 + i * 2048);
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
        for (int d = 0; d < 4; ++d) w0[j][d] = decode_word<kE5M2>(braw[j][d / 2], d & 1);

    uint32_t cur = 0;                           // slot of stage t
    uint32_t nxt = S::kStageBytes;              // slot of stage t + 1
    uint32_t prv = 2 * S::kStageBytes;          // slot of stage t - 1 = slot of stage t + 2
    for (int t = 0; t < stages; ++t) {
        // First k half.
#pragma unroll
        for (int m = 0; m < S::kMfmas; ++m) {
            const int i = m / RN;
            const int jj = m % RN;
            const int j = (i & 1) ? RN - 1 - jj : jj;
            acc[i][j] = mfma16(__builtin_bit_cast(half8, u32x4{w0[j][0], w0[j][1], w0[j][2], w0[j][3]}), as_f16(x0[i]),
                               acc[i][j]);
            if (jj == 0) x1[i] = read16(cur + a_rd1 + i * 2048);
            if (m >= S::kDecode1) {
                const int q = m - S::kDecode1;  // 4 RN dwords of second-half weights, one per MFMA
                w1[q / 4][q % 4] = decode_word<kE5M2>(braw[q / 4][2 + (q % 4) / 2], q & 1);
            }
            if (m >= S::kLateAt && (m - S::kLateAt) % S::kLateStep == 0 &&
                (m - S::kLateAt) / S::kLateStep < S::kLoadsPerStage - S::kLoadsEarly) {
                dma(S::kLoadsEarly + (m - S::kLateAt) / S::kLateStep, t + 2, prv);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Second k half.
#pragma unroll
        for (int m = 0; m < S::kMfmas; ++m) {
            const int i = m / RN;
            const int jj = m % RN;
            const int j = (i & 1) ? RN - 1 - jj : jj;
            acc[i][j] = mfma16(__builtin_bit_cast(half8, u32x4{w1[j][0], w1[j][1], w1[j][2], w1[j][3]}), as_f16(x1[i]),
                               acc[i][j]);
            if (m == 7) {
                // This wave's reads of slot t % 3 are complete and its loads of stage t + 1 have landed (those of
                // stage t + 2 may still be in flight); the barrier makes every wave's share of stage t + 1 visible,
                // after which slot t % 3 is free.
                __builtin_amdgcn_s_waitcnt(kLgkm0Imm);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(S::kLoadsPerStage));
                barrier_only();
            }
            if (m >= 8 && m < 8 + RN) braw[m - 8] = read16(nxt + b_rd + (m - 8) * 256);
            if (m >= 8 + RN && m < 8 + RN + RM) x0[m - 8 - RN] = read16(nxt + a_rd0 + (m - 8 - RN) * 2048);
            if (m >= S::kEarlyAt && (m - S::kEarlyAt) % S::kEarlyStep == 0 &&
                (m - S::kEarlyAt) / S::kEarlyStep < S::kLoadsEarly) {
                dma((m - S::kEarlyAt) / S::kEarlyStep, t + 3, cur);
            }
            if (m >= S::kDecode0) {
                const int q = 2 * (m - S::kDecode0);  // 4 RN dwords of stage t + 1's first-half weights, two per MFMA
                w0[q / 4][q % 4] = decode_word<kE5M2>(braw[q / 4][(q % 4) / 2], q & 1);
                w0[(q + 1) / 4][(q + 1) % 4] = decode_word<kE5M2>(braw[(q + 1) / 4][((q + 1) % 4) / 2], (q + 1) & 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const uint32_t freed = cur;
        cur = nxt;
        nxt = prv;
        prv = freed;
    }

    // The last iterations' loads (zeros) write LDS: let them land before the workgroup ends.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    const int row0 = m0 + wave_m * 16 * RM;
    const int col0 = n0 + wave_n * 16 * RN;
    if constexpr (kSplitK) {
        if (!join_split<S::kWaves, RM, RN>(p, acc, tile_id, split, wave, lane)) return;
    }
    if (p.col_scale) {
        if (p.bias) {
            store_wave_tiles_swap<RM, RN, kOutBf16, true, true, kRagged>(p, acc, row0, col0, lane, scale);
        } else {
            store_wave_tiles_swap<RM, RN, kOutBf16, false, true, kRagged>(p, acc, row0, col0, lane, scale);
        }
    } else if (p.bias) {
        store_wave_tiles_swap<RM, RN, kOutBf16, true, false, kRagged>(p, acc, row0, col0, lane, scale);
    } else {
        store_wave_tiles_swap<RM, RN, kOutBf16, false, false, kRagged>(p, acc, row0, col0, lane, scale);
    }
}

}  // namespace feather
