// Instantiates every tile of feather_tiles.h for ONE (weight format, activation dtype, output dtype)
// combination and dispatches a tile query to it. The build compiles this file once per combination,
// with FEATHER_B_E5M2, FEATHER_A_BF16 and FEATHER_OUT_BF16 set to 0 or 1, so the eight combinations
// compile in parallel. The instantiation flow (X-macro tile list -> template per tile) follows the
// reference's dispatch_scaled_mm (csrc/hip_kernel.cu:668-684).
#include "scaled_mm_launch.h"

#include "feather_tiles.h"
#include "scaled_mm_kernels.h"
#include "scaled_mm_wide.h"

#if !defined(FEATHER_B_E5M2) || !defined(FEATHER_A_BF16) || !defined(FEATHER_OUT_BF16)
#error "compile with -DFEATHER_B_E5M2=<0|1> -DFEATHER_A_BF16=<0|1> -DFEATHER_OUT_BF16=<0|1>"
#endif

namespace feather {
namespace {

constexpr bool kE5M2 = FEATHER_B_E5M2 != 0;
constexpr bool kABf16 = FEATHER_A_BF16 != 0;
constexpr bool kOutBf16 = FEATHER_OUT_BF16 != 0;
constexpr int kCus = 256;                // MI355X compute units

// Non-temporal weight loads (Params::stream_weight) go to launches whose M fits one tile row, so that each
// weight byte is read by one workgroup row. Ring tiles get the variant only at 64 rows or fewer: those are the
// tiles the heuristic streams big weights with at small M, and the 128-row tiles keep their instantiations.
template <int WM, int WN, int U, int RM, int RN, bool kSplitK, bool kDeep>
void launch_ring(const Params& q, dim3 grid, hipStream_t stream) {
    using S = DmaShape<WM, WN, U, RM, RN>;
    if constexpr (S::kBM <= 64) {
        if (q.stream_weight && q.M <= S::kBM) {
            hipLaunchKernelGGL((ring_dma_kernel<WM, WN, U, RM, RN, kE5M2, kABf16, kOutBf16, kSplitK, kDeep, true>),
                               grid, dim3(S::kThreads), 0, stream, q);
            return;
        }
    }
    hipLaunchKernelGGL((ring_dma_kernel<WM, WN, U, RM, RN, kE5M2, kABf16, kOutBf16, kSplitK, kDeep>), grid,
                       dim3(S::kThreads), 0, stream, q);
}

template <int KS, int WN, int U, int RM, int RN, bool kSplitK>
void launch_stream(const Params& p, dim3 grid, hipStream_t stream) {
    using S = StreamShape<KS, WN, U, RM, RN>;
    if (p.stream_weight && p.M <= S::kBM) {
        hipLaunchKernelGGL((stream_kernel<KS, WN, U, RM, RN, kE5M2, kABf16, kOutBf16, kSplitK, true>), grid,
                           dim3(S::kThreads), 0, stream, p);
    } else {
        hipLaunchKernelGGL((stream_kernel<KS, WN, U, RM, RN, kE5M2, kABf16, kOutBf16, kSplitK>), grid,
                           dim3(S::kThreads), 0, stream, p);
    }
}

template <int WM, int WN, int U, int RM, int RN, int PF>
bool try_tile(const TileQuery& t, const Params& p, hipStream_t stream) {
    if (t.warps_m != WM || t.warps_n != WN || t.unroll_k != U || t.repeat_m != RM || t.repeat_n != RN ||
        t.prefetch != (PF != 0)) {
        return false;
    }
    if constexpr (PF != 0 && is_wide_tile<WM, WN, U, RM, RN>()) {
        // One workgroup per CU, one wave per SIMD: the software-pipelined wide kernel.
        using S = WideShape<RN>;
        const int64_t tiles = ((p.M + S::kBM - 1) / S::kBM) * static_cast<int64_t>((p.N + S::kBN - 1) / S::kBN);
        const dim3 grid(static_cast<uint32_t>(tiles * p.splits));
        // M, N or K off the tile grid: the instantiation that masks every load per lane.
        const bool ragged = p.M % S::kBM != 0 || p.N % S::kBN != 0 || p.K % 64 != 0;
        const auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(S::kThreads), 0, stream, p); };
        if (p.splits > 1) {
            if (ragged) {
                go(wide_kernel<RN, kE5M2, kABf16, kOutBf16, true, true>);
            } else {
                go(wide_kernel<RN, kE5M2, kABf16, kOutBf16, true, false>);
            }
        } else if (ragged) {
            go(wide_kernel<RN, kE5M2, kABf16, kOutBf16, false, true>);
        } else {
            go(wide_kernel<RN, kE5M2, kABf16, kOutBf16, false, false>);
        }
    } else if constexpr (PF != 0) {
        using S = DmaShape<WM, WN, U, RM, RN>;
        const int64_t tiles = ((p.M + S::kBM - 1) / S::kBM) * static_cast<int64_t>((p.N + S::kBN - 1) / S::kBN);
        const int64_t blocks = tiles * p.splits;
        const dim3 grid(static_cast<uint32_t>(blocks));
        // Workgroups that take the ring kernel's reads-first schedule. Unsplit launches with fp16 activations
        // take it everywhere: partial last rounds included, it measured 1-4% faster than the interleaved order
        // there (same-box A/B, 128 x 256 and 128 x 128 tiles). With bf16 activations (register-staged) and in
        // split launches it pays only where a CU holds the tile's full complement of blocks: workgroups
        // dispatch in id order, breadth-first over the CUs, so that is every workgroup of a full round of
        // kCus * per_cu, and all of a last, partial round that still fills some CUs (those end last); a
        // partial round that fills none (at most per_cu - 1 blocks on any CU) keeps the interleaved schedule.
        const auto with_rounds = [&](int per_cu) {
            Params q = p;
            const int64_t slots = int64_t{kCus} * per_cu;
            const int64_t full = blocks / slots * slots;
            const bool everywhere = !kABf16 && p.splits == 1;
            q.reads_first_blocks = static_cast<int32_t>(
                everywhere || blocks - full > int64_t{kCus} * (per_cu - 1) ? blocks : full);
            return q;
        };
        if constexpr (S::kBM <= 64 && (!kABf16 || WN <= 2)) {
            // A 64-row tile takes the deep ring when every block of the launch is resident at once with it
            // (as many blocks per CU as its LDS allows): there the deeper lead hides the memory latency that
            // a small grid cannot hide with more blocks. Bigger grids keep the shallow ring's occupancy.
            // With bf16 activations the deep ring widens per fragment (each of the WN column waves widens
            // the block's rows again), which pays only while M <= 64 and WN <= 2.
            using D = DmaShape<WM, WN, U, RM, RN, true>;
            if ((!kABf16 || p.M <= 64) && blocks <= int64_t{kCus} * D::kBlocksPerCu) {
                const Params q = with_rounds(D::kBlocksPerCu);
                if (p.splits > 1) {
                    launch_ring<WM, WN, U, RM, RN, true, true>(q, grid, stream);
                } else {
                    launch_ring<WM, WN, U, RM, RN, false, true>(q, grid, stream);
                }
                return true;
            }
        }
        const Params q = with_rounds(S::kBlocksPerCu);
        if (p.splits > 1) {
            launch_ring<WM, WN, U, RM, RN, true, false>(q, grid, stream);
        } else {
            launch_ring<WM, WN, U, RM, RN, false, false>(q, grid, stream);
        }
    } else {
        using S = StreamShape<WM, WN, U, RM, RN>;
        const int64_t tiles = ((p.M + S::kBM - 1) / S::kBM) * static_cast<int64_t>((p.N + S::kBN - 1) / S::kBN);
        if (p.splits > 1) {
            launch_stream<WM, WN, U, RM, RN, true>(p, dim3(static_cast<uint32_t>(tiles * p.splits)), stream);
        } else {
            launch_stream<WM, WN, U, RM, RN, false>(p, dim3(static_cast<uint32_t>(tiles)), stream);
        }
    }
    return true;
}

}  // namespace

bool FEATHER_COMBO_FN(FEATHER_B_E5M2, FEATHER_A_BF16, FEATHER_OUT_BF16)(const TileQuery& t, const Params& p,
                                                                          hipStream_t stream) {
#define FEATHER_TRY_TILE(wm, wn, u, rm, rn, pf) || try_tile<wm, wn, u, rm, rn, pf>(t, p, stream)
    return false FEATHER_SCALED_MM_TILES(FEATHER_TRY_TILE);
#undef FEATHER_TRY_TILE
}

}  // namespace feather
