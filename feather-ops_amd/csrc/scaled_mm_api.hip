// C ABI of the gfx950 scaled matmul (include/feather_ops.h). Validates the contract on the host, so an
// out-of-contract call enqueues nothing, then routes to the instantiation of its dtype combination.
#include "feather_ops.h"
#include "feather_tiles.h"
#include "scaled_mm_launch.h"

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace feather {
namespace {

constexpr int64_t kMaxBufferBytes = (int64_t{1} << 31) - 1;  // buffer offsets are 31-bit (kOob marks "out")
constexpr int kMaxSplits = 32;
// The arrival counters occupy a fixed area at the start of every split workspace, whatever the shape, so
// a workspace reused across shapes never has partial sums where a later call keeps its counters.
constexpr int64_t kSplitCtrBytes = 64 * 1024;

// Non-temporal weight loads (feather_set_weight_streaming). A weight read once per launch and streamed from HBM
// loads 4-9% faster with the hint (MI355X, weights of 59-235 MB, working sets past the 256 MB MALL); a working
// set the MALL could hold (a small model, or one weight timed in a loop) loads up to a third slower, because
// non-temporal lines are not kept there. In auto mode the hint goes to weights from kStreamWeightMinBytes on:
// a model with weights that large does not fit the MALL, and below it the measured gains were small or losses.
constexpr int64_t kStreamWeightMinBytes = int64_t{48} << 20;
constexpr int kStreamOff = 0;
constexpr int kStreamOn = 1;
constexpr int kStreamAuto = 2;

// The process-wide mode; FEATHER_OPS_WEIGHT_STREAMING (0, 1 or 2) sets its first value, auto by default.
std::atomic<int>& stream_mode() {
    static std::atomic<int> mode{[] {
        const char* env = std::getenv("FEATHER_OPS_WEIGHT_STREAMING");
        if (env && std::strcmp(env, "0") == 0) return kStreamOff;
        if (env && std::strcmp(env, "1") == 0) return kStreamOn;
        return kStreamAuto;
    }()};
    return mode;
}

bool stream_weight(int64_t weight_bytes) {
    const int mode = stream_mode().load(std::memory_order_relaxed);
    return mode == kStreamOn || (mode == kStreamAuto && weight_bytes >= kStreamWeightMinBytes);
}

bool aligned(const void* ptr, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) == 0;
}

bool contract_ok(const uint16_t* a, const uint8_t* b, const float* scale, const uint16_t* bias, const uint16_t* c,
                 int64_t M, int64_t N, int64_t K, int has_scale, int has_bias) {
    if (M < 1 || N < 1 || K < 16) return false;
    if (N % 8 != 0 || K % 16 != 0) return false;
    if (!a || !b || !c) return false;
    if (has_scale && !scale) return false;
    if (has_bias && !bias) return false;
    if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16)) return false;
    if (has_bias && !aligned(bias, 8)) return false;
    if (has_scale == 2 && !aligned(scale, 16)) return false;
    const int64_t kb_rows = (K + 127) / 128 * 8;
    if (M * K * 2 > kMaxBufferBytes || M * N * 2 > kMaxBufferBytes || kb_rows * N * 16 > kMaxBufferBytes) {
        return false;
    }
    return true;
}

// True for a tile of the instantiated table.
bool is_tile(int wm, int wn, int u, int rm, int rn, bool prefetch) {
#define FEATHER_IS_TILE(twm, twn, tu, trm, trn, tpf) \
    || (((tpf) != 0) == prefetch && wm == (twm) && wn == (twn) && u == (tu) && rm == (trm) && rn == (trn))
    return false FEATHER_SCALED_MM_TILES(FEATHER_IS_TILE);
#undef FEATHER_IS_TILE
}

// Workspace of a split launch: the counter area (one uint32 per tile and join slot, at most kSplitCtrBytes),
// then the partial sums (splits fp32 tiles per output tile); none for splits = 1. -1 when the tile, the
// split count or the grid is out of contract. A ring tile joins per wave (WM * WN slots) and splits its
// 16*U-deep stages; a streaming tile (block BM = 16 * RM, BN = 16 * WN * RN) joins per 16 x 16 fragment
// (WN * RM * RN slots; WN when its block has one K slice) and splits its 64-deep groups.
struct SplitLayout {
    int64_t ctr_bytes = -1;
    int64_t total_bytes = -1;
};

SplitLayout split_layout(int64_t M, int64_t N, int64_t K, int wm, int wn, int u, int rm, int rn, bool prefetch,
                         int splits) {
    SplitLayout l;
    if (M < 1 || N < 1 || K < 16 || !is_tile(wm, wn, u, rm, rn, prefetch)) return l;
    const int64_t units = prefetch ? (K + 16 * u - 1) / (16 * u) : (K + 63) / 64;
    if (splits < 1 || splits > kMaxSplits || splits > units) return l;
    if (splits == 1) {  // the unsplit kernel: no workspace
        l.ctr_bytes = 0;
        l.total_bytes = 0;
        return l;
    }
    const int64_t bm = prefetch ? 16 * wm * rm : 16 * rm;
    const int64_t bn = 16 * wn * rn;
    const int64_t slots = prefetch ? wm * wn : (wm > 1 ? wn * rm * rn : wn);
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    if (tiles * slots * 4 > kSplitCtrBytes) return l;
    const int64_t total = kSplitCtrBytes + tiles * splits * bm * bn * 4;
    if (total > kMaxBufferBytes) return l;
    l.ctr_bytes = kSplitCtrBytes;
    l.total_bytes = total;
    return l;
}

// ---- the allocation-free split-K entry point's scratch -------------------------------------------------------

// Device memory of feather_scaled_mm_splitk_noalloc, in place of a caller's workspace: the same layout (the
// 64 KiB counter area, then the partial sums), sized for split launches with up to 64 MiB of fp32 partials
// (1024 workgroups of a 128 x 128 ring tile), the most the split heuristic launches. The array is part of the
// code object, so every GPU the library is loaded onto reserves its own copy until the process ends, whether
// or not the entry point is ever called. Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the current device.
constexpr int64_t kScratchBytes = kSplitCtrBytes + (int64_t{64} << 20);
static_assert(kScratchBytes == FEATHER_NOALLOC_SCRATCH_BYTES, "the size the public header promises");
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kMaxDevices];   // per device, from hipGetSymbolAddress
bool g_counters_cleared[kMaxDevices];  // the counter area has been cleared by a kernel that ran eagerly

// Zeroes the counter area with vector stores (a kernel rather than a memset, so that a launch recorded under
// graph capture replays correctly).
__global__ __launch_bounds__(256) void clear_counters_kernel(u32x4* ctr, int n16) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n16) ctr[i] = u32x4{0u, 0u, 0u, 0u};
}

// The current device's scratch, set up on the first call on that device (and until a clear has run outside
// graph capture, each call enqueues one on `stream` ahead of the kernel: a clear recorded into a graph only
// runs when the graph does). nullptr if the device or the symbol lookup fails.
uint8_t* device_scratch(hipStream_t stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
    }
    if (!g_counters_cleared[dev]) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &capture) != hipSuccess) return nullptr;
        u32x4* ctr = reinterpret_cast<u32x4*>(g_scratch_ptr[dev]);
        int n16 = static_cast<int>(kSplitCtrBytes / 16);
        void* args[] = {&ctr, &n16};
        if (hipLaunchKernel(reinterpret_cast<const void*>(clear_counters_kernel), dim3((n16 + 255) / 256), dim3(256),
                            args, 0, stream) != hipSuccess) {
            return nullptr;
        }
        g_counters_cleared[dev] = capture == hipStreamCaptureStatusNone;
    }
    return g_scratch_ptr[dev];
}

bool launch(const Params& p, bool use_fp8_e5m2, bool a_bf16, bool output_bf16, const TileQuery& t,
            hipStream_t stream) {
    const int combo = (use_fp8_e5m2 ? 4 : 0) | (a_bf16 ? 2 : 0) | (output_bf16 ? 1 : 0);
    switch (combo) {
        case 0: return launch_combo_000(t, p, stream);
        case 1: return launch_combo_001(t, p, stream);
        case 2: return launch_combo_010(t, p, stream);
        case 3: return launch_combo_011(t, p, stream);
        case 4: return launch_combo_100(t, p, stream);
        case 5: return launch_combo_101(t, p, stream);
        case 6: return launch_combo_110(t, p, stream);
        default: return launch_combo_111(t, p, stream);
    }
}

Params make_params(const uint16_t* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                   uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias) {
    Params p{};
    p.a = a;
    p.b = b_prepacked;
    p.scale = has_scale ? scale : nullptr;
    p.bias = has_bias ? bias : nullptr;
    p.c = c;
    p.M = static_cast<int32_t>(M);
    p.N = static_cast<int32_t>(N);
    p.K = static_cast<int32_t>(K);
    p.kb_total = static_cast<int32_t>((K + 127) / 128 * 8);
    p.col_scale = has_scale == 2 ? 1 : 0;
    p.splits = 1;
    p.stream_weight = stream_weight(int64_t{p.kb_total} * N * 16) ? 1 : 0;
    return p;
}

}  // namespace
}  // namespace feather

extern "C" bool launch_scaled_mm(const uint16_t* const a, const uint8_t* const b_prepacked, const float* const scale,
                                 const uint16_t* const bias, uint16_t* const c, const int64_t M, const int64_t N,
                                 const int64_t K, const int has_scale, const int has_bias, const bool use_fp8_e5m2,
                                 const bool a_bf16, const bool output_bf16, const int block_warps_m,
                                 const int block_warps_n, const int unroll_k, const int repeat_m, const int repeat_n,
                                 const bool prefetch, hipStream_t stream) {
    using namespace feather;
    if (!contract_ok(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias)) return false;
    const Params p = make_params(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias);
    const TileQuery t{block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch};
    return launch(p, use_fp8_e5m2, a_bf16, output_bf16, t, stream);
}

extern "C" int64_t feather_splitk_workspace_bytes(const int64_t M, const int64_t N, const int64_t K,
                                                  const int block_warps_m, const int block_warps_n,
                                                  const int unroll_k, const int repeat_m, const int repeat_n,
                                                  const bool prefetch, const int splits) {
    return feather::split_layout(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch,
                                 splits)
        .total_bytes;
}

extern "C" bool feather_scaled_mm_splitk(const uint16_t* const a, const uint8_t* const b_prepacked,
                                         const float* const scale, const uint16_t* const bias, uint16_t* const c,
                                         const int64_t M, const int64_t N, const int64_t K, const int has_scale,
                                         const int has_bias, const bool use_fp8_e5m2, const bool a_bf16,
                                         const bool output_bf16, const int block_warps_m, const int block_warps_n,
                                         const int unroll_k, const int repeat_m, const int repeat_n,
                                         const bool prefetch, const int splits, void* const workspace,
                                         const int64_t workspace_bytes, hipStream_t stream) {
    using namespace feather;
    if (!contract_ok(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias)) return false;
    const SplitLayout l =
        split_layout(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch, splits);
    if (l.total_bytes < 0) return false;
    if (splits > 1 && (!workspace || !aligned(workspace, 256) || workspace_bytes < l.total_bytes)) return false;
    Params p = make_params(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias);
    if (splits > 1) {
        p.splits = splits;
        p.split_ctr = static_cast<uint32_t*>(workspace);
        p.split_part = static_cast<uint8_t*>(workspace) + l.ctr_bytes;
    }
    const TileQuery t{block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch};
    return launch(p, use_fp8_e5m2, a_bf16, output_bf16, t, stream);
}

extern "C" bool feather_scaled_mm_splitk_noalloc(const uint16_t* const a, const uint8_t* const b_prepacked,
                                                 const float* const scale, const uint16_t* const bias,
                                                 uint16_t* const c, const int64_t M, const int64_t N, const int64_t K,
                                                 const int has_scale, const int has_bias, const bool use_fp8_e5m2,
                                                 const bool a_bf16, const bool output_bf16, const int block_warps_m,
                                                 const int block_warps_n, const int unroll_k, const int repeat_m,
                                                 const int repeat_n, const bool prefetch, const int splits,
                                                 hipStream_t stream) {
    using namespace feather;
    if (!contract_ok(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias)) return false;
    const SplitLayout l =
        split_layout(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch, splits);
    if (l.total_bytes < 0 || l.total_bytes > kScratchBytes) return false;
    Params p = make_params(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias);
    if (splits > 1) {
        uint8_t* const ws = device_scratch(stream);
        if (!ws) return false;
        p.splits = splits;
        p.split_ctr = reinterpret_cast<uint32_t*>(ws);
        p.split_part = ws + l.ctr_bytes;
    }
    const TileQuery t{block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch};
    return launch(p, use_fp8_e5m2, a_bf16, output_bf16, t, stream);
}

extern "C" int feather_set_weight_streaming(const int mode) {
    using namespace feather;
    if (mode == -1) return stream_mode().load();
    if (mode != kStreamOff && mode != kStreamOn && mode != kStreamAuto) return -1;
    return stream_mode().exchange(mode);
}
