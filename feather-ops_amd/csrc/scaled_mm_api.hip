// C ABI of the gfx950 scaled matmul (include/feather_ops.h). Validates the contract on the host, so an
// out-of-contract call enqueues nothing, then routes to the instantiation of its dtype combination.
#include "feather_ops.h"
#include "scaled_mm_launch.h"

#include <cstdint>

namespace feather {
namespace {

constexpr int64_t kMaxBufferBytes = (int64_t{1} << 31) - 1;  // buffer offsets are 31-bit (kOob marks "out")

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
    Params p{};
    p.a = a;
    p.b = b_prepacked;
    p.scale = has_scale ? scale : nullptr;
    p.col_scale = has_scale == 2 ? 1 : 0;
    p.bias = has_bias ? bias : nullptr;
    p.c = c;
    p.M = static_cast<int32_t>(M);
    p.N = static_cast<int32_t>(N);
    p.K = static_cast<int32_t>(K);
    p.kb_total = static_cast<int32_t>((K + 127) / 128 * 8);
    const TileQuery t{block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch};
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
