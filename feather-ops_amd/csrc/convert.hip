// bf16 -> fp16 elementwise conversion with round-toward-zero, the semantics of the reference's Triton
// kernel (feather_ops/convert.py:6-21, which runs v_cvt_pkrtz_f16_f32): values inside fp16's range that
// bf16 can hold are exact, finite values past 65504 saturate to +-65504, inf and NaN pass through, and
// values below fp16's normal range truncate toward zero. HBM-bound: 2 bytes read + 2 written per element.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "feather_ops.h"
#include "scaled_mm_kernels.h"

namespace feather {
namespace {

constexpr int kConvertThreads = 256;
constexpr int kPerThread = 8;  // one 16-byte load and one 16-byte store per work-item

__global__ __launch_bounds__(kConvertThreads) void bf16_to_fp16_kernel(const uint16_t* in, uint16_t* out, uint32_t n) {
    const rsrc_t src = make_rsrc(in, n * 2u);
    const rsrc_t dst = make_rsrc(out, n * 2u);
    const uint32_t base = (blockIdx.x * kConvertThreads + threadIdx.x) * kPerThread;
    if (base >= n) return;
    if (base + kPerThread <= n) {
        const u32x4 v = buf_load16(src, base * 2u);
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float lo = __builtin_bit_cast(float, v[i] << 16);
            const float hi = __builtin_bit_cast(float, v[i] & 0xffff0000u);
            r[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
        }
        __builtin_amdgcn_raw_buffer_store_b128(r, dst, static_cast<int>(base * 2u), 0, 0);
    } else {
        for (uint32_t i = base; i < n; ++i) {
            const float x = __builtin_bit_cast(float, static_cast<uint32_t>(in[i]) << 16);
            out[i] = __builtin_bit_cast(uint16_t, __builtin_amdgcn_cvt_pkrtz(x, 0.0f)[0]);
        }
    }
}

}  // namespace
}  // namespace feather

extern "C" bool feather_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    if (n < 0 || n >= (int64_t{1} << 30) || (n > 0 && (!in || !out))) return false;
    if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) return false;
    if (n == 0) return true;
    const int64_t per_block = feather::kConvertThreads * feather::kPerThread;
    const uint32_t blocks = static_cast<uint32_t>((n + per_block - 1) / per_block);
    hipLaunchKernelGGL(feather::bf16_to_fp16_kernel, dim3(blocks), dim3(feather::kConvertThreads), 0, stream, in, out,
                       static_cast<uint32_t>(n));
    return true;
}
