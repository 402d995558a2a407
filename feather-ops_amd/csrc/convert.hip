// bf16 -> fp16 elementwise conversion, in two roundings:
//   - round-toward-zero, the semantics of the reference's Triton kernel (feather_ops/convert.py:6-21, which
//     runs v_cvt_pkrtz_f16_f32): values inside fp16's range that bf16 can hold are exact, finite values past
//     65504 saturate to +-65504, inf and NaN pass through, and values below fp16's normal range truncate
//     toward zero;
//   - round-to-nearest-even with overflow to inf, the cast the naive path applies to bf16 activations
//     (feather_ops/naive.py:21, `a.to(torch.float16)`), with the very conversion the matmul kernels use when
//     they widen bf16 activations themselves (bf16x2_to_f16x2), so a matmul over the widened copy gives the
//     same bits as one over the bf16 original.
// HBM-bound: 2 bytes read + 2 written per element. Each work-item has 4 16-byte loads in flight before it
// converts and stores (64 bytes), which one load per work-item left too few of to cover HBM latency.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "feather_ops.h"
#include "scaled_mm_kernels.h"

namespace feather {
namespace {

constexpr int kConvertThreads = 256;
constexpr int kLoads = 4;                    // 16-byte loads per work-item
constexpr int kPerThread = 8 * kLoads;       // elements per work-item
constexpr int kPerBlock = kConvertThreads * kPerThread;

template <bool kRne>
__device__ __forceinline__ uint32_t convert2(uint32_t v) {
    if constexpr (kRne) {
        return bf16x2_to_f16x2(v);
    } else {
        const float lo = __builtin_bit_cast(float, v << 16);
        const float hi = __builtin_bit_cast(float, v & 0xffff0000u);
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
}

template <bool kRne>
__device__ __forceinline__ uint16_t convert1(uint16_t h) {
    return static_cast<uint16_t>(convert2<kRne>(static_cast<uint32_t>(h)) & 0xffffu);
}

template <bool kRne>
__global__ __launch_bounds__(kConvertThreads) void bf16_to_fp16_kernel(const uint16_t* in, uint16_t* out, uint32_t n) {
    const rsrc_t src = make_rsrc(in, n * 2u);
    const rsrc_t dst = make_rsrc(out, n * 2u);
    // Work-item t's 4 loads are 16-byte pieces t, t + 256, t + 512, t + 768 of its block's span: each load
    // instruction of a wave reads 1 KiB of contiguous memory.
    const uint32_t block0 = blockIdx.x * static_cast<uint32_t>(kPerBlock);
    if (block0 + kPerBlock <= n) {
        u32x4 v[kLoads];
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            v[i] = buf_load16(src, (block0 + (i * kConvertThreads + threadIdx.x) * 8u) * 2u);
        }
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            u32x4 r;
#pragma unroll
            for (int w = 0; w < 4; ++w) r[w] = convert2<kRne>(v[i][w]);
            __builtin_amdgcn_raw_buffer_store_b128(
                r, dst, static_cast<int>((block0 + (i * kConvertThreads + threadIdx.x) * 8u) * 2u), 0, 0);
        }
        return;
    }
    // The last, partial block: whole 8-element pieces with 16-byte accesses, the rest one element at a time.
    for (uint32_t piece = block0 / 8u + threadIdx.x; piece * 8u < n; piece += kConvertThreads) {
        const uint32_t base = piece * 8u;
        if (base + 8u <= n) {
            const u32x4 v = buf_load16(src, base * 2u);
            u32x4 r;
#pragma unroll
            for (int w = 0; w < 4; ++w) r[w] = convert2<kRne>(v[w]);
            __builtin_amdgcn_raw_buffer_store_b128(r, dst, static_cast<int>(base * 2u), 0, 0);
        } else {
            for (uint32_t i = base; i < n; ++i) out[i] = convert1<kRne>(in[i]);
        }
    }
}

template <bool kRne>
bool launch_convert(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    if (n < 0 || n >= (int64_t{1} << 30) || (n > 0 && (!in || !out))) return false;
    if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) return false;
    if (n == 0) return true;
    const uint32_t blocks = static_cast<uint32_t>((n + kPerBlock - 1) / kPerBlock);
    hipLaunchKernelGGL(bf16_to_fp16_kernel<kRne>, dim3(blocks), dim3(kConvertThreads), 0, stream, in, out,
                       static_cast<uint32_t>(n));
    return true;
}

}  // namespace
}  // namespace feather

extern "C" bool feather_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    return feather::launch_convert<false>(in, out, n, stream);
}

extern "C" bool feather_widen_bf16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    return feather::launch_convert<true>(in, out, n, stream);
}
