// Weight prepack on the GPU: b [K, N] fp8 codes (row-major; the GEMM's B, i.e. W^T) ->
// b_prepacked [K_pad / 16, N, 16] with K_pad = ceil(K / 128) * 128 and zero pad rows, so that
// b_prepacked[k / 16, n, k % 16] = b[k, n] (the layout of the reference's prepack_b_for_scaled_mm,
// feather_ops/scaled_mm.py:137-150). A pure byte permutation: bit-exact, dtype-agnostic.
//
// One block per (16-deep chunk, 128 columns): 256 work-items read the chunk's 16 rows x 128 columns
// with coalesced 8-byte loads (each row segment is 128 contiguous bytes) into LDS, then each work-item
// writes half of one column's 16 contiguous bytes. HBM-bound: 1 byte read and 1 written per element.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "feather_ops.h"
#include "scaled_mm_kernels.h"

namespace feather {
namespace {

constexpr int kPrepackThreads = 256;
constexpr int kPrepackCols = 128;

__global__ __launch_bounds__(kPrepackThreads) void prepack_kernel(const uint8_t* b, uint8_t* out, uint32_t K,
                                                                   uint32_t N, uint32_t col_tiles,
                                                                   uint32_t chunks) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[16][kPrepackCols];
    const uint32_t chunk = blockIdx.x / col_tiles;
    const uint32_t n0 = (blockIdx.x % col_tiles) * kPrepackCols;
    const rsrc_t src = make_rsrc(b, K * N);
    const rsrc_t dst = make_rsrc(out, chunks * N * 16u);
    const uint32_t t = threadIdx.x;

    // Load: work-item t takes row t / 16 of the chunk, columns 8 * (t % 16) .. + 7 (N % 8 == 0, so such a
    // group is all inside N or all past it). Rows past K are the zero padding.
    {
        const uint32_t k = chunk * 16u + t / 16u;
        const uint32_t col = n0 + 8u * (t % 16u);
        const uint32_t off = (k < K && col < N) ? k * N + col : kOob;
        *reinterpret_cast<u32x2*>(&tile[t / 16u][8u * (t % 16u)]) = buf_load8(src, off);
    }
    __syncthreads();

    // Store: work-item t writes bytes 8h .. 8h + 7 (h = t % 2) of column t / 2's 16-byte group.
    const uint32_t col = t / 2u;
    const uint32_t h = t % 2u;
    uint32_t w[2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t r = 8u * h + 4u * d;
        w[d] = static_cast<uint32_t>(tile[r][col]) | (static_cast<uint32_t>(tile[r + 1][col]) << 8) |
               (static_cast<uint32_t>(tile[r + 2][col]) << 16) | (static_cast<uint32_t>(tile[r + 3][col]) << 24);
    }
    const uint32_t n = n0 + col;
    buf_store8(u32x2{w[0], w[1]}, dst, n < N ? (chunk * N + n) * 16u + 8u * h : kOob);
}

}  // namespace
}  // namespace feather

extern "C" bool feather_prepack_b(const uint8_t* b, uint8_t* b_prepacked, int64_t K, int64_t N, hipStream_t stream) {
    if (K < 1 || N < 8 || N % 8 != 0 || !b || !b_prepacked) return false;
    if ((reinterpret_cast<uintptr_t>(b) & 7u) || (reinterpret_cast<uintptr_t>(b_prepacked) & 15u)) return false;
    const int64_t k_pad = (K + 127) / 128 * 128;
    if (k_pad * N >= (int64_t{1} << 31)) return false;  // 32-bit buffer offsets
    const uint32_t chunks = static_cast<uint32_t>(k_pad / 16);
    const uint32_t col_tiles = static_cast<uint32_t>((N + feather::kPrepackCols - 1) / feather::kPrepackCols);
    hipLaunchKernelGGL(feather::prepack_kernel, dim3(chunks * col_tiles), dim3(feather::kPrepackThreads), 0, stream, b,
                       b_prepacked, static_cast<uint32_t>(K), static_cast<uint32_t>(N), col_tiles, chunks);
    return true;
}
