// Sustained fp16 MFMA rate on gfx950 with data-dependent operands.
//
// Each wave runs a 64 x 128 (16x16x32) or the same work as 32x32x16 MFMAs over 24 operand fragments read once
// from memory, so consecutive MFMAs see different operands, as in a GEMM; the constant-operand runs show the
// clock without data-dependent switching power. Reported: TFLOP/s over the launch and the effective shader clock
// of wave 0 (s_memtime ticks over s_memrealtime's 100 MHz). The B-side fragments have a zero low byte, like an
// e5m2 code decoded to fp16.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

using half8 = _Float16 __attribute__((ext_vector_type(8)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));

constexpr int kIters = 2000;

// SHAPE 0: 16x16x32 (4 x 8 accumulators of 16x16), SHAPE 1: 32x32x16 (2 x 4 of 32x32), same FLOPs per iteration.
template <int SHAPE>
__global__ __launch_bounds__(256, 2) void mfma_loop(const half8* ops, float* out, unsigned long long* clk) {
    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * 4 + threadIdx.x / 64;
    half8 a[2][4], b[2][8];
    for (int s = 0; s < 2; ++s) {
        for (int i = 0; i < 4; ++i) a[s][i] = ops[(w * 24 + s * 12 + i) * 64 + lane];
        for (int j = 0; j < 8; ++j) b[s][j] = ops[(w * 24 + s * 12 + 4 + j) * 64 + lane];
    }
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    float sink = 0.f;
    if constexpr (SHAPE == 0) {
        f32x4 acc[4][8] = {};
        for (int it = 0; it < kIters; ++it) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[s][j], a[s][i], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half8 t = a[0][i];
                a[0][i] = a[1][i];
                a[1][i] = t;
            }
        }
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 8; ++j) sink += acc[i][j][0] + acc[i][j][3];
    } else {
        f32x16 acc[2][4] = {};
        for (int it = 0; it < kIters; ++it) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[s / 2][(s % 2) * 4 + j],
                                                                          a[s / 2][(s % 2) * 2 + i], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half8 t = a[0][i];
                a[0][i] = a[1][i];
                a[1][i] = t;
            }
        }
        for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 4; ++j) sink += acc[i][j][0] + acc[i][j][15];
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 256 + threadIdx.x] = sink;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clk[0] = t1 - t0;
        clk[1] = r1 - r0;
    }
}

template <int SHAPE>
void run(const char* name, const half8* ops, float* out, unsigned long long* clk, int blocks, hipStream_t s) {
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL((mfma_loop<SHAPE>), dim3(blocks), dim3(256), 0, s, ops, out, clk);
    CHECK(hipStreamSynchronize(s));
    hipEvent_t a, z;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&z));
    const int reps = 10;
    CHECK(hipEventRecord(a, s));
    for (int r = 0; r < reps; ++r) hipLaunchKernelGGL((mfma_loop<SHAPE>), dim3(blocks), dim3(256), 0, s, ops, out, clk);
    CHECK(hipEventRecord(z, s));
    CHECK(hipEventSynchronize(z));
    float ms;
    CHECK(hipEventElapsedTime(&ms, a, z));
    ms /= reps;
    unsigned long long h[2];
    CHECK(hipMemcpy(h, clk, sizeof h, hipMemcpyDeviceToHost));
    const double flop = 2.0 * 64 * 128 * 64 * kIters * 4.0 * blocks;
    printf("%-34s %4d blocks: %.3f ms, %5.0f TFLOP/s, shader clock %.2f GHz\n", name, blocks, ms,
           flop / (ms * 1e-3) / 1e12, h[0] / (h[1] / 100e6) / 1e9);
    fflush(stdout);
}

int main() {
    const int blocks = 512;  // two 4-wave blocks per CU: two waves per SIMD
    const size_t n = size_t(blocks) * 4 * 24 * 64;
    std::vector<_Float16> host(n * 8), konst(n * 8, (_Float16)0.5f);
    std::mt19937 g(1);
    std::normal_distribution<float> nd(0.f, 1.f);
    for (size_t i = 0; i < host.size(); ++i) {
        _Float16 h = (_Float16)nd(g);
        if ((i / (64 * 8)) % 12 >= 4) {  // B-side fragments: zero low byte
            uint16_t bits;
            std::memcpy(&bits, &h, 2);
            bits &= 0xff00;
            std::memcpy(&h, &bits, 2);
        }
        host[i] = h;
    }
    half8 *ops, *kops;
    CHECK(hipMalloc(&ops, n * sizeof(half8)));
    CHECK(hipMalloc(&kops, n * sizeof(half8)));
    CHECK(hipMemcpy(ops, host.data(), n * sizeof(half8), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(kops, konst.data(), n * sizeof(half8), hipMemcpyHostToDevice));
    float* out;
    CHECK(hipMalloc(&out, blocks * 256 * 4));
    unsigned long long* clk;
    CHECK(hipMalloc(&clk, 16));
    hipStream_t s;
    CHECK(hipStreamCreate(&s));
    for (int rep = 0; rep < 2; ++rep) {
        run<0>("16x16x32 random, 2 waves/SIMD", ops, out, clk, blocks, s);
        run<0>("16x16x32 random, 1 wave/SIMD", ops, out, clk, blocks / 2, s);
        run<0>("16x16x32 constant, 2 waves/SIMD", kops, out, clk, blocks, s);
        run<1>("32x32x16 random, 2 waves/SIMD", ops, out, clk, blocks, s);
        run<1>("32x32x16 constant, 2 waves/SIMD", kops, out, clk, blocks, s);
    }
    return 0;
}
