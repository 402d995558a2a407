// Clocks a memory instruction takes from the MFMA stream on gfx950, at one and at two waves per SIMD.
//
// A "stage" is 128 independent v_mfma_f32_16x16x32_f16 per wave (2048 clocks at full rate for one wave) with N
// memory instructions of one kind, issued in bursts of G back-to-back and spread evenly through the MFMAs
// (scheduling barriers keep the order; the accumulators are pinned to AGPRs so nothing else moves). Every loaded
// byte is used after the stage, so no load is narrowed or dead. Blocks hold more than half the LDS, so each CU runs
// exactly one block: 256 threads = one wave per SIMD, 512 threads = two waves per SIMD, all running the same code.
// Reported: the slowest wave's clocks per stage (s_memtime); the extra clocks per memory instruction are
// (stage - MFMA-only stage) / (N x waves per SIMD), i.e. what the SIMD loses per instruction.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

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
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr int kIters = 200;

__device__ __forceinline__ void mfma_agpr(f32x4& acc, half8 w, half8 x) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(w), "v"(x));
}

enum Kind { kNone, kDma, kLdsRead, kVgprLoad, kLdsWrite };

template <int KIND, int N, int G, int WAVES>
__global__ __launch_bounds__(256 * WAVES) void stage_loop(const uint8_t* src, uint32_t src_bytes, float* out,
                                                          unsigned long long* clk) {
    // 96 KiB (one wave per SIMD) or 128 KiB (two): more than half of the CU's 160 KiB, so one block per CU
    __shared__ __attribute__((aligned(1024))) uint8_t lds[WAVES == 1 ? 96 * 1024 : 128 * 1024];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)src_bytes, 0x00020000);
    half8 a[4], b[4];
    for (int i = 0; i < 4; ++i)
        for (int e = 0; e < 8; ++e) {
            a[i][e] = (_Float16)((lane + i * 3 + e) % 7 - 3);
            b[i][e] = (_Float16)((lane * 5 + i + e) % 5 - 2);
        }
    f32x4 acc[4][8];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    constexpr int kN = N > 0 ? N : 1;
    u32x4 reg[kN];
    for (int j = 0; j < kN; ++j) reg[j] = u32x4{(uint32_t)lane, 1u, 2u, 3u};
    uint8_t* const area = lds + wave * 16384;  // 16 KiB per wave, in bounds for every wave count
    const uint32_t voff = (uint32_t)((blockIdx.x * 4 * WAVES + wave) * 16384 + lane * 16) % (src_bytes - 16384);
    constexpr int kBursts = N > 0 ? N / G : 1;
    constexpr int kEvery = 128 / kBursts;
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < kIters; ++it) {
#pragma unroll
        for (int k = 0; k < 128; ++k) {
            mfma_agpr(acc[(k / 8) % 4][k % 8], b[k % 4], a[(k / 8) % 4]);
            if (N > 0 && k % kEvery == 3) {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const int j = (k / kEvery) * G + g;
                    const int slot = (j % 15) * 1024;
                    if constexpr (KIND == kDma) {
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            r, (__attribute__((address_space(3))) void*)(reinterpret_cast<uintptr_t>(area + slot)), 16,
                            (int)voff, slot, 0, 0);
                    } else if constexpr (KIND == kLdsRead) {
                        reg[j] = *reinterpret_cast<const u32x4*>(area + slot + lane * 16);
                    } else if constexpr (KIND == kVgprLoad) {
                        reg[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, slot, 0);
                    } else if constexpr (KIND == kLdsWrite) {
                        *reinterpret_cast<u32x4*>(area + slot + lane * 16) = reg[j];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr ((KIND == kLdsRead || KIND == kVgprLoad) && N > 0) {
            for (int j = 0; j < N; ++j) a[j % 4][0] += (_Float16)((reg[j][0] ^ reg[j][1] ^ reg[j][2] ^ reg[j][3]) & 1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // the last MFMAs write back
    float sink = 0;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 8; ++j) sink += acc[i][j][0];
    out[blockIdx.x * 1024 + threadIdx.x] = sink;
    if (lane == 0 && blockIdx.x == 0) clk[wave] = t1 - t0;
}

const char* kNames[] = {"MFMAs only", "buffer_load_dwordx4 ... lds", "ds_read_b128", "buffer_load_dwordx4 (VGPR)",
                        "ds_write_b128"};

template <int KIND, int N, int G, int WAVES>
double run(const uint8_t* src, uint32_t bytes, float* out, unsigned long long* clk, hipStream_t s, double base) {
    for (int w = 0; w < 3; ++w)
        hipLaunchKernelGGL((stage_loop<KIND, N, G, WAVES>), dim3(256), dim3(256 * WAVES), 0, s, src, bytes, out, clk);
    CHECK(hipStreamSynchronize(s));
    unsigned long long h[8] = {};
    CHECK(hipMemcpy(h, clk, sizeof(unsigned long long) * 4 * WAVES, hipMemcpyDeviceToHost));
    unsigned long long slowest = 0;
    for (int w = 0; w < 4 * WAVES; ++w) slowest = h[w] > slowest ? h[w] : slowest;
    const double per = double(slowest) / kIters;
    printf("%d wave(s)/SIMD  %-28s N=%2d burst %d: %5.0f clocks per stage", WAVES, kNames[KIND], N, G, per);
    if (N > 0) printf(", %5.1f clocks per instruction", (per - base) / (N * WAVES));
    printf("\n");
    fflush(stdout);
    return per;
}

int main() {
    const uint32_t bytes = 64u << 20;
    uint8_t* src;
    CHECK(hipMalloc(&src, bytes));
    CHECK(hipMemset(src, 1, bytes));
    float* out;
    CHECK(hipMalloc(&out, 256 * 1024 * 4));
    unsigned long long* clk;
    CHECK(hipMalloc(&clk, 64));
    hipStream_t s;
    CHECK(hipStreamCreate(&s));
    for (int rep = 0; rep < 2; ++rep) {
        const double b1 = run<kNone, 0, 1, 1>(src, bytes, out, clk, s, 0);
        run<kDma, 8, 1, 1>(src, bytes, out, clk, s, b1);
        run<kDma, 16, 1, 1>(src, bytes, out, clk, s, b1);
        run<kDma, 16, 4, 1>(src, bytes, out, clk, s, b1);
        run<kLdsRead, 16, 1, 1>(src, bytes, out, clk, s, b1);
        run<kLdsRead, 32, 1, 1>(src, bytes, out, clk, s, b1);
        run<kLdsRead, 16, 4, 1>(src, bytes, out, clk, s, b1);
        run<kVgprLoad, 16, 1, 1>(src, bytes, out, clk, s, b1);
        run<kLdsWrite, 16, 1, 1>(src, bytes, out, clk, s, b1);
        const double b2 = run<kNone, 0, 1, 2>(src, bytes, out, clk, s, 0);
        run<kDma, 8, 1, 2>(src, bytes, out, clk, s, b2);
        run<kDma, 16, 1, 2>(src, bytes, out, clk, s, b2);
        run<kLdsRead, 16, 1, 2>(src, bytes, out, clk, s, b2);
        run<kVgprLoad, 16, 1, 2>(src, bytes, out, clk, s, b2);
        run<kLdsWrite, 16, 1, 2>(src, bytes, out, clk, s, b2);
    }
    return 0;
}
