// Clocks a memory instruction takes from a wave's MFMA stream on gfx950, at one wave per SIMD.
//
// A "stage" is 128 independent v_mfma_f32_16x16x32_f16 (the MFMAs of a 128 x 128 x 64 wave tile; 2048 clocks
// at full rate) with N instructions of one kind spread through it, one after every 128 / N MFMAs (scheduling
// barriers keep the order; the accumulators are pinned to AGPRs so nothing else moves). The cost per extra
// instruction is (clocks per stage - clocks with none) / N. Addresses are in bounds and conflict-free.
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

// KIND 0: none, 1: buffer_load_dwordx4 ... lds, 2: buffer_load_dwordx4 into VGPRs, 3: ds_write_b128,
// 4: ds_read_b128
template <int KIND, int N>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void stage_loop(
    const uint8_t* src, uint32_t src_bytes, float* out, unsigned long long* clk) {
    constexpr int kN = N > 0 ? N : 1;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[64 * 1024];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)src_bytes, 0x00020000);
    half8 a[8], b[8];
    for (int i = 0; i < 8; ++i)
        for (int e = 0; e < 8; ++e) {
            a[i][e] = (_Float16)((lane + i * 3 + e) % 7 - 3);
            b[i][e] = (_Float16)((lane * 5 + i + e) % 5 - 2);
        }
    f32x4 acc[8][8];
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    u32x4 reg[kN];
    for (int n = 0; n < kN; ++n) reg[n] = u32x4{(uint32_t)lane, 1u, 2u, 3u};
    uint8_t* const area = lds + wave * 16384;  // 16 KiB per wave
    const uint32_t voff = (uint32_t)((blockIdx.x * 4 + wave) * 16384 + lane * 16) % (src_bytes - 16384);
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < kIters; ++it) {
#pragma unroll
        for (int k = 0; k < 128; ++k) {
            mfma_agpr(acc[(k / 8) % 8][k % 8], b[k % 8], a[(k / 8) % 8]);
            if (N > 0 && k % (128 / kN) == 3) {
                const int n = k / (128 / kN);
                const int slot = (n % 16) * 1024;
                if constexpr (KIND == 1) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        r, (__attribute__((address_space(3))) void*)(reinterpret_cast<uintptr_t>(area + slot)), 16,
                        (int)voff, slot, 0, 0);
                } else if constexpr (KIND == 2) {
                    reg[n] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, slot, 0);
                } else if constexpr (KIND == 3) {
                    *reinterpret_cast<u32x4*>(area + slot + lane * 16) = reg[n];
                } else if constexpr (KIND == 4) {
                    reg[n] = *reinterpret_cast<const u32x4*>(area + slot + lane * 16);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (KIND == 2 || KIND == 4) {  // use the loaded registers, so nothing is dead
            for (int n = 0; n < N; ++n) a[n % 8][0] += (_Float16)(reg[n][0] & 1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // the last MFMAs write back
    float sink = 0;
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) sink += acc[i][j][0];
    out[blockIdx.x * 256 + threadIdx.x] = sink;
    if (threadIdx.x == 0 && blockIdx.x == 0) clk[0] = t1 - t0;
}

template <int KIND, int N>
double run(const char* name, const uint8_t* src, uint32_t bytes, float* out, unsigned long long* clk, hipStream_t s,
           double base) {
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL((stage_loop<KIND, N>), dim3(256), dim3(256), 0, s, src, bytes, out, clk);
    CHECK(hipStreamSynchronize(s));
    unsigned long long h;
    CHECK(hipMemcpy(&h, clk, 8, hipMemcpyDeviceToHost));
    const double per = double(h) / kIters;
    printf("%-30s N=%2d: %5.0f clocks per 128 MFMAs", name, N, per);
    if (N > 0) printf(", %.1f clocks per instruction", (per - base) / N);
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
    CHECK(hipMalloc(&out, 256 * 256 * 4));
    unsigned long long* clk;
    CHECK(hipMalloc(&clk, 8));
    hipStream_t s;
    CHECK(hipStreamCreate(&s));
    for (int rep = 0; rep < 2; ++rep) {
        const double base = run<0, 0>("MFMAs only", src, bytes, out, clk, s, 0);
        run<1, 8>("buffer_load_dwordx4 lds", src, bytes, out, clk, s, base);
        run<1, 16>("buffer_load_dwordx4 lds", src, bytes, out, clk, s, base);
        run<2, 8>("buffer_load_dwordx4 (VGPR)", src, bytes, out, clk, s, base);
        run<2, 16>("buffer_load_dwordx4 (VGPR)", src, bytes, out, clk, s, base);
        run<3, 8>("ds_write_b128", src, bytes, out, clk, s, base);
        run<3, 16>("ds_write_b128", src, bytes, out, clk, s, base);
        run<4, 16>("ds_read_b128", src, bytes, out, clk, s, base);
        run<4, 32>("ds_read_b128", src, bytes, out, clk, s, base);
    }
    return 0;
}
