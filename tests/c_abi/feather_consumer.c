/*
 * A torch-free C consumer of include/feather_ops.h, compiled with gcc and linked against
 * libfeather_ops_gfx950.so: the role of the reference's cpp_benchmarks/benchmark_scaled_mm_hip.cpp:27-47,
 * 150-290 (declare the C ABI, hipMalloc the operands, launch, time with hipEvents), built from the header
 * instead of a hand-copied declaration, so a drift between header and library fails to compile or link.
 *
 *   feather_consumer refuse
 *       Host-only: every out-of-contract call must return false (nothing enqueued, no GPU needed), and the
 *       workspace query must answer without a GPU. Exit 0 when all hold.
 *   feather_consumer run DIR M N K A_BF16 OUT_BF16 WM WN U RM RN PREFETCH SPLITS
 *       GPU: reads DIR/a.bin ([M, K] 16-bit bits), DIR/b.bin ([K, N] fp8 e5m2 codes, the unpacked weight),
 *       DIR/scale.bin (one fp32) and DIR/bias.bin ([N] output-dtype bits); prepacks the weight on the GPU
 *       (feather_prepack_b), runs launch_scaled_mm and feather_scaled_mm_splitk with SPLITS on a zeroed
 *       workspace, writes DIR/c.bin and DIR/c_split.bin, and prints the average time of 20 launches. With
 *       A_BF16 it also widens the activations once (feather_widen_bf16) and runs launch_scaled_mm on the fp16
 *       copy, writing DIR/c_widened.bin (the same bits as c.bin by the header's contract).
 */
#include <hip/hip_runtime_api.h>

#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "feather_ops.h"

#define CHECK_HIP(cmd)                                                                                  \
    do {                                                                                                \
        hipError_t err_ = (cmd);                                                                        \
        if (err_ != hipSuccess) {                                                                       \
            fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(err_), __FILE__, __LINE__);   \
            exit(2);                                                                                    \
        }                                                                                               \
    } while (0)

static int failures = 0;

static void expect(bool got, bool want, const char* what) {
    if (got != want) {
        fprintf(stderr, "FAIL: %s returned %d, expected %d\n", what, (int)got, (int)want);
        ++failures;
    }
}

/* Fake, aligned, never-dereferenced device addresses: every call below is refused before any GPU work. */
#define PTR(type, addr) ((type)(uintptr_t)(addr))

static int refuse(void) {
    const uint16_t* a = PTR(const uint16_t*, 0x100000);
    const uint8_t* b = PTR(const uint8_t*, 0x200000);
    const float* s = PTR(const float*, 0x300000);
    const uint16_t* bias = PTR(const uint16_t*, 0x400000);
    uint16_t* c = PTR(uint16_t*, 0x500000);
    /* (M, N, K): N % 8, K % 16, K >= 16, M >= 1 */
    expect(launch_scaled_mm(a, b, s, bias, c, 16, 100, 64, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "N % 8 != 0");
    expect(launch_scaled_mm(a, b, s, bias, c, 16, 128, 40, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "K % 16 != 0");
    expect(launch_scaled_mm(a, b, s, bias, c, 0, 128, 64, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "M == 0");
    expect(launch_scaled_mm(a, b, s, bias, c, 16, 128, 0, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "K == 0");
    /* alignment and missing pointers */
    expect(launch_scaled_mm(PTR(const uint16_t*, 0x100008), b, s, bias, c, 16, 128, 64, 1, 1, true, false, false,
                            2, 2, 4, 4, 4, true, NULL),
           false, "a not 16-byte aligned");
    expect(launch_scaled_mm(a, b, s, PTR(const uint16_t*, 0x400002), c, 16, 128, 64, 1, 1, true, false, false, 2,
                            2, 4, 4, 4, true, NULL),
           false, "bias not 8-byte aligned");
    expect(launch_scaled_mm(a, b, NULL, bias, c, 16, 128, 64, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "has_scale without scale");
    expect(launch_scaled_mm(a, b, PTR(const float*, 0x300004), bias, c, 16, 128, 64, 2, 1, true, false, false, 2,
                            2, 4, 4, 4, true, NULL),
           false, "per-column scale not 16-byte aligned");
    expect(launch_scaled_mm(a, NULL, s, bias, c, 16, 128, 64, 1, 1, true, false, false, 2, 2, 4, 4, 4, true, NULL),
           false, "no weight");
    /* a 2 GiB output */
    expect(launch_scaled_mm(a, b, s, bias, c, 65536, 16384, 64, 1, 1, true, false, false, 2, 2, 4, 4, 4, true,
                            NULL),
           false, "output of 2 GiB");
    /* a tile that is not instantiated: the reference's only false case */
    expect(launch_scaled_mm(a, b, s, bias, c, 16, 128, 64, 1, 1, true, false, false, 3, 3, 3, 3, 3, true, NULL),
           false, "uninstantiated tile");

    /* split-K: workspace size, split count */
    const int64_t ws = feather_splitk_workspace_bytes(512, 5376, 5120, 2, 2, 4, 4, 4, true, 3);
    if (ws <= 64 * 1024) {
        fprintf(stderr, "FAIL: workspace query returned %lld\n", (long long)ws);
        ++failures;
    }
    if (feather_splitk_workspace_bytes(512, 5376, 5120, 2, 2, 4, 4, 4, true, 1) != 0) {
        fprintf(stderr, "FAIL: splits = 1 needs no workspace\n");
        ++failures;
    }
    if (feather_splitk_workspace_bytes(512, 5376, 5120, 2, 2, 4, 4, 4, true, 33) != -1) {
        fprintf(stderr, "FAIL: 33 splits are out of contract\n");
        ++failures;
    }
    void* wsp = PTR(void*, 0x600000);
    expect(feather_scaled_mm_splitk(a, b, s, bias, c, 512, 5376, 5120, 1, 1, true, false, false, 2, 2, 4, 4, 4,
                                    true, 3, wsp, ws - 1, NULL),
           false, "short workspace");
    expect(feather_scaled_mm_splitk(a, b, s, bias, c, 512, 5376, 5120, 1, 1, true, false, false, 2, 2, 4, 4, 4,
                                    true, 3, PTR(void*, 0x600010), ws, NULL),
           false, "workspace not 256-byte aligned");
    expect(feather_scaled_mm_splitk(a, b, s, bias, c, 512, 5376, 5120, 1, 1, true, false, false, 2, 2, 4, 4, 4,
                                    true, 3, NULL, ws, NULL),
           false, "no workspace");
    /* the other entry points */
    expect(feather_bf16_to_fp16(a, c, -1, NULL), false, "bf16_to_fp16 with n < 0");
    expect(feather_bf16_to_fp16(PTR(const uint16_t*, 0x100002), c, 16, NULL), false, "bf16_to_fp16 misaligned");
    expect(feather_bf16_to_fp16(a, c, 0, NULL), true, "bf16_to_fp16 with n == 0 (nothing to do)");
    expect(feather_widen_bf16(a, c, -1, NULL), false, "widen_bf16 with n < 0");
    expect(feather_widen_bf16(a, PTR(uint16_t*, 0x500008), 16, NULL), false, "widen_bf16 output misaligned");
    expect(feather_widen_bf16(a, c, 0, NULL), true, "widen_bf16 with n == 0 (nothing to do)");
    expect(feather_prepack_b(b, PTR(uint8_t*, 0x700000), 64, 12, NULL), false, "prepack with N % 8 != 0");
    expect(feather_prepack_b(b, PTR(uint8_t*, 0x700008), 64, 16, NULL), false, "prepack output misaligned");
    if (failures == 0) printf("refusals ok\n");
    return failures == 0 ? 0 : 1;
}

static void* read_file(const char* dir, const char* name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(2);
    }
    void* buf = malloc(bytes);
    if (!buf || fread(buf, 1, bytes, f) != bytes) {
        fprintf(stderr, "short read of %s\n", path);
        exit(2);
    }
    fclose(f);
    return buf;
}

static void write_file(const char* dir, const char* name, const void* data, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "wb");
    if (!f || fwrite(data, 1, bytes, f) != bytes) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

static int run(int argc, char** argv) {
    if (argc != 15) {
        fprintf(stderr, "usage: feather_consumer run DIR M N K A_BF16 OUT_BF16 WM WN U RM RN PREFETCH SPLITS\n");
        return 2;
    }
    const char* dir = argv[2];
    const int64_t M = atoll(argv[3]), N = atoll(argv[4]), K = atoll(argv[5]);
    const bool a_bf16 = atoi(argv[6]) != 0, out_bf16 = atoi(argv[7]) != 0;
    const int wm = atoi(argv[8]), wn = atoi(argv[9]), u = atoi(argv[10]), rm = atoi(argv[11]), rn = atoi(argv[12]);
    const bool prefetch = atoi(argv[13]) != 0;
    const int splits = atoi(argv[14]);
    const int64_t k_pad = (K + 127) / 128 * 128;
    const size_t a_bytes = (size_t)(M * K * 2), b_bytes = (size_t)(K * N), p_bytes = (size_t)(k_pad * N);
    const size_t c_bytes = (size_t)(M * N * 2);

    void* h_a = read_file(dir, "a.bin", a_bytes);
    void* h_b = read_file(dir, "b.bin", b_bytes);
    void* h_s = read_file(dir, "scale.bin", 4);
    void* h_bias = read_file(dir, "bias.bin", (size_t)N * 2);

    uint16_t *d_a, *d_bias, *d_c;
    uint8_t *d_b, *d_p;
    float* d_s;
    void* d_ws = NULL;
    CHECK_HIP(hipMalloc((void**)&d_a, a_bytes));
    CHECK_HIP(hipMalloc((void**)&d_b, b_bytes));
    CHECK_HIP(hipMalloc((void**)&d_p, p_bytes));
    CHECK_HIP(hipMalloc((void**)&d_s, 4));
    CHECK_HIP(hipMalloc((void**)&d_bias, (size_t)N * 2));
    CHECK_HIP(hipMalloc((void**)&d_c, c_bytes));
    CHECK_HIP(hipMemcpy(d_a, h_a, a_bytes, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_b, h_b, b_bytes, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_s, h_s, 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_bias, h_bias, (size_t)N * 2, hipMemcpyHostToDevice));

    hipStream_t stream;
    CHECK_HIP(hipStreamCreate(&stream));
    if (!feather_prepack_b(d_b, d_p, K, N, stream)) {
        fprintf(stderr, "feather_prepack_b refused the call\n");
        return 1;
    }
    if (!launch_scaled_mm(d_a, d_p, d_s, d_bias, d_c, M, N, K, 1, 1, true, a_bf16, out_bf16, wm, wn, u, rm, rn,
                          prefetch, stream)) {
        fprintf(stderr, "launch_scaled_mm refused the call\n");
        return 1;
    }
    CHECK_HIP(hipGetLastError());
    CHECK_HIP(hipStreamSynchronize(stream));
    void* h_c = malloc(c_bytes);
    CHECK_HIP(hipMemcpy(h_c, d_c, c_bytes, hipMemcpyDeviceToHost));
    write_file(dir, "c.bin", h_c, c_bytes);

    /* bf16 activations widened once up front, then the fp16-activation launch: the same output bits */
    if (a_bf16) {
        uint16_t* d_a16;
        CHECK_HIP(hipMalloc((void**)&d_a16, a_bytes));
        CHECK_HIP(hipMemset(d_c, 0, c_bytes));
        if (!feather_widen_bf16(d_a, d_a16, M * K, stream) ||
            !launch_scaled_mm(d_a16, d_p, d_s, d_bias, d_c, M, N, K, 1, 1, true, false, out_bf16, wm, wn, u, rm, rn,
                              prefetch, stream)) {
            fprintf(stderr, "feather_widen_bf16 or the launch after it refused the call\n");
            return 1;
        }
        CHECK_HIP(hipGetLastError());
        CHECK_HIP(hipStreamSynchronize(stream));
        CHECK_HIP(hipMemcpy(h_c, d_c, c_bytes, hipMemcpyDeviceToHost));
        write_file(dir, "c_widened.bin", h_c, c_bytes);
        CHECK_HIP(hipFree(d_a16));
    }

    /* the same product split along K, through a caller-owned workspace zeroed once */
    const int64_t ws_bytes = feather_splitk_workspace_bytes(M, N, K, wm, wn, u, rm, rn, prefetch, splits);
    if (ws_bytes < 0) {
        fprintf(stderr, "split count out of contract\n");
        return 1;
    }
    if (ws_bytes > 0) {
        CHECK_HIP(hipMalloc(&d_ws, (size_t)ws_bytes));
        CHECK_HIP(hipMemset(d_ws, 0, (size_t)ws_bytes));
    }
    CHECK_HIP(hipMemset(d_c, 0, c_bytes));
    if (!feather_scaled_mm_splitk(d_a, d_p, d_s, d_bias, d_c, M, N, K, 1, 1, true, a_bf16, out_bf16, wm, wn, u, rm,
                                  rn, prefetch, splits, d_ws, ws_bytes, stream)) {
        fprintf(stderr, "feather_scaled_mm_splitk refused the call\n");
        return 1;
    }
    CHECK_HIP(hipGetLastError());
    CHECK_HIP(hipStreamSynchronize(stream));
    CHECK_HIP(hipMemcpy(h_c, d_c, c_bytes, hipMemcpyDeviceToHost));
    write_file(dir, "c_split.bin", h_c, c_bytes);

    /* timing, as the reference's benchmark does: hipEvents around back-to-back launches */
    hipEvent_t start, stop;
    CHECK_HIP(hipEventCreate(&start));
    CHECK_HIP(hipEventCreate(&stop));
    const int iters = 20;
    CHECK_HIP(hipEventRecord(start, stream));
    for (int i = 0; i < iters; ++i) {
        launch_scaled_mm(d_a, d_p, d_s, d_bias, d_c, M, N, K, 1, 1, true, a_bf16, out_bf16, wm, wn, u, rm, rn,
                         prefetch, stream);
    }
    CHECK_HIP(hipEventRecord(stop, stream));
    CHECK_HIP(hipEventSynchronize(stop));
    float ms = 0.0f;
    CHECK_HIP(hipEventElapsedTime(&ms, start, stop));
    printf("launch_scaled_mm %lldx%lldx%lld: %.3f us per launch (%d launches)\n", (long long)M, (long long)N,
           (long long)K, 1e3 * ms / iters, iters);

    CHECK_HIP(hipEventDestroy(start));
    CHECK_HIP(hipEventDestroy(stop));
    CHECK_HIP(hipStreamDestroy(stream));
    if (d_ws) CHECK_HIP(hipFree(d_ws));
    CHECK_HIP(hipFree(d_c));
    CHECK_HIP(hipFree(d_bias));
    CHECK_HIP(hipFree(d_s));
    CHECK_HIP(hipFree(d_p));
    CHECK_HIP(hipFree(d_b));
    CHECK_HIP(hipFree(d_a));
    free(h_a);
    free(h_b);
    free(h_s);
    free(h_bias);
    free(h_c);
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 2 && strcmp(argv[1], "refuse") == 0) return refuse();
    if (argc >= 2 && strcmp(argv[1], "run") == 0) return run(argc, argv);
    fprintf(stderr, "usage: feather_consumer refuse | run DIR M N K A_BF16 OUT_BF16 WM WN U RM RN PREFETCH SPLITS\n");
    return 2;
}
