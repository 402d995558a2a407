/*
 * C ABI of the gfx950 scaled matmul library (libfeather_ops_gfx950.so). Plain pointers and sizes, no
 * torch types: this is the boundary a C/C++ benchmark, a ctypes/cffi binding or the thin torch extension
 * (feather-ops_amd/csrc/extension.cpp) binds.
 */
#ifndef FEATHER_OPS_H
#define FEATHER_OPS_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same declaration as <hip/hip_runtime_api.h>, so this header needs no HIP include. */
typedef struct ihipStream_t* hipStream_t;

/*
 * c[M, N] = round_out((a[M, K] @ decode(b)) * scale) (+ bias), enqueued on `stream` (asynchronous).
 *
 * Replaces the reference's `extern "C" bool launch_scaled_mm(...)` (csrc/hip_kernel.cu:687-713), as
 * declared by its consumer cpp_benchmarks/benchmark_scaled_mm_hip.cpp:27-47: same symbol, same arguments.
 *
 *   a            [M, K] row-major, fp16 bits (a_bf16 = false) or bf16 bits (a_bf16 = true); bf16 is
 *                widened to fp16 with round-to-nearest-even, as feather_ops/naive.py:21 does.
 *   b_prepacked  [K_pad/16, N, 16] fp8 codes, e5m2 (use_fp8_e5m2 = true) or e4m3fn (false), K_pad a
 *                multiple of 128 with zero pad rows (feather_ops/scaled_mm.py:137-150).
 *   scale        fp32 in device memory, read by the kernel: one per-tensor value (has_scale == 1, or any
 *                non-zero value other than 2), N per-output-column values (has_scale == 2, 16-byte aligned;
 *                an extension: the reference kernel takes only the per-tensor form, its naive path
 *                feather_ops/naive.py:29-33 both), or ignored (has_scale == 0).
 *   bias         N values of the output dtype (has_bias != 0), added after the downcast, or ignored.
 *   c            [M, N] row-major output, fp16 (output_bf16 = false) or bf16 (true), rounded to nearest even.
 *   tile         (block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, prefetch): one entry of
 *                feather_ops/tiles.py SCALED_MM_TILES (gfx950 meaning documented there).
 *
 * Contract (checked here; a violation returns false and enqueues nothing): M >= 1, N >= 1 with
 * N % 8 == 0 (the reference requires N % 16 == 0), K >= 16 with K % 16 == 0, a, b_prepacked and c
 * 16-byte aligned, bias 8-byte aligned, a/c/b_prepacked each under 2 GiB. The kernel reads
 * b_prepacked rows up to ceil(K / 128) * 8. Returns false for a tile that is not instantiated (the
 * reference's only false case) and true once the kernel is enqueued; launch errors are left to the
 * caller (hipGetLastError), as in the reference.
 */
bool launch_scaled_mm(const uint16_t* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                      uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias,
                      bool use_fp8_e5m2, bool a_bf16, bool output_bf16, int block_warps_m, int block_warps_n,
                      int unroll_k, int repeat_m, int repeat_n, bool prefetch, hipStream_t stream);

/*
 * Split-K form of launch_scaled_mm for grids with fewer output tiles than the GPU has compute units: the
 * same arguments and contract (any instantiated tile, ring or streaming), and each tile's K range cut into
 * `splits` contiguous ranges computed by separate workgroups. The partial sums (fp32) meet in
 * `workspace`; the last workgroup of a tile to finish adds them in split order and stores the tile, so
 * results are deterministic and differ from the unsplit launch only by fp32 summation order.
 *
 * No counterpart in the reference: its kernel has no split-K (README.md:21 mentions an unreleased branch
 * without a speedup on its GPU). The workspace is the caller's, like a BLAS handle's:
 *   - at least feather_splitk_workspace_bytes(...) bytes, 256-byte aligned;
 *   - its first 64 KiB (the arrival counters) all zero before its first use; every completed call leaves
 *     them zero again, whatever its shape, so zero the workspace once, not per call;
 *   - calls that share a workspace must be ordered (one stream); concurrent calls need their own.
 * splits = 1 runs the unsplit kernel and ignores the workspace. Returns false (nothing enqueued) for a
 * contract violation, a tile that is not instantiated, splits outside 1 .. min(32, units of K) (a ring
 * tile's units are its ceil(K / (16 * unroll_k)) stages, a streaming tile's the ceil(K / 64) groups), more
 * than 16384 join counters (tiles x slots: a ring tile's waves, a streaming tile's 16 x 16 fragments), or
 * a missing or short workspace.
 */
bool feather_scaled_mm_splitk(const uint16_t* a, const uint8_t* b_prepacked, const float* scale,
                              const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale,
                              int has_bias, bool use_fp8_e5m2, bool a_bf16, bool output_bf16, int block_warps_m,
                              int block_warps_n, int unroll_k, int repeat_m, int repeat_n, bool prefetch,
                              int splits, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * feather_scaled_mm_splitk without a workspace argument and without any allocation: the partial sums and
 * arrival counters live in a static device array of the library (64 KiB of counters + 64 MiB of partials on
 * each GPU it runs on), so callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc) can still split K. The array is part of the library's
 * code object: loading the library onto a GPU reserves it there until the process ends, whether or not
 * this function is ever called. It calls no hipMalloc, hipFree or allocating library routine; its first
 * call on a device looks the array up (hipGetSymbolAddress) and enqueues a small kernel on `stream` that
 * zeroes the counters. Make that first call on a device outside graph capture: later calls under capture
 * record only the split launch, and each replay finds the counters zero, as every completed launch leaves
 * them. (A first call made under capture records the clearing kernel into the graph ahead of the launch,
 * and so does every captured call until one has run outside capture; it returns false if the runtime
 * refuses the symbol lookup during capture.)
 *
 * No counterpart in the reference. Same arguments, contract and results as feather_scaled_mm_splitk,
 * minus the workspace. Returns false (nothing enqueued) where that function would, and also when the
 * launch needs more than the static array holds, i.e. when feather_splitk_workspace_bytes(...) exceeds
 * FEATHER_NOALLOC_SCRATCH_BYTES. Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams or threads without ordering) race and must not be made.
 */
#define FEATHER_NOALLOC_SCRATCH_BYTES (65536 + 67108864) /* 64 KiB of counters + 64 MiB of partial sums */
bool feather_scaled_mm_splitk_noalloc(const uint16_t* a, const uint8_t* b_prepacked, const float* scale,
                                      const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K,
                                      int has_scale, int has_bias, bool use_fp8_e5m2, bool a_bf16, bool output_bf16,
                                      int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n,
                                      bool prefetch, int splits, hipStream_t stream);

/*
 * Workspace bytes feather_scaled_mm_splitk needs for this shape, tile and split count (host only, no GPU
 * call): 0 for splits = 1, -1 if they are outside its contract. Always under 2 GiB.
 */
int64_t feather_splitk_workspace_bytes(int64_t M, int64_t N, int64_t K, int block_warps_m, int block_warps_n,
                                       int unroll_k, int repeat_m, int repeat_n, bool prefetch, int splits);

/*
 * Process-wide choice of non-temporal weight loads, for the three scaled_mm entry points above; returns the
 * previous mode, the current one for mode = -1, or -1 (nothing changed) for any other value. Results do not
 * depend on it: it is a cache hint. A launch whose M fits one row of its tile (so that it reads every weight
 * byte once) then loads the weight non-temporally:
 *   0  never;
 *   1  always;
 *   2  (auto, the default) when the prepacked weight holds at least 48 MiB.
 * The hint pays when the weight streams from HBM on every launch (a model far larger than the GPU's 256 MB
 * MALL: 4-9% on weights of 59-235 MB) and costs when the caller's working set would stay in the MALL (up to
 * a third slower): mode 0 suits small models and one weight timed in a loop. The environment variable
 * FEATHER_OPS_WEIGHT_STREAMING (0, 1 or 2) sets the first value. No counterpart in the reference, whose
 * GPUs have no such cache.
 */
int feather_set_weight_streaming(int mode);

/*
 * out[i] = bf16 -> fp16 of in[i] with round-toward-zero (finite overflow saturates to +-65504, inf/NaN
 * pass through), n elements, enqueued on `stream`. Replaces the reference's Triton kernel behind
 * feather_ops/convert.py:24-34 (bf16_to_fp16), which has no C entry point of its own. in/out 16-byte
 * aligned, n < 2^30; returns false (nothing enqueued) otherwise.
 */
bool feather_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream);

/*
 * out[i] = bf16 -> fp16 of in[i] with round-to-nearest-even (overflow to +-inf, inf/NaN pass through), n
 * elements, enqueued on `stream`: the cast feather_ops/naive.py:21 applies to bf16 activations
 * (`a.to(torch.float16)`), and the conversion launch_scaled_mm applies when a_bf16 is true, bit for bit, so
 * launch_scaled_mm over the widened copy with a_bf16 = false returns what it returns over the original with
 * a_bf16 = true. No counterpart in the reference, whose kernel always widens in place; here the heuristic's
 * launches widen once up front for wide weights, where the fp16-activation kernel's speed repays the pass.
 * in/out 16-byte aligned, n < 2^30; returns false (nothing enqueued) otherwise.
 */
bool feather_widen_bf16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream);

/*
 * b_prepacked[k / 16][n][k % 16] = b[k][n] for a [K, N] row-major fp8 weight b (the GEMM's B = W^T),
 * with the K_pad - K rows past K (K_pad = ceil(K / 128) * 128) written as zeros: the layout
 * launch_scaled_mm reads, produced on the GPU and enqueued on `stream`. Restates the reference's Python
 * prepack_b_for_scaled_mm (feather_ops/scaled_mm.py:137-150), which has no C entry point of its own.
 * Requires K >= 1, N >= 8 and N % 8 == 0, b 8-byte and b_prepacked 16-byte aligned, K_pad * N < 2^31;
 * returns false (nothing enqueued) otherwise. b_prepacked holds K_pad / 16 * N * 16 bytes.
 */
bool feather_prepack_b(const uint8_t* b, uint8_t* b_prepacked, int64_t K, int64_t N, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FEATHER_OPS_H */
