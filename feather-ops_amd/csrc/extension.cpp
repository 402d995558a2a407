// The `feather_ops` torch library and the `feather_ops._C` Python module (reference: csrc/extension.cpp:1-23
// plus the op registration of csrc/hip_kernel.cu:716-846). Host code only: it validates the tensors,
// takes the current stream of a's device, and calls the C ABI of libfeather_ops_gfx950.so
// (include/feather_ops.h). Built against torch's stable ABI, like the reference.
#include <Python.h>

#include <torch/csrc/stable/accelerator.h>
#include <torch/csrc/stable/library.h>
#include <torch/csrc/stable/tensor.h>

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <optional>

#include "feather_ops.h"

namespace {

using torch::stable::Tensor;
using ST = torch::headeronly::ScalarType;

bool is_aligned(const void* p, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// What the C ABI needs of one validated scaled_mm call.
struct Operands {
    int64_t M, N, K;
    int scale_mode;  // 0: none, 1: per tensor, 2: per output column
    bool e5m2, a_bf16, out_bf16;
    int32_t device_index;
};

// Preconditions and messages of feather_ops::scaled_mm, following csrc/hip_kernel.cu:729-801; N is relaxed
// from a multiple of 16 to a multiple of 8 (16-byte output rows stay aligned, partial 16-column tiles are
// masked), and scale may also hold one value per output column (the per-channel scale of
// feather_ops/naive.py:29-33).
Operands check_operands(const Tensor& a, const Tensor& b_prepacked, const std::optional<Tensor>& scale,
                        const std::optional<Tensor>& bias, const Tensor& c, const int64_t block_warps_m,
                        const int64_t block_warps_n) {
    STD_TORCH_CHECK(a.is_cuda(), "a must be a CUDA tensor");
    STD_TORCH_CHECK(b_prepacked.is_cuda(), "b_prepacked must be a CUDA tensor");
    STD_TORCH_CHECK(c.is_cuda(), "c must be a CUDA tensor");
    const auto device_index = a.get_device_index();
    STD_TORCH_CHECK(b_prepacked.get_device_index() == device_index, "b_prepacked must be on the same device as a");
    STD_TORCH_CHECK(c.get_device_index() == device_index, "c must be on the same device as a");

    const auto a_type = a.scalar_type();
    STD_TORCH_CHECK(a_type == ST::Half || a_type == ST::BFloat16, "a must be float16 or bfloat16");
    STD_TORCH_CHECK(c.scalar_type() == ST::Half || c.scalar_type() == ST::BFloat16, "c must be float16 or bfloat16");
    const auto b_type = b_prepacked.scalar_type();
    STD_TORCH_CHECK(b_type == ST::Float8_e4m3fn || b_type == ST::Float8_e5m2,
                    "b_prepacked must be float8_e4m3fn or float8_e5m2");

    STD_TORCH_CHECK(a.dim() == 2, "a must be 2D");
    STD_TORCH_CHECK(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)");
    STD_TORCH_CHECK(c.dim() == 2, "c must be 2D");

    const int64_t M = a.size(0);
    const int64_t K = a.size(1);
    const int64_t N = b_prepacked.size(1);
    STD_TORCH_CHECK(K % 16 == 0, "K must be divisible by 16");
    STD_TORCH_CHECK(K >= 16, "K must be at least 16");
    STD_TORCH_CHECK(N % 8 == 0, "N must be divisible by 8");
    STD_TORCH_CHECK(b_prepacked.size(0) >= K / 16, "b_prepacked.shape[0] must be at least K/16 (", K / 16, ")");
    STD_TORCH_CHECK(b_prepacked.size(0) % 8 == 0, "b_prepacked.shape[0] must be a multiple of 8 (K padded to 128)");
    STD_TORCH_CHECK(b_prepacked.size(2) == 16, "b_prepacked.shape[2] must be 16");
    STD_TORCH_CHECK(c.size(0) == M, "c.shape[0] must equal M");
    STD_TORCH_CHECK(c.size(1) == N, "c.shape[1] must equal N");

    STD_TORCH_CHECK(a.stride(0) == K, "a.stride(0) must equal K (", K, ")");
    STD_TORCH_CHECK(a.stride(1) == 1, "a.stride(1) must be 1");
    STD_TORCH_CHECK(b_prepacked.stride(0) == N * 16, "b_prepacked.stride(0) must equal N*16 (", N * 16, ")");
    STD_TORCH_CHECK(b_prepacked.stride(1) == 16, "b_prepacked.stride(1) must be 16");
    STD_TORCH_CHECK(b_prepacked.stride(2) == 1, "b_prepacked.stride(2) must be 1");
    STD_TORCH_CHECK(c.stride(0) == N, "c.stride(0) must equal N (", N, ")");
    STD_TORCH_CHECK(c.stride(1) == 1, "c.stride(1) must be 1");

    if (scale.has_value()) {
        const Tensor& s = *scale;
        STD_TORCH_CHECK(s.is_cuda(), "scale must be a CUDA tensor");
        STD_TORCH_CHECK(s.get_device_index() == device_index, "scale must be on the same device as a");
        STD_TORCH_CHECK(s.scalar_type() == ST::Float, "scale must be float32");
        STD_TORCH_CHECK(s.numel() == 1 || s.numel() == N,
                        "scale must have one element (per tensor) or N elements (per output column)");
        if (s.numel() == N) {
            STD_TORCH_CHECK(s.dim() == 1, "a per-column scale must be 1D");
            STD_TORCH_CHECK(s.stride(0) == 1, "a per-column scale must be contiguous");
            STD_TORCH_CHECK(is_aligned(s.const_data_ptr(), 16), "a per-column scale must be 16-byte aligned");
        }
    }
    // 1: one per-tensor value; 2: one value per output column (N >= 8, so the two never coincide).
    const int scale_mode = !scale.has_value() ? 0 : scale->numel() == 1 ? 1 : 2;
    if (bias.has_value()) {
        const Tensor& b = *bias;
        STD_TORCH_CHECK(b.is_cuda(), "bias must be a CUDA tensor");
        STD_TORCH_CHECK(b.get_device_index() == device_index, "bias must be on the same device as a");
        STD_TORCH_CHECK(b.scalar_type() == c.scalar_type(), "bias must have the same dtype as c");
        STD_TORCH_CHECK(b.numel() == N, "bias must have N elements");
        STD_TORCH_CHECK(b.numel() == 0 || b.stride(b.dim() - 1) == 1, "bias must be contiguous");
        STD_TORCH_CHECK(is_aligned(b.const_data_ptr(), 8), "bias data pointer must be 8-byte aligned");
    }

    const int64_t threads = 64 * block_warps_m * block_warps_n;
    STD_TORCH_CHECK(threads <= 1024, "Block size exceeds HIP thread-per-block limit");
    STD_TORCH_CHECK(M * K * 2 < (int64_t{1} << 31) && M * N * 2 < (int64_t{1} << 31) &&
                        b_prepacked.size(0) * N * 16 < (int64_t{1} << 31),
                    "a, b_prepacked and c must each be smaller than 2 GiB");
    if (M > 0) {
        STD_TORCH_CHECK(is_aligned(a.const_data_ptr(), 16), "a data pointer must be 16-byte aligned");
        STD_TORCH_CHECK(is_aligned(b_prepacked.const_data_ptr(), 16),
                        "b_prepacked data pointer must be 16-byte aligned");
        STD_TORCH_CHECK(is_aligned(c.const_data_ptr(), 16), "c data pointer must be 16-byte aligned");
    }
    return Operands{M, N, K, scale_mode, b_type == ST::Float8_e5m2, a_type == ST::BFloat16,
                    c.scalar_type() == ST::BFloat16, device_index};
}

hipStream_t current_stream(int32_t device_index) {
    void* raw_stream = nullptr;
    TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device_index, &raw_stream));
    return static_cast<hipStream_t>(raw_stream);
}

void check_launch(bool launched, const char* what) {
    STD_TORCH_CHECK(launched, "Unsupported config");
    const hipError_t err = hipGetLastError();
    STD_TORCH_CHECK(err == hipSuccess, what, " kernel launch failed: ", hipGetErrorString(err));
}

// feather_ops::scaled_mm (csrc/hip_kernel.cu:716-823 of the reference).
void scaled_mm(const Tensor& a, const Tensor& b_prepacked, const std::optional<Tensor>& scale,
               const std::optional<Tensor>& bias, Tensor& c, const int64_t block_warps_m, const int64_t block_warps_n,
               const int64_t unroll_k, const int64_t repeat_m, const int64_t repeat_n, const bool prefetch) {
    const Operands o = check_operands(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n);
    if (o.M == 0) return;
    torch::stable::accelerator::DeviceGuard guard(o.device_index);
    const bool launched = launch_scaled_mm(
        static_cast<const uint16_t*>(a.const_data_ptr()), static_cast<const uint8_t*>(b_prepacked.const_data_ptr()),
        scale.has_value() ? static_cast<const float*>(scale->const_data_ptr()) : nullptr,
        bias.has_value() ? static_cast<const uint16_t*>(bias->const_data_ptr()) : nullptr,
        static_cast<uint16_t*>(c.mutable_data_ptr()), o.M, o.N, o.K, o.scale_mode, bias.has_value() ? 1 : 0, o.e5m2,
        o.a_bf16, o.out_bf16, static_cast<int>(block_warps_m), static_cast<int>(block_warps_n),
        static_cast<int>(unroll_k), static_cast<int>(repeat_m), static_cast<int>(repeat_n), prefetch,
        current_stream(o.device_index));
    check_launch(launched, "scaled_mm");
}

// feather_ops::scaled_mm_splitk: scaled_mm with each tile's K range split over
// `splits` workgroups that meet in `workspace` (uint8, the caller's; all zero before its first use, and
// every completed call leaves it reusable; see feather_scaled_mm_splitk). No counterpart in the reference.
void scaled_mm_splitk(const Tensor& a, const Tensor& b_prepacked, const std::optional<Tensor>& scale,
                      const std::optional<Tensor>& bias, Tensor& c, Tensor& workspace, const int64_t splits,
                      const int64_t block_warps_m, const int64_t block_warps_n, const int64_t unroll_k,
                      const int64_t repeat_m, const int64_t repeat_n, const bool prefetch) {
    const Operands o = check_operands(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n);
    STD_TORCH_CHECK(workspace.is_cuda() && workspace.get_device_index() == o.device_index,
                    "workspace must be on the same device as a");
    STD_TORCH_CHECK(workspace.scalar_type() == ST::Byte && workspace.dim() == 1 && workspace.stride(0) == 1,
                    "workspace must be a contiguous 1-D uint8 tensor");
    STD_TORCH_CHECK(splits >= 1 && splits <= 32, "splits must be in 1 .. 32");
    if (o.M == 0) return;
    const int64_t need = feather_splitk_workspace_bytes(o.M, o.N, o.K, static_cast<int>(block_warps_m),
                                                        static_cast<int>(block_warps_n), static_cast<int>(unroll_k),
                                                        static_cast<int>(repeat_m), static_cast<int>(repeat_n),
                                                        prefetch, static_cast<int>(splits));
    STD_TORCH_CHECK(need >= 0, "Unsupported config");
    STD_TORCH_CHECK(splits == 1 || workspace.numel() >= need, "workspace must hold at least ", need, " bytes");
    STD_TORCH_CHECK(splits == 1 || is_aligned(workspace.const_data_ptr(), 256),
                    "workspace data pointer must be 256-byte aligned");
    torch::stable::accelerator::DeviceGuard guard(o.device_index);
    const bool launched = feather_scaled_mm_splitk(
        static_cast<const uint16_t*>(a.const_data_ptr()), static_cast<const uint8_t*>(b_prepacked.const_data_ptr()),
        scale.has_value() ? static_cast<const float*>(scale->const_data_ptr()) : nullptr,
        bias.has_value() ? static_cast<const uint16_t*>(bias->const_data_ptr()) : nullptr,
        static_cast<uint16_t*>(c.mutable_data_ptr()), o.M, o.N, o.K, o.scale_mode, bias.has_value() ? 1 : 0, o.e5m2,
        o.a_bf16, o.out_bf16, static_cast<int>(block_warps_m), static_cast<int>(block_warps_n),
        static_cast<int>(unroll_k), static_cast<int>(repeat_m), static_cast<int>(repeat_n), prefetch,
        static_cast<int>(splits), workspace.mutable_data_ptr(), workspace.numel(), current_stream(o.device_index));
    check_launch(launched, "scaled_mm_splitk");
}

// bf16 -> fp16 of x into out, both contiguous on one device: round toward zero (feather_ops::bf16_to_fp16,
// the reference's bf16_to_fp16) or round to nearest even (feather_ops::widen_bf16, the activations' cast).
void convert_bf16(const Tensor& x, Tensor& out, bool nearest, const char* name) {
    STD_TORCH_CHECK(x.is_cuda() && out.is_cuda(), "x and out must be CUDA tensors");
    STD_TORCH_CHECK(x.get_device_index() == out.get_device_index(), "x and out must be on one device");
    STD_TORCH_CHECK(x.scalar_type() == ST::BFloat16, "x must be bfloat16");
    STD_TORCH_CHECK(out.scalar_type() == ST::Half, "out must be float16");
    STD_TORCH_CHECK(x.is_contiguous() && out.is_contiguous(), "x and out must be contiguous");
    STD_TORCH_CHECK(x.numel() == out.numel(), "x and out must have the same number of elements");
    STD_TORCH_CHECK(x.numel() < (int64_t{1} << 30), "x must have fewer than 2^30 elements");
    if (x.numel() == 0) return;
    STD_TORCH_CHECK(is_aligned(x.const_data_ptr(), 16) && is_aligned(out.mutable_data_ptr(), 16),
                    "x and out data pointers must be 16-byte aligned");
    const auto device_index = x.get_device_index();
    torch::stable::accelerator::DeviceGuard guard(device_index);
    void* raw_stream = nullptr;
    TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device_index, &raw_stream));
    const auto* in_bits = static_cast<const uint16_t*>(x.const_data_ptr());
    auto* out_bits = static_cast<uint16_t*>(out.mutable_data_ptr());
    const auto stream = static_cast<hipStream_t>(raw_stream);
    const bool launched = nearest ? feather_widen_bf16(in_bits, out_bits, x.numel(), stream)
                                  : feather_bf16_to_fp16(in_bits, out_bits, x.numel(), stream);
    STD_TORCH_CHECK(launched, name, ": unsupported arguments");
    const hipError_t err = hipGetLastError();
    STD_TORCH_CHECK(err == hipSuccess, name, " kernel launch failed: ", hipGetErrorString(err));
}

void bf16_to_fp16(const Tensor& x, Tensor& out) { convert_bf16(x, out, false, "bf16_to_fp16"); }

void widen_bf16(const Tensor& x, Tensor& out) { convert_bf16(x, out, true, "widen_bf16"); }

// feather_ops::prepack_b: out[k // 16, n, k % 16] = b[k, n] for a [K, N] fp8 weight, K zero-padded to a
// multiple of 128 (the reference's prepack_b_for_scaled_mm layout, feather_ops/scaled_mm.py:137-150).
void prepack_b(const Tensor& b, Tensor& out) {
    STD_TORCH_CHECK(b.is_cuda() && out.is_cuda(), "b and out must be CUDA tensors");
    STD_TORCH_CHECK(b.get_device_index() == out.get_device_index(), "b and out must be on one device");
    STD_TORCH_CHECK(b.scalar_type() == ST::Float8_e5m2 || b.scalar_type() == ST::Float8_e4m3fn,
                    "b must be float8_e5m2 or float8_e4m3fn");
    STD_TORCH_CHECK(out.scalar_type() == b.scalar_type(), "out must have b's dtype");
    STD_TORCH_CHECK(b.dim() == 2 && out.dim() == 3, "b must be 2-D [K, N] and out 3-D [K_pad/16, N, 16]");
    STD_TORCH_CHECK(b.is_contiguous() && out.is_contiguous(), "b and out must be contiguous");
    const int64_t K = b.size(0);
    const int64_t N = b.size(1);
    const int64_t k_pad = (K + 127) / 128 * 128;
    STD_TORCH_CHECK(K >= 1 && N % 8 == 0 && N >= 8, "prepack_b needs K >= 1 and N a positive multiple of 8");
    STD_TORCH_CHECK(out.size(0) == k_pad / 16 && out.size(1) == N && out.size(2) == 16,
                    "out must be [ceil(K/128)*8, N, 16]");
    STD_TORCH_CHECK(k_pad * N < (int64_t{1} << 31), "the prepacked weight must be smaller than 2 GiB");
    STD_TORCH_CHECK(is_aligned(b.const_data_ptr(), 8) && is_aligned(out.mutable_data_ptr(), 16),
                    "b must be 8-byte and out 16-byte aligned");
    const auto device_index = b.get_device_index();
    torch::stable::accelerator::DeviceGuard guard(device_index);
    void* raw_stream = nullptr;
    TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device_index, &raw_stream));
    const bool launched = feather_prepack_b(static_cast<const uint8_t*>(b.const_data_ptr()),
                                            static_cast<uint8_t*>(out.mutable_data_ptr()), K, N,
                                            static_cast<hipStream_t>(raw_stream));
    STD_TORCH_CHECK(launched, "prepack_b: unsupported arguments");
    const hipError_t err = hipGetLastError();
    STD_TORCH_CHECK(err == hipSuccess, "prepack_b kernel launch failed: ", hipGetErrorString(err));
}

}  // namespace

STABLE_TORCH_LIBRARY(feather_ops, m) {
    m.def(
        "scaled_mm(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, Tensor(a!) c, int block_warps_m, "
        "int block_warps_n, int unroll_k, int repeat_m, int repeat_n, bool prefetch) -> ()");
    m.def(
        "scaled_mm_splitk(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, Tensor(a!) c, "
        "Tensor(b!) workspace, int splits, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, "
        "int repeat_n, bool prefetch=True) -> ()");
    m.def("bf16_to_fp16(Tensor x, Tensor(a!) out) -> ()");
    m.def("widen_bf16(Tensor x, Tensor(a!) out) -> ()");
    m.def("prepack_b(Tensor b, Tensor(a!) out) -> ()");
}

STABLE_TORCH_LIBRARY_IMPL(feather_ops, CUDA, m) {
    m.impl("scaled_mm", TORCH_BOX(&scaled_mm));
    m.impl("scaled_mm_splitk", TORCH_BOX(&scaled_mm_splitk));
    m.impl("bf16_to_fp16", TORCH_BOX(&bf16_to_fp16));
    m.impl("widen_bf16", TORCH_BOX(&widen_bf16));
    m.impl("prepack_b", TORCH_BOX(&prepack_b));
}

extern "C" PyObject* PyInit__C(void) {
    static PyModuleDef module = {PyModuleDef_HEAD_INIT, "_C", nullptr, -1, nullptr, nullptr, nullptr, nullptr, nullptr};
    return PyModule_Create(&module);
}
