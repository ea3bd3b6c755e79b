// torch.library custom ops over libpaia_gemv.so: the thin PyTorch-ROCm layer of the paia_gemv package.
//
// Namespace torch.ops.paia_gemv. Each op validates its tensors, resolves the variant (-1 = the library's per-shape
// pick), and calls the C ABI on torch's current HIP stream of the operand's device, so the ops compose with torch
// streams and HIP graph capture. Functional ops allocate their output; the *_out ops write a caller-given output and
// allocate nothing. Meta kernels give shapes for tracing.
//
// The reference reaches its kernels through ctypes only (src/paia_gemv/loader.py:28-99); these ops are the additional
// Tensor-level surface (same semantics, same return-code errors surfaced as RuntimeError).
//
// x is [K], [1, K] or [M, K] with M <= 16 (y is [N], [1, N] or [M, N]). One activation row runs the M = 1 GEMV
// kernels and `variant` indexes their table; M > 1 runs the small-batch kernels (paia_gemv_batch_*: row-streaming or
// matrix-core) and `variant` indexes the batch table of that format. -1 is the library's choice in both cases.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cstdint>
#include <optional>

#include "paia_gemv.h"

namespace {

enum Kind { kBF16 = 0, kFP8 = 1, kINT4 = 2, kINT4ZP = 3 };

void check_rc(int rc, const char* what)
{
    TORCH_CHECK(rc == 0, what, " failed with code ", rc,
                " (-1 bad variant, -2 bad shape/alignment, >0 hipError_t)");
}

void* stream_of(const at::Tensor& t)
{
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

constexpr int64_t kMaxRows = 16;   // activation rows the small-batch kernels take

// Every operand must live on the GPU the kernel runs on: the kernels dereference the raw pointers, so a host tensor
// (the dispatcher picks the GPU kernel when any argument is on the GPU) or another GPU's tensor must be refused here.
void on_device_of(const at::Tensor& W, const at::Tensor& t, const char* name)
{
    TORCH_CHECK(t.device() == W.device(), name, " must be on the device of the weights (", W.device(), "), found ",
                t.device());
}
void on_device_of(const at::Tensor& W, const std::optional<at::Tensor>& t, const char* name)
{
    if (t.has_value()) on_device_of(W, *t, name);
}
void check_weights(const at::Tensor& W, int64_t N, int64_t K)
{
    TORCH_CHECK(W.is_cuda(), "the weights must be on a GPU, found ", W.device());
    TORCH_CHECK(N <= INT32_MAX && K <= INT32_MAX, "N and K must fit in 32 bits (the C ABI takes int)");
}

int64_t x_len(const at::Tensor& x)
{
    TORCH_CHECK(x.dim() == 1 || (x.dim() == 2 && x.size(0) >= 1 && x.size(0) <= kMaxRows),
                "x must be [K] or [M, K] with 1 <= M <= 16");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    return x.size(-1);
}

int64_t x_rows(const at::Tensor& x) { return x.dim() == 2 ? x.size(0) : 1; }

std::vector<int64_t> y_shape(const at::Tensor& x, int64_t N)
{
    if (x.dim() == 2) return {x.size(0), N};
    return {N};
}

void check_out(const at::Tensor& out, const at::Tensor& x, int64_t N)
{
    TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.is_contiguous() && out.numel() == x_rows(x) * N,
                "out must be a contiguous bfloat16 tensor with M*N elements");
}

const void* opt_ptr(const std::optional<at::Tensor>& t, int64_t N)
{
    if (!t.has_value()) return nullptr;
    TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->is_contiguous() && t->numel() == N,
                "bias must be a contiguous bfloat16 tensor with N elements");
    return t->data_ptr();
}

int pick(int64_t variant, int kind, int64_t N, int64_t K)
{
    return variant >= 0 ? (int)variant : paia_gemv_pick_variant(kind, (int)N, (int)K);
}

// -------------------------------------------------------------------------------------------------------------
void gemv_bf16_out(const at::Tensor& W, const at::Tensor& x, const std::optional<at::Tensor>& bias, int64_t variant,
                   at::Tensor& out)
{
    TORCH_CHECK(W.dim() == 2 && W.scalar_type() == at::kBFloat16 && W.is_contiguous(), "W must be bf16 [N, K]");
    const int64_t N = W.size(0), K = W.size(1);
    check_weights(W, N, K);
    TORCH_CHECK(x_len(x) == K, "x length must equal K");
    check_out(out, x, N);
    on_device_of(W, x, "x");
    on_device_of(W, bias, "bias");
    on_device_of(W, out, "out");
    c10::DeviceGuard g(W.device());
    const int64_t M = x_rows(x);
    if (M > 1) {
        check_rc(paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr(), opt_ptr(bias, N), out.data_ptr(), (int)M, (int)N,
                                      (int)K, (int)variant, stream_of(W)),
                 "paia_gemv_batch_bf16");
        return;
    }
    check_rc(paia_gemv_bf16_bias(W.data_ptr(), x.data_ptr(), opt_ptr(bias, N), out.data_ptr(), (int)N, (int)K,
                                 pick(variant, kBF16, N, K), stream_of(W)),
             "paia_gemv_bf16");
}
at::Tensor gemv_bf16(const at::Tensor& W, const at::Tensor& x, const std::optional<at::Tensor>& bias, int64_t variant)
{
    at::Tensor out = at::empty(y_shape(x, W.size(0)), x.options());
    gemv_bf16_out(W, x, bias, variant, out);
    return out;
}

void gemv_fp8_out(const at::Tensor& Wq, const at::Tensor& scale, const at::Tensor& x,
                  const std::optional<at::Tensor>& bias, int64_t variant, at::Tensor& out)
{
    TORCH_CHECK(Wq.dim() == 2 && Wq.element_size() == 1 && Wq.is_contiguous(), "Wq must be 1-byte e4m3 [N, K]");
    const int64_t N = Wq.size(0), K = Wq.size(1);
    check_weights(Wq, N, K);
    TORCH_CHECK(scale.scalar_type() == at::kFloat && scale.numel() == N && scale.is_contiguous(), "scale: fp32 [N]");
    TORCH_CHECK(x_len(x) == K, "x length must equal K");
    check_out(out, x, N);
    on_device_of(Wq, scale, "scale");
    on_device_of(Wq, x, "x");
    on_device_of(Wq, bias, "bias");
    on_device_of(Wq, out, "out");
    c10::DeviceGuard g(Wq.device());
    const int64_t M = x_rows(x);
    if (M > 1) {
        check_rc(paia_gemv_batch_fp8(Wq.data_ptr(), scale.data_ptr(), x.data_ptr(), opt_ptr(bias, N), out.data_ptr(),
                                     (int)M, (int)N, (int)K, (int)variant, stream_of(Wq)),
                 "paia_gemv_batch_fp8");
        return;
    }
    check_rc(paia_gemv_fp8_bias(Wq.data_ptr(), scale.data_ptr(), x.data_ptr(), opt_ptr(bias, N), out.data_ptr(),
                                (int)N, (int)K, pick(variant, kFP8, N, K), stream_of(Wq)),
             "paia_gemv_fp8");
}
at::Tensor gemv_fp8(const at::Tensor& Wq, const at::Tensor& scale, const at::Tensor& x,
                    const std::optional<at::Tensor>& bias, int64_t variant)
{
    at::Tensor out = at::empty(y_shape(x, Wq.size(0)), x.options());
    gemv_fp8_out(Wq, scale, x, bias, variant, out);
    return out;
}

// Packed INT4 weights: uint8 [N, K/2] or int32 [N, K/8] (the same bytes on a little-endian machine).
int64_t int4_K(const at::Tensor& Wq)
{
    TORCH_CHECK(Wq.dim() == 2 && Wq.is_contiguous(), "Wq must be a contiguous 2-D tensor");
    if (Wq.scalar_type() == at::kByte) return Wq.size(1) * 2;
    TORCH_CHECK(Wq.scalar_type() == at::kInt, "Wq must be uint8 [N, K/2] or int32 [N, K/8]");
    return Wq.size(1) * 8;
}

void gemv_int4_out(const at::Tensor& Wq, const at::Tensor& scales, const at::Tensor& x, int64_t variant,
                   at::Tensor& out)
{
    const int64_t N = Wq.size(0), K = int4_K(Wq);
    check_weights(Wq, N, K);
    TORCH_CHECK(scales.scalar_type() == at::kHalf && scales.is_contiguous() && scales.numel() == N * (K / 128),
                "scales: fp16 [N, K/128]");
    TORCH_CHECK(x_len(x) == K, "x length must equal K");
    check_out(out, x, N);
    on_device_of(Wq, scales, "scales");
    on_device_of(Wq, x, "x");
    on_device_of(Wq, out, "out");
    c10::DeviceGuard g(Wq.device());
    const int64_t M = x_rows(x);
    if (M > 1) {
        check_rc(paia_gemv_batch_int4(Wq.data_ptr(), scales.data_ptr(), x.data_ptr(), out.data_ptr(), (int)M, (int)N,
                                      (int)K, (int)variant, stream_of(Wq)),
                 "paia_gemv_batch_int4");
        return;
    }
    check_rc(paia_gemv_int4(Wq.data_ptr(), scales.data_ptr(), x.data_ptr(), out.data_ptr(), (int)N, (int)K,
                            pick(variant, kINT4, N, K), stream_of(Wq)),
             "paia_gemv_int4");
}
at::Tensor gemv_int4(const at::Tensor& Wq, const at::Tensor& scales, const at::Tensor& x, int64_t variant)
{
    at::Tensor out = at::empty(y_shape(x, Wq.size(0)), x.options());
    gemv_int4_out(Wq, scales, x, variant, out);
    return out;
}

void gemv_int4_zp_out(const at::Tensor& Wq, const at::Tensor& scales, const at::Tensor& zeros, const at::Tensor& x,
                      const std::optional<at::Tensor>& bias, int64_t variant, at::Tensor& out)
{
    const int64_t N = Wq.size(0), K = int4_K(Wq), G = K / 128;
    check_weights(Wq, N, K);
    TORCH_CHECK(scales.scalar_type() == at::kBFloat16 && scales.is_contiguous() && scales.numel() == N * G,
                "scales: bf16 [N, K/128]");
    TORCH_CHECK(zeros.scalar_type() == at::kByte && zeros.is_contiguous() && zeros.numel() == N * ((G + 1) / 2),
                "zeros: uint8 [N, ceil(K/256)] (two 4-bit zero points per byte along the groups)");
    TORCH_CHECK(x_len(x) == K, "x length must equal K");
    check_out(out, x, N);
    on_device_of(Wq, scales, "scales");
    on_device_of(Wq, zeros, "zeros");
    on_device_of(Wq, x, "x");
    on_device_of(Wq, bias, "bias");
    on_device_of(Wq, out, "out");
    c10::DeviceGuard g(Wq.device());
    const int64_t M = x_rows(x);
    if (M > 1) {
        check_rc(paia_gemv_batch_int4_zp(Wq.data_ptr(), scales.data_ptr(), zeros.data_ptr(), x.data_ptr(),
                                         opt_ptr(bias, N), out.data_ptr(), (int)M, (int)N, (int)K, (int)variant,
                                         stream_of(Wq)),
                 "paia_gemv_batch_int4_zp");
        return;
    }
    check_rc(paia_gemv_int4_zp(Wq.data_ptr(), scales.data_ptr(), zeros.data_ptr(), x.data_ptr(), opt_ptr(bias, N),
                               out.data_ptr(), (int)N, (int)K, pick(variant, kINT4ZP, N, K), stream_of(Wq)),
             "paia_gemv_int4_zp");
}
at::Tensor gemv_int4_zp(const at::Tensor& Wq, const at::Tensor& scales, const at::Tensor& zeros, const at::Tensor& x,
                        const std::optional<at::Tensor>& bias, int64_t variant)
{
    at::Tensor out = at::empty(y_shape(x, Wq.size(0)), x.options());
    gemv_int4_zp_out(Wq, scales, zeros, x, bias, variant, out);
    return out;
}

at::Tensor dequant_fp8(const at::Tensor& Wq, const at::Tensor& scale)
{
    TORCH_CHECK(Wq.dim() == 2 && Wq.element_size() == 1 && Wq.is_contiguous(), "Wq must be 1-byte e4m3 [N, K]");
    const int64_t N = Wq.size(0), K = Wq.size(1);
    check_weights(Wq, N, K);
    TORCH_CHECK(scale.scalar_type() == at::kFloat && scale.numel() == N && scale.is_contiguous(), "scale: fp32 [N]");
    on_device_of(Wq, scale, "scale");
    at::Tensor out = at::empty({N, K}, Wq.options().dtype(at::kFloat));
    c10::DeviceGuard g(Wq.device());
    check_rc(paia_dequant_fp8(Wq.data_ptr(), scale.data_ptr(), out.data_ptr(), (int)N, (int)K, stream_of(Wq)),
             "paia_dequant_fp8");
    return out;
}

at::Tensor dequant_int4(const at::Tensor& Wq, const at::Tensor& scales)
{
    const int64_t N = Wq.size(0), K = int4_K(Wq);
    TORCH_CHECK(scales.scalar_type() == at::kHalf && scales.is_contiguous() && scales.numel() == N * (K / 128),
                "scales: fp16 [N, K/128]");
    check_weights(Wq, N, K);
    on_device_of(Wq, scales, "scales");
    at::Tensor out = at::empty({N, K}, Wq.options().dtype(at::kFloat));
    c10::DeviceGuard g(Wq.device());
    check_rc(paia_dequant_int4(Wq.data_ptr(), scales.data_ptr(), out.data_ptr(), (int)N, (int)K, stream_of(Wq)),
             "paia_dequant_int4");
    return out;
}

at::Tensor dequant_int4_zp(const at::Tensor& Wq, const at::Tensor& scales, const at::Tensor& zeros)
{
    const int64_t N = Wq.size(0), K = int4_K(Wq), G = K / 128;
    TORCH_CHECK(scales.scalar_type() == at::kBFloat16 && scales.is_contiguous() && scales.numel() == N * G,
                "scales: bf16 [N, K/128]");
    TORCH_CHECK(zeros.scalar_type() == at::kByte && zeros.is_contiguous() && zeros.numel() == N * ((G + 1) / 2),
                "zeros: uint8 [N, ceil(K/256)]");
    check_weights(Wq, N, K);
    on_device_of(Wq, scales, "scales");
    on_device_of(Wq, zeros, "zeros");
    at::Tensor out = at::empty({N, K}, Wq.options().dtype(at::kFloat));
    c10::DeviceGuard g(Wq.device());
    check_rc(paia_dequant_int4_zp(Wq.data_ptr(), scales.data_ptr(), zeros.data_ptr(), out.data_ptr(), (int)N, (int)K,
                                  stream_of(Wq)),
             "paia_dequant_int4_zp");
    return out;
}

// ---- quantizers (fp32 W [N, K] on the device) ----------------------------------------------------------------
void check_w32(const at::Tensor& W, int64_t kmult)
{
    TORCH_CHECK(W.dim() == 2 && W.scalar_type() == at::kFloat && W.is_contiguous(), "W must be contiguous fp32 [N, K]");
    TORCH_CHECK(W.size(1) % kmult == 0, "K must be a multiple of ", kmult);
    check_weights(W, W.size(0), W.size(1));
}

std::tuple<at::Tensor, at::Tensor> quantize_fp8_rowwise(const at::Tensor& W)
{
    check_w32(W, 16);
    const int64_t N = W.size(0), K = W.size(1);
    at::Tensor q = at::empty({N, K}, W.options().dtype(at::kByte));
    at::Tensor scale = at::empty({N}, W.options());
    c10::DeviceGuard g(W.device());
    check_rc(paia_quantize_fp8_rowwise(W.data_ptr(), q.data_ptr(), scale.data_ptr(), (int)N, (int)K, stream_of(W)),
             "paia_quantize_fp8_rowwise");
    return {q, scale};
}

std::tuple<at::Tensor, at::Tensor> quantize_int4_g128(const at::Tensor& W)
{
    check_w32(W, 128);
    const int64_t N = W.size(0), K = W.size(1);
    at::Tensor packed = at::empty({N, K / 2}, W.options().dtype(at::kByte));
    at::Tensor scales = at::empty({N, K / 128}, W.options().dtype(at::kHalf));
    c10::DeviceGuard g(W.device());
    check_rc(paia_quantize_int4_g128(W.data_ptr(), packed.data_ptr(), scales.data_ptr(), (int)N, (int)K, stream_of(W)),
             "paia_quantize_int4_g128");
    return {packed, scales};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> quantize_int4_zp_g128(const at::Tensor& W)
{
    check_w32(W, 128);
    const int64_t N = W.size(0), K = W.size(1), G = K / 128;
    at::Tensor packed = at::empty({N, K / 2}, W.options().dtype(at::kByte));
    at::Tensor scales = at::empty({N, G}, W.options().dtype(at::kBFloat16));
    at::Tensor zeros = at::empty({N, (G + 1) / 2}, W.options().dtype(at::kByte));
    c10::DeviceGuard g(W.device());
    check_rc(paia_quantize_int4_zp_g128(W.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), (int)N,
                                        (int)K, stream_of(W)),
             "paia_quantize_int4_zp_g128");
    return {packed, scales, zeros};
}

std::tuple<at::Tensor, at::Tensor> quantize_fp8_rowwise_meta(const at::Tensor& W)
{
    return {at::empty({W.size(0), W.size(1)}, W.options().dtype(at::kByte)), at::empty({W.size(0)}, W.options())};
}
std::tuple<at::Tensor, at::Tensor> quantize_int4_g128_meta(const at::Tensor& W)
{
    return {at::empty({W.size(0), W.size(1) / 2}, W.options().dtype(at::kByte)),
            at::empty({W.size(0), W.size(1) / 128}, W.options().dtype(at::kHalf))};
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> quantize_int4_zp_g128_meta(const at::Tensor& W)
{
    const int64_t G = W.size(1) / 128;
    return {at::empty({W.size(0), W.size(1) / 2}, W.options().dtype(at::kByte)),
            at::empty({W.size(0), G}, W.options().dtype(at::kBFloat16)),
            at::empty({W.size(0), (G + 1) / 2}, W.options().dtype(at::kByte))};
}

// ---- Meta (shape-only) kernels ------------------------------------------------------------------------------
at::Tensor gemv_bf16_meta(const at::Tensor& W, const at::Tensor& x, const std::optional<at::Tensor>&, int64_t)
{
    return at::empty(y_shape(x, W.size(0)), x.options());
}
at::Tensor gemv_fp8_meta(const at::Tensor& Wq, const at::Tensor&, const at::Tensor& x, const std::optional<at::Tensor>&,
                         int64_t)
{
    return at::empty(y_shape(x, Wq.size(0)), x.options());
}
at::Tensor gemv_int4_meta(const at::Tensor& Wq, const at::Tensor&, const at::Tensor& x, int64_t)
{
    return at::empty(y_shape(x, Wq.size(0)), x.options());
}
at::Tensor gemv_int4_zp_meta(const at::Tensor& Wq, const at::Tensor&, const at::Tensor&, const at::Tensor& x,
                             const std::optional<at::Tensor>&, int64_t)
{
    return at::empty(y_shape(x, Wq.size(0)), x.options());
}
at::Tensor dequant_fp8_meta(const at::Tensor& Wq, const at::Tensor&)
{
    return at::empty({Wq.size(0), Wq.size(1)}, Wq.options().dtype(at::kFloat));
}
at::Tensor dequant_int4_meta(const at::Tensor& Wq, const at::Tensor&)
{
    return at::empty({Wq.size(0), int4_K(Wq)}, Wq.options().dtype(at::kFloat));
}
at::Tensor dequant_int4_zp_meta(const at::Tensor& Wq, const at::Tensor&, const at::Tensor&)
{
    return at::empty({Wq.size(0), int4_K(Wq)}, Wq.options().dtype(at::kFloat));
}
void out_meta_bf16(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t, at::Tensor&) {}
void out_meta_fp8(const at::Tensor&, const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t,
                  at::Tensor&) {}
void out_meta_int4(const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t, at::Tensor&) {}
void out_meta_int4_zp(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                      const std::optional<at::Tensor>&, int64_t, at::Tensor&) {}

}  // namespace

TORCH_LIBRARY(paia_gemv, m)
{
    m.def("gemv_bf16(Tensor W, Tensor x, Tensor? bias=None, int variant=-1) -> Tensor");
    m.def("gemv_bf16_out(Tensor W, Tensor x, Tensor? bias, int variant, Tensor(a!) out) -> ()");
    m.def("gemv_fp8(Tensor Wq, Tensor scale, Tensor x, Tensor? bias=None, int variant=-1) -> Tensor");
    m.def("gemv_fp8_out(Tensor Wq, Tensor scale, Tensor x, Tensor? bias, int variant, Tensor(a!) out) -> ()");
    m.def("gemv_int4(Tensor Wq, Tensor scales, Tensor x, int variant=-1) -> Tensor");
    m.def("gemv_int4_out(Tensor Wq, Tensor scales, Tensor x, int variant, Tensor(a!) out) -> ()");
    m.def("gemv_int4_zp(Tensor Wq, Tensor scales, Tensor zeros, Tensor x, Tensor? bias=None, int variant=-1) -> Tensor");
    m.def("gemv_int4_zp_out(Tensor Wq, Tensor scales, Tensor zeros, Tensor x, Tensor? bias, int variant, "
          "Tensor(a!) out) -> ()");
    m.def("dequant_fp8(Tensor Wq, Tensor scale) -> Tensor");
    m.def("dequant_int4(Tensor Wq, Tensor scales) -> Tensor");
    m.def("dequant_int4_zp(Tensor Wq, Tensor scales, Tensor zeros) -> Tensor");
    m.def("quantize_fp8_rowwise(Tensor W) -> (Tensor, Tensor)");
    m.def("quantize_int4_g128(Tensor W) -> (Tensor, Tensor)");
    m.def("quantize_int4_zp_g128(Tensor W) -> (Tensor, Tensor, Tensor)");
}

// torch on ROCm dispatches HIP tensors under the CUDA key.
TORCH_LIBRARY_IMPL(paia_gemv, CUDA, m)
{
    m.impl("gemv_bf16", &gemv_bf16);
    m.impl("gemv_bf16_out", &gemv_bf16_out);
    m.impl("gemv_fp8", &gemv_fp8);
    m.impl("gemv_fp8_out", &gemv_fp8_out);
    m.impl("gemv_int4", &gemv_int4);
    m.impl("gemv_int4_out", &gemv_int4_out);
    m.impl("gemv_int4_zp", &gemv_int4_zp);
    m.impl("gemv_int4_zp_out", &gemv_int4_zp_out);
    m.impl("dequant_fp8", &dequant_fp8);
    m.impl("dequant_int4", &dequant_int4);
    m.impl("dequant_int4_zp", &dequant_int4_zp);
    m.impl("quantize_fp8_rowwise", &quantize_fp8_rowwise);
    m.impl("quantize_int4_g128", &quantize_int4_g128);
    m.impl("quantize_int4_zp_g128", &quantize_int4_zp_g128);
}

TORCH_LIBRARY_IMPL(paia_gemv, Meta, m)
{
    m.impl("gemv_bf16", &gemv_bf16_meta);
    m.impl("gemv_bf16_out", &out_meta_bf16);
    m.impl("gemv_fp8", &gemv_fp8_meta);
    m.impl("gemv_fp8_out", &out_meta_fp8);
    m.impl("gemv_int4", &gemv_int4_meta);
    m.impl("gemv_int4_out", &out_meta_int4);
    m.impl("gemv_int4_zp", &gemv_int4_zp_meta);
    m.impl("gemv_int4_zp_out", &out_meta_int4_zp);
    m.impl("dequant_fp8", &dequant_fp8_meta);
    m.impl("dequant_int4", &dequant_int4_meta);
    m.impl("dequant_int4_zp", &dequant_int4_zp_meta);
    m.impl("quantize_fp8_rowwise", &quantize_fp8_rowwise_meta);
    m.impl("quantize_int4_g128", &quantize_int4_g128_meta);
    m.impl("quantize_int4_zp_g128", &quantize_int4_zp_g128_meta);
}
