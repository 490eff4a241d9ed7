// kernels/libharp_async_op.so — PyTorch-ROCm operator library for the QK
// RMSNorm and RoPE operators of HARP's async runtime, on the GPU.
//
// Registers namespace async_op with the reference's schemas for the four
// operators the attention producer uses (async_rt/csrc/async_op_api.cc:54-57):
//   rmsnorm_forward_out(input, weight, output!, rms!, eps)
//   rmsnorm_backward_out(input, grad_output, weight, rms, grad_input!, grad_weight!)
//   rope_forward_impl(x, freqs_cis, output!)
//   rope_backward_impl(grad_output, freqs_cis, grad_x!)
// plus the fused pair the model applies back to back (attn.py:78-89):
//   qk_norm_rope_forward(x, weight, freqs_cis, output!, rms!, eps)
//   qk_norm_rope_backward(input, grad_output, weight, rms, freqs_cis,
//                         grad_input!, grad_weight!)
// The reference registers these for the CPU key of its own async_op library
// (an aarch64 build).  This one defines them as a fragment of the namespace,
// so a library holding the namespace's other operators (silu, tanh, add, ...)
// can be loaded next to it, as long as it does not define these six names.
//
// Implementations are registered for the CUDA dispatch key (PyTorch-ROCm
// tensors on a HIP device carry it) and call libharp_ra.so through
// include/harp_qk_norm_rope.h on the current HIP stream.  The CPU key raises.
//
// Tensor conventions: x / output / gradients are [B, H, S, D] views with unit
// D stride (fewer dims are read as [1, .., S, D]); weight and grad_weight are
// [D] bf16 or fp32 (an undefined or empty weight means none); rms is fp32
// with B*H*S elements in (b, h, s) order; freqs_cis is the complex [S, D/2] or
// [B, S, D/2] table (or its torch.view_as_real flattened to [.., S, D]).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <array>

#include "harp_qk_norm_rope.h"

namespace {

void check_status(int rc, const char* op) {
  TORCH_CHECK(rc == HARP_QK_OK, "async_op.", op, ": ", harp_qk_last_error(), " (status ", rc, ")");
}

// [B, H, S, D] view of t (leading unit dims added for fewer dims)
at::Tensor as4(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.dim() >= 1 && t.dim() <= 4, name, " must have 1 to 4 dims, got ", t.dim());
  at::Tensor v = t;
  while (v.dim() < 4) v = v.unsqueeze(0);
  return v;
}

std::array<int64_t, 4> strides4(const at::Tensor& t) { return {t.stride(0), t.stride(1), t.stride(2), t.stride(3)}; }

void check_bf16_on(const at::Tensor& t, const at::Tensor& ref, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be on a HIP device");
  TORCH_CHECK(t.device() == ref.device(), name, " must be on the same device as the input");
  TORCH_CHECK(t.scalar_type() == at::kBFloat16, name, " must be bfloat16, got ", t.scalar_type());
}

void check_same_shape(const at::Tensor& a, const at::Tensor& b, const char* name) {
  TORCH_CHECK(a.sizes() == b.sizes(), name, " must have shape ", b.sizes(), ", got ", a.sizes());
}

// weight / grad_weight: NULL (absent) or a contiguous [D] bf16 / fp32 tensor
const void* vec_ptr(const at::Tensor& w, const at::Tensor& ref, int64_t D, int* dtype, const char* name) {
  if (!w.defined() || w.numel() == 0) {
    *dtype = HARP_QK_BF16;
    return nullptr;
  }
  TORCH_CHECK(w.is_cuda() && w.device() == ref.device(), name, " must be on the input's device");
  TORCH_CHECK(w.numel() == D && w.is_contiguous(), name, " must be a contiguous tensor of ", D, " elements");
  if (w.scalar_type() == at::kFloat) *dtype = HARP_QK_F32;
  else if (w.scalar_type() == at::kBFloat16) *dtype = HARP_QK_BF16;
  else TORCH_CHECK(false, name, " must be float32 or bfloat16, got ", w.scalar_type());
  return w.data_ptr();
}

float* rms_ptr(const at::Tensor& rms, const at::Tensor& ref, int64_t rows, const char* name) {
  TORCH_CHECK(rms.is_cuda() && rms.device() == ref.device(), name, " must be on the input's device");
  TORCH_CHECK(rms.scalar_type() == at::kFloat, name, " must be float32");
  TORCH_CHECK(rms.numel() == rows && rms.is_contiguous(), name, " must be contiguous with ", rows, " elements");
  return rms.data_ptr<float>();
}

// freqs_cis -> fp32 [.., S, D] (cos, sin) pairs as rope.cc:197-204 builds
// them, plus the batch and row strides in floats
struct Freqs {
  at::Tensor t;
  int64_t sb = 0, ss = 0;
};
Freqs freqs_of(const at::Tensor& f, const at::Tensor& x4) {
  TORCH_CHECK(f.is_cuda() && f.device() == x4.device(), "freqs_cis must be on the input's device");
  at::Tensor r = f.is_complex() ? at::view_as_real(f).flatten(-2) : f;
  TORCH_CHECK(r.scalar_type() == at::kFloat, "freqs_cis must be complex64 (or its float32 view_as_real)");
  r = r.contiguous();
  TORCH_CHECK(r.dim() == 2 || r.dim() == 3, "freqs_cis must be [S, D/2] or [B, S, D/2] complex, got ", f.sizes());
  const int64_t B = x4.size(0), S = x4.size(2), D = x4.size(3);
  TORCH_CHECK(r.size(-1) == D && r.size(-2) == S, "freqs_cis must cover S=", S, " rows of D/2=", D / 2,
              " pairs, got ", f.sizes());
  if (r.dim() == 3) TORCH_CHECK(r.size(0) == B || r.size(0) == 1, "freqs_cis batch must be 1 or ", B);
  Freqs q;
  q.t = r;
  q.ss = r.stride(-2);
  q.sb = (r.dim() == 3 && r.size(0) > 1) ? r.stride(0) : 0;
  return q;
}

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  if (bytes == 0) return at::Tensor();
  return at::empty({(int64_t)((bytes + 3) / 4)}, like.options().dtype(at::kFloat));
}

hipStream_t stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.get_device()).stream(); }

// ---------------------------------------------------------------------------
void rmsnorm_forward_out_hip(const at::Tensor& input, const at::Tensor& weight, at::Tensor& output, at::Tensor& rms,
                             double eps) {
  check_bf16_on(input, input, "input");
  check_bf16_on(output, input, "output");
  check_same_shape(output, input, "output");
  const c10::DeviceGuard guard(input.device());
  const at::Tensor x4 = as4(input, "input"), o4 = as4(output, "output");
  const int64_t B = x4.size(0), H = x4.size(1), S = x4.size(2), D = x4.size(3);
  int wdt;
  const void* w = vec_ptr(weight, input, D, &wdt, "weight");
  float* r = rms_ptr(rms, input, B * H * S, "rms");
  const auto xs = strides4(x4), os = strides4(o4);
  check_status(harp_qk_rmsnorm_forward(x4.data_ptr(), xs.data(), o4.data_ptr(), os.data(), w, wdt, r, (float)eps,
                                       (int)B, (int)H, (int)S, (int)D, stream_of(input)),
               "rmsnorm_forward_out");
}

void rmsnorm_backward_out_hip(const at::Tensor& input, const at::Tensor& grad_output, const at::Tensor& weight,
                              const at::Tensor& rms, at::Tensor& grad_input, at::Tensor& grad_weight) {
  check_bf16_on(input, input, "input");
  check_bf16_on(grad_output, input, "grad_output");
  check_bf16_on(grad_input, input, "grad_input");
  check_same_shape(grad_output, input, "grad_output");
  check_same_shape(grad_input, input, "grad_input");
  const c10::DeviceGuard guard(input.device());
  const at::Tensor x4 = as4(input, "input"), g4 = as4(grad_output, "grad_output"), dx4 = as4(grad_input, "grad_input");
  const int64_t B = x4.size(0), H = x4.size(1), S = x4.size(2), D = x4.size(3);
  int wdt, gwdt;
  const void* w = vec_ptr(weight, input, D, &wdt, "weight");
  void* gw = const_cast<void*>(vec_ptr(grad_weight, input, D, &gwdt, "grad_weight"));
  const float* r = rms_ptr(rms, input, B * H * S, "rms");
  const size_t wsb = harp_qk_backward_workspace_bytes((int)B, (int)H, (int)S, (int)D);
  TORCH_CHECK(wsb != (size_t)-1, "async_op.rmsnorm_backward_out: ", harp_qk_last_error());
  at::Tensor ws = workspace(wsb, input);
  const auto xs = strides4(x4), gs = strides4(g4), dxs = strides4(dx4);
  check_status(harp_qk_rmsnorm_backward(x4.data_ptr(), xs.data(), g4.data_ptr(), gs.data(), w, wdt, r,
                                        dx4.data_ptr(), dxs.data(), gw, gwdt, (int)B, (int)H, (int)S, (int)D,
                                        ws.defined() ? ws.data_ptr() : nullptr, wsb, stream_of(input)),
               "rmsnorm_backward_out");
}

void rope_forward_impl_hip(const at::Tensor& x, const at::Tensor& freqs_cis, at::Tensor& output) {
  check_bf16_on(x, x, "x");
  check_bf16_on(output, x, "output");
  check_same_shape(output, x, "output");
  const c10::DeviceGuard guard(x.device());
  const at::Tensor x4 = as4(x, "x"), o4 = as4(output, "output");
  const Freqs f = freqs_of(freqs_cis, x4);
  const auto xs = strides4(x4), os = strides4(o4);
  check_status(harp_qk_rope_forward(x4.data_ptr(), xs.data(), f.t.data_ptr<float>(), f.sb, f.ss, o4.data_ptr(),
                                    os.data(), (int)x4.size(0), (int)x4.size(1), (int)x4.size(2), (int)x4.size(3),
                                    stream_of(x)),
               "rope_forward_impl");
}

void rope_backward_impl_hip(const at::Tensor& grad_output, const at::Tensor& freqs_cis, at::Tensor& grad_x) {
  check_bf16_on(grad_output, grad_output, "grad_output");
  check_bf16_on(grad_x, grad_output, "grad_x");
  check_same_shape(grad_x, grad_output, "grad_x");
  const c10::DeviceGuard guard(grad_output.device());
  const at::Tensor g4 = as4(grad_output, "grad_output"), dx4 = as4(grad_x, "grad_x");
  const Freqs f = freqs_of(freqs_cis, g4);
  const auto gs = strides4(g4), dxs = strides4(dx4);
  check_status(harp_qk_rope_backward(g4.data_ptr(), gs.data(), f.t.data_ptr<float>(), f.sb, f.ss, dx4.data_ptr(),
                                     dxs.data(), (int)g4.size(0), (int)g4.size(1), (int)g4.size(2), (int)g4.size(3),
                                     stream_of(grad_output)),
               "rope_backward_impl");
}

void qk_norm_rope_forward_hip(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& freqs_cis,
                              at::Tensor& output, at::Tensor& rms, double eps) {
  check_bf16_on(x, x, "x");
  check_bf16_on(output, x, "output");
  check_same_shape(output, x, "output");
  const c10::DeviceGuard guard(x.device());
  const at::Tensor x4 = as4(x, "x"), o4 = as4(output, "output");
  const int64_t B = x4.size(0), H = x4.size(1), S = x4.size(2), D = x4.size(3);
  int wdt;
  const void* w = vec_ptr(weight, x, D, &wdt, "weight");
  float* r = rms_ptr(rms, x, B * H * S, "rms");
  const Freqs f = freqs_of(freqs_cis, x4);
  const auto xs = strides4(x4), os = strides4(o4);
  check_status(harp_qk_norm_rope_forward(x4.data_ptr(), xs.data(), w, wdt, (float)eps, f.t.data_ptr<float>(), f.sb,
                                         f.ss, o4.data_ptr(), os.data(), r, (int)B, (int)H, (int)S, (int)D,
                                         stream_of(x)),
               "qk_norm_rope_forward");
}

void qk_norm_rope_backward_hip(const at::Tensor& input, const at::Tensor& grad_output, const at::Tensor& weight,
                               const at::Tensor& rms, const at::Tensor& freqs_cis, at::Tensor& grad_input,
                               at::Tensor& grad_weight) {
  check_bf16_on(input, input, "input");
  check_bf16_on(grad_output, input, "grad_output");
  check_bf16_on(grad_input, input, "grad_input");
  check_same_shape(grad_output, input, "grad_output");
  check_same_shape(grad_input, input, "grad_input");
  const c10::DeviceGuard guard(input.device());
  const at::Tensor x4 = as4(input, "input"), g4 = as4(grad_output, "grad_output"), dx4 = as4(grad_input, "grad_input");
  const int64_t B = x4.size(0), H = x4.size(1), S = x4.size(2), D = x4.size(3);
  int wdt, gwdt;
  const void* w = vec_ptr(weight, input, D, &wdt, "weight");
  void* gw = const_cast<void*>(vec_ptr(grad_weight, input, D, &gwdt, "grad_weight"));
  const float* r = rms_ptr(rms, input, B * H * S, "rms");
  const Freqs f = freqs_of(freqs_cis, x4);
  const size_t wsb = harp_qk_backward_workspace_bytes((int)B, (int)H, (int)S, (int)D);
  TORCH_CHECK(wsb != (size_t)-1, "async_op.qk_norm_rope_backward: ", harp_qk_last_error());
  at::Tensor ws = workspace(wsb, input);
  const auto xs = strides4(x4), gs = strides4(g4), dxs = strides4(dx4);
  check_status(harp_qk_norm_rope_backward(g4.data_ptr(), gs.data(), x4.data_ptr(), xs.data(), w, wdt, r,
                                          f.t.data_ptr<float>(), f.sb, f.ss, dx4.data_ptr(), dxs.data(), gw, gwdt,
                                          (int)B, (int)H, (int)S, (int)D, ws.defined() ? ws.data_ptr() : nullptr,
                                          wsb, stream_of(input)),
               "qk_norm_rope_backward");
}

[[noreturn]] void no_cpu(const char* op) {
  TORCH_CHECK(false, "async_op.", op, ": this library runs on a HIP device only (CPU tensors given)");
}
void rmsnorm_forward_out_cpu(const at::Tensor&, const at::Tensor&, at::Tensor&, at::Tensor&, double) {
  no_cpu("rmsnorm_forward_out");
}
void rmsnorm_backward_out_cpu(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, at::Tensor&,
                              at::Tensor&) {
  no_cpu("rmsnorm_backward_out");
}
void rope_forward_impl_cpu(const at::Tensor&, const at::Tensor&, at::Tensor&) { no_cpu("rope_forward_impl"); }
void rope_backward_impl_cpu(const at::Tensor&, const at::Tensor&, at::Tensor&) { no_cpu("rope_backward_impl"); }
void qk_norm_rope_forward_cpu(const at::Tensor&, const at::Tensor&, const at::Tensor&, at::Tensor&, at::Tensor&,
                              double) {
  no_cpu("qk_norm_rope_forward");
}
void qk_norm_rope_backward_cpu(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                               const at::Tensor&, at::Tensor&, at::Tensor&) {
  no_cpu("qk_norm_rope_backward");
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(async_op, m) {
  m.def("rmsnorm_forward_out(Tensor input, Tensor weight, Tensor(a!) output, Tensor(b!) rms, float eps) -> ()");
  m.def(
      "rmsnorm_backward_out(Tensor input, Tensor grad_output, Tensor weight, Tensor rms, Tensor(a!) grad_input, "
      "Tensor(b!) grad_weight) -> ()");
  m.def("rope_forward_impl(Tensor x, Tensor freqs_cis, Tensor(a!) output) -> ()");
  m.def("rope_backward_impl(Tensor grad_output, Tensor freqs_cis, Tensor(b!) grad_x) -> ()");
  m.def(
      "qk_norm_rope_forward(Tensor x, Tensor weight, Tensor freqs_cis, Tensor(a!) output, Tensor(b!) rms, "
      "float eps) -> ()");
  m.def(
      "qk_norm_rope_backward(Tensor input, Tensor grad_output, Tensor weight, Tensor rms, Tensor freqs_cis, "
      "Tensor(a!) grad_input, Tensor(b!) grad_weight) -> ()");
}

TORCH_LIBRARY_IMPL(async_op, CUDA, m) {
  m.impl("rmsnorm_forward_out", &rmsnorm_forward_out_hip);
  m.impl("rmsnorm_backward_out", &rmsnorm_backward_out_hip);
  m.impl("rope_forward_impl", &rope_forward_impl_hip);
  m.impl("rope_backward_impl", &rope_backward_impl_hip);
  m.impl("qk_norm_rope_forward", &qk_norm_rope_forward_hip);
  m.impl("qk_norm_rope_backward", &qk_norm_rope_backward_hip);
}

TORCH_LIBRARY_IMPL(async_op, CPU, m) {
  m.impl("rmsnorm_forward_out", &rmsnorm_forward_out_cpu);
  m.impl("rmsnorm_backward_out", &rmsnorm_backward_out_cpu);
  m.impl("rope_forward_impl", &rope_forward_impl_cpu);
  m.impl("rope_backward_impl", &rope_backward_impl_cpu);
  m.impl("qk_norm_rope_forward", &qk_norm_rope_forward_cpu);
  m.impl("qk_norm_rope_backward", &qk_norm_rope_backward_cpu);
}
