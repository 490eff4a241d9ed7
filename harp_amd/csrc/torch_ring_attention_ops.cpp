// kernels/libring_attention_ops.so — PyTorch-ROCm operator library for the
// ring-attention block, a drop-in for the reference's library of the same
// name (gemm/ring_attention/Makefile:9-12, loaded by train.py:151).
//
// Registers namespace ring_attention_ops with the reference's two schemas
// (gemm/ring_attention/torch_ring_attention_ops.cpp:260-263) extended only by
// trailing defaulted arguments, so every existing positional call parses:
//   ring_attention_forward(q, k, v, out!, m_i!, l_i!, sp_size, scale,
//                          ring_rank=0, kv_lens=None, kv_chunk_len=0)
//   ring_attention_backward(q, grad_q!, k, dK!, v, dV!, grad_out, m_i, l_i, D,
//                           sp_size, scale, ring_rank=0, kv_lens=None,
//                           kv_chunk_len=0)
// plus ring_attention_delta(grad_out, out) -> D, the rowsum(dO*O) preprocess
// of src/models/z_image/module/attn.py:41 as one kernel.
//
// Implementations are registered for the CUDA dispatch key (PyTorch-ROCm
// tensors on a HIP device carry it) and call libharp_ra.so through its C ABI
// on the current HIP stream; they never synchronise.  The CPU key validates
// the call's shapes, then raises: this build has no CPU path.
//
// Single-GPU ring semantics: k and v hold every KV chunk of the ring,
// concatenated along dim 2; dK / dV have k's shape and receive the local
// queries' contribution to each chunk.  kv_lens optionally gives the valid
// (unmasked) rows of each chunk.  The chunk length is
//   * kv_chunk_len when it is > 0 (k.size(2) must be sp_size * kv_chunk_len);
//   * else, when kv_lens is given, k.size(2) / sp_size;
//   * else (the reference's positional call) k.size(2) when sp_size == 1, or
//     q.size(2) when k.size(2) == sp_size * q.size(2).
// Any other reference-shaped call is rejected.  In particular HARP's own call
// (attn.py:29: k / v hold only the local chunk, the other sp_size - 1 chunks
// live on peer ranks, ring_attn.cpp:2424-2426) cannot be served on one GPU
// and raises instead of silently attending over the local keys only.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <array>
#include <tuple>
#include <vector>

#include "harp_ring_attn.h"

namespace {

// Element strides of a [B, H, T, D] view.  A size-1 dim may carry any stride
// in torch; the kernels derive buffer ranges from the T stride, so a single
// row reports a T stride of at least one row.
std::array<int64_t, 4> strides4(const at::Tensor& t) {
  std::array<int64_t, 4> s = {t.stride(0), t.stride(1), t.stride(2), t.stride(3)};
  if (t.size(2) == 1 && s[2] < t.size(3)) s[2] = (t.size(3) + 7) / 8 * 8;
  return s;
}

void check_status(int rc, const char* op) {
  TORCH_CHECK(rc == HARP_RA_OK, "ring_attention_ops.", op, ": ", harp_ra_last_error(), " (status ", rc, ")");
}

void check_device(const at::Tensor& t, const at::Tensor& ref, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be on a HIP device");
  TORCH_CHECK(t.device() == ref.device(), name, " must be on the same device as q");
}

void check_bhtd(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.dim() == 4, name, " must be a [B, H, T, D] tensor, got ", t.dim(), " dims");
}

int dtype_code(const at::Tensor& t, const char* name) {
  if (t.scalar_type() == at::kFloat) return HARP_RA_F32;
  if (t.scalar_type() == at::kBFloat16) return HARP_RA_BF16;
  TORCH_CHECK(false, name, " must be float32 or bfloat16, got ", t.scalar_type());
}

void check_stats(const at::Tensor& t, const at::Tensor& q, const char* name) {
  TORCH_CHECK(t.dim() == 4 && t.size(0) == q.size(0) && t.size(1) == q.size(1) && t.size(2) == q.size(2) &&
                  t.size(3) == 1,
              name, " must be [B, H, T, 1] matching q");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

struct Chunks {
  std::vector<const void*> k, v;
  std::vector<void*> dk, dv;
  std::vector<int32_t> lens;
  int chunk_len = 0;
};

Chunks split_chunks(const char* op, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t sp_size,
                    at::OptionalIntArrayRef kv_lens, int64_t kv_chunk_len) {
  TORCH_CHECK(sp_size >= 1 && sp_size <= HARP_RA_MAX_CHUNKS, "ring_attention_ops.", op, ": sp_size must be in [1, ",
              HARP_RA_MAX_CHUNKS, "], got ", sp_size);
  TORCH_CHECK(k.sizes() == v.sizes(), "k and v must have the same shape");
  TORCH_CHECK(k.size(0) == q.size(0) && k.size(1) == q.size(1) && k.size(3) == q.size(3),
              "k/v must match q on B, H and D");
  TORCH_CHECK(k.strides() == v.strides(), "k and v must have the same strides");
  TORCH_CHECK(kv_chunk_len >= 0, "ring_attention_ops.", op, ": kv_chunk_len must be >= 0, got ", kv_chunk_len);
  const int64_t rows = k.size(2);
  int64_t chunk = 0;
  if (kv_chunk_len > 0) {
    TORCH_CHECK(rows == sp_size * kv_chunk_len, "ring_attention_ops.", op, ": k.size(2)=", rows,
                " must equal sp_size * kv_chunk_len = ", sp_size, " * ", kv_chunk_len);
    chunk = kv_chunk_len;
  } else if (kv_lens.has_value()) {
    TORCH_CHECK(rows % sp_size == 0, "ring_attention_ops.", op, ": with kv_lens, k/v hold all sp_size KV chunks along ",
                "dim 2: k.size(2)=", rows, " is not a multiple of sp_size=", sp_size);
    chunk = rows / sp_size;
  } else if (sp_size == 1) {
    chunk = rows;
  } else if (rows == sp_size * q.size(2)) {
    chunk = q.size(2);
  } else if (rows == q.size(2)) {
    TORCH_CHECK(false, "ring_attention_ops.", op, ": k/v hold only the local chunk (k.size(2) == q.size(2) == ", rows,
                ") with sp_size=", sp_size,
                " > 1: the other ranks' chunks would come from peers, which one GPU does not have. Pass all ",
                "sp_size chunks concatenated along dim 2 (k.size(2) == sp_size * q.size(2)), or give kv_chunk_len ",
                "(k.size(2) == sp_size * kv_chunk_len)");
  } else {
    TORCH_CHECK(false, "ring_attention_ops.", op, ": k.size(2)=", rows, " does not match sp_size=", sp_size,
                " chunks of q.size(2)=", q.size(2), " rows; pass kv_chunk_len (k.size(2) == sp_size * kv_chunk_len) ",
                "for another chunk length");
  }
  Chunks c;
  c.chunk_len = static_cast<int>(chunk);
  const int64_t step = chunk * k.stride(2) * k.element_size();
  for (int64_t i = 0; i < sp_size; ++i) {
    c.k.push_back(static_cast<const char*>(k.data_ptr()) + i * step);
    c.v.push_back(static_cast<const char*>(v.data_ptr()) + i * step);
  }
  if (kv_lens.has_value()) {
    TORCH_CHECK(static_cast<int64_t>(kv_lens->size()) == sp_size, "kv_lens must have sp_size entries");
    for (int64_t x : *kv_lens) {
      TORCH_CHECK(x >= 0 && x <= c.chunk_len, "kv_lens entries must be in [0, ", c.chunk_len, "]");
      c.lens.push_back(static_cast<int32_t>(x));
    }
  }
  return c;
}

// Device scratch from the caching allocator (empty when none is needed).
at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  return at::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
}
void* ws_ptr(const at::Tensor& ws) { return ws.numel() ? ws.data_ptr() : nullptr; }

std::tuple<at::Tensor, at::Tensor, at::Tensor> forward_hip(const at::Tensor& q, const at::Tensor& k,
                                                           const at::Tensor& v, at::Tensor out, at::Tensor m_i,
                                                           at::Tensor l_i, int64_t sp_size, double scale,
                                                           int64_t ring_rank, at::OptionalIntArrayRef kv_lens,
                                                           int64_t kv_chunk_len) {
  check_bhtd(q, "q");
  check_bhtd(k, "k");
  check_bhtd(v, "v");
  check_bhtd(out, "out");
  for (const at::Tensor* t : {&k, &v, (const at::Tensor*)&out, (const at::Tensor*)&m_i, (const at::Tensor*)&l_i})
    check_device(*t, q, "tensor");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                  v.scalar_type() == at::kBFloat16,
              "q, k, v must be bfloat16");
  TORCH_CHECK(out.scalar_type() == at::kFloat, "out must be float32");
  TORCH_CHECK(out.sizes() == q.sizes(), "out must have q's shape");
  check_stats(m_i, q, "m_i");
  check_stats(l_i, q, "l_i");
  TORCH_CHECK(l_i.scalar_type() == at::kFloat, "l_i must be float32");
  const int m_code = dtype_code(m_i, "m_i");
  Chunks ch = split_chunks("ring_attention_forward", q, k, v, sp_size, kv_lens, kv_chunk_len);
  const c10::DeviceGuard guard(q.device());
  const int B = q.size(0), H = q.size(1), T = q.size(2), D = q.size(3);
  const int32_t* lens = ch.lens.empty() ? nullptr : ch.lens.data();
  const size_t ws_bytes = harp_ra_forward_workspace_bytes(B, H, T, D, sp_size, ch.chunk_len, lens);
  check_status(ws_bytes != SIZE_MAX ? HARP_RA_OK : HARP_RA_EINVAL, "ring_attention_forward");
  at::Tensor ws = workspace(ws_bytes, q);
  const auto qs = strides4(q), ks = strides4(k), os = strides4(out);
  hipStream_t stream = c10::hip::getCurrentHIPStream(q.get_device()).stream();
  const int rc = harp_ra_forward(q.data_ptr(), qs.data(), ch.k.data(), ch.v.data(), ks.data(), ch.chunk_len, lens,
                                 out.data_ptr<float>(), os.data(), m_i.data_ptr(), m_code, l_i.data_ptr<float>(), B,
                                 H, T, D, static_cast<int>(sp_size), static_cast<int>(ring_rank),
                                 static_cast<float>(scale), ws_ptr(ws), ws_bytes, stream);
  check_status(rc, "ring_attention_forward");
  return std::make_tuple(out, m_i, l_i);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> backward_hip(const at::Tensor& q, at::Tensor grad_q,
                                                            const at::Tensor& k, at::Tensor dK, const at::Tensor& v,
                                                            at::Tensor dV, const at::Tensor& grad_out,
                                                            const at::Tensor& m_i, const at::Tensor& l_i,
                                                            const at::Tensor& D, int64_t sp_size, double scale,
                                                            int64_t ring_rank, at::OptionalIntArrayRef kv_lens,
                                                            int64_t kv_chunk_len) {
  const std::array<const at::Tensor*, 7> ops4 = {&q, &grad_q, &k, &dK, &v, &dV, &grad_out};
  for (const at::Tensor* t : ops4) check_bhtd(*t, "gradient operand");
  const std::array<const at::Tensor*, 9> dev_ops = {&grad_q, &k, &dK, &v, &dV, &grad_out, &m_i, &l_i, &D};
  for (const at::Tensor* t : dev_ops) check_device(*t, q, "tensor");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                  v.scalar_type() == at::kBFloat16 && grad_out.scalar_type() == at::kBFloat16,
              "q, k, v, grad_out must be bfloat16");
  TORCH_CHECK(grad_q.sizes() == q.sizes(), "grad_q must have q's shape");
  TORCH_CHECK(grad_out.sizes() == q.sizes(), "grad_out must have q's shape");
  TORCH_CHECK(dK.sizes() == k.sizes() && dV.sizes() == k.sizes(), "dK and dV must have k's shape");
  TORCH_CHECK(dK.scalar_type() == dV.scalar_type(), "dK and dV must have the same dtype");
  TORCH_CHECK(dK.strides() == dV.strides(), "dK and dV must have the same strides");
  check_stats(m_i, q, "m_i");
  check_stats(l_i, q, "l_i");
  check_stats(D, q, "D");
  TORCH_CHECK(l_i.scalar_type() == at::kFloat && D.scalar_type() == at::kFloat, "l_i and D must be float32");
  const int m_code = dtype_code(m_i, "m_i");
  const int dq_code = dtype_code(grad_q, "grad_q");
  const int dkv_code = dtype_code(dK, "dK");
  Chunks ch = split_chunks("ring_attention_backward", q, k, v, sp_size, kv_lens, kv_chunk_len);
  const int64_t dstep = ch.chunk_len * dK.stride(2) * dK.element_size();
  for (int64_t i = 0; i < sp_size; ++i) {
    ch.dk.push_back(static_cast<char*>(dK.data_ptr()) + i * dstep);
    ch.dv.push_back(static_cast<char*>(dV.data_ptr()) + i * dstep);
  }
  const c10::DeviceGuard guard(q.device());
  const int B = q.size(0), H = q.size(1), T = q.size(2), Dh = q.size(3);
  const int32_t* lens = ch.lens.empty() ? nullptr : ch.lens.data();
  const size_t ws_bytes = harp_ra_backward_workspace_bytes(B, H, T, Dh, sp_size, ch.chunk_len, lens);
  check_status(ws_bytes != SIZE_MAX ? HARP_RA_OK : HARP_RA_EINVAL, "ring_attention_backward");
  at::Tensor ws = workspace(ws_bytes, q);
  const auto qs = strides4(q), dqs = strides4(grad_q), ks = strides4(k), dks = strides4(dK), gs = strides4(grad_out);
  hipStream_t stream = c10::hip::getCurrentHIPStream(q.get_device()).stream();
  const int rc = harp_ra_backward(
      q.data_ptr(), qs.data(), grad_q.data_ptr(), dqs.data(), dq_code, ch.k.data(), ch.v.data(), ks.data(),
      ch.dk.data(), ch.dv.data(), dks.data(), dkv_code, ch.chunk_len, lens, grad_out.data_ptr(), gs.data(),
      m_i.data_ptr(), m_code, l_i.data_ptr<float>(), D.data_ptr<float>(), B, H, T, Dh, static_cast<int>(sp_size),
      static_cast<int>(ring_rank), static_cast<float>(scale), ws_ptr(ws), ws_bytes, stream);
  check_status(rc, "ring_attention_backward");
  return std::make_tuple(grad_q, dK, dV);
}

at::Tensor delta_hip(const at::Tensor& grad_out, const at::Tensor& out) {
  check_bhtd(grad_out, "grad_out");
  check_bhtd(out, "out");
  check_device(out, grad_out, "out");
  TORCH_CHECK(grad_out.scalar_type() == at::kBFloat16, "grad_out must be bfloat16");
  TORCH_CHECK(out.scalar_type() == at::kFloat, "out must be float32");
  TORCH_CHECK(out.sizes() == grad_out.sizes(), "out must have grad_out's shape");
  const c10::DeviceGuard guard(out.device());
  at::Tensor D = at::empty({out.size(0), out.size(1), out.size(2), 1}, out.options());
  const auto gs = strides4(grad_out), os = strides4(out);
  hipStream_t stream = c10::hip::getCurrentHIPStream(out.get_device()).stream();
  const int rc = harp_ra_delta(grad_out.data_ptr(), gs.data(), out.data_ptr<float>(), os.data(), D.data_ptr<float>(),
                               out.size(0), out.size(1), out.size(2), out.size(3), stream);
  check_status(rc, "ring_attention_delta");
  return D;
}

[[noreturn]] void no_cpu_path(const char* op) {
  TORCH_CHECK(false, "ring_attention_ops.", op,
              ": this MI355X build runs on HIP devices only; move the tensors to the GPU (there is no CPU path)");
}

// The CPU key runs the shape contract first, so a call that could never run
// on the GPU either reports that, then refuses the CPU tensors.
std::tuple<at::Tensor, at::Tensor, at::Tensor> forward_cpu(const at::Tensor& q, const at::Tensor& k,
                                                           const at::Tensor& v, at::Tensor, at::Tensor, at::Tensor,
                                                           int64_t sp_size, double, int64_t,
                                                           at::OptionalIntArrayRef kv_lens, int64_t kv_chunk_len) {
  check_bhtd(q, "q");
  check_bhtd(k, "k");
  check_bhtd(v, "v");
  (void)split_chunks("ring_attention_forward", q, k, v, sp_size, kv_lens, kv_chunk_len);
  no_cpu_path("ring_attention_forward");
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> backward_cpu(const at::Tensor& q, at::Tensor, const at::Tensor& k,
                                                            at::Tensor, const at::Tensor& v, at::Tensor,
                                                            const at::Tensor&, const at::Tensor&, const at::Tensor&,
                                                            const at::Tensor&, int64_t sp_size, double, int64_t,
                                                            at::OptionalIntArrayRef kv_lens, int64_t kv_chunk_len) {
  check_bhtd(q, "q");
  check_bhtd(k, "k");
  check_bhtd(v, "v");
  (void)split_chunks("ring_attention_backward", q, k, v, sp_size, kv_lens, kv_chunk_len);
  no_cpu_path("ring_attention_backward");
}
at::Tensor delta_cpu(const at::Tensor&, const at::Tensor&) { no_cpu_path("ring_attention_delta"); }

}  // namespace

TORCH_LIBRARY(ring_attention_ops, m) {
  m.def(
      "ring_attention_forward(Tensor q, Tensor k, Tensor v, Tensor(a!) out, Tensor(b!) m_i, Tensor(c!) l_i, "
      "int sp_size, float scale, int ring_rank=0, int[]? kv_lens=None, int kv_chunk_len=0) -> (Tensor(a!), Tensor(b!), "
      "Tensor(c!))");
  m.def(
      "ring_attention_backward(Tensor q, Tensor(a!) grad_q, Tensor k, Tensor(b!) dK, Tensor v, Tensor(c!) dV, "
      "Tensor grad_out, Tensor m_i, Tensor l_i, Tensor D, int sp_size, float scale, int ring_rank=0, "
      "int[]? kv_lens=None, int kv_chunk_len=0) -> (Tensor(a!), Tensor(b!), Tensor(c!))");
  m.def("ring_attention_delta(Tensor grad_out, Tensor out) -> Tensor");
}

TORCH_LIBRARY_IMPL(ring_attention_ops, CUDA, m) {
  m.impl("ring_attention_forward", &forward_hip);
  m.impl("ring_attention_backward", &backward_hip);
  m.impl("ring_attention_delta", &delta_hip);
}

TORCH_LIBRARY_IMPL(ring_attention_ops, CPU, m) {
  m.impl("ring_attention_forward", &forward_cpu);
  m.impl("ring_attention_backward", &backward_cpu);
  m.impl("ring_attention_delta", &delta_cpu);
}
