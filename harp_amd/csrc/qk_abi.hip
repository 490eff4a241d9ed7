// C ABI of the QK-RMSNorm / RoPE kernels: argument validation and kernel
// sequencing.  See include/harp_qk_norm_rope.h.
//
// Host flow mirrors the reference operators (async_rt/csrc/rms_norm.cc:447-522,
// async_rt/csrc/rope.cc:186-249): the reference walks rows on CPU threads
// (at::parallel_for); here one launch covers every row of every head, and the
// RMSNorm weight gradient is reduced from per-block partial sums by two small
// launches instead of per-thread buffers.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <utility>
#include <string>
#include <vector>

#include "../../include/harp_qk_norm_rope.h"
#include "proj_kernels.h"
#include "qk_kernels.h"

using namespace harp_qk;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}
int ok() {
  g_last_error.clear();
  return HARP_QK_OK;
}

int check_shape(int B, int H, int S, int D, bool rope) {
  if (B < 1 || H < 1 || S < 1 || D < 1) return fail(HARP_QK_EINVAL, "B, H, S, D must be positive");
  if (D % 8 != 0) return fail(HARP_QK_EUNSUPPORTED, "D=%d must be a multiple of 8", D);
  if (D > 256) return fail(HARP_QK_EUNSUPPORTED, "D=%d > 256 is not supported", D);
  if (rope && D % 2 != 0) return fail(HARP_QK_EINVAL, "RoPE needs an even D");
  if ((int64_t)B * H * S > ((int64_t)1 << 40)) return fail(HARP_QK_EUNSUPPORTED, "too many rows");
  return HARP_QK_OK;
}

// bf16 [B,H,S,D] view read or written with 16-byte accesses
int check_view(const void* p, const int64_t* st, const char* name) {
  if (!p) return fail(HARP_QK_EINVAL, "%s is NULL", name);
  if (!st) return fail(HARP_QK_EINVAL, "%s strides are NULL", name);
  if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return fail(HARP_QK_EINVAL, "%s must be 16-byte aligned", name);
  if (st[3] != 1) return fail(HARP_QK_EINVAL, "%s must have unit stride in D (got %lld)", name, (long long)st[3]);
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || st[i] % 8 != 0)
      return fail(HARP_QK_EINVAL, "%s stride[%d]=%lld must be a non-negative multiple of 8 elements", name, i,
                  (long long)st[i]);
  return HARP_QK_OK;
}

int check_freqs(const float* f, int64_t fsb, int64_t fss) {
  if (!f) return fail(HARP_QK_EINVAL, "freqs is NULL");
  if ((reinterpret_cast<uintptr_t>(f) & 15u) != 0) return fail(HARP_QK_EINVAL, "freqs must be 16-byte aligned");
  if (fsb < 0 || fss < 0 || fsb % 4 != 0 || fss % 4 != 0)
    return fail(HARP_QK_EINVAL, "freqs strides (%lld, %lld) must be non-negative multiples of 4 floats",
                (long long)fsb, (long long)fss);
  return HARP_QK_OK;
}

int check_dtype(int dt, const char* name) {
  if (dt != HARP_QK_F32 && dt != HARP_QK_BF16) return fail(HARP_QK_EINVAL, "%s dtype must be F32 or BF16", name);
  return HARP_QK_OK;
}

// the weight is read with 16-byte loads
int check_weight(const void* w, int dt) {
  int rc;
  if ((rc = check_dtype(dt, "weight"))) return rc;
  if ((reinterpret_cast<uintptr_t>(w) & 15u) != 0) return fail(HARP_QK_EINVAL, "weight must be 16-byte aligned");
  return HARP_QK_OK;
}

Strides4 s3(const int64_t* st) { return Strides4{st[0], st[1], st[2]}; }

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(HARP_QK_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HARP_QK_OK;
}

size_t bwd_ws_bytes(const QkShape& sh) { return bwd_workspace_floats(sh) * sizeof(float); }

// Library-owned grow-only workspace for callers that pass workspace == NULL,
// one buffer per (device, stream): calls on one stream run in order and so
// never overlap on their buffer, and calls on different streams never share
// one.  A buffer that must grow is freed only after its stream has drained
// (earlier calls may still read it).  At most kMaxOwned buffers are kept: a
// call on a new stream when the table is full frees the least recently used
// buffer first, after waiting for its whole device (its stream may no longer
// exist).  This path calls hipMalloc / hipFree, so it cannot be captured into
// a HIP graph; callers that capture pass their own workspace.
constexpr size_t kMaxOwned = 8;
struct OwnedWorkspace {
  struct Buf {
    int dev;
    hipStream_t stream;
    void* ptr;
    size_t bytes;
    uint64_t last_use;
  };
  std::mutex mu;
  std::vector<Buf> bufs;
  uint64_t clock = 0;
};
OwnedWorkspace& owned() {
  static OwnedWorkspace w;
  return w;
}
int resolve_workspace(void** ws, size_t* ws_bytes, size_t need, hipStream_t stream) {
  if (*ws) {
    if (*ws_bytes < need)
      return fail(HARP_QK_ENOMEM, "workspace of %zu bytes is smaller than the %zu bytes needed", *ws_bytes, need);
    if ((reinterpret_cast<uintptr_t>(*ws) & 15u) != 0) return fail(HARP_QK_EINVAL, "workspace must be 16-byte aligned");
    return HARP_QK_OK;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HARP_QK_ELAUNCH, "hipGetDevice failed");
  OwnedWorkspace& w = owned();
  std::lock_guard<std::mutex> lk(w.mu);
  OwnedWorkspace::Buf* b = nullptr;
  for (auto& x : w.bufs)
    if (x.dev == dev && x.stream == stream) b = &x;
  if (!b) {
    if (w.bufs.size() >= kMaxOwned) {
      size_t lru = 0;
      for (size_t i = 1; i < w.bufs.size(); ++i)
        if (w.bufs[i].last_use < w.bufs[lru].last_use) lru = i;
      OwnedWorkspace::Buf& e = w.bufs[lru];
      if (e.ptr) {
        if (e.dev != dev && hipSetDevice(e.dev) != hipSuccess) return fail(HARP_QK_ELAUNCH, "hipSetDevice failed");
        const bool synced = hipDeviceSynchronize() == hipSuccess;
        if (synced) (void)hipFree(e.ptr);
        if (e.dev != dev && hipSetDevice(dev) != hipSuccess) return fail(HARP_QK_ELAUNCH, "hipSetDevice failed");
        if (!synced) return fail(HARP_QK_ELAUNCH, "hipDeviceSynchronize failed");
      }
      w.bufs.erase(w.bufs.begin() + (std::ptrdiff_t)lru);
    }
    w.bufs.push_back(OwnedWorkspace::Buf{dev, stream, nullptr, 0, 0});
    b = &w.bufs.back();
  }
  b->last_use = ++w.clock;
  if (b->bytes < need) {
    if (b->ptr) {
      if (hipStreamSynchronize(stream) != hipSuccess) return fail(HARP_QK_ELAUNCH, "hipStreamSynchronize failed");
      (void)hipFree(b->ptr);
      b->ptr = nullptr;
      b->bytes = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, need) != hipSuccess) return fail(HARP_QK_ENOMEM, "hipMalloc of %zu workspace bytes failed", need);
    b->ptr = p;
    b->bytes = need;
  }
  *ws = b->ptr;
  *ws_bytes = b->bytes;
  return HARP_QK_OK;
}

// Scratch of the allocation-free backward (harp_qk_norm_rope_backward_noalloc):
// the weight-gradient partials of at most kQkBwdMaxBlocks row blocks plus their
// group sums, for any D <= 256: (2048 + 32) x 256 floats = 2.03 MiB, held by
// every device the library runs on until the process ends.  In host code the
// name is only a stand-in; kernels get the device address that
// hipGetSymbolAddress returns for the current device (scratch_ptr below).
constexpr size_t kScratchFloats =
    (size_t)(kQkBwdMaxBlocks + (kQkBwdMaxBlocks + kWgGroupRows - 1) / kWgGroupRows) * 256;
static __device__ __align__(256) float scratch[kScratchFloats];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_ptr(float** out) {
  static std::mutex mu;
  static std::vector<std::pair<int, float*>> table;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HARP_QK_ELAUNCH, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(mu);
  for (const auto& e : table)
    if (e.first == dev) {
      *out = e.second;
      return HARP_QK_OK;
    }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(HARP_QK_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
  table.emplace_back(dev, static_cast<float*>(p));
  *out = static_cast<float*>(p);
  return HARP_QK_OK;
}

int forward(int mode, const void* x, const int64_t* xs, const void* weight, int wdt, float eps, const float* freqs,
            int64_t fsb, int64_t fss, void* out, const int64_t* os, float* rms, int B, int H, int S, int D,
            void* stream) {
  int rc;
  if ((rc = check_shape(B, H, S, D, mode & 2))) return rc;
  if ((rc = check_view(x, xs, "x"))) return rc;
  if ((rc = check_view(out, os, "out"))) return rc;
  if (mode & 1) {
    if (weight && (rc = check_weight(weight, wdt))) return rc;
    if (!(eps >= 0.f) || eps != eps) return fail(HARP_QK_EINVAL, "eps must be a non-negative number");
  }
  if ((mode & 2) && (rc = check_freqs(freqs, fsb, fss))) return rc;
  QkFwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.sh = QkShape{B, H, S, D};
  p.x = static_cast<const uint16_t*>(x);
  p.sx = s3(xs);
  p.out = static_cast<uint16_t*>(out);
  p.so = s3(os);
  p.weight = weight;
  p.weight_f32 = (wdt == HARP_QK_F32);
  p.eps = eps;
  p.rms = rms;
  p.freqs = freqs;
  p.f_stride_b = fsb;
  p.f_stride_s = fss;
  if ((rc = launched(launch_qk_forward(p, mode, static_cast<hipStream_t>(stream)), "QK forward"))) return rc;
  return ok();
}

int backward(int mode, const void* dy, const int64_t* dys, const void* x, const int64_t* xs, const void* weight,
             int wdt, const float* rms, const float* freqs, int64_t fsb, int64_t fss, void* dx, const int64_t* dxs,
             void* gw, int gwdt, int B, int H, int S, int D, void* ws, size_t wsb, void* stream) {
  int rc;
  if ((rc = check_shape(B, H, S, D, mode & 2))) return rc;
  if ((rc = check_view(dy, dys, "grad_output"))) return rc;
  if ((rc = check_view(dx, dxs, "grad_input"))) return rc;
  if ((mode & 2) && (rc = check_freqs(freqs, fsb, fss))) return rc;
  const QkShape sh{B, H, S, D};
  if (mode & 1) {
    if ((rc = check_view(x, xs, "input"))) return rc;
    if (!rms) return fail(HARP_QK_EINVAL, "rms is NULL");
    if (weight && (rc = check_weight(weight, wdt))) return rc;
    if (gw && (rc = check_dtype(gwdt, "grad_weight"))) return rc;
    if ((rc = resolve_workspace(&ws, &wsb, bwd_ws_bytes(sh), static_cast<hipStream_t>(stream)))) return rc;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  QkBwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.sh = sh;
  p.dy = static_cast<const uint16_t*>(dy);
  p.sdy = s3(dys);
  p.dx = static_cast<uint16_t*>(dx);
  p.sdx = s3(dxs);
  p.x = static_cast<const uint16_t*>(x);
  if (mode & 1) p.sx = s3(xs);
  p.weight = weight;
  p.weight_f32 = (wdt == HARP_QK_F32);
  p.rms = rms;
  p.freqs = freqs;
  p.f_stride_b = fsb;
  p.f_stride_s = fss;
  p.wpart = static_cast<float*>(ws);
  if ((rc = launched(launch_qk_backward(p, mode, st), "QK backward"))) return rc;
  if ((mode & 1) && gw) {
    if ((rc = launched(launch_wgrad_reduce(p.wpart, bwd_blocks(sh), D, gw, gwdt == HARP_QK_F32, st),
                       "weight-gradient reduction")))
      return rc;
  }
  return ok();
}

}  // namespace

extern "C" {

const char* harp_qk_last_error(void) { return g_last_error.c_str(); }

size_t harp_qk_backward_workspace_bytes(int batch, int h_num, int s_len, int h_len) {
  if (check_shape(batch, h_num, s_len, h_len, false)) return (size_t)-1;
  return bwd_ws_bytes(QkShape{batch, h_num, s_len, h_len});
}

int harp_qk_rmsnorm_forward(const void* x, const int64_t* x_strides, void* out, const int64_t* out_strides,
                            const void* weight, int weight_dtype, float* rms, float eps, int batch, int h_num,
                            int s_len, int h_len, void* stream) {
  return forward(1, x, x_strides, weight, weight_dtype, eps, nullptr, 0, 0, out, out_strides, rms, batch, h_num,
                 s_len, h_len, stream);
}

int harp_qk_rmsnorm_backward(const void* x, const int64_t* x_strides, const void* dy, const int64_t* dy_strides,
                             const void* weight, int weight_dtype, const float* rms, void* dx,
                             const int64_t* dx_strides, void* grad_weight, int grad_weight_dtype, int batch, int h_num,
                             int s_len, int h_len, void* workspace, size_t workspace_bytes, void* stream) {
  return backward(1, dy, dy_strides, x, x_strides, weight, weight_dtype, rms, nullptr, 0, 0, dx, dx_strides,
                  grad_weight, grad_weight_dtype, batch, h_num, s_len, h_len, workspace, workspace_bytes, stream);
}

int harp_qk_rope_forward(const void* x, const int64_t* x_strides, const float* freqs, int64_t f_stride_b,
                         int64_t f_stride_s, void* out, const int64_t* out_strides, int batch, int h_num, int s_len,
                         int h_len, void* stream) {
  return forward(2, x, x_strides, nullptr, HARP_QK_BF16, 0.f, freqs, f_stride_b, f_stride_s, out, out_strides,
                 nullptr, batch, h_num, s_len, h_len, stream);
}

int harp_qk_rope_backward(const void* dy, const int64_t* dy_strides, const float* freqs, int64_t f_stride_b,
                          int64_t f_stride_s, void* dx, const int64_t* dx_strides, int batch, int h_num, int s_len,
                          int h_len, void* stream) {
  return backward(2, dy, dy_strides, nullptr, nullptr, nullptr, HARP_QK_BF16, nullptr, freqs, f_stride_b,
                  f_stride_s, dx, dx_strides, nullptr, HARP_QK_BF16, batch, h_num, s_len, h_len, nullptr, 0, stream);
}

int harp_qk_norm_rope_forward(const void* x, const int64_t* x_strides, const void* weight, int weight_dtype,
                              float eps, const float* freqs, int64_t f_stride_b, int64_t f_stride_s, void* out,
                              const int64_t* out_strides, float* rms, int batch, int h_num, int s_len, int h_len,
                              void* stream) {
  return forward(3, x, x_strides, weight, weight_dtype, eps, freqs, f_stride_b, f_stride_s, out, out_strides, rms,
                 batch, h_num, s_len, h_len, stream);
}

int harp_qk_norm_rope_backward(const void* dy, const int64_t* dy_strides, const void* x, const int64_t* x_strides,
                               const void* weight, int weight_dtype, const float* rms, const float* freqs,
                               int64_t f_stride_b, int64_t f_stride_s, void* dx, const int64_t* dx_strides,
                               void* grad_weight, int grad_weight_dtype, int batch, int h_num, int s_len, int h_len,
                               void* workspace, size_t workspace_bytes, void* stream) {
  return backward(3, dy, dy_strides, x, x_strides, weight, weight_dtype, rms, freqs, f_stride_b, f_stride_s, dx,
                  dx_strides, grad_weight, grad_weight_dtype, batch, h_num, s_len, h_len, workspace,
                  workspace_bytes, stream);
}

int harp_qk_norm_rope_backward_noalloc(const void* dy, const int64_t* dy_strides, const void* x,
                                       const int64_t* x_strides, const void* weight, int weight_dtype,
                                       const float* rms, const float* freqs, int64_t f_stride_b, int64_t f_stride_s,
                                       void* dx, const int64_t* dx_strides, void* grad_weight, int grad_weight_dtype,
                                       int batch, int h_num, int s_len, int h_len, void* stream) {
  int rc;
  if ((rc = check_shape(batch, h_num, s_len, h_len, true))) return rc;
  const size_t need = bwd_ws_bytes(QkShape{batch, h_num, s_len, h_len});
  if (need > sizeof(scratch))
    return fail(HARP_QK_EUNSUPPORTED, "the weight-gradient partials need %zu bytes, more than the %zu-byte static scratch",
                need, sizeof(scratch));
  float* ws = nullptr;
  if ((rc = scratch_ptr(&ws))) return rc;
  return backward(3, dy, dy_strides, x, x_strides, weight, weight_dtype, rms, freqs, f_stride_b, f_stride_s, dx,
                  dx_strides, grad_weight, grad_weight_dtype, batch, h_num, s_len, h_len, ws, sizeof(scratch), stream);
}

int harp_qkv_project(const void* x, int64_t ld_x, int batch, int seq, int k_dim, int n_out, const float* freqs,
                     int64_t f_stride_b, int64_t f_stride_s, const harp_qkv_out_t* outs, int n_outs, void* stream) {
  using harp_proj::kHeadDim;
  using harp_proj::kKTile;
  auto aligned16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  constexpr int64_t kMaxLd = (int64_t)1 << 22;  // a 256-row tile spans < 2^32 bytes
  if (!x || !aligned16(x)) return fail(HARP_QK_EINVAL, "x must be a 16-byte aligned device pointer");
  if (batch < 1 || seq < 1) return fail(HARP_QK_EINVAL, "batch=%d and seq=%d must be positive", batch, seq);
  if ((int64_t)batch * seq >= ((int64_t)1 << 31)) return fail(HARP_QK_EUNSUPPORTED, "batch * seq >= 2^31");
  if (k_dim < kKTile || k_dim % kKTile)
    return fail(HARP_QK_EUNSUPPORTED, "k_dim=%d must be a positive multiple of %d", k_dim, kKTile);
  if (n_out < kHeadDim || n_out % kHeadDim)
    return fail(HARP_QK_EUNSUPPORTED, "n_out=%d must be a positive multiple of %d (heads of 128)", n_out, kHeadDim);
  if (ld_x < k_dim || ld_x % 8 || ld_x > kMaxLd)
    return fail(HARP_QK_EINVAL, "ld_x=%lld must be a multiple of 8 in [k_dim, 2^22]", (long long)ld_x);
  if (!outs || n_outs < 1 || n_outs > harp_proj::kMaxOuts)
    return fail(HARP_QK_EINVAL, "outs must hold 1 to %d outputs (got %d)", harp_proj::kMaxOuts, n_outs);
  int rc;
  if (freqs && (rc = check_freqs(freqs, f_stride_b, f_stride_s))) return rc;
  harp_proj::ProjParams p{};
  p.x = (const uint16_t*)x;
  p.ldx = ld_x;
  p.M = batch * seq;
  p.S = seq;
  p.K = k_dim;
  p.heads = n_out / kHeadDim;
  p.freqs = freqs;
  p.f_stride_b = f_stride_b;
  p.f_stride_s = f_stride_s;
  p.n_outs = n_outs;
  for (int i = 0; i < n_outs; ++i) {
    const harp_qkv_out_t& o = outs[i];
    if (!o.weight || !aligned16(o.weight)) return fail(HARP_QK_EINVAL, "outs[%d].weight must be 16-byte aligned", i);
    if (o.ld_weight < k_dim || o.ld_weight % 8 || o.ld_weight > kMaxLd)
      return fail(HARP_QK_EINVAL, "outs[%d].ld_weight=%lld must be a multiple of 8 in [k_dim, 2^22]", i,
                  (long long)o.ld_weight);
    if (!o.y || !aligned16(o.y)) return fail(HARP_QK_EINVAL, "outs[%d].y must be 16-byte aligned", i);
    if (o.ld_y < n_out || o.ld_y % 8)
      return fail(HARP_QK_EINVAL, "outs[%d].ld_y=%lld must be a multiple of 8 >= n_out", i, (long long)o.ld_y);
    if (o.y_lin && !aligned16(o.y_lin)) return fail(HARP_QK_EINVAL, "outs[%d].y_lin must be 16-byte aligned", i);
    if (o.norm_weight) {
      if ((rc = check_weight(o.norm_weight, o.norm_weight_dtype))) return rc;
    } else if (o.y_lin || o.rms) {
      return fail(HARP_QK_EINVAL, "outs[%d]: y_lin and rms belong to outputs with a norm_weight", i);
    }
    harp_proj::ProjOut& q = p.out[i];
    q.w = (const uint16_t*)o.weight;
    q.ldw = o.ld_weight;
    q.y = (uint16_t*)o.y;
    q.ldy = o.ld_y;
    q.y_lin = (uint16_t*)o.y_lin;
    q.norm_w = o.norm_weight;
    q.norm_w_f32 = o.norm_weight && o.norm_weight_dtype == HARP_QK_F32;
    q.eps = o.eps;
    q.rms = o.rms;
  }
  if ((rc = launched(harp_proj::launch_proj(p, (hipStream_t)stream), "qkv projection"))) return rc;
  return ok();
}

}  // extern "C"
