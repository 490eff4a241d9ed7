// C ABI of libharp_ra.so: argument validation, kernel sequencing and optional
// kernel timing for the ring-attention block.  See include/harp_ring_attn.h.
//
// Host flow mirrors the reference's operator bodies:
//   forward  (ring_attn.cpp:2412-2575): the reference packs K/V/Q into SME
//            panels (:2452-2485) and then loops over ring steps (:2488-2568)
//            and normalises (:2569-2573); here a single fused kernel launch
//            streams every chunk's K/V tiles through LDS (no panel copies).
//   backward (ring_attn.cpp:2577-2829): packs (:2664-2717), per-step S/dP
//            recompute and dQ/dK/dV GEMMs (:2723-2816), dQ owner sum
//            (:2817-2828); here a dK/dV kernel (KV-stationary, like the
//            reference) and a dQ kernel whose fp32 register accumulators
//            replace the dQ slot reduction.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/harp_ring_attn.h"
#include "ra_kernels.h"

using namespace harp_ra;

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
  return HARP_RA_OK;
}


bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// bf16 operand that is read with 16-byte vector loads.  Its rows are walked
// through buffer ranges of rows x row stride, so a row stride below D (0 for
// an expanded view) would cut every row short: rejected.  B and H strides may
// be 0 (a broadcast input).
int check_bf16_view(const void* p, const int64_t* s, int D, const char* name) {
  if (!p) return fail(HARP_RA_EINVAL, "%s is NULL", name);
  if (!s) return fail(HARP_RA_EINVAL, "%s strides are NULL", name);
  if (!aligned16(p)) return fail(HARP_RA_EINVAL, "%s must be 16-byte aligned", name);
  if (s[3] != 1) return fail(HARP_RA_EINVAL, "%s must have unit stride in D (got %lld)", name, (long long)s[3]);
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || s[i] % 8 != 0)
      return fail(HARP_RA_EINVAL, "%s stride[%d]=%lld must be a non-negative multiple of 8 elements", name, i,
                  (long long)s[i]);
  if (s[2] < D)
    return fail(HARP_RA_EINVAL, "%s row stride %lld is below D=%d: rows would overlap", name, (long long)s[2], D);
  return HARP_RA_OK;
}

// fp32 input read element by element (the forward's out, for the delta)
int check_plain_view(const void* p, const int64_t* s, const char* name) {
  if (!p) return fail(HARP_RA_EINVAL, "%s is NULL", name);
  if (!s) return fail(HARP_RA_EINVAL, "%s strides are NULL", name);
  if (s[3] != 1) return fail(HARP_RA_EINVAL, "%s must have unit stride in D (got %lld)", name, (long long)s[3]);
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0) return fail(HARP_RA_EINVAL, "%s stride[%d] must be non-negative", name, i);
  return HARP_RA_OK;
}

// Output view [B, H, rows, D] written element by element: unit D stride, and
// no two elements at one address (else stores from different threads race).
// Sufficient test: with the dims of extent > 1 sorted by stride, each stride
// exceeds the span of the smaller ones.
int check_out_view(const void* p, const int64_t* s, int B, int H, int rows, int D, const char* name) {
  if (!p) return fail(HARP_RA_EINVAL, "%s is NULL", name);
  if (!s) return fail(HARP_RA_EINVAL, "%s strides are NULL", name);
  if (s[3] != 1) return fail(HARP_RA_EINVAL, "%s must have unit stride in D (got %lld)", name, (long long)s[3]);
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0) return fail(HARP_RA_EINVAL, "%s stride[%d] must be non-negative", name, i);
  const int64_t ext[4] = {B, H, rows, D};
  int idx[4], n = 0;
  for (int i = 0; i < 4; ++i)
    if (ext[i] > 1) idx[n++] = i;
  for (int i = 1; i < n; ++i)  // insertion sort by stride
    for (int j = i; j > 0 && s[idx[j]] < s[idx[j - 1]]; --j) std::swap(idx[j], idx[j - 1]);
  int64_t span = 0;  // largest offset reachable through the dims so far
  for (int i = 0; i < n; ++i) {
    if (s[idx[i]] <= span)
      return fail(HARP_RA_EINVAL, "%s strides make elements overlap (stride[%d]=%lld)", name, idx[i],
                  (long long)s[idx[i]]);
    span += (ext[idx[i]] - 1) * s[idx[i]];
  }
  return HARP_RA_OK;
}

// Streamed operands are read through 32-bit buffer offsets: every [rows][D]
// view the kernels walk (one (b, h) of a chunk, of q or of grad_out) must
// span less than 2^31 bytes, counted over at least 128 rows: the copies of a
// 128-row tile form their offsets before the buffer's range check zero-fills
// the rows past a short view, so those offsets must not wrap either.
int check_extent(int rows, const int64_t* s, const char* name) {
  const int64_t span_rows = rows > 128 ? rows : 128;
  if (span_rows * s[2] * 2 >= ((int64_t)1 << 31))
    return fail(HARP_RA_EUNSUPPORTED,
                "%s: %d rows (at least 128 counted) x row stride %lld elements exceeds the 2 GiB buffer range", name,
                rows, (long long)s[2]);
  return HARP_RA_OK;
}

int check_dims(int batch, int h_num, int t_num, int h_len) {
  if (batch < 1 || h_num < 1 || t_num < 1 || h_len < 1)
    return fail(HARP_RA_EINVAL, "sizes must be positive (B=%d H=%d T=%d D=%d)", batch, h_num, t_num, h_len);
  if (h_len % 8 != 0) return fail(HARP_RA_EUNSUPPORTED, "head dim D=%d must be a multiple of 8", h_len);
  if (h_len > 128) return fail(HARP_RA_EUNSUPPORTED, "head dim D=%d > 128 is not supported", h_len);
  if (batch > 65535 || h_num > 65535) return fail(HARP_RA_EUNSUPPORTED, "B and H must be <= 65535");
  return HARP_RA_OK;
}

// Chunk geometry shared by forward/backward/workspace sizing.
struct Geometry {
  int n = 0;
  int len[kMaxChunks] = {};
};

int make_geometry(int sp_size, int kv_chunk_len, const int32_t* kv_valid_lens, Geometry* g) {
  if (sp_size < 1 || sp_size > HARP_RA_MAX_CHUNKS)
    return fail(HARP_RA_EINVAL, "sp_size=%d must be in [1, %d]", sp_size, HARP_RA_MAX_CHUNKS);
  if (kv_chunk_len < 1) return fail(HARP_RA_EINVAL, "kv_chunk_len=%d must be positive", kv_chunk_len);
  if (kv_chunk_len > (1 << 26)) return fail(HARP_RA_EUNSUPPORTED, "kv_chunk_len=%d is too large", kv_chunk_len);
  g->n = sp_size;
  for (int c = 0; c < sp_size; ++c) {
    const int len = kv_valid_lens ? kv_valid_lens[c] : kv_chunk_len;
    if (len < 0 || len > kv_chunk_len)
      return fail(HARP_RA_EINVAL, "kv_valid_lens[%d]=%d must be in [0, kv_chunk_len=%d]", c, len, kv_chunk_len);
    g->len[c] = len;
  }
  return HARP_RA_OK;
}

size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }

// Compute units of the current device (0 if the query fails).
int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

// KV splits of the forward and dQ kernels.  Their grids have one 8-wave
// block (one CU) per 256-query tile and (b, h); when that leaves at least
// half of the CUs idle, each tile's ring steps are split over up to N blocks
// (never more splits than chunks), whose partial results are merged after.
int kv_splits(int batch, int h_num, int t_num, const Geometry& g) {
  const int64_t blocks = (int64_t)((t_num + kQueryBlockRows - 1) / kQueryBlockRows) * h_num * batch;
  const int cus = device_cus();
  if (g.n < 2 || cus < 2 || blocks * 2 > cus) return 1;
  const int64_t fill = cus / blocks;
  return (int)(fill < g.n ? fill : g.n);
}

// Forward: no scratch, except the KV splits' partial O (fp32 [n][B,H,T,D])
// and row statistics (fp32 m and l, [n][B,H,T] each).
struct FwdLayout {
  int n_split;
  size_t o, m, l, bytes;  // byte offsets
};
FwdLayout fwd_layout(int batch, int h_num, int t_num, int h_len, const Geometry& g) {
  FwdLayout w{kv_splits(batch, h_num, t_num, g), 0, 0, 0, 0};
  if (w.n_split < 2) return w;
  const size_t rows = (size_t)batch * h_num * t_num;
  w.m = round256(sizeof(float) * w.n_split * rows * h_len);
  w.l = w.m + round256(sizeof(float) * w.n_split * rows);
  w.bytes = w.l + round256(sizeof(float) * w.n_split * rows);
  return w;
}
size_t fwd_ws(int batch, int h_num, int t_num, int h_len, const Geometry& g) {
  return fwd_layout(batch, h_num, t_num, h_len, g).bytes;
}

// Backward: the per-query statistics, written once per call by the dQ
// kernel for the dK/dV kernel, in two fp32 planes of B*H*T rows; then, with
// KV splits, the dQ kernel's partials (fp32 [n][B,H,T,D]).
struct BwdLayout {
  int n_split;
  size_t stats, dq, bytes;  // byte offsets
};
BwdLayout bwd_layout(int batch, int h_num, int t_num, int h_len, const Geometry& g) {
  BwdLayout w{kv_splits(batch, h_num, t_num, g), 0, 0, 0};
  const size_t rows = (size_t)batch * h_num * t_num;
  w.dq = round256(2 * sizeof(float) * rows);
  w.bytes = w.dq + (w.n_split > 1 ? round256(sizeof(float) * w.n_split * rows * h_len) : 0);
  return w;
}
size_t bwd_ws(int batch, int h_num, int t_num, int h_len, const Geometry& g) {
  return bwd_layout(batch, h_num, t_num, h_len, g).bytes;
}

// Library-owned grow-only workspace, one per device (used when the caller
// passes workspace == NULL).
struct OwnedWorkspace {
  std::mutex mu;
  void* ptr[64] = {};
  size_t bytes[64] = {};
};
OwnedWorkspace& owned() {
  static OwnedWorkspace w;
  return w;
}

int resolve_workspace(void** ws, size_t* ws_bytes, size_t need) {
  if (need == 0) return HARP_RA_OK;
  if (*ws) {
    if (*ws_bytes < need)
      return fail(HARP_RA_ENOMEM, "workspace of %zu bytes is smaller than the %zu bytes needed", *ws_bytes, need);
    if ((reinterpret_cast<uintptr_t>(*ws) & 255u) != 0) return fail(HARP_RA_EINVAL, "workspace must be 256-byte aligned");
    return HARP_RA_OK;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(HARP_RA_ELAUNCH, "hipGetDevice failed");
  OwnedWorkspace& w = owned();
  std::lock_guard<std::mutex> lock(w.mu);
  if (w.bytes[dev] < need) {
    if (w.ptr[dev]) {
      // earlier calls may still use the old buffer on any stream
      if (hipDeviceSynchronize() != hipSuccess) return fail(HARP_RA_ELAUNCH, "hipDeviceSynchronize failed");
      (void)hipFree(w.ptr[dev]);
      w.ptr[dev] = nullptr;
      w.bytes[dev] = 0;
    }
    const size_t grow = need + need / 4;  // grow-only with headroom, like the reference's x1.25 slots
    if (hipMalloc(&w.ptr[dev], grow) != hipSuccess) {
      w.ptr[dev] = nullptr;
      return fail(HARP_RA_ENOMEM, "hipMalloc of %zu workspace bytes failed", grow);
    }
    w.bytes[dev] = grow;
  }
  *ws = w.ptr[dev];
  *ws_bytes = w.bytes[dev];
  return HARP_RA_OK;
}

// Optional per-kernel event timing (harp_ra_timing_enable / _read).
struct Timing {
  bool on = false;
  struct Rec {
    int kind;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> pool;
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Timing& timing() {
  static Timing t;
  return t;
}

// Brackets one kernel launch with timing events when timing is enabled.
struct TimedLaunch {
  int kind;
  hipStream_t st;
  hipEvent_t a = nullptr, b = nullptr;
  TimedLaunch(int k, hipStream_t s) : kind(k), st(s) {
    Timing& t = timing();
    if (!t.on) return;
    a = t.get();
    b = t.get();
    if (a && b) (void)hipEventRecord(a, st);
  }
  ~TimedLaunch() {
    if (!a || !b) return;
    (void)hipEventRecord(b, st);
    timing().recs.push_back({kind, a, b});
  }
};

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(HARP_RA_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HARP_RA_OK;
}

}  // namespace

extern "C" {

const char* harp_ra_last_error(void) { return g_last_error.c_str(); }

const char* harp_ra_version(void) { return "harp_ra 0.1.0 (gfx950)"; }

int harp_ra_timing_enable(int enable) {
  timing().on = (enable != 0);
  return ok();
}

int harp_ra_timing_read(double* ms, int* launches, int n_kinds) {
  if (!ms || !launches || n_kinds < 1) return fail(HARP_RA_EINVAL, "timing_read needs output arrays");
  for (int i = 0; i < n_kinds; ++i) {
    ms[i] = 0.0;
    launches[i] = 0;
  }
  Timing& t = timing();
  int rc = HARP_RA_OK;
  for (auto& r : t.recs) {
    float e = 0.f;
    if (hipEventElapsedTime(&e, r.a, r.b) != hipSuccess) rc = HARP_RA_ELAUNCH;
    if (r.kind < n_kinds) {
      ms[r.kind] += e;
      launches[r.kind] += 1;
    }
    t.pool.push_back(r.a);
    t.pool.push_back(r.b);
  }
  t.recs.clear();
  if (rc) return fail(rc, "hipEventElapsedTime failed (were the streams synchronised?)");
  return ok();
}

size_t harp_ra_forward_workspace_bytes(int batch, int h_num, int t_num, int h_len, int sp_size, int kv_chunk_len,
                                       const int32_t* kv_valid_lens) {
  Geometry g;
  if (check_dims(batch, h_num, t_num, h_len) != HARP_RA_OK) return SIZE_MAX;
  if (make_geometry(sp_size, kv_chunk_len, kv_valid_lens, &g) != HARP_RA_OK) return SIZE_MAX;
  return fwd_ws(batch, h_num, t_num, h_len, g);
}

size_t harp_ra_backward_workspace_bytes(int batch, int h_num, int t_num, int h_len, int sp_size, int kv_chunk_len,
                                        const int32_t* kv_valid_lens) {
  Geometry g;
  if (check_dims(batch, h_num, t_num, h_len) != HARP_RA_OK) return SIZE_MAX;
  if (make_geometry(sp_size, kv_chunk_len, kv_valid_lens, &g) != HARP_RA_OK) return SIZE_MAX;
  return bwd_ws(batch, h_num, t_num, h_len, g);
}

int harp_ra_forward(const void* q, const int64_t* q_strides, const void* const* k_chunks,
                    const void* const* v_chunks, const int64_t* kv_strides, int kv_chunk_len,
                    const int32_t* kv_valid_lens, float* out, const int64_t* out_strides, void* m_i, int m_i_dtype,
                    float* l_i, int batch, int h_num, int t_num, int h_len, int sp_size, int ring_rank, float scale,
                    void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_dims(batch, h_num, t_num, h_len))) return rc;
  Geometry g;
  if ((rc = make_geometry(sp_size, kv_chunk_len, kv_valid_lens, &g))) return rc;
  if (ring_rank < 0 || ring_rank >= sp_size)
    return fail(HARP_RA_EINVAL, "ring_rank=%d must be in [0, sp_size=%d)", ring_rank, sp_size);
  if (!std::isfinite(scale) || !(scale > 0.f)) return fail(HARP_RA_EINVAL, "scale must be finite and positive");
  if ((rc = check_bf16_view(q, q_strides, h_len, "q"))) return rc;
  if (!k_chunks || !v_chunks) return fail(HARP_RA_EINVAL, "k_chunks / v_chunks are NULL");
  for (int c = 0; c < sp_size; ++c) {
    if ((rc = check_bf16_view(k_chunks[c], kv_strides, h_len, "k chunk"))) return rc;
    if ((rc = check_bf16_view(v_chunks[c], kv_strides, h_len, "v chunk"))) return rc;
  }
  if ((rc = check_out_view(out, out_strides, batch, h_num, t_num, h_len, "out"))) return rc;
  if ((rc = check_extent(kv_chunk_len, kv_strides, "k/v chunk"))) return rc;
  if (!m_i || !l_i) return fail(HARP_RA_EINVAL, "m_i / l_i are NULL");
  if (m_i_dtype != HARP_RA_F32 && m_i_dtype != HARP_RA_BF16) return fail(HARP_RA_EINVAL, "m_i_dtype must be F32 or BF16");

  const FwdLayout wl = fwd_layout(batch, h_num, t_num, h_len, g);
  if ((rc = resolve_workspace(&workspace, &workspace_bytes, wl.bytes))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);

  FwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = static_cast<const bf16*>(q);
  p.sqb = q_strides[0];
  p.sqh = q_strides[1];
  p.sqt = q_strides[2];
  p.skb = kv_strides[0];
  p.skh = kv_strides[1];
  p.skt = kv_strides[2];
  p.out = out;
  p.sob = out_strides[0];
  p.soh = out_strides[1];
  p.sot = out_strides[2];
  p.m = m_i;
  p.m_bf16 = (m_i_dtype == HARP_RA_BF16);
  p.l = l_i;
  p.B = batch;
  p.H = h_num;
  p.T = t_num;
  p.D = h_len;
  p.scale = scale;
  p.ct.n = sp_size;
  for (int c = 0; c < sp_size; ++c) {
    p.ct.k[c] = static_cast<const bf16*>(k_chunks[c]);
    p.ct.v[c] = static_cast<const bf16*>(v_chunks[c]);
    p.ct.len[c] = g.len[c];
    p.ct.order[c] = (c + ring_rank) % sp_size;
  }
  p.n_split = wl.n_split;
  FwdMergeParams mp;
  std::memset(&mp, 0, sizeof(mp));
  if (wl.n_split > 1) {
    // the kernel writes per-split partials (fp32, [n][B,H,T,D] and [n][B,H,T]);
    // the merge writes out / m_i / l_i
    char* ws = static_cast<char*>(workspace);
    mp.part_o = reinterpret_cast<const float*>(ws + wl.o);
    mp.part_m = reinterpret_cast<const float*>(ws + wl.m);
    mp.part_l = reinterpret_cast<const float*>(ws + wl.l);
    mp.n_split = wl.n_split;
    mp.out = out;
    mp.sob = p.sob;
    mp.soh = p.soh;
    mp.sot = p.sot;
    mp.m = m_i;
    mp.m_bf16 = p.m_bf16;
    mp.l = l_i;
    mp.B = batch;
    mp.H = h_num;
    mp.T = t_num;
    mp.D = h_len;
    p.out = reinterpret_cast<float*>(ws + wl.o);
    p.sot = h_len;
    p.soh = (int64_t)t_num * h_len;
    p.sob = (int64_t)h_num * p.soh;
    p.split_o = (int64_t)batch * p.sob;
    p.m = ws + wl.m;
    p.m_bf16 = 0;
    p.l = reinterpret_cast<float*>(ws + wl.l);
    p.split_ml = (int64_t)batch * h_num * t_num;
  }
  {
    TimedLaunch tl(HARP_RA_KERNEL_FWD, st);  // the merge is timed with the forward
    if ((rc = launched(launch_fwd(p, st), "forward"))) return rc;
    if (wl.n_split > 1 && (rc = launched(launch_fwd_merge(mp, st), "forward merge"))) return rc;
  }
  return ok();
}

int harp_ra_delta(const void* grad_out, const int64_t* do_strides, const float* out, const int64_t* out_strides,
                  float* delta, int batch, int h_num, int t_num, int h_len, void* stream) {
  int rc;
  if ((rc = check_dims(batch, h_num, t_num, h_len))) return rc;
  if ((rc = check_bf16_view(grad_out, do_strides, h_len, "grad_out"))) return rc;
  if ((rc = check_plain_view(out, out_strides, "out"))) return rc;
  if (!delta) return fail(HARP_RA_EINVAL, "delta is NULL");
  DeltaParams p;
  p.dout = static_cast<const bf16*>(grad_out);
  p.sdb = do_strides[0];
  p.sdh = do_strides[1];
  p.sdt = do_strides[2];
  p.out = out;
  p.sob = out_strides[0];
  p.soh = out_strides[1];
  p.sot = out_strides[2];
  p.delta = delta;
  p.B = batch;
  p.H = h_num;
  p.T = t_num;
  p.D = h_len;
  {
    TimedLaunch tl(HARP_RA_KERNEL_DELTA, static_cast<hipStream_t>(stream));
    if ((rc = launched(launch_delta(p, static_cast<hipStream_t>(stream)), "delta"))) return rc;
  }
  return ok();
}

int harp_ra_backward(const void* q, const int64_t* q_strides, void* grad_q, const int64_t* dq_strides, int dq_dtype,
                     const void* const* k_chunks, const void* const* v_chunks, const int64_t* kv_strides,
                     void* const* dk_chunks, void* const* dv_chunks, const int64_t* dkv_strides, int dkv_dtype,
                     int kv_chunk_len, const int32_t* kv_valid_lens, const void* grad_out, const int64_t* do_strides,
                     const void* m_i, int m_i_dtype, const float* l_i, const float* delta, int batch, int h_num,
                     int t_num, int h_len, int sp_size, int ring_rank, float scale, void* workspace,
                     size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_dims(batch, h_num, t_num, h_len))) return rc;
  Geometry g;
  if ((rc = make_geometry(sp_size, kv_chunk_len, kv_valid_lens, &g))) return rc;
  if (ring_rank < 0 || ring_rank >= sp_size)
    return fail(HARP_RA_EINVAL, "ring_rank=%d must be in [0, sp_size=%d)", ring_rank, sp_size);
  if (!std::isfinite(scale) || !(scale > 0.f)) return fail(HARP_RA_EINVAL, "scale must be finite and positive");
  if ((rc = check_bf16_view(q, q_strides, h_len, "q"))) return rc;
  if ((rc = check_bf16_view(grad_out, do_strides, h_len, "grad_out"))) return rc;
  if ((rc = check_out_view(grad_q, dq_strides, batch, h_num, t_num, h_len, "grad_q"))) return rc;
  if (dq_dtype != HARP_RA_F32 && dq_dtype != HARP_RA_BF16) return fail(HARP_RA_EINVAL, "dq_dtype must be F32 or BF16");
  // at head dim 128 the dQ kernel stores bf16 rows four elements (8 bytes)
  // per lane store too
  if (dq_dtype == HARP_RA_BF16 && h_len == 128) {
    for (int i = 0; i < 3; ++i)
      if (dq_strides[i] % 4 != 0)
        return fail(HARP_RA_EINVAL, "bf16 grad_q stride[%d]=%lld must be a multiple of 4 elements at h_len 128", i,
                    (long long)dq_strides[i]);
    if ((reinterpret_cast<uintptr_t>(grad_q) & 7u) != 0)
      return fail(HARP_RA_EINVAL, "bf16 grad_q must be 8-byte aligned at h_len 128");
  }
  if (dkv_dtype != HARP_RA_F32 && dkv_dtype != HARP_RA_BF16)
    return fail(HARP_RA_EINVAL, "dkv_dtype must be F32 or BF16");
  if (!k_chunks || !v_chunks || !dk_chunks || !dv_chunks) return fail(HARP_RA_EINVAL, "chunk pointer arrays are NULL");
  // at head dim 128 the dK / dV kernel writes bf16 rows four elements (8
  // bytes) per lane store; the kernel for other head dims stores elements
  const bool dkv_wide = dkv_dtype == HARP_RA_BF16 && h_len == 128;
  if (dkv_wide)
    for (int i = 0; i < 3; ++i)
      if (dkv_strides && dkv_strides[i] % 4 != 0)
        return fail(HARP_RA_EINVAL, "bf16 dK / dV stride[%d]=%lld must be a multiple of 4 elements at h_len 128", i,
                    (long long)dkv_strides[i]);
  for (int c = 0; c < sp_size; ++c) {
    if ((rc = check_bf16_view(k_chunks[c], kv_strides, h_len, "k chunk"))) return rc;
    if ((rc = check_bf16_view(v_chunks[c], kv_strides, h_len, "v chunk"))) return rc;
    if ((rc = check_out_view(dk_chunks[c], dkv_strides, batch, h_num, kv_chunk_len, h_len, "dK chunk"))) return rc;
    if ((rc = check_out_view(dv_chunks[c], dkv_strides, batch, h_num, kv_chunk_len, h_len, "dV chunk"))) return rc;
    if (dkv_wide &&
        ((reinterpret_cast<uintptr_t>(dk_chunks[c]) | reinterpret_cast<uintptr_t>(dv_chunks[c])) & 7u) != 0)
      return fail(HARP_RA_EINVAL, "bf16 dK / dV chunks must be 8-byte aligned at h_len 128");
  }
  if ((rc = check_extent(kv_chunk_len, kv_strides, "k/v chunk"))) return rc;
  if ((rc = check_extent(t_num, q_strides, "q"))) return rc;
  if ((rc = check_extent(t_num, do_strides, "grad_out"))) return rc;
  if (!m_i || !l_i || !delta) return fail(HARP_RA_EINVAL, "m_i / l_i / delta are NULL");
  if (m_i_dtype != HARP_RA_F32 && m_i_dtype != HARP_RA_BF16) return fail(HARP_RA_EINVAL, "m_i_dtype must be F32 or BF16");

  const BwdLayout wl = bwd_layout(batch, h_num, t_num, h_len, g);
  if ((rc = resolve_workspace(&workspace, &workspace_bytes, wl.bytes))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);

  BwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = static_cast<const bf16*>(q);
  p.sqb = q_strides[0];
  p.sqh = q_strides[1];
  p.sqt = q_strides[2];
  p.dout = static_cast<const bf16*>(grad_out);
  p.sdb = do_strides[0];
  p.sdh = do_strides[1];
  p.sdt = do_strides[2];
  p.skb = kv_strides[0];
  p.skh = kv_strides[1];
  p.skt = kv_strides[2];
  p.sdkb = dkv_strides[0];
  p.sdkh = dkv_strides[1];
  p.sdkt = dkv_strides[2];
  p.dkv_f32 = (dkv_dtype == HARP_RA_F32);
  p.dq = grad_q;
  p.sdqb = dq_strides[0];
  p.sdqh = dq_strides[1];
  p.sdqt = dq_strides[2];
  p.dq_f32 = (dq_dtype == HARP_RA_F32);
  p.m = m_i;
  p.m_bf16 = (m_i_dtype == HARP_RA_BF16);
  p.l = l_i;
  p.delta = delta;
  p.B = batch;
  p.H = h_num;
  p.T = t_num;
  p.D = h_len;
  p.scale = scale;
  p.inv_scale = 1.f / scale;
  p.ct.n = sp_size;
  int key_tiles = 0;
  for (int c = 0; c < sp_size; ++c) {
    p.ct.k[c] = static_cast<const bf16*>(k_chunks[c]);
    p.ct.v[c] = static_cast<const bf16*>(v_chunks[c]);
    p.ct.dk[c] = static_cast<bf16*>(dk_chunks[c]);
    p.ct.dv[c] = static_cast<bf16*>(dv_chunks[c]);
    p.ct.len[c] = g.len[c];
    p.ct.order[c] = (c + ring_rank) % sp_size;
    p.ct.tile0[c] = key_tiles;
    p.ct_rows[c] = kv_chunk_len;
    key_tiles += (kv_chunk_len + kDkdvBlockKeys - 1) / kDkdvBlockKeys;
  }
  p.n_key_tiles = key_tiles;
  if ((int64_t)key_tiles * h_num * batch > INT32_MAX || (int64_t)((t_num + 127) / 128) * h_num * batch > INT32_MAX)
    return fail(HARP_RA_EUNSUPPORTED, "grid too large");
  char* ws = static_cast<char*>(workspace);
  p.stats = reinterpret_cast<float*>(ws + wl.stats);
  p.n_split = 1;
  // dQ first: it writes the per-query statistics planes the dK/dV kernel reads
  BwdParams pk = p;
  DqMergeParams mp;
  std::memset(&mp, 0, sizeof(mp));
  if (wl.n_split > 1) {
    // per-split fp32 partials [n][B,H,T,D], summed into grad_q by the merge
    mp.part = reinterpret_cast<const float*>(ws + wl.dq);
    mp.n_split = wl.n_split;
    mp.dq = grad_q;
    mp.sdqb = p.sdqb;
    mp.sdqh = p.sdqh;
    mp.sdqt = p.sdqt;
    mp.dq_f32 = p.dq_f32;
    mp.B = batch;
    mp.H = h_num;
    mp.T = t_num;
    mp.D = h_len;
    p.n_split = wl.n_split;
    p.dq = ws + wl.dq;
    p.dq_f32 = 1;
    p.sdqt = h_len;
    p.sdqh = (int64_t)t_num * h_len;
    p.sdqb = (int64_t)h_num * p.sdqh;
    p.split_dq = (int64_t)batch * p.sdqb;
  }
  {
    TimedLaunch tl(HARP_RA_KERNEL_DQ, st);  // the merge is timed with the dQ kernel
    if ((rc = launched(launch_dq(p, st), "dQ"))) return rc;
    if (wl.n_split > 1 && (rc = launched(launch_dq_merge(mp, st), "dQ merge"))) return rc;
  }
  {
    TimedLaunch tl(HARP_RA_KERNEL_DKDV, st);
    if ((rc = launched(launch_dkdv(pk, st), "dK/dV"))) return rc;
  }
  return ok();
}

}  // extern "C"
