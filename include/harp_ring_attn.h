/*
 * harp_ring_attn.h — C ABI of the MI355X (gfx950) ring-attention block.
 *
 * libharp_ra.so exports exactly the functions declared here.  Every entry
 * point takes plain device pointers, element strides and sizes, runs
 * asynchronously on the given HIP stream (NULL = the default stream), never
 * synchronises the host, and returns an int status (HARP_RA_OK on success);
 * harp_ra_last_error() gives the calling thread's last message.  Arguments
 * are validated on the host before any HIP call is made.
 *
 * Tensors are described as [B, H, T, D] with element strides {b, h, t, d};
 * d must be 1.  The reference's q/k/v and grad tensors are [B,H,T,D] views
 * over token-major [B,T,H,D] storage, i.e. strides {T*H*D, D, H*D, 1}
 * (gemm/ring_attention/torch_ring_attention_ops.cpp:40-67); any strides with
 * d == 1 are accepted.  bf16 tensors need a 16-byte aligned base and b/h/t
 * strides that are multiples of 8 elements.  m_i, l_i and delta are
 * contiguous [B, H, T].
 *
 * Ring semantics on one GPU: the KV side is sp_size chunks (the ring's
 * ranks), each a [B, H, kv_chunk_len, D] view at k_chunks[c] / v_chunks[c]
 * sharing kv_strides.  kv_valid_lens[c] (NULL = all kv_chunk_len) keys of
 * chunk c are valid; the rest are masked out (key-padding mask).  Chunks are
 * visited in ring order c = (s + ring_rank) % sp_size, s = 0..sp_size-1
 * (gemm/ring_attention/ring_attn.cpp:2497).
 */
#ifndef HARP_RING_ATTN_H
#define HARP_RING_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifndef HARP_RA_API
#define HARP_RA_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  HARP_RA_OK = 0,
  HARP_RA_EINVAL = 1,       /* bad pointer, size, stride, alignment or dtype */
  HARP_RA_EUNSUPPORTED = 2, /* valid request this build does not handle (e.g. D > 128) */
  HARP_RA_ENOMEM = 3,       /* workspace too small / allocation failed */
  HARP_RA_ELAUNCH = 4       /* HIP launch or runtime error */
};

enum { HARP_RA_F32 = 0, HARP_RA_BF16 = 1 };

#define HARP_RA_MAX_CHUNKS 16

/*
 * Forward: O = softmax(scale * Q K^T) V over all sp_size chunks, with
 * O written as fp32 (divided by l), m_i (natural-log domain; fp32, or bf16
 * when m_i_dtype == HARP_RA_BF16) and l_i = sum exp(scale*Q K^T - m_i), so
 * that m_i + log(l_i) = LSE exactly for either m_i dtype.  m_i is the
 * reference point of the kernel's exps, at most 8 ln 2 below the row max of
 * scale*Q K^T (the reference's m_i is that max; only m_i + log(l_i) is
 * consumed).  A row without keys gets m_i = -inf, l_i = 0.
 * Replaces: ring_attention_forward(__bf16* Q, __bf16* K, __bf16* V, float* out,
 *   int t_num, int h_num, int h_len, int sp_size, __bf16* m_i, float* l_i,
 *   float scale)  — gemm/ring_attention/ring_attn.cpp:2412-2414, called from
 *   ring_attention_forward_op, torch_ring_attention_ops.cpp:177-215.
 * workspace: harp_ra_forward_workspace_bytes() bytes of device memory, or
 * NULL to use a grow-only per-device buffer owned by the library (calls with
 * a NULL workspace that overlap on one device then race).
 */
HARP_RA_API int harp_ra_forward(const void* q, const int64_t* q_strides,
                    const void* const* k_chunks, const void* const* v_chunks,
                    const int64_t* kv_strides, int kv_chunk_len,
                    const int32_t* kv_valid_lens,
                    float* out, const int64_t* out_strides,
                    void* m_i, int m_i_dtype, float* l_i,
                    int batch, int h_num, int t_num, int h_len,
                    int sp_size, int ring_rank, float scale,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward of one rank's share: dQ for the local rows and Q_local's
 * contribution to dK/dV of every chunk (pad keys receive 0), accumulated in
 * fp32 and written once as fp32 or bf16 (dq_dtype / dkv_dtype).  P is
 * recomputed from LSE = m_i + log(l_i); delta = rowsum(dO * O).
 * Replaces: ring_attention_backward(__bf16* Q, __bf16* grad_Q, __bf16* K,
 *   __bf16* dK, __bf16* V, __bf16* dV, __bf16* grad_out, int t_num,
 *   int h_num, int h_len, int sp_size, float* m_i, float* l_i, float* D,
 *   float scale) — gemm/ring_attention/ring_attn.cpp:2577-2581, called from
 *   ring_attention_backward_op, torch_ring_attention_ops.cpp:217-257.
 * workspace: harp_ra_backward_workspace_bytes() bytes of device memory
 * (256-byte aligned), or NULL to use a grow-only per-device buffer owned by
 * the library (calls with a NULL workspace that overlap on one device then
 * race; that path may call hipMalloc, so graph-captured calls pass one).
 * bf16 dQ, dK and dV at h_len 128 are stored 8 bytes per lane: grad_q and
 * every dK / dV chunk pointer must then be 8-byte aligned and every
 * dq_strides / dkv_strides entry a multiple of 4 elements (HARP_RA_EINVAL
 * otherwise).  fp32 gradients, and bf16 at other head dims, only need the
 * view rules of the other outputs.
 */
HARP_RA_API int harp_ra_backward(const void* q, const int64_t* q_strides,
                     void* grad_q, const int64_t* dq_strides, int dq_dtype,
                     const void* const* k_chunks, const void* const* v_chunks,
                     const int64_t* kv_strides,
                     void* const* dk_chunks, void* const* dv_chunks,
                     const int64_t* dkv_strides, int dkv_dtype,
                     int kv_chunk_len, const int32_t* kv_valid_lens,
                     const void* grad_out, const int64_t* do_strides,
                     const void* m_i, int m_i_dtype, const float* l_i,
                     const float* delta,
                     int batch, int h_num, int t_num, int h_len,
                     int sp_size, int ring_rank, float scale,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * delta[b,h,t] = sum_d grad_out[b,h,t,d] * out[b,h,t,d] in fp32 (grad_out
 * bf16, out fp32).  Replaces the caller-side
 *   D = torch.sum(grad_out.to(torch.float32) * out, dim=-1, keepdim=True)
 * of CPURingAttention.backward, src/models/z_image/module/attn.py:41.
 */
HARP_RA_API int harp_ra_delta(const void* grad_out, const int64_t* do_strides,
                  const float* out, const int64_t* out_strides, float* delta,
                  int batch, int h_num, int t_num, int h_len, void* stream);

/*
 * Device workspace the forward / backward need for these sizes on the
 * current device ((size_t)-1 when the arguments are invalid; 0 = none
 * needed).  The forward keeps all staging in LDS; the backward needs 8 bytes
 * per query row (B*H*T, rounded up to 256 bytes) for its per-query
 * statistics, prepared once per call.  When the forward / dQ grids would
 * leave at least half of the device's compute units idle (fewer than
 * CUs / 2 tiles of 256 queries over B and H) and there are several chunks,
 * the ring steps are split over up to sp_size blocks per tile: the forward
 * then needs n * B*H*T * (4*h_len + 8) bytes for the splits' partial O, m
 * and l, and the backward n * B*H*T * 4*h_len more for the dQ partials (each
 * part rounded up to 256 bytes).  Replaces the reference's grow-only scratch sizing
 * (RingAttnHbmWorkspace::ensure_slot, ring_attn.cpp:620-840, sized at
 * :2428-2450 and :2595-2656).
 */
HARP_RA_API size_t harp_ra_forward_workspace_bytes(int batch, int h_num, int t_num, int h_len, int sp_size,
                                       int kv_chunk_len, const int32_t* kv_valid_lens);
HARP_RA_API size_t harp_ra_backward_workspace_bytes(int batch, int h_num, int t_num, int h_len,
                                        int sp_size, int kv_chunk_len,
                                        const int32_t* kv_valid_lens);

/* Last error message of the calling thread ("" if none).  The reference
 * reports errors with abort_with_message (ring_attn.cpp:1451-1461). */
HARP_RA_API const char* harp_ra_last_error(void);

/*
 * Kernel-level timing for benchmarks (no reference counterpart; the
 * reference's only timing is torch.profiler / RECORD_FUNCTION around whole
 * ops, train.py:422-441).  While enabled, every kernel launch records a HIP
 * event pair on its own stream.  harp_ra_timing_read() must be called after
 * the caller has synchronised those streams; it writes, per kernel kind
 * (HARP_RA_KERNEL_*), the summed milliseconds and launch counts since the
 * last read, then clears them.  Not thread-safe with concurrent calls.
 */
enum {
  HARP_RA_KERNEL_STATS = 0, /* kept for the numbering: the dQ kernel prepares the
                               backward's statistics, so this kind counts no launches */
  HARP_RA_KERNEL_FWD = 1,
  HARP_RA_KERNEL_DELTA = 2,
  HARP_RA_KERNEL_DKDV = 3,
  HARP_RA_KERNEL_DQ = 4,
  HARP_RA_KERNEL_KINDS = 5
};
HARP_RA_API int harp_ra_timing_enable(int enable);
HARP_RA_API int harp_ra_timing_read(double* ms, int* launches, int n_kinds);

/* Library version string. No reference counterpart. */
HARP_RA_API const char* harp_ra_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HARP_RING_ATTN_H */
