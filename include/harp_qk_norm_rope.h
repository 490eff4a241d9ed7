/*
 * harp_qk_norm_rope.h — C ABI of the MI355X (gfx950) kernels for the step
 * before the ring-attention block: per-head RMSNorm of Q and K and the rotary
 * embedding (RoPE), forward and backward, separately and fused.
 *
 * In HARP these run on the CPU as async_op operators (ARM SVE): the model
 * applies norm_q / norm_k and then RoPE to the head-split projections
 * (src/models/z_image/module/attn.py:74-89).  libharp_ra.so exports the
 * functions declared here next to those of harp_ring_attn.h.
 *
 * Conventions (as harp_ring_attn.h): plain device pointers, element strides
 * {b, h, s, d} of [B, H, S, D] views with d == 1, asynchronous on the given
 * HIP stream (NULL = default stream), int status (HARP_QK_OK = 0) and
 * harp_qk_last_error() for the message.  bf16 rows are read and written with
 * 16-byte accesses: bf16 bases 16-byte aligned, b/h/s strides multiples of 8
 * elements, D a multiple of 8 (and even, for RoPE), 8 <= D <= 256; the RMSNorm
 * weight (16-byte aligned) is read with 16-byte loads too.
 *
 * freqs is the RoPE table as fp32 (cos, sin) pairs: torch.view_as_real of
 * the complex [S, D/2] (or [B, S, D/2]) freqs_cis, flattened to [.., S, D];
 * f_stride_b (0 = shared by every batch) and f_stride_s are float strides,
 * multiples of 4, and the base is 16-byte aligned.
 *
 * Numerics follow the reference kernels: fp32 arithmetic, every bf16 result
 * truncated to its high 16 bits (async_rt/csrc/async_op_math.h:24-35),
 * rms = sqrt(sum(x^2)/D + eps) kept in fp32.
 */
#ifndef HARP_QK_NORM_ROPE_H
#define HARP_QK_NORM_ROPE_H

#include <stddef.h>
#include <stdint.h>

#ifndef HARP_QK_API
#define HARP_QK_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  HARP_QK_OK = 0,
  HARP_QK_EINVAL = 1,       /* bad pointer, size, stride, alignment or dtype */
  HARP_QK_EUNSUPPORTED = 2, /* valid request this build does not handle (e.g. D > 256) */
  HARP_QK_ENOMEM = 3,       /* workspace too small / allocation failed */
  HARP_QK_ELAUNCH = 4       /* HIP launch or runtime error */
};

enum { HARP_QK_F32 = 0, HARP_QK_BF16 = 1 };

/*
 * RMSNorm forward: out = (x / rms) * weight, rms = sqrt(mean(x^2) + eps) per
 * row, written to rms[(b*H + h)*S + s] (fp32) when rms is not NULL.  weight is
 * [D] (bf16 or fp32 per weight_dtype) or NULL.
 * Replaces: rmsnorm_forward_out(Tensor input, Tensor weight, Tensor(a!) output,
 *   Tensor(b!) rms, float eps) — async_rt/csrc/rms_norm.cc:447-482 (kernel
 *   :20-105), schema async_rt/csrc/async_op_api.cc:54.
 */
HARP_QK_API int harp_qk_rmsnorm_forward(const void* x, const int64_t* x_strides, void* out,
                                        const int64_t* out_strides, const void* weight, int weight_dtype,
                                        float* rms, float eps, int batch, int h_num, int s_len, int h_len,
                                        void* stream);

/*
 * RMSNorm backward: dx from dy, the forward input x and the saved rms;
 * grad_weight (bf16 or fp32 per grad_weight_dtype, may be NULL) = sum over
 * all rows of dy * x / rms.  workspace: harp_qk_backward_workspace_bytes()
 * bytes of device memory, or NULL for a library-owned one.  The library keeps
 * one such buffer per (device, stream), grown with hipMalloc when a call needs
 * more (after the stream drains): calls on different streams never share it,
 * but a NULL-workspace call allocates and so cannot be captured into a HIP
 * graph; callers that capture pass a workspace.  At most 8 such buffers are
 * kept until the process ends: a NULL-workspace call on a ninth stream first
 * frees the least recently used one, after a device-wide synchronisation.
 * Replaces: rmsnorm_backward_out(Tensor input, Tensor grad_output, Tensor
 *   weight, Tensor rms, Tensor(a!) grad_input, Tensor(b!) grad_weight) —
 *   async_rt/csrc/rms_norm.cc:484-522 (kernel :107-240), schema
 *   async_op_api.cc:55.  The reference binding passes a NULL weight-gradient
 *   pointer to its kernel (rms_norm.cc:500-512) and so returns zeros; this
 *   entry point computes the sum the kernel accumulates (rms_norm.cc:222-229).
 */
HARP_QK_API int harp_qk_rmsnorm_backward(const void* x, const int64_t* x_strides, const void* dy,
                                         const int64_t* dy_strides, const void* weight, int weight_dtype,
                                         const float* rms, void* dx, const int64_t* dx_strides, void* grad_weight,
                                         int grad_weight_dtype, int batch, int h_num, int s_len, int h_len,
                                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * RoPE forward: pairs (x[2i], x[2i+1]) times (cos, sin) of row s as complex
 * numbers.
 * Replaces: rope_forward_impl(Tensor x, Tensor freqs_cis, Tensor(a!) output) —
 *   async_rt/csrc/rope.cc:186-215 (kernel :9-86), schema async_op_api.cc:56.
 */
HARP_QK_API int harp_qk_rope_forward(const void* x, const int64_t* x_strides, const float* freqs, int64_t f_stride_b,
                                     int64_t f_stride_s, void* out, const int64_t* out_strides, int batch, int h_num,
                                     int s_len, int h_len, void* stream);

/*
 * RoPE backward: the same pairs times the conjugate.
 * Replaces: rope_backward_impl(Tensor grad_output, Tensor freqs_cis, Tensor(b!)
 *   grad_x) — async_rt/csrc/rope.cc:217-249 (kernel :88-183), schema
 *   async_op_api.cc:57.
 */
HARP_QK_API int harp_qk_rope_backward(const void* dy, const int64_t* dy_strides, const float* freqs,
                                      int64_t f_stride_b, int64_t f_stride_s, void* dx, const int64_t* dx_strides,
                                      int batch, int h_num, int s_len, int h_len, void* stream);

/*
 * Fused RMSNorm then RoPE in one pass over the rows (read x once, write out
 * once), the intermediate truncated to bf16 exactly as between the two
 * reference operators; rms as harp_qk_rmsnorm_forward.  No reference
 * counterpart as one operator: it replaces the pair norm_q/norm_k ->
 * ApplyRotaryComplexFn of src/models/z_image/module/attn.py:78-89.
 */
HARP_QK_API int harp_qk_norm_rope_forward(const void* x, const int64_t* x_strides, const void* weight,
                                          int weight_dtype, float eps, const float* freqs, int64_t f_stride_b,
                                          int64_t f_stride_s, void* out, const int64_t* out_strides, float* rms,
                                          int batch, int h_num, int s_len, int h_len, void* stream);

/*
 * Fused backward: RoPE backward of dy (truncated to bf16, as the reference's
 * intermediate gradient), then RMSNorm backward against x and rms.  No
 * reference counterpart as one operator (the reverse of the pair above).
 */
HARP_QK_API int harp_qk_norm_rope_backward(const void* dy, const int64_t* dy_strides, const void* x,
                                           const int64_t* x_strides, const void* weight, int weight_dtype,
                                           const float* rms, const float* freqs, int64_t f_stride_b,
                                           int64_t f_stride_s, void* dx, const int64_t* dx_strides,
                                           void* grad_weight, int grad_weight_dtype, int batch, int h_num,
                                           int s_len, int h_len, void* workspace, size_t workspace_bytes,
                                           void* stream);

/*
 * harp_qk_norm_rope_backward without a workspace argument, and allocating
 * nothing: no reference counterpart.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The weight-gradient partials go to a static device
 * array of the library, 2.03 MiB per device (enough for any h_len <= 256),
 * held until the process ends; sizes beyond it return HARP_QK_EUNSUPPORTED.
 * Every call on one device shares that array: calls that overlap on one device
 * (e.g. on two streams) race and must not be issued; calls ordered on one
 * stream are safe.  Everything else as harp_qk_norm_rope_backward.
 */
HARP_QK_API int harp_qk_norm_rope_backward_noalloc(const void* dy, const int64_t* dy_strides, const void* x,
                                                   const int64_t* x_strides, const void* weight, int weight_dtype,
                                                   const float* rms, const float* freqs, int64_t f_stride_b,
                                                   int64_t f_stride_s, void* dx, const int64_t* dx_strides,
                                                   void* grad_weight, int grad_weight_dtype, int batch, int h_num,
                                                   int s_len, int h_len, void* stream);

/* Device workspace the two backward entry points with RMSNorm need
 * ((size_t)-1 when the arguments are invalid): the weight-gradient partial
 * sums of up to 2048 row blocks and their 64-row group sums, at most
 * (2048 + 32) x h_len floats. */
HARP_QK_API size_t harp_qk_backward_workspace_bytes(int batch, int h_num, int s_len, int h_len);

/*
 * The producer of the ring-attention block's q, k and v in one launch: up to
 * three projections y = x W^T (nn.Linear without bias) of the hidden states
 * x [batch * seq, k_dim] (row stride ld_x, token b * seq + s), each written
 * as y [batch * seq, n_out] (row stride ld_y): the token-major [B, S, H, 128]
 * layout the ring-attention operators read as [B, H, S, 128] views.
 * For an output with a norm_weight, every 128-feature head of the product,
 * rounded to bf16 to nearest (as the Linear layer's output), is normalised
 * as by harp_qk_norm_rope_forward (RMSNorm with eps and the [128] weight,
 * then RoPE with row s of freqs when freqs is not NULL; fp32 arithmetic, bf16
 * results truncated) before its only store; y_lin (may be NULL) receives the
 * bf16 product itself and rms (may be NULL) the fp32 rms at
 * (b * (n_out / 128) + h) * seq + s, the two tensors
 * harp_qk_norm_rope_backward takes.  An output without norm_weight is the
 * plain product (its y_lin and rms must be NULL).
 * Requirements: n_out a positive multiple of 128 and k_dim of 64 (else
 * HARP_QK_EUNSUPPORTED); k_dim <= ld_x, ld_weight <= 2^22 and n_out <= ld_y,
 * all multiples of 8 elements; x, weights, y, y_lin, norm weights 16-byte
 * aligned; batch * seq < 2^31.  freqs as for harp_qk_rope_forward with
 * D = 128 (pair p of token (b, s) at freqs + b*f_stride_b + s*f_stride_s + 2p).
 * Outputs must not overlap each other or the inputs.  Asynchronous on stream;
 * no workspace, no allocation.
 * Replaces: the three projections and the norm_q / norm_k and RoPE calls of
 *   Z_Attention.forward, src/models/z_image/module/attn.py:69-89 (nn.Linear,
 *   then async_rt/csrc/rms_norm.cc:20-105 and rope.cc:9-86 on the CPU).
 */
typedef struct harp_qkv_out {
  const void* weight;      /* [n_out, k_dim] bf16, row stride ld_weight */
  int64_t ld_weight;
  void* y;                 /* [batch * seq, n_out] bf16, row stride ld_y */
  int64_t ld_y;
  void* y_lin;             /* NULL, or like y: the bf16 product before RMSNorm */
  const void* norm_weight; /* NULL (plain projection) or [128] */
  int norm_weight_dtype;   /* HARP_QK_BF16 or HARP_QK_F32 */
  float eps;
  float* rms;              /* NULL or [batch * (n_out / 128) * seq] fp32 */
} harp_qkv_out_t;

HARP_QK_API int harp_qkv_project(const void* x, int64_t ld_x, int batch, int seq, int k_dim, int n_out,
                                 const float* freqs, int64_t f_stride_b, int64_t f_stride_s,
                                 const harp_qkv_out_t* outs, int n_outs, void* stream);

/* Last error message of the calling thread ("" if none). */
HARP_QK_API const char* harp_qk_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HARP_QK_NORM_ROPE_H */
