// Parameter blocks and launchers of the QK-RMSNorm / RoPE kernels
// (internal to libharp_ra.so; the C ABI is include/harp_qk_norm_rope.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace harp_qk {

struct QkShape {
  int B, H, S, D;
};
struct Strides4 {
  int64_t b, h, s;  // element strides of a [B, H, S, D] view (D stride 1)
};

struct QkFwdParams {
  QkShape sh;
  const uint16_t* x;  // bf16
  Strides4 sx;
  uint16_t* out;      // bf16
  Strides4 so;
  const void* weight;  // RMSNorm weight [D] (bf16, or fp32 if weight_f32), NULL = none
  int weight_f32;
  float eps;
  float* rms;          // [B*H*S] fp32, written by RMSNorm (NULL: not kept)
  const float* freqs;  // RoPE table, fp32 (cos, sin) pairs
  int64_t f_stride_b, f_stride_s;
};

struct QkBwdParams {
  QkShape sh;
  const uint16_t* dy;  // gradient of the op's output, bf16
  Strides4 sdy;
  uint16_t* dx;        // gradient of the op's input, bf16
  Strides4 sdx;
  const uint16_t* x;   // RMSNorm input (bf16)
  Strides4 sx;
  const void* weight;
  int weight_f32;
  const float* rms;    // saved by the forward
  const float* freqs;
  int64_t f_stride_b, f_stride_s;
  float* wpart;        // [blocks][D] fp32 weight-gradient partials, then the
                       // reduction's group sums (workspace, bwd_workspace_floats)
};

// Blocks of the backward kernel (each a contiguous range of rows); bounds the
// weight-gradient workspace (one partial row of D floats per block).
constexpr int kQkBwdMaxBlocks = 2048;
int bwd_blocks(const QkShape& sh);
// Partial rows per group of the first level of the weight-gradient reduction;
// the workspace holds the partials and then one row per group.
constexpr int kWgGroupRows = 64;
inline size_t bwd_workspace_floats(const QkShape& sh) {
  const size_t nblk = (size_t)bwd_blocks(sh);
  return (nblk + (nblk + kWgGroupRows - 1) / kWgGroupRows) * (size_t)sh.D;
}

// mode: 1 = RMSNorm, 2 = RoPE, 3 = RMSNorm then RoPE (forward) /
// RoPE backward then RMSNorm backward (backward)
hipError_t launch_qk_forward(const QkFwdParams& p, int mode, hipStream_t st);
hipError_t launch_qk_backward(const QkBwdParams& p, int mode, hipStream_t st);
hipError_t launch_wgrad_reduce(const float* wpart, int nblk, int D, void* gw, int gw_f32, hipStream_t st);

}  // namespace harp_qk
