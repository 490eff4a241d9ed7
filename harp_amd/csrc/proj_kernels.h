// Parameter block and launcher of the fused q/k/v projection kernel
// (internal to libharp_ra.so; the C ABI, harp_qkv_project, is in
// include/harp_qk_norm_rope.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace harp_proj {

constexpr int kHeadDim = 128;       // features of one head (one wave's share)
constexpr int kBlockHeads = 2;      // heads per block
constexpr int kBlockTokens = 256;   // tokens per block
constexpr int kKTile = 64;        // contraction elements per LDS tile
constexpr int kMaxOuts = 3;       // q, k, v in one launch

// One projection y = x W^T of the launch (an nn.Linear without bias).
struct ProjOut {
  const uint16_t* w;  // [n_out, K] bf16, row stride ldw
  int64_t ldw;
  uint16_t* y;        // [M, n_out] bf16, row stride ldy
  int64_t ldy;
  uint16_t* y_lin;    // [M, n_out] bf16 pre-norm product (row stride ldy), NULL = not written
  const void* norm_w; // RMSNorm weight [128] (bf16, or fp32 if norm_w_f32), NULL = plain projection
  int norm_w_f32;
  float eps;
  float* rms;         // [B * heads * S] fp32 at (b * heads + h) * S + s, NULL = not written
};

struct ProjParams {
  const uint16_t* x;  // [M, K] bf16 hidden states (M = B * S tokens), row stride ldx
  int64_t ldx;
  int M, S, K, heads;  // heads = n_out / 128
  // RoPE table, fp32 (cos, sin) pairs: pair p of token (b, s) at
  // freqs + b * f_stride_b + s * f_stride_s + 2p; NULL = no RoPE
  const float* freqs;
  int64_t f_stride_b, f_stride_s;
  int n_outs;
  ProjOut out[kMaxOuts];
  // set by launch_proj: blocks per output of the main grid, the first block of
  // the last output left to the tail launch, and its first unit there
  int n_lin, keep_last, tail_bid0;
};

// LDS bytes of the main kernel: two stages of the x and W tiles
constexpr int kProjLdsBytes = 2 * (kBlockTokens + kBlockHeads * kHeadDim) * kKTile * 2;

hipError_t launch_proj(const ProjParams& p, hipStream_t stream);

}  // namespace harp_proj
