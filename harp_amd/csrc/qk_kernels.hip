// gfx950 kernels for the step before the ring-attention block: per-head
// RMSNorm of Q and K and the rotary embedding (RoPE), forward and backward,
// separately and fused.
//
// Reference math (HARP's async runtime, ARM SVE, run on the CPU):
//   rmsnormForwardKernelBF16   async_rt/csrc/rms_norm.cc:20-105
//     rms = sqrt(sum(x^2) / D + eps), out = bf16((x * (1 / rms)) * w), rms saved
//   rmsnormBackwardKernelBF16  async_rt/csrc/rms_norm.cc:107-240
//     xn = x / rms, g = dy * w, dx = bf16((g - xn * sum(g * xn) / D) / rms),
//     grad_w = sum over rows of dy * xn
//   ropeForwardKernelBF16      async_rt/csrc/rope.cc:9-86
//     pairs (x[2i], x[2i+1]) times (f[2i], f[2i+1]) as complex numbers
//   ropeBackwardKernelBF16     async_rt/csrc/rope.cc:88-183
//     times the conjugate of f
// Every bf16 result is truncated (the reference stores the high 16 bits of
// the fp32 value, async_rt/csrc/async_op_math.h:24-35), so these kernels do
// the same and match the reference's results to the last bit wherever the
// fp32 arithmetic agrees (sums of squares are reduced in a different order,
// which can move a result by one bf16 unit).
//
// Layout: x and every per-row tensor are [B, H, S, D] views with unit D
// stride (the ring-attention kernels read Q and K token-major, strides
// (S*H*D, D, H*D, 1)).  freqs is fp32 [B or 1, S, D] with (cos, sin)
// interleaved, i.e. torch.view_as_real of the complex [.., S, D/2] table.
//
// Mapping: 16 lanes per row (4 rows per wave, 16 per 256-thread block), each
// lane owns NCH chunks of 8 consecutive elements (chunk j of lane i covers
// elements 8*(16*j + i) ..); a row's reductions are 4 xor-shuffles among its
// 16 lanes.  All loads are 16-byte (bf16) or 32-byte (fp32 freqs) per lane.
// The kernels are HBM-bound: per row they read and write D bf16 once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qk_kernels.h"

namespace harp_qk {

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// fp32 -> bf16 by truncation, as the reference stores bf16
__device__ __forceinline__ uint16_t f32_to_bf16_trunc(float f) { return (uint16_t)(__float_as_uint(f) >> 16); }

__device__ __forceinline__ float row_sum16(float v) {
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 16);
  return v;
}

// Position of a thread's row.  Rows are visited with the head fastest, then
// the token, then the batch: in the token-major layout the rows of one token
// are one contiguous run, and they share one row of the RoPE table.  The
// per-row rms is stored at (b*H + h)*S + s either way.
struct RowPos {
  int64_t visit;  // visit index over (b, s, h), h fastest
  int64_t row;    // (b*H + h)*S + s
  int b, h, s;
  int sub;        // lane within the row's 16
  bool ok;
};
// Block index -> logical block with the 8 XCDs (workgroups are dealt to them
// round-robin) each taking one contiguous range of logical blocks: the rows
// of one token, its RoPE table row and the neighbouring rms entries of a head
// are then fetched into, and merged in, one XCD's L2 instead of up to eight.
__device__ __forceinline__ int64_t xcd_block(int64_t i, int64_t n) {
  const int64_t q = n / 8, r = n % 8, x = i % 8, local = i / 8;
  return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}
__device__ __forceinline__ RowPos row_at(const QkShape& sh, int64_t visit) {
  RowPos r;
  r.visit = visit;
  r.sub = threadIdx.x & 15;
  r.ok = visit < (int64_t)sh.B * sh.H * sh.S;
  const int64_t v = r.ok ? visit : 0;
  r.h = (int)(v % sh.H);
  const int64_t bs = v / sh.H;
  r.s = (int)(bs % sh.S);
  r.b = (int)(bs / sh.S);
  r.row = ((int64_t)r.b * sh.H + r.h) * sh.S + r.s;
  return r;
}
__device__ __forceinline__ int64_t elem_off(const Strides4& st, const RowPos& r) {
  return (int64_t)r.b * st.b + (int64_t)r.h * st.h + (int64_t)r.s * st.s;
}

template <int NCH>
__device__ __forceinline__ void load_row(const uint16_t* base, int D, int sub, float (&v)[NCH][8]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e0 = 8 * (16 * j + sub);
    if (e0 < D) {
      const u16x8 u = *(const u16x8*)(base + e0);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = bf16_to_f32(u[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = 0.f;
    }
  }
}
template <int NCH>
__device__ __forceinline__ void store_row(uint16_t* base, int D, int sub, const float (&v)[NCH][8]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e0 = 8 * (16 * j + sub);
    if (e0 < D) {
      u16x8 u;
#pragma unroll
      for (int k = 0; k < 8; ++k) u[k] = f32_to_bf16_trunc(v[j][k]);
      *(u16x8*)(base + e0) = u;
    }
  }
}
// weight (bf16 or fp32) chunk as fp32; absent weight = 1.  The weight is a
// separate allocation of D elements: 16-byte loads stay inside it because D
// is a multiple of 8 and allocations are at least 16-byte aligned.
template <int NCH>
__device__ __forceinline__ void load_weight(const void* w, int w_f32, int D, int sub, float (&v)[NCH][8]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e0 = 8 * (16 * j + sub);
    if (!w || e0 >= D) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = 1.f;
    } else if (w_f32) {
      const f32x4 a = *(const f32x4*)((const float*)w + e0), c = *(const f32x4*)((const float*)w + e0 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[j][k] = a[k];
        v[j][k + 4] = c[k];
      }
    } else {
      const u16x8 u = *(const u16x8*)((const uint16_t*)w + e0);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = bf16_to_f32(u[k]);
    }
  }
}
template <int NCH>
__device__ __forceinline__ void load_freqs(const float* f, int D, int sub, float (&v)[NCH][8]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e0 = 8 * (16 * j + sub);
    if (e0 < D) {
      const f32x4 a = *(const f32x4*)(f + e0), c = *(const f32x4*)(f + e0 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[j][k] = a[k];
        v[j][k + 4] = c[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[j][k] = 0.f;
    }
  }
}

// RMSNorm forward of one row (rms_norm.cc:39-103): returns rms, v becomes
// bf16-truncated (x * (1 / rms)) * w, kept as fp32 values.
template <int NCH>
__device__ __forceinline__ float rmsnorm_row(float (&v)[NCH][8], const float (&w)[NCH][8], int D, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(v[j][k], v[j][k], ss);
  ss = row_sum16(ss);
  const float rms = __fsqrt_rn(__fdiv_rn(ss, (float)D) + eps);
  const float inv = __fdiv_rn(1.f, rms);
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) v[j][k] = bf16_to_f32(f32_to_bf16_trunc(__fmul_rn(__fmul_rn(v[j][k], inv), w[j][k])));
  return rms;
}
// RoPE of one row (rope.cc:34-38): complex multiply by f, or by conj(f)
// (rope.cc:115-134), then bf16-truncated.  The reference forms each part with
// one rounded product and one fused multiply-add.
template <int NCH, bool CONJ>
__device__ __forceinline__ void rope_row(float (&v)[NCH][8], const float (&f)[NCH][8]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
      const float xr = v[j][k], xi = v[j][k + 1], fr = f[j][k], fi = f[j][k + 1];
      float re, im;
      if (CONJ) {
        re = __builtin_fmaf(xi, fi, __fmul_rn(xr, fr));
        im = __builtin_fmaf(-xr, fi, __fmul_rn(xi, fr));
      } else {
        re = __builtin_fmaf(-xi, fi, __fmul_rn(xr, fr));
        im = __builtin_fmaf(xi, fr, __fmul_rn(xr, fi));
      }
      v[j][k] = bf16_to_f32(f32_to_bf16_trunc(re));
      v[j][k + 1] = bf16_to_f32(f32_to_bf16_trunc(im));
    }
}

// RMSNorm backward of one row (rms_norm.cc:139-230): dy becomes dx (fp32,
// not yet truncated); wgrad accumulates dy * xn.
template <int NCH>
__device__ __forceinline__ void rmsnorm_bwd_row(const float (&x)[NCH][8], float (&dy)[NCH][8],
                                                const float (&w)[NCH][8], float rms, int D, float (&wgrad)[NCH][8]) {
  const float inv = __fdiv_rn(1.f, rms);
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) dot = __builtin_fmaf(__fmul_rn(dy[j][k], w[j][k]), __fmul_rn(x[j][k], inv), dot);
  dot = row_sum16(dot);
  const float coeff = __fdiv_rn(dot, (float)D);
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float xn = __fmul_rn(x[j][k], inv);
      const float g = __fmul_rn(dy[j][k], w[j][k]);
      wgrad[j][k] = __builtin_fmaf(dy[j][k], xn, wgrad[j][k]);
      dy[j][k] = __fmul_rn(__fsub_rn(g, __fmul_rn(xn, coeff)), inv);
    }
}

// ---------------------------------------------------------------------------
// Forward: MODE 1 = RMSNorm, 2 = RoPE, 3 = RMSNorm then RoPE (fused; the
// intermediate is truncated to bf16 exactly as between the two reference ops)
// ---------------------------------------------------------------------------
template <int NCH, int MODE>
__global__ __launch_bounds__(256) void qk_forward_kernel(QkFwdParams p) {
  const RowPos r = row_at(p.sh, xcd_block(blockIdx.x, gridDim.x) * 16 + (threadIdx.x >> 4));
  if (!r.ok) return;  // whole 16-lane groups exit together
  float v[NCH][8];
  load_row<NCH>(p.x + elem_off(p.sx, r), p.sh.D, r.sub, v);
  if (MODE & 1) {
    float w[NCH][8];
    load_weight<NCH>(p.weight, p.weight_f32, p.sh.D, r.sub, w);
    const float rms = rmsnorm_row<NCH>(v, w, p.sh.D, p.eps);
    if (r.sub == 0 && p.rms) p.rms[r.row] = rms;
  }
  if (MODE & 2) {
    float f[NCH][8];
    load_freqs<NCH>(p.freqs + (int64_t)r.b * p.f_stride_b + (int64_t)r.s * p.f_stride_s, p.sh.D, r.sub, f);
    rope_row<NCH, false>(v, f);
  }
  store_row<NCH>(p.out + elem_off(p.so, r), p.sh.D, r.sub, v);
}

// ---------------------------------------------------------------------------
// Backward: MODE 1 = RMSNorm, 2 = RoPE, 3 = RoPE backward then RMSNorm
// backward (fused).  Each block walks a contiguous range of 16-row groups
// (kQkBwdMaxBlocks blocks at most).  With RMSNorm it writes its fp32
// weight-gradient partial sums to wpart[block][D]; the partials are summed
// in a second kernel (deterministic, no atomics).
// ---------------------------------------------------------------------------
template <int NCH, int MODE>
__global__ __launch_bounds__(256) void qk_backward_kernel(QkBwdParams p) {
  __shared__ float wsum[16][NCH * 128 + 4];
  const int64_t rows = (int64_t)p.sh.B * p.sh.H * p.sh.S;
  float wg[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) wg[j][k] = 0.f;
  float w[NCH][8];
  if (MODE & 1) load_weight<NCH>(p.weight, p.weight_f32, p.sh.D, threadIdx.x & 15, w);
  const int64_t groups = (rows + 15) / 16, per = (groups + gridDim.x - 1) / gridDim.x;
  const int64_t g0 = xcd_block(blockIdx.x, gridDim.x) * per, g1 = min(g0 + per, groups);
  for (int64_t gi = g0; gi < g1; ++gi) {
    const RowPos r = row_at(p.sh, gi * 16 + (threadIdx.x >> 4));
    if (!r.ok) break;  // only the last group has short rows; whole 16-lane groups leave together
    float g[NCH][8];
    load_row<NCH>(p.dy + elem_off(p.sdy, r), p.sh.D, r.sub, g);
    if (MODE & 2) {
      float f[NCH][8];
      load_freqs<NCH>(p.freqs + (int64_t)r.b * p.f_stride_b + (int64_t)r.s * p.f_stride_s, p.sh.D, r.sub, f);
      rope_row<NCH, true>(g, f);
    }
    if (MODE & 1) {
      float x[NCH][8];
      load_row<NCH>(p.x + elem_off(p.sx, r), p.sh.D, r.sub, x);
      rmsnorm_bwd_row<NCH>(x, g, w, p.rms[r.row], p.sh.D, wg);
    }
    store_row<NCH>(p.dx + elem_off(p.sdx, r), p.sh.D, r.sub, g);
  }
  if (MODE & 1) {
    // block partial of the weight gradient: sum the 16 row groups through LDS
    const int grp = threadIdx.x >> 4, sub = threadIdx.x & 15;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) wsum[grp][8 * (16 * j + sub) + k] = wg[j][k];
    __syncthreads();
    for (int e = threadIdx.x; e < p.sh.D; e += 256) {
      float acc = 0.f;
#pragma unroll
      for (int gi = 0; gi < 16; ++gi) acc += wsum[gi][e];
      p.wpart[(int64_t)blockIdx.x * p.sh.D + e] = acc;
    }
  }
}

// grad_weight[e] = sum over blocks of wpart[block][e], in two launches of the
// kernel below with a fixed order (so the result is deterministic): level 1
// sums groups of kWgGroupRows partial rows into level2[group][e], level 2 sums
// the groups and stores grad_weight as fp32 or bf16 (truncated, like the
// reference's other bf16 stores).  Two small launches over many CUs beat one
// launch over a few: a CU's own fetch rate bounds a single block.
//
// Block (x, g) sums rows [g*group_rows, (g+1)*group_rows) of src[nrows][D] for
// columns 16x .. 16x+15: its 16 row lanes take every 16th row (64-byte row
// segments, independent loads in flight) and LDS adds the lane sums in order.
template <bool FINAL>
__global__ __launch_bounds__(256) void wgrad_sum_kernel(const float* src, int nrows, int group_rows, int D, void* dst,
                                                        int dst_f32) {
  __shared__ float part[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int e = blockIdx.x * 16 + tx;
  const int i0 = blockIdx.y * group_rows, i1 = min(i0 + group_rows, nrows);
  float acc = 0.f;
  if (e < D) {
#pragma unroll 4
    for (int i = i0 + ty; i < i1; i += 16) acc += src[(int64_t)i * D + e];
  }
  part[ty][tx] = acc;
  __syncthreads();
  if (ty != 0 || e >= D) return;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) v += part[k][tx];
  if (!FINAL) ((float*)dst)[(int64_t)blockIdx.y * D + e] = v;
  else if (dst_f32) ((float*)dst)[e] = v;
  else ((uint16_t*)dst)[e] = f32_to_bf16_trunc(v);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
template <int NCH>
static hipError_t fwd_t(const QkFwdParams& p, int mode, hipStream_t st) {
  const int64_t rows = (int64_t)p.sh.B * p.sh.H * p.sh.S;
  const dim3 grid((unsigned)((rows + 15) / 16));
  switch (mode) {
    case 1: hipLaunchKernelGGL((qk_forward_kernel<NCH, 1>), grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((qk_forward_kernel<NCH, 2>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((qk_forward_kernel<NCH, 3>), grid, dim3(256), 0, st, p); break;
  }
  return hipGetLastError();
}
hipError_t launch_qk_forward(const QkFwdParams& p, int mode, hipStream_t st) {
  return p.sh.D <= 128 ? fwd_t<1>(p, mode, st) : fwd_t<2>(p, mode, st);
}

int bwd_blocks(const QkShape& sh) {
  const int64_t rows = (int64_t)sh.B * sh.H * sh.S;
  const int64_t need = (rows + 15) / 16;
  return (int)(need < kQkBwdMaxBlocks ? need : kQkBwdMaxBlocks);
}

template <int NCH>
static hipError_t bwd_t(const QkBwdParams& p, int mode, hipStream_t st) {
  const dim3 grid((unsigned)bwd_blocks(p.sh));
  switch (mode) {
    case 1: hipLaunchKernelGGL((qk_backward_kernel<NCH, 1>), grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((qk_backward_kernel<NCH, 2>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((qk_backward_kernel<NCH, 3>), grid, dim3(256), 0, st, p); break;
  }
  return hipGetLastError();
}
hipError_t launch_qk_backward(const QkBwdParams& p, int mode, hipStream_t st) {
  return p.sh.D <= 128 ? bwd_t<1>(p, mode, st) : bwd_t<2>(p, mode, st);
}

hipError_t launch_wgrad_reduce(const float* wpart, int nblk, int D, void* gw, int gw_f32, hipStream_t st) {
  float* level2 = const_cast<float*>(wpart) + (size_t)nblk * D;
  const int ngroups = (nblk + kWgGroupRows - 1) / kWgGroupRows;
  const unsigned cols = (unsigned)((D + 15) / 16);
  hipLaunchKernelGGL(wgrad_sum_kernel<false>, dim3(cols, (unsigned)ngroups), dim3(256), 0, st, wpart, nblk,
                     kWgGroupRows, D, (void*)level2, 1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(wgrad_sum_kernel<true>, dim3(cols, 1u), dim3(256), 0, st, (const float*)level2, ngroups, ngroups,
                     D, gw, gw_f32);
  return hipGetLastError();
}

}  // namespace harp_qk
