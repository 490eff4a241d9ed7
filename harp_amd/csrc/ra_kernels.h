// Kernel parameter blocks and host launchers (internal to libharp_ra.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ra_common.h"

namespace harp_ra {

struct FwdParams {
  const bf16* q;
  int64_t sqb, sqh, sqt;
  int64_t skb, skh, skt;  // strides shared by every K/V chunk
  float* out;
  int64_t sob, soh, sot;
  void* m;                // [B,H,T] contiguous, fp32 or bf16
  int m_bf16;
  float* l;               // [B,H,T] contiguous
  int B, H, T, D;
  float scale;
  int n_split;            // KV splits (grid dimension y); > 1: out / m / l are per-split partials
  int64_t split_o;        // elements between the splits' out buffers
  int64_t split_ml;       // elements between the splits' m / l buffers
  ChunkTable ct;
};

// Combines the KV splits of the forward: per query row, the splits'
// normalised O, row max m and sum l (fp32, [n][B,H,T(,D)] contiguous) merge
// as O = sum_s w_s O_s / sum_s w_s with w_s = l_s exp(m_s - max_s m_s).
struct FwdMergeParams {
  const float* part_o;
  const float* part_m;
  const float* part_l;
  int n_split;
  float* out;
  int64_t sob, soh, sot;
  void* m;
  int m_bf16;
  float* l;
  int B, H, T, D;
};

// Sums the KV splits' dQ partials (fp32, already scaled, [n][B,H,T,D]).
struct DqMergeParams {
  const float* part;
  int n_split;
  void* dq;
  int64_t sdqb, sdqh, sdqt;
  int dq_f32;
  int B, H, T, D;
};

struct DeltaParams {
  const bf16* dout;
  int64_t sdb, sdh, sdt;
  const float* out;
  int64_t sob, soh, sot;
  float* delta;  // [B,H,T] contiguous
  int B, H, T, D;
};

struct BwdParams {
  const bf16* q;
  int64_t sqb, sqh, sqt;
  const bf16* dout;
  int64_t sdb, sdh, sdt;
  int64_t skb, skh, skt;       // K/V chunk strides
  int64_t sdkb, sdkh, sdkt;    // dK/dV chunk strides
  int dkv_f32;
  void* dq;
  int64_t sdqb, sdqh, sdqt;
  int dq_f32;
  const void* m;
  int m_bf16;
  const float* l;
  const float* delta;
  float* stats;             // workspace [2][B*H*T]: -(m + ln l) / scale, -D (written by the dQ kernel)
  int n_split;              // KV splits of the dQ kernel (grid dimension y); > 1: dq is per-split partials
  int64_t split_dq;         // elements between the splits' dQ buffers
  int n_key_tiles;          // kDkdvBlockKeys-key blocks per (b, h) over all chunks
  int ct_rows[kMaxChunks];  // stored rows of chunk c (dK/dV rows written, pads get 0)
  int B, H, T, D;
  float scale;
  float inv_scale;  // 1 / scale (a kernel argument, so it stays in an SGPR)
  ChunkTable ct;
};

// The backward's per-query statistics.  The dQ kernel (split 0 of every
// query tile) computes them for its rows, uses them and writes them to the
// two planes of p.stats, which the dK/dV kernel, launched after it, reads:
// plane 0 = -(m + ln l) / scale (-inf for a row without keys), plane 1 = -D.
__device__ __forceinline__ float bwd_stat_lse(const BwdParams& p, int64_t i) {
  const float mm = p.m_bf16 ? (float)((const bf16*)p.m)[i] : ((const float*)p.m)[i];
  const float ll = p.l[i];
  return (ll > 0.f) ? -(mm + __logf(ll)) * p.inv_scale : -INFINITY;
}

// Keys per dK/dV block (the host sizes the grid and the chunk table with it).
constexpr int kDkdvBlockKeys = 256;

hipError_t launch_fwd(const FwdParams& p, hipStream_t st);
// the forward with the hand-scheduled main loop (fwd_asm.hip), used by
// launch_fwd where it applies
bool fwd_asm_applies(const FwdParams& p);
hipError_t launch_fwd_asm(const FwdParams& p, hipStream_t st);
hipError_t launch_fwd_merge(const FwdMergeParams& p, hipStream_t st);
hipError_t launch_dq_merge(const DqMergeParams& p, hipStream_t st);
// Query rows per block of the forward and dQ kernels (the host sizes KV splits with it).
constexpr int kQueryBlockRows = 256;
hipError_t launch_delta(const DeltaParams& p, hipStream_t st);
hipError_t launch_dq(const BwdParams& p, hipStream_t st);
// the dQ kernel with the hand-scheduled main loop (dq_asm.hip), used by
// launch_dq where it applies
bool dq_asm_applies(const BwdParams& p);
hipError_t launch_dq_asm(const BwdParams& p, hipStream_t st);
hipError_t launch_dkdv(const BwdParams& p, hipStream_t st);
// the dK/dV kernel with the hand-scheduled main loop (dkdv_asm.hip), used by
// launch_dkdv where it applies
bool dkdv_asm_applies(const BwdParams& p);
hipError_t launch_dkdv_asm(const BwdParams& p, hipStream_t st);

}  // namespace harp_ra
