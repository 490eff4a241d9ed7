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
  ChunkTable ct;
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
  float* stats;             // workspace [2][B*H*T]: -(m + ln l) / scale, -D (stats_prep_kernel)
  int n_key_tiles;          // kDkdvBlockKeys-key blocks per (b, h) over all chunks
  int ct_rows[kMaxChunks];  // stored rows of chunk c (dK/dV rows written, pads get 0)
  int B, H, T, D;
  float scale;
  float inv_scale;  // 1 / scale (a kernel argument, so it stays in an SGPR)
  ChunkTable ct;
};

// Keys per dK/dV block (the host sizes the grid and the chunk table with it).
constexpr int kDkdvBlockKeys = 256;

hipError_t launch_fwd(const FwdParams& p, hipStream_t st);
hipError_t launch_delta(const DeltaParams& p, hipStream_t st);
hipError_t launch_stats_prep(const BwdParams& p, hipStream_t st);
hipError_t launch_dq(const BwdParams& p, hipStream_t st);
hipError_t launch_dkdv(const BwdParams& p, hipStream_t st);

}  // namespace harp_ra
