// Device probe: the sustained dense bf16 MFMA rate of this GPU and the shader
// clock it runs at while doing only that.
//
// Every wave streams v_mfma_f32_32x32x16_bf16 (the instruction all ring-
// attention kernels here use) from registers: four independent accumulator
// chains, operands drawn from a per-lane hash of the seed (bf16 values in
// [-1, 1), so the multiplier inputs toggle like real data; all-zero operands
// draw far less power and run at a higher clock).  No LDS, no global traffic
// inside the loop.  The result bounds what any MFMA-bound kernel can reach on
// this board under its power limit, independently of the published peak
// (256 CU x 2.4 GHz x 4096 FLOP/clk).
//
// Clock: each block's first wave reads the shader-clock counter (s_memtime)
// and the constant-rate counter (s_memrealtime) around its loop; the average
// ratio, times the constant counter's rate, is the average shader clock.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ra_common.h"
#include "ra_kernels.h"

namespace harp_ra {

__device__ __forceinline__ uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// bf16 with a random sign and mantissa and an exponent in [2^-8, 1)
__device__ __forceinline__ bf16x8 random_bf16x8(uint32_t seed) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t h = hash32(seed * 8u + (uint32_t)i);
    const uint16_t bits = (uint16_t)((h & 0x807fu) | ((119u + ((h >> 8) & 7u)) << 7));
    v[i] = __builtin_bit_cast(bf16, bits);
  }
  return v;
}

__global__ __launch_bounds__(256) void mfma_probe_kernel(uint32_t seed, int iters, float* sink, long long* clocks) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  bf16x8 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = random_bf16x8(hash32(seed) ^ (gid * 8u + (uint32_t)j));
    b[j] = random_bf16x8(hash32(seed + 1u) ^ (gid * 8u + 4u + (uint32_t)j));
  }
  const long long t0 = clock64(), r0 = wall_clock64();
  f32x16 c0 = zero16(), c1 = zero16(), c2 = zero16(), c3 = zero16();
  for (int i = 0; i < iters; ++i) {
    c0 = mfma32x32x16(a[0], b[0], c0);
    c1 = mfma32x32x16(a[1], b[1], c1);
    c2 = mfma32x32x16(a[2], b[2], c2);
    c3 = mfma32x32x16(a[3], b[3], c3);
  }
  const long long t1 = clock64(), r1 = wall_clock64();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  sink[gid] = s;
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

hipError_t launch_mfma_probe(int blocks, int iters, uint32_t seed, float* sink, long long* clocks, hipStream_t st) {
  hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, st, seed, iters, sink, clocks);
  return hipGetLastError();
}

}  // namespace harp_ra
