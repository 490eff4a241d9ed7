// Bench-only device probe (kernels/libharp_probe.so, loaded by bench.py; not
// part of the drop-in libraries): the sustained dense bf16 MFMA rate of this
// GPU and the shader clock it runs at while doing only that.
//
// Every wave streams v_mfma_f32_32x32x16_bf16 (the instruction all ring-
// attention kernels use) from registers: four independent accumulator
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
//
// C ABI (ctypes in harp_amd/_lib.py):
//   int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops, double* shader_ghz);
//   const char* harp_probe_last_error(void);
// Status 0 = ok, 1 = bad argument, 3 = allocation failed, 4 = launch failed.
// Synchronous on the null stream; allocates and frees its own small buffers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

namespace {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kOk = 0, kEinval = 1, kEnomem = 3, kElaunch = 4;

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

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

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}
int ok() {
  g_last_error.clear();
  return kOk;
}
int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(kElaunch, "%s launch failed: %s", what, hipGetErrorString(e));
  return kOk;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) const char* harp_probe_last_error(void) { return g_last_error.c_str(); }

__attribute__((visibility("default"))) int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops,
                                                                double* shader_ghz) {
  if (!tflops || !shader_ghz) return fail(kEinval, "probe outputs are NULL");
  if (iters < 16 || iters > (1 << 20)) return fail(kEinval, "iters=%d must be in [16, 2^20]", iters);
  int dev = 0, cus = 0, wall_khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ||
      hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev) || cus < 1 || wall_khz < 1)
    return fail(kElaunch, "device query failed");
  const int blocks = 8 * cus;  // 32 waves per CU, 8 per SIMD
  float* sink = nullptr;
  long long* clocks = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = kOk;
  std::vector<long long> h(2 * (size_t)blocks);
  float best_ms = 0.f;
  if (hipMalloc(&sink, sizeof(float) * 256 * (size_t)blocks) != hipSuccess ||
      hipMalloc(&clocks, sizeof(long long) * 2 * (size_t)blocks) != hipSuccess) {
    rc = fail(kEnomem, "probe buffers: hipMalloc failed");
  } else if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = fail(kElaunch, "probe events: hipEventCreate failed");
  } else {
    // one warm-up launch (clocks ramp), then the timed one
    for (int rep = 0; rep < 2 && rc == kOk; ++rep) {
      (void)hipEventRecord(e0, nullptr);
      hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, nullptr, seed + (uint32_t)rep, iters,
                         sink, clocks);
      if ((rc = launched("MFMA probe"))) break;
      (void)hipEventRecord(e1, nullptr);
      if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&best_ms, e0, e1) != hipSuccess)
        rc = fail(kElaunch, "probe timing failed");
    }
    if (rc == kOk &&
        hipMemcpy(h.data(), clocks, sizeof(long long) * h.size(), hipMemcpyDeviceToHost) != hipSuccess)
      rc = fail(kElaunch, "probe clock readback failed");
  }
  if (rc == kOk) {
    double shader = 0.0, wall = 0.0;
    for (int i = 0; i < blocks; ++i) {
      shader += (double)h[2 * i];
      wall += (double)h[2 * i + 1];
    }
    const double flop = (double)blocks * 4.0 /* waves */ * 4.0 * iters * 32.0 * 32.0 * 16.0 * 2.0;
    *tflops = (best_ms > 0.f) ? flop / (best_ms * 1e-3) / 1e12 : 0.0;
    *shader_ghz = (wall > 0.0) ? shader / wall * wall_khz * 1e-6 : 0.0;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (sink) (void)hipFree(sink);
  if (clocks) (void)hipFree(clocks);
  return rc == kOk ? ok() : rc;
}

}  // extern "C"
