// Bench-only device probe (kernels/libharp_bench_probe.so, built by
// __graft_entry__.build() and loaded by bench.py; not part of the drop-in
// libraries and not loaded by anything on the operator path): the sustained
// dense bf16 MFMA rate of this GPU, and the shader clock it runs at, for two
// operand paths.
//
// 1. harp_probe_mfma_rate: every wave streams v_mfma_f32_32x32x16_bf16 (the
//    instruction all ring-attention kernels use) from registers: four
//    independent accumulator chains, operands drawn from a per-lane hash of
//    the seed (bf16 values in [-1, 1), so the multiplier inputs toggle like
//    real data; all-zero operands draw far less power and run at a higher
//    clock).  32 waves per CU.  No LDS, no global traffic inside the loop.
// 2. harp_probe_mfma_lds_rate: the attention kernels' operand path -- 8
//    waves per CU, one operand of every MFMA read from LDS by ds_read_b128,
//    1 KB per MFMA per wave (a 32x16 bf16 fragment), issued one MFMA ahead of
//    its use.  The other operand stays in registers, as Q, dO or P do in the
//    kernels.
// The published peak is 256 CU x 2.4 GHz x 4096 FLOP/clk; under a dense MFMA
// stream on random data the board holds a lower clock, which these two rates
// measure.
//
// Clock: each block's first wave reads the shader-clock counter (s_memtime)
// and the constant-rate counter (s_memrealtime) around its loop; the average
// ratio, times the constant counter's rate, is the average shader clock.
//
// C ABI (ctypes in bench.py):
//   int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops, double* shader_ghz);
//   int harp_probe_mfma_lds_rate(int iters, uint32_t seed, double* tflops, double* shader_ghz);
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

// 8 waves, 64 KB of random bf16 in LDS.  The LDS reads and the MFMAs that
// consume the previous step's fragments are one asm block, so the compiler
// cannot sink the reads down to their use (which would expose their latency)
// and the reads of step i + 1 overlap the MFMAs of step i.  Every fragment
// address is lane * 16 + group * 4096 + k * 1024 + 16 bytes <= 65536.
constexpr int kLdsProbeWaves = 8;
constexpr int kLdsProbeFrags = 64 * 64;  // bf16x8 fragments, 64 KB

__global__ __launch_bounds__(64 * kLdsProbeWaves) void mfma_lds_probe_kernel(uint32_t seed, int iters, float* sink,
                                                                            long long* clocks) {
  __shared__ __attribute__((aligned(16))) bf16x8 lds[kLdsProbeFrags];
  const uint32_t gid = blockIdx.x * (64u * kLdsProbeWaves) + threadIdx.x;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < kLdsProbeFrags; i += 64 * kLdsProbeWaves)
    lds[i] = random_bf16x8(hash32(seed + 7u) ^ (blockIdx.x * (uint32_t)kLdsProbeFrags + (uint32_t)i));
  __syncthreads();
  bf16x8 b[4], x[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b[j] = random_bf16x8(hash32(seed + 1u) ^ (gid * 8u + 4u + (uint32_t)j));
    x[0][j] = lds[j * 64 + lane];
    x[1][j] = x[0][j];
  }
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&lds[lane];
  f32x16 c0 = zero16(), c1 = zero16(), c2 = zero16(), c3 = zero16();
  auto step = [&](const bf16x8* u, bf16x8* w, uint32_t addr) {
    asm volatile(
        "ds_read_b128 %4, %16 offset:0\n\t"
        "v_mfma_f32_32x32x16_bf16 %0, %8, %12, %0\n\t"
        "ds_read_b128 %5, %16 offset:1024\n\t"
        "v_mfma_f32_32x32x16_bf16 %1, %9, %13, %1\n\t"
        "ds_read_b128 %6, %16 offset:2048\n\t"
        "v_mfma_f32_32x32x16_bf16 %2, %10, %14, %2\n\t"
        "ds_read_b128 %7, %16 offset:3072\n\t"
        "v_mfma_f32_32x32x16_bf16 %3, %11, %15, %3\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
        : "v"(u[0]), "v"(u[1]), "v"(u[2]), "v"(u[3]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(addr));
  };
  auto addr_of = [&](int i) { return base + (uint32_t)((i & 15) * 4096); };
  const long long t0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; i += 2) {
    step(x[0], x[1], addr_of(i + 1));
    step(x[1], x[0], addr_of(i + 2));
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

// mix 0: register-fed, 32 waves per CU; mix 1: LDS-fed, 8 waves per CU
int run_probe(int mix, int iters, uint32_t seed, double* tflops, double* shader_ghz) {
  if (!tflops || !shader_ghz) return fail(kEinval, "probe outputs are NULL");
  if (iters < 16 || iters > (1 << 20) || iters % 2) return fail(kEinval, "iters=%d must be even, in [16, 2^20]", iters);
  int dev = 0, cus = 0, wall_khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ||
      hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev) || cus < 1 || wall_khz < 1)
    return fail(kElaunch, "device query failed");
  const int threads = mix == 0 ? 256 : 64 * kLdsProbeWaves;
  const int blocks = mix == 0 ? 8 * cus : cus;  // 32 or 8 waves per CU
  float* sink = nullptr;
  long long* clocks = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = kOk;
  std::vector<long long> h(2 * (size_t)blocks);
  float ms = 0.f;
  if (hipMalloc(&sink, sizeof(float) * threads * (size_t)blocks) != hipSuccess ||
      hipMalloc(&clocks, sizeof(long long) * 2 * (size_t)blocks) != hipSuccess) {
    rc = fail(kEnomem, "probe buffers: hipMalloc failed");
  } else if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = fail(kElaunch, "probe events: hipEventCreate failed");
  } else {
    // one warm-up launch (clocks ramp), then the timed one
    for (int rep = 0; rep < 2 && rc == kOk; ++rep) {
      (void)hipEventRecord(e0, nullptr);
      if (mix == 0)
        hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(threads), 0, nullptr, seed + (uint32_t)rep, iters,
                           sink, clocks);
      else
        hipLaunchKernelGGL(mfma_lds_probe_kernel, dim3(blocks), dim3(threads), 0, nullptr, seed + (uint32_t)rep,
                           iters, sink, clocks);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) {
        rc = fail(kElaunch, "MFMA probe launch failed: %s", hipGetErrorString(e));
        break;
      }
      (void)hipEventRecord(e1, nullptr);
      if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
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
    // four MFMAs per wave and step
    const double flop = (double)blocks * (threads / 64) * 4.0 * iters * 32.0 * 32.0 * 16.0 * 2.0;
    *tflops = (ms > 0.f) ? flop / (ms * 1e-3) / 1e12 : 0.0;
    *shader_ghz = (wall > 0.0) ? shader / wall * wall_khz * 1e-6 : 0.0;
    g_last_error.clear();
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (sink) (void)hipFree(sink);
  if (clocks) (void)hipFree(clocks);
  return rc;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) const char* harp_probe_last_error(void) { return g_last_error.c_str(); }

__attribute__((visibility("default"))) int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops,
                                                                double* shader_ghz) {
  return run_probe(0, iters, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_mfma_lds_rate(int iters, uint32_t seed, double* tflops,
                                                                    double* shader_ghz) {
  return run_probe(1, iters, seed, tflops, shader_ghz);
}

}  // extern "C"
