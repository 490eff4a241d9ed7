// Bench-only device probe (kernels/libharp_probe.so, loaded by bench.py; not
// part of the drop-in libraries): the sustained dense bf16 MFMA rate of this
// GPU, and the shader clock it runs at, for three instruction mixes.
//
// 1. harp_probe_mfma_rate: every wave streams v_mfma_f32_32x32x16_bf16 (the
//    instruction all ring-attention kernels use) from registers: four
//    independent accumulator chains, operands drawn from a per-lane hash of
//    the seed (bf16 values in [-1, 1), so the multiplier inputs toggle like
//    real data; all-zero operands draw far less power and run at a higher
//    clock).  32 waves per CU.  No LDS, no global traffic inside the loop.
// 2. harp_probe_mfma_lds_rate(softmax = 0): the attention kernels' operand
//    path -- 8 waves per CU (two per SIMD, as the kernels run), and one
//    operand of every MFMA read from LDS by ds_read_b128, 1 KB per MFMA per
//    wave (a 32x16 bf16 fragment), issued one MFMA ahead of its use.  The
//    other operand stays in registers, as Q, dO or P do in the kernels.
// 3. harp_probe_mfma_lds_rate(softmax = 1): the same plus one v_exp_f32 and
//    three FMAs per MFMA, the forward kernel's per-MFMA softmax work.
// 4. harp_probe_kernel_mix(kernel): mix 2 at one attention kernel's measured
//    per-MFMA work (hardware counters of the kernel at the headline shape):
//    VALU instructions, of which v_exp_f32, and the bytes of direct-to-LDS
//    copies it streams from L2 (buffer_load_dwordx4 ... lds, 1 KB per wave
//    instruction, from a 1 MiB L2-resident buffer into a separate LDS area):
//      kernel 0, forward: 4.5 VALU (1 exp), 128 B of copies per MFMA
//      kernel 1, dK/dV:   2.5 VALU (0.5 exp), 64 B (its LDS reads are
//                         1.1 KB per MFMA, the probe's 1 KB)
//      kernel 2, dQ:      3.33 VALU (0.67 exp), 85 B
//    Nothing in it depends on anything but its own registers: it is the rate
//    that kernel's instruction mix allows on this board under its power
//    limit, with no latency exposed and no wave waiting for another.
// 5. harp_probe_fwd_asm_loop: the D = 128 forward's own generated loop
//    (HARP_FWD_ASM_PROBE in fwd_asm.inc: the same instruction stream, with
//    the copy cursor wrapping around one 1 MiB K and one 1 MiB V source of
//    random bf16 instead of walking a chunk table), one 4-wave block per CU:
//    the steady-state rate of that loop on this board, the ceiling of
//    fwd_asm_kernel.
// 6. harp_probe_dq_asm_loop: the same for the D = 128 dQ kernel's generated
//    loop (HARP_DQ_ASM_PROBE in dq_asm.inc), with random Q and dO and
//    per-query statistics of the size the headline shape has: the ceiling of
//    dq_asm_kernel.
// 7. harp_probe_dkdv_asm_loop: the same for the D = 128 dK/dV kernel's
//    generated loop (HARP_DKDV_ASM_PROBE in dkdv_asm.inc: its copies re-read
//    one 32-query block of random Q and dO), random K and V, statistics that
//    put P near 2^-16 as at the headline shape: the ceiling of
//    dkdv_asm_kernel.
// The board is power-limited under MFMA load: LDS reads and VALU work take
// power from the MFMA stream, so mixes 2 and 3 run at a lower clock than 1.
// They bound what a kernel with that operand path can reach, independently
// of the published peak (256 CU x 2.4 GHz x 4096 FLOP/clk).
//
// Clock: each block's first wave reads the shader-clock counter (s_memtime)
// and the constant-rate counter (s_memrealtime) around its loop; the average
// ratio, times the constant counter's rate, is the average shader clock.
//
// C ABI (ctypes in harp_amd/_lib.py):
//   int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops, double* shader_ghz);
//   int harp_probe_mfma_lds_rate(int iters, uint32_t seed, int softmax, double* tflops, double* shader_ghz);
//   int harp_probe_kernel_mix(int kernel, int iters, uint32_t seed, double* tflops, double* shader_ghz);
//   int harp_probe_fwd_asm_loop(int key_blocks, uint32_t seed, double* tflops, double* shader_ghz);
//   int harp_probe_dq_asm_loop(int key_blocks, uint32_t seed, double* tflops, double* shader_ghz);
//   int harp_probe_dkdv_asm_loop(int query_blocks, uint32_t seed, double* tflops, double* shader_ghz);
//   const char* harp_probe_last_error(void);
// Status 0 = ok, 1 = bad argument, 3 = allocation failed, 4 = launch failed.
// Synchronous on the null stream; allocates and frees its own small buffers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstring>
#include <cstdio>
#include <string>
#include <vector>

#include "../dkdv_asm.inc"
#include "../dq_asm.inc"
#include "../fwd_asm.inc"

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

// Mixes 2 to 4: 8 waves, 64 KB of random bf16 in LDS (plus 16 KB as the
// copies' destination).  The LDS reads and the MFMAs that consume the
// previous step's fragments are one asm block, so the compiler cannot sink
// the reads down to their use (which would expose their latency) and the
// reads of step i + 1 overlap the MFMAs of step i.  Every fragment address is
// lane * 16 + group * 4096 + k * 1024 + 16 bytes <= 65536.
constexpr int kLdsProbeWaves = 8;
constexpr int kLdsProbeFrags = 64 * 64;  // bf16x8 fragments, 64 KB
constexpr int kCopyLdsBytes = 2048 * kLdsProbeWaves;  // two 1 KB slots per wave
constexpr uint32_t kCopySrcBytes = 1u << 20;         // L2-resident copy source

// VALU work of one step (4 MFMAs): E exps and F FMAs on eight independent
// chains whose values stay in (-3, 1).  The step's address arithmetic and
// each copy's offset update add about 0.25 and 2 / COPY_EVERY / 4 VALU
// instructions per MFMA; the mixes below count them.
template <int E, int F>
__device__ __forceinline__ void valu_work(float (&e)[8]) {
#pragma unroll
  for (int k = 0; k < E; ++k) e[k % 8] = __builtin_amdgcn_exp2f(e[k % 8]);
#pragma unroll
  for (int k = 0; k < F; ++k) e[(k + E) % 8] = __builtin_fmaf(e[(k + E) % 8], 0.5f, -1.5f);
}

// Steps cycle through three (exp, FMA) counts; a copy is issued every
// COPY_EVERY steps (0: none).
template <int E0, int F0, int E1, int F1, int E2, int F2, int COPY_EVERY>
__global__ __launch_bounds__(64 * kLdsProbeWaves) void mfma_lds_probe_kernel(uint32_t seed, int iters, float* sink,
                                                                            long long* clocks, const void* copy_src) {
  __shared__ __attribute__((aligned(16))) bf16x8 lds[kLdsProbeFrags + kCopyLdsBytes / 16];
  const uint32_t gid = blockIdx.x * (64u * kLdsProbeWaves) + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
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
  float e[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) e[k] = -0.01f * (float)(lane + k);
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&lds[lane];
  // copies: source offsets walk the 1 MiB buffer (wave-dependent start),
  // destination alternates between the wave's two 1 KB slots
  const uint64_t src = (uint64_t)(uintptr_t)copy_src;
  uint32_t rsrc[4] = {(uint32_t)src, (uint32_t)(src >> 32) & 0xffffu, COPY_EVERY ? kCopySrcBytes : 0u, 0x00020000u};
  const uint32_t copy_lds =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&lds[kLdsProbeFrags] + (uint32_t)wave * 2048u;
  uint32_t voff = ((uint32_t)(blockIdx.x * kLdsProbeWaves + wave) * 8192u + (uint32_t)lane * 16u) & (kCopySrcBytes - 1u);
  int n_copy = 0;
  auto copy = [&]() {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 rs = {(uint32_t)__builtin_amdgcn_readfirstlane(rsrc[0]),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rsrc[1]),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rsrc[2]), rsrc[3]};
    // at most four copies of this wave in flight
    asm volatile(
        "s_waitcnt vmcnt(3)\n\t"
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(copy_lds + (uint32_t)(n_copy & 1) * 1024u), "v"(voff), "s"(rs)
        : "memory", "m0");
    voff = (voff + 1024u) & (kCopySrcBytes - 1u);
    ++n_copy;
  };
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
  // six steps per iteration: the fragment double buffer (2) times the
  // three-step VALU cycle
  for (int i = 0; i < iters; i += 6) {
#define HARP_PROBE_STEP(k, E, F)                                   \
  step(x[(k) & 1], x[((k) + 1) & 1], addr_of(i + (k) + 1));        \
  valu_work<E, F>(e);                                              \
  if (COPY_EVERY && ((i + (k)) % (COPY_EVERY ? COPY_EVERY : 1)) == 0) copy();
    HARP_PROBE_STEP(0, E0, F0)
    HARP_PROBE_STEP(1, E1, F1)
    HARP_PROBE_STEP(2, E2, F2)
    HARP_PROBE_STEP(3, E0, F0)
    HARP_PROBE_STEP(4, E1, F1)
    HARP_PROBE_STEP(5, E2, F2)
#undef HARP_PROBE_STEP
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy may outlive the workgroup
  const long long t1 = clock64(), r1 = wall_clock64();
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += e[k];
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  sink[gid] = s;
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// Mix 5: the forward's generated loop on synthetic data (see the header).
// Register tuples, LDS layout and per-lane addresses as fwd_asm_kernel sets
// them up (fwd_asm.hip); keys are 1 MiB of K rows and 1 MiB of V rows
// (4096 x 128 bf16 each), read 32 rows per block and wrapped around.
typedef int v32i __attribute__((ext_vector_type(32)));
constexpr int kFaSrcRows = 4096;
__device__ __forceinline__ int fa_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__global__ __launch_bounds__(256, 1) void fwd_asm_probe_kernel(uint32_t seed, int nb, const uint16_t* kv, float c2,
                                                              float* sink, long long* clocks) {
  __shared__ __attribute__((aligned(16))) char lds[131072];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  {
    uint4* vb7 = (uint4*)(lds + 65536 + 7 * 8192);
    vb7[tid] = make_uint4(0u, 0u, 0u, 0u);
    vb7[tid + 256] = make_uint4(0u, 0u, 0u, 0u);
  }
  v32i q0, q1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const bf16x8 a = random_bf16x8(hash32(seed) ^ (blockIdx.x * 4096u + (uint32_t)tid * 16u + (uint32_t)k));
    const bf16x8 b = random_bf16x8(hash32(seed) ^ (blockIdx.x * 4096u + (uint32_t)tid * 16u + 8u + (uint32_t)k));
    const uint4 ua = __builtin_bit_cast(uint4, a), ub = __builtin_bit_cast(uint4, b);
    q0[4 * k] = (int)ua.x, q0[4 * k + 1] = (int)ua.y, q0[4 * k + 2] = (int)ua.z, q0[4 * k + 3] = (int)ua.w;
    q1[4 * k] = (int)ub.x, q1[4 * k + 1] = (int)ub.y, q1[4 * k + 2] = (int)ub.z, q1[4 * k + 3] = (int)ub.w;
  }
  asm volatile("" : "+{a[128:159]}"(q0), "+{a[160:191]}"(q1));
  v32i misc, misc2;
  {
    int mv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) mv[i] = 0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) mv[ks] = (int)(lds0 + l32 * 256 + (((2 * ks + g) ^ fa_swz(l32)) << 4));
    const int j = lane >> 4, sr = (lane >> 2) & 3, m = lane & 3;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int row = 8 * hh + 4 * g + sr;
        mv[8 + hh * 4 + db] =
            (int)(lds0 + 65536 + 2 * (row * 128 + (((4 * db + cl) ^ fa_swz(row)) << 3) + 4 * (m & 1)));
      }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = (2 * wave + i) * 4 + (lane >> 4);
      mv[16 + i] = r * 256 + (((lane & 15) ^ fa_swz(r)) << 4);
    }
    mv[18] = mv[19] = mv[20] = mv[21] = mv[26] = mv[27] = __float_as_int(-INFINITY);
#pragma unroll
    for (int i = 0; i < 32; ++i) misc[i] = mv[i];
#pragma unroll
    for (int i = 0; i < 32; ++i) misc2[i] = 0;
    misc2[1] = 4 * g;
    misc2[2] = __float_as_int(-INFINITY);
  }
  asm volatile("" : "+{v[32:63]}"(misc), "+{v[192:223]}"(misc2));
  v32i frag, pp, s0, s1, o0, o1, o2, o3;
  const uint64_t kp0 = (uint64_t)(uintptr_t)kv, vp0 = kp0 + (uint64_t)kFaSrcRows * 256u;
  const uint32_t dbase = lds0 + (uint32_t)wave * 2048u;
  const long long t0 = clock64(), r0 = wall_clock64();
  asm volatile(HARP_FWD_ASM_PROBE
               : "+{v[32:63]}"(misc), "={v[64:95]}"(frag), "={v[96:127]}"(pp), "={v[128:159]}"(s0),
                 "={v[160:191]}"(s1), "+{v[192:223]}"(misc2), "={a[0:31]}"(o0), "={a[32:63]}"(o1),
                 "={a[64:95]}"(o2), "={a[96:127]}"(o3), "+{a[128:159]}"(q0), "+{a[160:191]}"(q1)
               : [c2] "s"(c2), [dbase] "s"(dbase), [sbytes] "s"(256u), [blkb] "s"(8192u), [nb] "s"(nb),
                 [kp0] "s"(kp0), [vp0] "s"(vp0), [left0] "s"(kFaSrcRows), [step0] "s"(0)
               : "memory", "vcc", HARP_FWD_ASM_SGPR_CLOBBERS);
  const long long t1 = clock64(), r1 = wall_clock64();
  float acc = __int_as_float(misc[22]) + __int_as_float(misc[23]);
#pragma unroll
  for (int i = 0; i < 32; ++i) acc += __int_as_float(o0[i]) + __int_as_float(o3[i]);
  sink[blockIdx.x * 256 + tid] = acc;
  if (tid == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// Register tuples, LDS layout and per-lane addresses as dq_asm_kernel sets
// them up (dq_asm.hip); the same wrapped 1 MiB K and V sources as above.
// LSE2 = 16 (the log2 row sum of 2^16 keys with scores of unit spread, so P
// is about 2^-16 as at the headline shape) and D = 0.5.
__global__ __launch_bounds__(256, 1) void dq_asm_probe_kernel(uint32_t seed, int nb, const uint16_t* kv, float c2,
                                                             float* sink, long long* clocks) {
  __shared__ __attribute__((aligned(16))) char lds[131072];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  {
    uint4* kb7 = (uint4*)(lds + 7 * 8192);
    kb7[tid] = make_uint4(0u, 0u, 0u, 0u);
    kb7[tid + 256] = make_uint4(0u, 0u, 0u, 0u);
  }
  // random Q; dO from it by sign flips and swapped bf16 halves (operands
  // that toggle like independent data, without a second generator's registers)
  v32i q0, q1, g0, g1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t h = hash32(seed) ^ (blockIdx.x * 4096u + (uint32_t)tid * 16u + (uint32_t)k);
    const uint4 ua = __builtin_bit_cast(uint4, random_bf16x8(h)), ub = __builtin_bit_cast(uint4, random_bf16x8(h + 8u));
    q0[4 * k] = (int)ua.x, q0[4 * k + 1] = (int)ua.y, q0[4 * k + 2] = (int)ua.z, q0[4 * k + 3] = (int)ua.w;
    q1[4 * k] = (int)ub.x, q1[4 * k + 1] = (int)ub.y, q1[4 * k + 2] = (int)ub.z, q1[4 * k + 3] = (int)ub.w;
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    g0[i] = (int)((uint32_t)q1[i] ^ 0x80008000u);
    g1[i] = (int)(((uint32_t)q0[i] >> 16) | ((uint32_t)q0[i] << 16));
  }
  asm volatile("" : "+{a[128:159]}"(q0), "+{a[160:191]}"(q1), "+{a[192:223]}"(g0), "+{a[224:255]}"(g1));
  v32i misc;
  {
    int mv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) mv[i] = 0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      mv[ks] = (int)(lds0 + l32 * 256 + (((2 * ks + g) ^ fa_swz(l32)) << 4));
      mv[8 + ks] = mv[ks] + 65536;
    }
    const int j = lane >> 4, sr = (lane >> 2) & 3, m = lane & 3;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int row = 8 * hh + 4 * g + sr;
        mv[16 + hh * 4 + db] = (int)(lds0 + 2 * (row * 128 + (((4 * db + cl) ^ fa_swz(row)) << 3) + 4 * (m & 1)));
      }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = (2 * wave + i) * 4 + (lane >> 4);
      mv[24 + i] = r * 256 + (((lane & 15) ^ fa_swz(r)) << 4);
    }
    mv[26] = mv[27] = __float_as_int(16.0f);
    mv[28] = mv[29] = (int)seed;
    // unused slots: a value the compiler cannot fold (known-zero elements get
    // reused as constants after the loop, which keeps the whole tuple alive)
    mv[30] = mv[31] = (int)seed;
#pragma unroll
    for (int i = 0; i < 32; ++i) misc[i] = mv[i];
  }
  v32i fr0, fr1, s0, s1, d0, d1, o0, o1, o2, o3;
  // -D = -0.5 for every query: the initial dP^T accumulators
  v32i negd;
#pragma unroll
  for (int i = 0; i < 32; ++i) negd[i] = __float_as_int(-0.5f);
  const uint64_t kp0 = (uint64_t)(uintptr_t)kv, vp0 = kp0 + (uint64_t)kFaSrcRows * 256u;
  const uint32_t dbase = lds0 + (uint32_t)wave * 2048u;
  const long long t0 = clock64(), r0 = wall_clock64();
  asm volatile(HARP_DQ_ASM_PROBE
               : "+{v[0:31]}"(negd), "+{v[32:63]}"(misc), "={v[64:95]}"(fr0), "={v[96:127]}"(fr1),
                 "={v[128:159]}"(s0),
                 "={v[160:191]}"(s1), "={v[192:223]}"(d0), "={v[224:255]}"(d1), "={a[0:31]}"(o0),
                 "={a[32:63]}"(o1), "={a[64:95]}"(o2), "={a[96:127]}"(o3), "+{a[128:159]}"(q0),
                 "+{a[160:191]}"(q1), "+{a[192:223]}"(g0), "+{a[224:255]}"(g1)
               : [c2] "s"(c2), [dbase] "s"(dbase), [sbytes] "s"(256u), [blkb] "s"(8192u), [nb] "s"(nb),
                 [kp0] "s"(kp0), [vp0] "s"(vp0), [left0] "s"(kFaSrcRows), [step0] "s"(0)
               : "memory", "vcc", HARP_DQ_ASM_SGPR_CLOBBERS);
  const long long t1 = clock64(), r1 = wall_clock64();
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) acc += __int_as_float(o0[i]) + __int_as_float(o3[i]);
  // the lane index read again: the loop statement binds v32..v255, so no
  // per-lane value is kept across it
  int lane_e;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  float* sk = sink;
  asm volatile("" : "+s"(sk));  // the pointer stays scalar across the loop
  sk[blockIdx.x * 256 + wave * 64 + lane_e] = acc;
  if (wave == 0 && lane_e == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// Register tuples, LDS layout and per-lane addresses as dkdv_asm_kernel sets
// them up (dkdv_asm.hip): Q rows at the source's start, dO rows 1 MiB in, V
// rows from 512 KiB in, the statistics planes (fp32, written by the host) in
// its last 512 bytes; K from the per-lane hash.
constexpr int kDkBuf = 16384, kDkVOff = 5 * kDkBuf, kDkVRow = 272, kDkStats = kDkVOff + 256 * kDkVRow;
constexpr int kDkStatsPerWave = 5 * 512;
__global__ __launch_bounds__(256, 1) void dkdv_asm_probe_kernel(uint32_t seed, int nb, const uint16_t* src,
                                                               float c2, float* sink, long long* clocks) {
  __shared__ __attribute__((aligned(16))) char lds[kDkStats + 4 * kDkStatsPerWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  {
    const char* vsrc = (const char*)src + (512 << 10);
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int idx = i * 256 + tid, row = idx >> 4, ch = idx & 15;
      *(uint4*)(lds + kDkVOff + row * kDkVRow + ch * 16) = *(const uint4*)(vsrc + row * 256 + ch * 16);
    }
    uint4* b4 = (uint4*)(lds + 4 * kDkBuf);
#pragma unroll
    for (int i = 0; i < 4; ++i) b4[i * 256 + tid] = make_uint4(0u, 0u, 0u, 0u);
  }
  v32i kb0, kb1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t h = hash32(seed) ^ (blockIdx.x * 4096u + (uint32_t)tid * 16u + (uint32_t)k);
    const uint4 ua = __builtin_bit_cast(uint4, random_bf16x8(h)), ub = __builtin_bit_cast(uint4, random_bf16x8(h + 8u));
    kb0[4 * k] = (int)ua.x, kb0[4 * k + 1] = (int)ua.y, kb0[4 * k + 2] = (int)ua.z, kb0[4 * k + 3] = (int)ua.w;
    kb1[4 * k] = (int)ub.x, kb1[4 * k + 1] = (int)ub.y, kb1[4 * k + 2] = (int)ub.z, kb1[4 * k + 3] = (int)ub.w;
  }
  __syncthreads();
  v32i misc;
  {
    int mv[32];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) mv[ks] = (int)(lds0 + l32 * 256 + (((2 * ks + g) ^ fa_swz(l32)) << 4));
    const int j = lane >> 4, sr = (lane >> 2) & 3, m = lane & 3;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int row = 8 * hh + 4 * g + sr;
        mv[8 + hh * 4 + db] =
            (int)(lds0 + kDkBuf + 2 * (row * 128 + (((4 * db + cl) ^ fa_swz(row)) << 3) + 4 * (m & 1)));
      }
    mv[16] = (int)(lds0 + kDkVOff + (wave * 64 + l32) * kDkVRow + g * 16);
    mv[17] = (int)(lds0 + kDkStats + wave * kDkStatsPerWave + g * 16);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = (2 * wave + i) * 4 + (lane >> 4);
      mv[18 + i] = mv[20 + i] = r * 256 + (((lane & 15) ^ fa_swz(r)) << 4);
    }
    mv[22] = lane * 4;
#pragma unroll
    for (int i = 23; i < 32; ++i) mv[i] = mv[16];
#pragma unroll
    for (int i = 0; i < 32; ++i) misc[i] = mv[i];
  }
  const uint64_t qp = (uint64_t)(uintptr_t)src, gp = qp + (1u << 20);
  const uint64_t sp0 = qp + (2u << 20) - 512u, sp1 = sp0 + 256u;
  const uint32_t dbase = lds0 + (uint32_t)wave * 2048u;
  const uint32_t stb = lds0 + kDkStats + (uint32_t)wave * kDkStatsPerWave;
  v32i sacc, dacc, pbds, init, frag, o0, o1, o2, o3, o4, o5, o6, o7;
  const long long t0 = clock64(), r0 = wall_clock64();
  asm volatile(HARP_DKDV_ASM_PROBE
               : "+{v[0:31]}"(misc), "+{v[32:63]}"(kb0), "+{v[64:95]}"(kb1), "={v[96:127]}"(sacc),
                 "={v[128:159]}"(dacc), "={v[160:191]}"(pbds), "={v[192:223]}"(init), "={v[224:255]}"(frag),
                 "={a[0:31]}"(o0), "={a[32:63]}"(o1), "={a[64:95]}"(o2), "={a[96:127]}"(o3), "={a[128:159]}"(o4),
                 "={a[160:191]}"(o5), "={a[192:223]}"(o6), "={a[224:255]}"(o7)
               : [c2] "s"(__float_as_uint(c2)), [dbase] "s"(dbase), [sbase] "s"(stb), [qp] "s"(qp), [gp] "s"(gp),
                 [sp0] "s"(sp0), [sp1] "s"(sp1), [qnr] "s"(8192u), [gnr] "s"(8192u), [snr] "s"(256u),
                 [qstep] "s"(8192u), [gstep] "s"(8192u), [nb] "s"(nb)
               : "memory", "vcc", HARP_DKDV_ASM_SGPR_CLOBBERS);
  const long long t1 = clock64(), r1 = wall_clock64();
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) acc += __int_as_float(o0[i]) + __int_as_float(o7[i]);
  // the lane index read again and the sink pointer kept scalar: the loop
  // statement binds every VGPR
  int lane_e;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  float* sk = sink;
  asm volatile("" : "+s"(sk));
  sk[blockIdx.x * 256 + wave * 64 + lane_e] = acc;
  if (wave == 0 && lane_e == 0) {
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

// mix 0: register-fed, 32 waves per CU; mix 1 / 2: LDS-fed (without / with
// the softmax VALU), 8 waves per CU; mix 3 / 4 / 5: the forward / dK/dV / dQ
// kernel's per-MFMA work, 8 waves per CU
int launch_mix(int mix, int blocks, int threads, uint32_t sd, int iters, float* sink, long long* clocks,
               const void* src) {
  const dim3 g((unsigned)blocks), t((unsigned)threads);
  switch (mix) {
    case 0: hipLaunchKernelGGL(mfma_probe_kernel, g, t, 0, nullptr, sd, iters, sink, clocks); break;
    case 1:
      hipLaunchKernelGGL((mfma_lds_probe_kernel<0, 0, 0, 0, 0, 0, 0>), g, t, 0, nullptr, sd, iters, sink, clocks, src);
      break;
    case 2:
      hipLaunchKernelGGL((mfma_lds_probe_kernel<4, 12, 4, 12, 4, 12, 0>), g, t, 0, nullptr, sd, iters, sink, clocks,
                         src);
      break;
    case 3:  // forward: 4.5 VALU (1 exp) per MFMA, a 1 KB copy per 8 MFMAs
      hipLaunchKernelGGL((mfma_lds_probe_kernel<4, 12, 4, 12, 4, 12, 2>), g, t, 0, nullptr, sd, iters, sink, clocks,
                         src);
      break;
    case 4:  // dK/dV: 2.5 VALU (0.5 exp), a copy per 16 MFMAs
      hipLaunchKernelGGL((mfma_lds_probe_kernel<2, 6, 2, 6, 2, 7, 4>), g, t, 0, nullptr, sd, iters, sink, clocks, src);
      break;
    case 6:  // the forward's generated loop: iters = 32-key blocks
      hipLaunchKernelGGL(fwd_asm_probe_kernel, g, t, 0, nullptr, sd, iters, (const uint16_t*)src,
                         0.08838834764f * 1.44269504f, sink, clocks);
      break;
    case 8:  // the dK/dV kernel's generated loop: iters = 32-query blocks
      hipLaunchKernelGGL(dkdv_asm_probe_kernel, g, t, 0, nullptr, sd, iters, (const uint16_t*)src,
                         0.08838834764f * 1.44269504f, sink, clocks);
      break;
    case 7:  // the dQ kernel's generated loop: iters = 32-key blocks
      hipLaunchKernelGGL(dq_asm_probe_kernel, g, t, 0, nullptr, sd, iters, (const uint16_t*)src,
                         0.08838834764f * 1.44269504f, sink, clocks);
      break;
    default:  // dQ: 3.33 VALU (0.67 exp), a copy per 12 MFMAs
      hipLaunchKernelGGL((mfma_lds_probe_kernel<3, 9, 3, 9, 2, 9, 3>), g, t, 0, nullptr, sd, iters, sink, clocks,
                         src);
      break;
  }
  return launched("MFMA probe");
}

int run_probe(int mix, int iters, uint32_t seed, double* tflops, double* shader_ghz) {
  if (!tflops || !shader_ghz) return fail(kEinval, "probe outputs are NULL");
  if (iters < 16 || iters > (1 << 20) || iters % 2) return fail(kEinval, "iters=%d must be even, in [16, 2^20]", iters);
  if (mix > 0 && mix < 6) iters = (iters + 5) / 6 * 6;  // the LDS-fed loops run six steps per iteration
  int dev = 0, cus = 0, wall_khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ||
      hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev) || cus < 1 || wall_khz < 1)
    return fail(kElaunch, "device query failed");
  const int threads = (mix == 0 || mix >= 6) ? 256 : 64 * kLdsProbeWaves;
  const int waves_per_block = threads / 64;
  const int blocks = mix == 0 ? 8 * cus : cus;  // 32 or 8 waves per CU
  float* sink = nullptr;
  long long* clocks = nullptr;
  void* src = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = kOk;
  std::vector<long long> h(2 * (size_t)blocks);
  float best_ms = 0.f;
  if (hipMalloc(&sink, sizeof(float) * threads * (size_t)blocks) != hipSuccess ||
      hipMalloc(&clocks, sizeof(long long) * 2 * (size_t)blocks) != hipSuccess ||
      hipMalloc(&src, 2 * kCopySrcBytes) != hipSuccess) {
    rc = fail(kEnomem, "probe buffers: hipMalloc failed");
  } else if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = fail(kElaunch, "probe events: hipEventCreate failed");
  } else {
    // the copies' source: random bytes, so their data path toggles like real data
    std::vector<uint32_t> r(2 * kCopySrcBytes / 4);
    for (size_t i = 0; i < r.size(); ++i) r[i] = (uint32_t)(i * 2654435761u) ^ (seed * 0x9e3779b9u) ^ (uint32_t)(i >> 7);
    if (mix >= 6) {  // finite bf16 keys and values in [-1.7, 1.7]: pairs of (sign, exponent 117-127, mantissa)
      for (size_t i = 0; i < r.size(); ++i) {
        const uint32_t h = r[i] * 0x85ebca6bu;
        const uint32_t lo = (h & 0x807fu) | ((117u + (h >> 7) % 11u) << 7);
        const uint32_t hi = ((h >> 16) & 0x807fu) | ((117u + (h >> 23) % 11u) << 7);
        r[i] = lo | (hi << 16);
      }
    }
    if (mix == 8) {  // the dK/dV loop's statistics planes: S' c = S c - 16 (P near 2^-16), D = 0.5
      const float c2 = 0.08838834764f * 1.44269504f, lse = -16.f / c2, dlt = -0.5f;
      float* st = (float*)(r.data() + r.size() - 128);
      for (int i = 0; i < 64; ++i) {
        st[i] = lse;
        st[64 + i] = dlt;
      }
    }
    if (hipMemcpy(src, r.data(), 2 * kCopySrcBytes, hipMemcpyHostToDevice) != hipSuccess)
      rc = fail(kElaunch, "probe copy source upload failed");
    // one warm-up launch (clocks ramp), then the timed one
    for (int rep = 0; rep < 2 && rc == kOk; ++rep) {
      (void)hipEventRecord(e0, nullptr);
      if ((rc = launch_mix(mix, blocks, threads, seed + (uint32_t)rep, iters, sink, clocks, src))) break;
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
    // mixes 0-5: four MFMAs per wave and step; per wave and key block, mix 6:
    // 32 (S, O), mix 7: 48 (S, dP, dQ)
    const double per = mix == 6 ? 32.0 : (mix == 7 ? 48.0 : (mix == 8 ? 64.0 : 4.0));
    const double flop = (double)blocks * waves_per_block * per * iters * 32.0 * 32.0 * 16.0 * 2.0;
    *tflops = (best_ms > 0.f) ? flop / (best_ms * 1e-3) / 1e12 : 0.0;
    *shader_ghz = (wall > 0.0) ? shader / wall * wall_khz * 1e-6 : 0.0;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (sink) (void)hipFree(sink);
  if (clocks) (void)hipFree(clocks);
  if (src) (void)hipFree(src);
  return rc == kOk ? ok() : rc;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) const char* harp_probe_last_error(void) { return g_last_error.c_str(); }

__attribute__((visibility("default"))) int harp_probe_mfma_rate(int iters, uint32_t seed, double* tflops,
                                                                double* shader_ghz) {
  return run_probe(0, iters, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_mfma_lds_rate(int iters, uint32_t seed, int softmax,
                                                                    double* tflops, double* shader_ghz) {
  if (softmax != 0 && softmax != 1) return fail(kEinval, "softmax=%d must be 0 or 1", softmax);
  return run_probe(1 + softmax, iters, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_fwd_asm_loop(int key_blocks, uint32_t seed, double* tflops,
                                                                   double* shader_ghz) {
  return run_probe(6, key_blocks, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_dq_asm_loop(int key_blocks, uint32_t seed, double* tflops,
                                                                  double* shader_ghz) {
  return run_probe(7, key_blocks, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_dkdv_asm_loop(int query_blocks, uint32_t seed, double* tflops,
                                                                    double* shader_ghz) {
  return run_probe(8, query_blocks, seed, tflops, shader_ghz);
}

__attribute__((visibility("default"))) int harp_probe_kernel_mix(int kernel, int iters, uint32_t seed, double* tflops,
                                                                 double* shader_ghz) {
  if (kernel < 0 || kernel > 2) return fail(kEinval, "kernel=%d must be 0 (forward), 1 (dK/dV) or 2 (dQ)", kernel);
  return run_probe(3 + kernel, iters, seed, tflops, shader_ghz);
}

}  // extern "C"
