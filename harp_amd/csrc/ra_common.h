// Shared device-side definitions for the gfx950 ring-attention kernels.
//
// Layout conventions (CDNA4 wave64 MFMA, v_mfma_f32_32x32x16_bf16):
//   A operand: lane l holds A[row = l%32][k-set of 8 picked by l/32]
//   B operand: lane l holds B[k-set of 8 picked by l/32][col = l%32]
//   C/D (16 fp32 per lane): C[row = 8*(r/4) + 4*(l/32) + r%4][col = l%32]
// A and B of one instruction always use the same k-set for a lane, so the
// order of k inside a k-step is free; the kernels exploit that to feed a
// C-layout accumulator (16 rows per lane) straight back as the next GEMM's
// k-operand without any lane shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "acc_layout.h"

namespace harp_ra {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxChunks = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Per-call description of the N KV chunks of the ring (passed by value).
struct ChunkTable {
  const bf16* k[kMaxChunks];  // chunk base pointers ([B,H,Tc,D] views, shared strides)
  const bf16* v[kMaxChunks];
  bf16* dk[kMaxChunks];       // backward outputs (same strides as dkv_strides)
  bf16* dv[kMaxChunks];
  int len[kMaxChunks];        // valid keys of chunk c
  int tile0[kMaxChunks];      // first 128-key tile index of chunk c (backward grid)
  int order[kMaxChunks];      // ring order: chunk visited at step s
  int n;                      // number of chunks (sp_size)
};

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// 16 x 16 x 32: lane L holds A row L % 16, B column L % 16, each with
// k = 8 (L / 16) .. + 7; C column L % 16, rows 4 (L / 16) .. + 3 (measured on
// the MI355X with an in-bounds probe, as v_permlane16_swap's lane exchange)
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// v_permlane16_swap on each dword of two fragments: afterwards x holds
// (x row 0, y row 0, x row 2, y row 2) and y (x row 1, y row 1, x row 3,
// y row 3), rows being the wave's four 16-lane groups
__device__ __forceinline__ void permlane16_swap(bf16x8& x, bf16x8& y) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  u32x4 a = __builtin_bit_cast(u32x4, x), b = __builtin_bit_cast(u32x4, y);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const auto r = __builtin_amdgcn_permlane16_swap(a[w], b[w], false, false);
    a[w] = r[0];
    b[w] = r[1];
  }
  x = __builtin_bit_cast(bf16x8, a);
  y = __builtin_bit_cast(bf16x8, b);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// exp2 clamped to [0, 1]: the median against (0, 1) folds into the clamp bit
// of v_exp_f32, so it costs no instruction.
__device__ __forceinline__ float exp2_unit(float x) {
  return __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(x), 0.f, 1.f);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.f;
  return z;
}

// Lane index computed anew (v_mbcnt) in an asm the compiler cannot merge with
// an earlier one: an epilogue that derives its lane-dependent indices from it
// keeps no such value live (or spilled) across the main loop.
// A wave-uniform 32-bit value in an SGPR, for an inline-asm "s" operand.  A
// value the compiler knows to be uniform but computes with VALU instructions
// (a float product, say) is otherwise handed to an asm statement in a VGPR
// whatever the constraint, and the assembler accepts that wherever only VALU
// instructions read the operand.  The volatile readfirstlane cannot be folded.
// The compiler's hazard pass does not look into the statement, so it waits
// itself: v_readfirstlane right after the VALU write of its source reads the
// old value (measured: without the wait some waves saw the multiplicand).
__device__ __forceinline__ uint32_t sgpr_of(float x) {
  uint32_t r;
  asm volatile("s_nop 4\n\tv_readfirstlane_b32 %0, %1" : "=s"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ int lane_id_fresh() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// c_row(r, g): row of the 32x32 C layout held in accumulator register r by
// lane-half g (acc_layout.h, shared with host code).

// ---------------------------------------------------------------------------
// Direct-to-LDS copies through buffer descriptors
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t rsrc_t __attribute__((ext_vector_type(4)));  // buffer resource (V#), SGPR quad

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every valid range: loads 0

// Raw buffer descriptor: base address, stride 0, num_records = bytes, and the
// dword-3 format word of an untyped buffer.  The base and size are
// wave-uniform by construction; readfirstlane tells the compiler so, which
// keeps the descriptor in SGPRs.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  rsrc_t r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;
  r.z = __builtin_amdgcn_readfirstlane(bytes);
  r.w = 0x00020000u;
  return r;
}

// Buffer resource over rows [row0, row0 + rows) of a [rows][stride] bf16 view.
__device__ __forceinline__ rsrc_t rows_rsrc(const bf16* base, int64_t stride, int row0, int rows) {
  return make_rsrc(base + (int64_t)row0 * stride, (uint32_t)((int64_t)(rows > 0 ? rows : 0) * stride * 2));
}

// One direct-to-LDS copy: every lane's 16 bytes at buffer offset voff land at
// LDS byte address lds + 16 * lane (M0 holds the wave-uniform base; one wait
// state separates the M0 write from its use).
// Issued as inline asm on purpose: the compiler cannot tell which LDS buffer
// an LDS-DMA load writes, so for the builtin it makes every later LDS read
// wait for the load (s_waitcnt vmcnt(0)), which turns the double-buffered
// prefetch into a synchronous load per tile.  Completion is instead ordered
// explicitly: wait_lds_loads() then a barrier, before any wave reads the
// buffer, and no load targets a buffer until a barrier shows that every wave
// has finished reading it.
__device__ __forceinline__ void lds_dma_b128(rsrc_t rs, uint32_t lds, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rs)
      : "memory", "m0");
}

// The same with 4 bytes per lane: lane i's dword lands at lds + 4 * i.
__device__ __forceinline__ void lds_dma_b32(rsrc_t rs, uint32_t lds, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rs)
      : "memory", "m0");
}

// Wait for this thread's direct-to-LDS loads (a barrier then publishes them).
__device__ __forceinline__ void wait_lds_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// The same but leaving this thread's last N vector-memory loads in flight
// (they complete in issue order): with three tile buffers, the copies of the
// tile after the next one stay outstanding while the next one is waited for.
template <int N>
__device__ __forceinline__ void wait_lds_loads_but() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Settle a value loaded from global memory before the main loop.  The
// direct-to-LDS loads are invisible to the compiler, but they count in the
// same hardware vmcnt: a wait the compiler places inside the loop for a
// prologue load would also wait for the tile loads just issued.  An asm that
// reads (and nominally rewrites) the value makes the compiler wait once,
// here, and leaves nothing for it to wait on inside the loop.
__device__ __forceinline__ void settle(bf16x8& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void settle(float& x) { asm volatile("" : "+v"(x)); }

// Scheduling fence: the compiler may not move any instruction across it.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// XOR swizzle of 16-byte chunks within a 256-byte LDS row: a permutation
// of the 16 chunk positions for any 16 consecutive rows.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Max / sum of a value over the two halves of the wave (lanes l and l ^ 32).
__device__ __forceinline__ float wave_half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Block index -> (tile, head, batch) with all tiles of one (b, h) kept on one
// XCD (workgroups are dealt to the 8 XCDs round-robin), so a head's streamed
// operands are fetched into that XCD's L2 once for all of its tiles.
__device__ __forceinline__ void decode_block(int n_tiles, int H, int& tile, int& h, int& b) {
  const int total = (int)gridDim.x;
  int lin = (int)blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  tile = lin % n_tiles;
  const int bh = lin / n_tiles;
  h = bh % H;
  b = bh / H;
}

// Position of a streamed KV tile in the ring: ring step, first key, and the
// visited chunk's valid length and K / V bases (offset to this (b, h)).  The
// cursor lives in scalar registers, so moving to the next tile reads the
// chunk table (kernel arguments: dependent scalar loads of ~200 cycles each)
// only when it crosses into the next chunk, not on every tile.
struct KvCursor {
  int step, k0, len;
  const bf16* k;
  const bf16* v;
};
// first non-empty chunk from ring step `step` on, before step `end`
// (step == end: past the end)
__device__ __forceinline__ void kv_enter(const ChunkTable& ct, int64_t kvo, int step, int end, KvCursor& c) {
  while (step < end && ct.len[ct.order[step]] == 0) ++step;
  c.step = step;
  c.k0 = 0;
  if (step < end) {
    const int ch = ct.order[step];
    c.len = ct.len[ch];
    c.k = ct.k[ch] + kvo;
    c.v = ct.v[ch] + kvo;
  }
}
// the tile after the one of tile_keys keys at c
__device__ __forceinline__ KvCursor kv_next(const ChunkTable& ct, int64_t kvo, const KvCursor& c, int tile_keys,
                                             int end) {
  KvCursor n = c;
  n.k0 = c.k0 + tile_keys;
  if (n.k0 >= c.len) kv_enter(ct, kvo, c.step + 1, end, n);
  return n;
}

// KV split (grid dimension y): split s of n visits ring steps
// [s * N / n, (s + 1) * N / n) and writes its results at offset s times the
// split stride of its output buffers (the host points those at per-split
// partial buffers; with n == 1 this is the whole ring and offset 0).
struct KvSplit {
  int begin, end, index;
};
__device__ __forceinline__ KvSplit kv_split(int n_chunks) {
  const int s = (int)blockIdx.y, n = (int)gridDim.y;
  return KvSplit{s * n_chunks / n, (s + 1) * n_chunks / n, s};
}

}  // namespace harp_ra
