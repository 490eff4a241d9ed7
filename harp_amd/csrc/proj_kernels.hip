// gfx950 kernel for the producer of the ring-attention block's q, k and v:
// the three Linear projections of the attention module with the QK RMSNorm
// and the rotary embedding fused into the GEMM epilogue.
//
// Reference (HARP's model code and async runtime, run on the CPU):
//   q = to_q(x), k = to_k(x), v = to_v(x)       src/models/z_image/module/attn.py:69-76
//                                               (nn.Linear, bias=False:
//                                               standalone_transformer.py:214-216)
//   q = norm_q(q), k = norm_k(k)                attn.py:78-81, RMSNorm over each
//                                               head's 128 features
//                                               (async_rt/csrc/rms_norm.cc:20-105)
//   q, k = RoPE(q, freqs), RoPE(k, freqs)       attn.py:83-89 (async_rt/csrc/rope.cc:9-86)
// Unfused, that is three GEMMs writing q, k, v, then a pass that reads q and k
// back, normalises, rotates and writes them again.  Here one launch computes
// every 256-token x 256-feature tile (two heads) of q, k and v, and finishes
// the tiles of q and k in registers before their only store.
//
// Numerics: fp32 accumulation of bf16 products; the product is rounded to
// bf16 to nearest (as the Linear layer's output is), then normalised and
// rotated exactly as the separate QK kernels do (qk_kernels.hip): fp32
// arithmetic, rms = sqrt(sum(x^2) / 128 + eps), out = trunc_bf16((x * (1 /
// rms)) * w), RoPE on the truncated values, truncated again.  The sum of
// squares is reduced in a different order than in the separate kernel.
//
// Tiling (C^T = W x^T, so a lane holds one token and 16 features per
// accumulator, the layout of the attention kernels):
//   block  = 8 waves, 2 heads (256 features) x 256 tokens; grid (token tiles
//            x head pairs, outputs);
//   wave   = 1 head (128 features) x 64 tokens: 4 x 2 v_mfma_f32_32x32x16_bf16
//            accumulators.  Per 16-element k-step it reads four W and two x
//            fragments (6 KB) from LDS for eight MFMAs, and a head's RMSNorm
//            needs no exchange between waves;
//   k-tile = 64 elements: x tile 256 x 64 and W tile 256 x 64 (32 KB each),
//            copied global -> LDS by buffer_load ... lds into two stages.
// Work units are 256-token x 2-head tiles.  When they leave the last round of
// the CUs at most half full (1152 units on 256 CUs at the headline shape: 4.5
// rounds), the units of that round run in a second launch as two 128-token
// halves each (the same kernel with 32 tokens per wave), which fill one round
// at half the time, instead of half the CUs idling through a whole one.
// Pipeline: one barrier per tile, in its last k-step, after which nobody
// reads tile t's stage any more (its last fragments are in registers) and
// tile t + 1 is complete; the copies of tile t + 2 then go into tile t's
// stage, between the MFMAs of that last k-step, and have until the barrier
// of the next tile to land.  Fragment reads run on across tile boundaries.
#include "proj_kernels.h"
#include "ra_common.h"

namespace harp_proj {

using harp_ra::bf16;
using harp_ra::bf16x8;
using harp_ra::f32x16;
using harp_ra::f32x4;
using harp_ra::lds_dma_b128;
using harp_ra::lds_void;
using harp_ra::make_rsrc;
using harp_ra::mfma32x32x16;
using harp_ra::rsrc_t;
using harp_ra::sched_fence;
using harp_ra::wait_lds_loads;
using harp_ra::zero16;

namespace {

constexpr int kWaves = 8;
constexpr int kStages = 2;
constexpr int kFeatures = kBlockHeads * kHeadDim;     // 256
constexpr int kRowBytes = kKTile * 2;                 // 128: one row of a tile
constexpr int kWBytes = kFeatures * kRowBytes;        // 32 KB
constexpr int kWPerWave = kWBytes / 1024 / kWaves;    // 1 KB copy instructions per wave and tile: 4
constexpr int kHeadPairGroup = 4;  // head pairs per group of the block order
static_assert(kWBytes % (1024 * kWaves) == 0, "copies split evenly");
static_assert(kStages * (kBlockTokens * kRowBytes + kWBytes) == kProjLdsBytes, "LDS budget");
static_assert(kWaves == 2 * (kBlockTokens / 64), "waves = heads x token groups of 64");

template <int I>
struct Int {
  static constexpr int value = I;
  constexpr operator int() const { return I; }
};

// Tile layout: rows of 64 bf16 (128 bytes = 8 chunks of 16 bytes); chunk c of
// row r sits at position c ^ ((r >> 1) & 7).  A fragment read (ds_read_b128,
// served 16 lanes per cycle: rows r0 .. r0 + 15 at one chunk, r0 % 16 == 0)
// then touches every 16-byte bank group of the 256-byte bank line once:
// r & 1 picks the half line and (r >> 1) & 7 a distinct position in it.
__device__ __forceinline__ int tile_pos(int r, int c) { return c ^ ((r >> 1) & 7); }

// Source byte offset (within the tile's rows) of 16-byte LDS slot `slot`:
// the copy instruction that fills slots 64 i .. 64 i + 63 reads rows
// 8 i .. 8 i + 7 whole (128 bytes each).  tile_pos is its own inverse for a
// fixed row, so position -> chunk is the same XOR.
__device__ __forceinline__ uint32_t slot_src(int slot, int64_t ld) {
  const int r = slot >> 3;
  return (uint32_t)(r * ld * 2 + tile_pos(r, slot & 7) * 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ uint32_t f32_to_bf16_trunc(float f) { return __float_as_uint(f) >> 16; }
// round to nearest even, as a Linear layer's bf16 output
__device__ __forceinline__ float round_bf16(float f) { return (float)(bf16)f; }
__device__ __forceinline__ uint32_t bf16_bits(float f) { return __float_as_uint(f) >> 16; }  // f exact in bf16

__device__ __forceinline__ float half_wave_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int NJ>
struct Frags {
  bf16x8 a[4];   // W rows: 32 features each (the wave's head)
  bf16x8 b[NJ];  // x rows: 32 tokens each
};

}  // namespace

// TPW tokens per wave (64: the main grid, 256-token blocks; 32: the tail,
// 128-token halves of the last round's units)
template <int TPW>
__global__ __launch_bounds__(64 * kWaves, 1) void proj_kernel(ProjParams p) {
  constexpr int NJ = TPW / 32;                            // 32-token blocks per wave
  constexpr int kTok = 4 * TPW;                           // tokens per block
  constexpr int kXBytes = kTok * kRowBytes;               // 32 or 16 KB
  constexpr int kXPerWave = kXBytes / 1024 / kWaves;      // 4 or 2
  constexpr int kDmaPerWave = kXPerWave + kWPerWave;      // 8 or 6 copies per tile
  constexpr int kMfma = 4 * NJ;                           // MFMAs per k-step
  static_assert(kXBytes % (1024 * kWaves) == 0, "copies split evenly");
  // the stages: x tiles, then W tiles; after the main loop each wave's
  // TPW x 256 bytes serve as its staging rows for the output stores
  __shared__ __attribute__((aligned(16))) char lds[kStages * (kXBytes + kWBytes)];
  __shared__ float norm_wf[kHeadDim];  // RMSNorm weight as fp32
  static_assert(kWaves * TPW * 2 * kHeadDim <= kStages * (kXBytes + kWBytes), "staging fits the stages");
  auto Xs = [&](int s) { return lds + s * kXBytes; };
  auto Ws = [&](int s) { return lds + kStages * kXBytes + s * kWBytes; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int hh = wave & 1, tg = wave >> 1;  // head of the pair, token group (TPW)

  // this block's unit (bid in the main grid's order) and output
  int bid, y, half = 0;
  if (TPW == 64) {
    bid = (int)blockIdx.x;
    y = (int)blockIdx.y;
    if (y == p.n_outs - 1 && bid >= p.keep_last) return;  // left to the tail launch
  } else {
    bid = p.tail_bid0 + (int)blockIdx.x / 2;
    half = (int)blockIdx.x & 1;
    y = p.n_outs - 1;
  }

  // block -> (token tile, head pair).  Workgroups are dealt to the 8 XCDs
  // round-robin; the remap gives each XCD a contiguous range of the order
  // below, which walks groups of 4 head pairs, within a group the token
  // tiles, and within a token tile the group's pairs.  The 32 blocks an XCD
  // runs at once then cover 8 token tiles x 4 head pairs, and per k-tile read
  // 12 tiles through its L2 (against 2 + 24 in token-tile-major order).
  const int n_hp = (p.heads + kBlockHeads - 1) / kBlockHeads;
  const int total = p.n_lin;
  int lin = bid;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  const int n_mt = total / n_hp;
  const int grp = lin / (n_mt * kHeadPairGroup), gs = min(kHeadPairGroup, n_hp - grp * kHeadPairGroup);
  const int rem = lin - grp * n_mt * kHeadPairGroup;
  const int mt = rem / gs, hp = grp * kHeadPairGroup + rem % gs;
  // (constant indices: a kernel-argument array indexed at run time would be
  // copied to scratch memory)
  const ProjOut o = y == 0 ? p.out[0] : (y == 1 ? p.out[1] : p.out[2]);
  const int m0 = mt * kBlockTokens + half * kTok;
  const int rows_x = min(kTok, p.M - m0);
  if (rows_x <= 0) return;  // the empty second half of a partial last token tile
  const int rows_w = min(kFeatures, (p.heads - hp * kBlockHeads) * kHeadDim);  // an odd last head
  const bf16* xb = (const bf16*)p.x + (int64_t)m0 * p.ldx;
  const bf16* wb = (const bf16*)o.w + (int64_t)hp * kFeatures * o.ldw;
  const uint32_t x_bytes = (uint32_t)((int64_t)rows_x * p.ldx * 2);
  const uint32_t w_bytes = (uint32_t)((int64_t)rows_w * o.ldw * 2);

  // this wave's copy instructions: x tile instructions wave + 8k, W tile
  // instructions wave + 8k (1 KB of LDS each)
  uint32_t xsrc[kXPerWave], wsrc[kWPerWave];
#pragma unroll
  for (int k = 0; k < kXPerWave; ++k) xsrc[k] = slot_src((wave + kWaves * k) * 64 + lane, p.ldx);
#pragma unroll
  for (int k = 0; k < kWPerWave; ++k) wsrc[k] = slot_src((wave + kWaves * k) * 64 + lane, o.ldw);
  // descriptors of tile t's rows: they start at column t * 64 and end past
  // the last valid row (rows beyond load 0); `live` false gives empty
  // ranges (the copies then write zeros and read nothing)
  auto x_rsrc = [&](int t, bool live) {
    const int k0 = t * kKTile;
    return make_rsrc(xb + k0, live ? x_bytes - (uint32_t)k0 * 2 : 0u);
  };
  auto w_rsrc = [&](int t, bool live) {
    const int k0 = t * kKTile;
    return make_rsrc(wb + k0, live ? w_bytes - (uint32_t)k0 * 2 : 0u);
  };
  // copy j (0 .. kDmaPerWave - 1) of a tile into stage s
  auto dma = [&](const rsrc_t& xr, const rsrc_t& wr, int s, int j) {
    if (j < kXPerWave) {
      const uint32_t dst = (uint32_t)(uintptr_t)(lds_void*)(Xs(s) + (wave + kWaves * j) * 1024);
      lds_dma_b128(xr, __builtin_amdgcn_readfirstlane(dst), xsrc[j]);
    } else {
      const uint32_t dst =
          (uint32_t)(uintptr_t)(lds_void*)(Ws(s) + (wave + kWaves * (j - kXPerWave)) * 1024);
      lds_dma_b128(wr, __builtin_amdgcn_readfirstlane(dst), wsrc[j - kXPerWave]);
    }
  };

  // lane part of a fragment's LDS offset at k-step ks: row l32 of a 32-row
  // block (block bases are multiples of 32 rows, which leave the swizzle
  // unchanged), chunk 2 ks + g
  int foff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) foff[ks] = l32 * kRowBytes + (tile_pos(l32, 2 * ks + g) << 4);
  auto load = [&](int s, int ks) {
    Frags<NJ> f;
    const char* xs = Xs(s) + tg * TPW * kRowBytes + foff[ks];
    const char* ws = Ws(s) + hh * kHeadDim * kRowBytes + foff[ks];
#pragma unroll
    for (int j = 0; j < NJ; ++j) f.b[j] = *(const bf16x8*)(xs + 32 * j * kRowBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = *(const bf16x8*)(ws + 32 * i * kRowBytes);
    return f;
  };

  f32x16 acc[4][NJ];  // [feature block][token block]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = zero16();
  // the MFMAs of one k-step, with a tile's copies (into stage s) spread
  // between them when `copy` is set
  auto mma = [&](const Frags<NJ>& f, bool copy, const rsrc_t& xr, const rsrc_t& wr, int s) {
#pragma unroll
    for (int u = 0; u < kMfma; ++u) {
      acc[u / NJ][u % NJ] = mfma32x32x16(f.a[u / NJ], f.b[u % NJ], acc[u / NJ][u % NJ]);
      if (copy) {
#pragma unroll
        for (int j = u * kDmaPerWave / kMfma; j < (u + 1) * kDmaPerWave / kMfma; ++j) dma(xr, wr, s, j);
      }
    }
  };

  // the RMSNorm weight, loaded now and moved to LDS after the main loop (an
  // ordinary load, older than every copy below: the copy waits also cover it)
  const bool norm = o.norm_w != nullptr;
  float wreg = 0.f;
  if (norm && tid < kHeadDim)
    wreg = o.norm_w_f32 ? ((const float*)o.norm_w)[tid] : bf16_bits_to_f32(((const uint16_t*)o.norm_w)[tid]);

  const int nt = p.K / kKTile;
  // prologue: tiles 0 and 1 in flight, tile 0 published
  {
    const rsrc_t x0 = x_rsrc(0, true), w0 = w_rsrc(0, true);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) dma(x0, w0, 0, j);
    const rsrc_t x1 = x_rsrc(1, nt > 1), w1 = w_rsrc(1, nt > 1);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) dma(x1, w1, 1, j);
    // this wave's copies of tile 0 (tile 1's may stay in flight)
    if constexpr (kDmaPerWave == 8) {
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else {
      static_assert(kDmaPerWave == 6, "prologue wait");
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    }
  }
  __syncthreads();
  Frags<NJ> f0 = load(0, 0), f1;

  // tile t in stage S (a compile-time constant: the loop is unrolled over the
  // two stages).  After the last tile the fragment reads of "tile t + 1"
  // read a stale stage and the copies of "tile t + 2" are empty: both stay in
  // bounds, their results are never used, and the loop has no branches.
  auto tile = [&](auto SC, int t) {
    constexpr int S = decltype(SC)::value, S1 = S ^ 1;
    f1 = load(S, 1);
    sched_fence();
    mma(f0, false, {}, {}, S);
    sched_fence();
    f0 = load(S, 2);
    sched_fence();
    mma(f1, false, {}, {}, S);
    sched_fence();
    f1 = load(S, 3);
    sched_fence();
    mma(f0, false, {}, {}, S);
    sched_fence();
    // every wave has its last fragments of tile t (the barrier waits for
    // their reads), and tile t + 1 is complete: its copies were issued in the
    // last k-step of tile t - 1
    wait_lds_loads();
    __syncthreads();
    const bool more2 = t + 2 < nt;
    const rsrc_t xr = x_rsrc(t + 2, more2), wr = w_rsrc(t + 2, more2);
    f0 = load(S1, 0);
    sched_fence();
    mma(f1, true, xr, wr, S);  // tile t + 2 into tile t's stage
    sched_fence();
  };
#pragma unroll 1
  for (int t = 0; t < nt; t += kStages) {
    tile(Int<0>{}, t);
    if (t + 1 < nt) tile(Int<1>{}, t + 1);
  }
  // the last tiles issued (empty) copies; none may still write the LDS when
  // the workgroup ends
  wait_lds_loads();
  if (norm && tid < kHeadDim) norm_wf[tid] = wreg;
  // every wave is past its fragment reads: the stages become staging rows
  __syncthreads();

  // ---- epilogue: this lane holds tokens m0 + TPW tg + 32 j + l32 and
  // features 32 i + c_row(r, g) of head h, i in 0..3, j < NJ
  const int h = hp * kBlockHeads + hh;
  if (h >= p.heads) return;
  const int lane_e = harp_ra::lane_id_fresh(), l32e = lane_e & 31, ge = lane_e >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = round_bf16(acc[i][j][r]);

  // Output stores go through LDS: the wave's TPW rows of 256 bytes (its
  // head's 128 bf16 features per token), 16-byte chunk c of row r at position
  // c ^ (r & 15), then out 16 bytes per lane, 16 lanes per token row.  Its
  // own rows only, and LDS operations of one wave stay in order: no barrier.
  char* const stg = lds + wave * (TPW * 2 * kHeadDim);
  auto stage_put = [&](int j, int i, int q, uint32_t lo, uint32_t hi) {  // features 32i + 8q + 4g ..
    const int r = 32 * j + l32e;
    *(uint2*)(stg + r * 256 + (((4 * i + q) ^ (r & 15)) << 4) + ge * 8) = make_uint2(lo, hi);
  };
  auto stage_flush = [&](uint16_t* base) {
#pragma unroll
    for (int k = 0; k < TPW / 4; ++k) {
      const int r = 4 * k + (lane_e >> 4), c = lane_e & 15;
      const uint4 v = *(const uint4*)(stg + r * 256 + ((c ^ (r & 15)) << 4));
      const int64_t m = m0 + TPW * tg + r;
      if (m < p.M) *(uint4*)(base + m * o.ldy + h * kHeadDim + c * 8) = v;
    }
  };
  auto put_rounded = [&]() {  // the bf16 products
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          stage_put(j, i, q, bf16_bits(acc[i][j][4 * q]) | (bf16_bits(acc[i][j][4 * q + 1]) << 16),
                    bf16_bits(acc[i][j][4 * q + 2]) | (bf16_bits(acc[i][j][4 * q + 3]) << 16));
  };
  if (!norm) {
    put_rounded();
    stage_flush(o.y);
    return;
  }

  // RoPE table row of the lane's token in token block j, pairs d0 / 2 ..
  // d0 / 2 + 1 for the 16 groups d0 = 32 i + 8 q + 4 g (one token block at
  // a time: both would not fit beside the accumulators)
  const bool rope = p.freqs != nullptr;
  f32x4 fq[4][4];
  auto load_freqs = [&](int j) {
    const int64_t m = min((int64_t)m0 + TPW * tg + 32 * j + l32e, (int64_t)p.M - 1);
    const int b = (int)(m / p.S), s = (int)(m % p.S);
    const float* fr = p.freqs + (int64_t)b * p.f_stride_b + (int64_t)s * p.f_stride_s;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) fq[i][q] = *(const f32x4*)(fr + 32 * i + 8 * q + 4 * ge);
  };
  // loaded before any store (a load issued after a store would wait for it)
  if (rope) load_freqs(0);
  if (o.y_lin) {
    put_rounded();
    stage_flush(o.y_lin);
  }

  // RMSNorm: sum of squares over the head's 128 features = this lane's 64 +
  // its partner lane's 64 (the other half of the wave); both get the same sum
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (rope && j > 0) load_freqs(j);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss = __builtin_fmaf(acc[i][j][r], acc[i][j][r], ss);
    ss = half_wave_sum(ss);
    const float rms = __fsqrt_rn(__fdiv_rn(ss, (float)kHeadDim) + o.eps);
    const float inv = __fdiv_rn(1.f, rms);
    const int64_t m = m0 + TPW * tg + 32 * j + l32e;
    if (ge == 0 && o.rms && m < p.M) {
      const int b = (int)(m / p.S), s = (int)(m % p.S);
      o.rms[((int64_t)b * p.heads + h) * p.S + s] = rms;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d0 = 32 * i + 8 * q + 4 * ge;
        const f32x4 w = *(const f32x4*)(norm_wf + d0);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = bf16_bits_to_f32(f32_to_bf16_trunc(__fmul_rn(__fmul_rn(acc[i][j][4 * q + e], inv), w[e])));
        if (rope) {
          // pairs (d0, d0 + 1) and (d0 + 2, d0 + 3): RoPE pairs d0 / 2 and d0 / 2 + 1
          const f32x4 f = fq[i][q];
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            const float xr = y[e], xi = y[e + 1], cr = f[e], ci = f[e + 1];
            y[e] = __builtin_fmaf(-xi, ci, __fmul_rn(xr, cr));
            y[e + 1] = __builtin_fmaf(xi, cr, __fmul_rn(xr, ci));
          }
        }
        stage_put(j, i, q, f32_to_bf16_trunc(y[0]) | (f32_to_bf16_trunc(y[1]) << 16),
                  f32_to_bf16_trunc(y[2]) | (f32_to_bf16_trunc(y[3]) << 16));
      }
  }
  stage_flush(o.y);
}

namespace {
// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cached[dev] = n;
  }
  return cached[dev];
}
}  // namespace

hipError_t launch_proj(const ProjParams& p_in, hipStream_t stream) {
  ProjParams p = p_in;
  const int n_mt = (p.M + kBlockTokens - 1) / kBlockTokens;
  const int n_hp = (p.heads + kBlockHeads - 1) / kBlockHeads;
  const int L = n_mt * n_hp;
  p.n_lin = L;
  p.keep_last = L;
  p.tail_bid0 = L;
  // units left over for the last round of the CUs: when they fill at most
  // half of it, run them as 128-token halves in a second launch
  const int cus = device_cus();
  const int64_t units = (int64_t)p.n_outs * L;
  const int r = cus > 0 ? (int)(units % cus) : 0;
  const bool split = r > 0 && 2 * r <= cus && units > cus && r <= L;
  if (split) p.keep_last = p.tail_bid0 = L - r;
  hipLaunchKernelGGL(proj_kernel<64>, dim3((unsigned)L, (unsigned)p.n_outs), dim3(64 * kWaves), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  hipLaunchKernelGGL(proj_kernel<32>, dim3((unsigned)(2 * r)), dim3(64 * kWaves), 0, stream, p);
  return hipGetLastError();
}

}  // namespace harp_proj
