// gfx950 kernels for the ring-attention block, forward and backward.
//
// Reference math: gemm/ring_attention/ring_attn.cpp
//   forward  ring_attention_forward   :2412-2575  (Q-stationary online softmax over KV chunks)
//   backward ring_attention_backward  :2577-2829  (S/dP recompute, P = exp(S-m)/l, dS, dQ/dK/dV)
// D = rowsum(dO * O) is the caller's preprocess (src/models/z_image/module/attn.py:41).
//
// Work split on one GPU (one rank's share, all ring steps in one launch each):
//   fwd_kernel    per 256-query tile: S^T = K Q^T -> online softmax (lane = query)
//                 -> O^T += V^T P^T, over every 64-key tile of every chunk in ring order.
//   delta_kernel  D = rowsum(dO * O) (fp32).
//   dq_kernel     per 256-query tile: recompute S^T, dP^T, dS^T; dQ^T += K^T dS^T.
//   dkdv_kernel   per 256-key block (KV-stationary like the reference): per 64-query
//                 tile recompute S, dP; dV += P^T dO, dK += dS^T Q.
//
// Memory path: every streamed 64-row tile is copied global -> LDS by
// buffer_load_dwordx4 ... lds (no register staging).  The buffer range check
// zero-fills rows past a chunk's valid length and columns past D.  Two LDS
// buffers alternate: after the barrier that publishes tile t, the loads of
// tile t+1 go into the buffer every wave has finished reading, and overlap
// the MFMA work on tile t.  Within each MFMA phase the LDS operand fragments
// are issued two steps ahead of the MFMAs that consume them.
// Accumulation is fp32 in registers; P and dS are rounded to bf16 only as
// MFMA operands; exp is v_exp_f32 (exp2) with log2(e) folded into the scale.
#include "cq_epilogue.h"
#include "ra_common.h"
#include "ra_kernels.h"

namespace harp_ra {


// LDS is 64 banks x 4 bytes (256 bytes per cycle); 16-byte accesses are
// served 16 lanes per cycle, 8-byte accesses 32 lanes per cycle.  Two tile
// layouts, both free of bank conflicts for the accesses they get:
//  * PadTile (tiles read only as MFMA row fragments): rows padded to DP+8
//    elements, so 16 consecutive rows start 16 bytes apart modulo 256 and a
//    16-row x one-chunk ds_read_b128 touches every bank once; every fragment
//    offset is a per-lane base plus an immediate.
//  * XorTile (tiles also read transposed): 256-byte rows, chunk c of row r at
//    position c ^ swz(r) with swz(r) = 4*(r%4) + (r/4)%4, a permutation over
//    any 16 rows.  Row reads (16 rows x one chunk) and ds_read_b64_tr_b16
//    (rows r0+4g+{0..3} x chunks 4db+{0..3} -> positions
//    4*(db ^ (r%4)) + ((c%4) ^ ((r/4)%4))) hit distinct banks.
// Both are written by direct-to-LDS loads: one wave instruction fills 64
// consecutive 16-byte slots; slot() maps a slot to its (row, chunk).

template <int DP>
struct XorTile {
  static constexpr int W = 128;
  static constexpr int NCH = DP / 8;  // 16-byte data chunks per row
  static constexpr int ELEMS = 64 * W;
  static constexpr int SLOTS = ELEMS / 8;
  static __device__ __forceinline__ void slot(int s, int& r, int& c) {
    r = s >> 4;
    c = (s & 15) ^ swz(r);
  }
};

template <int DP>
struct PadTile {
  static constexpr int W = DP + 8;
  static constexpr int NCH = DP / 8;
  static constexpr int SPR = W / 8;  // slots per row (the last one is padding)
  static constexpr int ELEMS = 64 * W;
  static constexpr int SLOTS = ELEMS / 8;
  static __device__ __forceinline__ void slot(int s, int& r, int& c) {
    r = s / SPR;
    c = s % SPR;
  }
};


// This wave's share of the direct-to-LDS copies of one 64-row tile: slot
// instruction i (64 slots) goes to waves round-robin; voff holds each lane's
// byte offset (relative to the tile's first row) or kOOB for padding slots
// and columns past D, which the range check turns into zeros.
//
// Pair (head dims <= 64, G an XorTile<128>): the tile holds 128 rows of at
// most 64 columns, row R at physical row R % 64 in chunks 8 (R / 64) + 0..7,
// so that every slot of every copy carries data and 128 rows take the LDS of
// 64.  Row fragments of rows 64 + x are those of row x at k-step ks + 4, and
// transposed fragments at d block db + 2.
template <class G, int NW, bool Pair = false>
struct DirectLoader {
  static constexpr int kInstTot = G::SLOTS / 64;
  static constexpr int kInst = (kInstTot + NW - 1) / NW;
  uint32_t voff[kInst];
  int wave;
  __device__ __forceinline__ void init(int64_t row_stride, int D, int wave_, int lane) {
    wave = wave_;
#pragma unroll
    for (int k = 0; k < kInst; ++k) {
      const int inst = wave + k * NW;
      int r, c;
      G::slot(inst * 64 + lane, r, c);
      if constexpr (Pair) {
        const int dc = c & 7;  // data chunk of row r + 64 (c / 8)
        const bool ok = inst < kInstTot && dc * 8 < D;
        voff[k] = ok ? (uint32_t)((r + 64 * (c >> 3)) * row_stride * 2 + dc * 16) : kOOB;
      } else {
        const bool ok = inst < kInstTot && c < G::NCH && c * 8 < D;
        voff[k] = ok ? (uint32_t)(r * row_stride * 2 + c * 16) : kOOB;
      }
    }
  }
  // this wave's k-th copy instruction of the tile (k < kInst)
  __device__ __forceinline__ void load_one(rsrc_t rs, bf16* tile, int k) const {
    const int inst = wave + k * NW;
    if (kInstTot % NW == 0 || inst < kInstTot) {
      const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)(tile + inst * 512);
      lds_dma_b128(rs, __builtin_amdgcn_readfirstlane(lds), voff[k]);
    }
  }
  __device__ __forceinline__ void load(rsrc_t rs, bf16* tile) const {
#pragma unroll
    for (int k = 0; k < kInst; ++k) load_one(rs, tile, k);
  }
};

// Row fragment T[rb*32 + l32][16*ks + 8*g .. +7] of a PadTile: per-lane base,
// immediate per (rb, ks).
template <int DP>
struct PadRows {
  using G = PadTile<DP>;
  int base;
  __device__ __forceinline__ void init(int lane) { base = (lane & 31) * G::W + 8 * (lane >> 5); }
  __device__ __forceinline__ bf16x8 frag(const bf16* t, int rb, int ks) const {
    return *(const bf16x8*)(t + base + rb * 32 * G::W + ks * 16);
  }
};

// Lane offsets for the two read patterns of an XorTile.
template <int DP, int KSTEPS>
struct XorLanes {
  using G = XorTile<DP>;
  static constexpr int NDB = DP / 32;
  // row reads: T[rb*32 + l32][16*ks + 8*g .. +7] at rb*32*W + row_off[ks]
  int row_off[KSTEPS];
  // transposed reads: rows r0 + 8*hh + 4g + s, columns 32*db + l32 (r0 % 16 == 0)
  //   at r0*W + tr_off[hh][db]
  int tr_off[2][NDB];
  __device__ __forceinline__ void init(int lane, bool rows = true) {
    const int l32 = lane & 31, g = lane >> 5;
    if (rows) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) row_off[ks] = l32 * G::W + (((2 * ks + g) ^ swz(l32)) << 3);
    }
    const int j = lane >> 4, s = (lane >> 2) & 3, m = lane & 3;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 8 * hh + 4 * g + s;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        tr_off[hh][db] = row * G::W + (((4 * db + cl) ^ swz(row)) << 3) + 4 * (m & 1);
    }
  }
  __device__ __forceinline__ bf16x8 row_frag(const bf16* t, int rb, int ks) const {
    return *(const bf16x8*)(t + rb * 32 * G::W + row_off[ks]);
  }
  // the same row fragment from two per-lane registers (row base and
  // swizzle) instead of KSTEPS offsets: (2ks + g) ^ swz(l32) = 2ks ^ (g ^ swz(l32))
  int row_base, row_x;
  // transposed reads from NDB offsets plus one per-lane delta: the hh = 1
  // offset differs from hh = 0 by 8 rows and by flipping bit 1 of the chunk
  // index, the same for every db
  int tr_lean[NDB], tr_delta;
  __device__ __forceinline__ void init_tr_lean(int lane) {
    const int g = lane >> 5, j = lane >> 4, s = (lane >> 2) & 3, m = lane & 3;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int row = 4 * g + s;
      tr_lean[db] = row * G::W + (((4 * db + cl) ^ swz(row)) << 3) + 4 * (m & 1);
    }
    const int row1 = 8 + 4 * g + s;
    tr_delta = row1 * G::W + (((cl) ^ swz(row1)) << 3) - ((4 * g + s) * G::W + (((cl) ^ swz(4 * g + s)) << 3));
  }
  __device__ __forceinline__ bf16x8 tr_frag_lean(const bf16* t, int r0, int db) const {
    const bf16* p0 = t + r0 * G::W + tr_lean[db];
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p0);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + tr_delta));
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = lo[i];
      r[i + 4] = hi[i];
    }
    return r;
  }
  __device__ __forceinline__ void init_rows_lean(int lane) {
    const int l32 = lane & 31, g = lane >> 5;
    row_base = l32 * G::W;
    row_x = g ^ swz(l32);
  }
  __device__ __forceinline__ bf16x8 row_frag_lean(const bf16* t, int rb, int ks) const {
    return *(const bf16x8*)(t + rb * 32 * G::W + row_base + (((2 * ks) ^ row_x) << 3));
  }
  // k-operand fragment read transposed: T[r0 + {4g+0..3, 8+4g+0..3}][32*db + l32]
  // ds_read_b64_tr_b16: in each 16-lane group, lane i slot s' receives element
  // i%4 of the 8 bytes addressed by lane 4s' + i/4 of that group.
  __device__ __forceinline__ bf16x8 tr_frag(const bf16* t, int r0, int db) const {
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + r0 * G::W + tr_off[0][db]));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + r0 * G::W + tr_off[1][db]));
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = lo[i];
      r[i + 4] = hi[i];
    }
    return r;
  }
};


// Wave issue priority (s_setprio, 0..3) within a tile.  Two waves share a
// SIMD and the issue arbiter otherwise favours the older one, which then
// runs a whole phase ahead and idles at the next barrier while its partner
// finishes alone.  The level falls as a wave moves through the tile, so the
// wave that lags gets precedence and both reach the barrier together.
template <int LEVEL>
__device__ __forceinline__ void prio() {
  __builtin_amdgcn_s_setprio(LEVEL);
}


// Compile-time step index: converts to int, and generic lambdas can read it
// as a constant expression (decltype(i)::value).
template <int I>
struct Int {
  static constexpr int value = I;
  constexpr operator int() const { return I; }
};

// N MFMA steps whose LDS operand fragments are issued PF steps ahead:
// load(i) returns step i's fragments, mma(i, frags) issues its MFMAs.  The
// fences keep each step's reads above the MFMAs of the earlier steps, so the
// s_waitcnt before an MFMA leaves the later reads in flight.  The steps are
// expanded by template recursion, so every step index is a compile-time
// constant however long the pipeline is.
template <int I, int N, int PF, class Load, class Mma, class F>
__device__ __forceinline__ void pipeline_steps(const Load& load, const Mma& mma, F* f) {
  if constexpr (I < N) {
    if constexpr (I + PF < N) f[(I + PF) % (PF + 1)] = load(Int<I + PF>{});
    sched_fence();
    mma(Int<I>{}, f[I % (PF + 1)]);
    sched_fence();
    pipeline_steps<I + 1, N, PF>(load, mma, f);
  }
}
template <int I, int N, class Load, class F>
__device__ __forceinline__ void pipeline_fill(const Load& load, F* f) {
  if constexpr (I < N) {
    f[I] = load(Int<I>{});
    pipeline_fill<I + 1, N>(load, f);
  }
}
template <int N, int PF, class Load, class Mma>
__device__ __forceinline__ void pipelined(const Load& load, const Mma& mma) {
  using F = decltype(load(Int<0>{}));
  F f[PF + 1];
  pipeline_fill<0, (PF < N ? PF : N)>(load, f);
  pipeline_steps<0, N, PF>(load, mma, f);
}

struct Frag2 {
  bf16x8 a, b;
};
struct Frag3 {
  bf16x8 a, b, c;
};

// DPP row_newbcast:R -- every lane of each 16-lane row receives lane R of
// that row.  With x[l] = v(l % 16, l / 32) (rows 0,1 equal; rows 2,3 equal),
// lane l receives v(R, l / 32): a per-register value that depends only on
// the lane's half of the wave, without LDS traffic.
template <int R>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + R, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_bcast(float x, int r) {  // r must fold to a constant
  switch (r) {
    case 0: return row_bcast<0>(x);
    case 1: return row_bcast<1>(x);
    case 2: return row_bcast<2>(x);
    case 3: return row_bcast<3>(x);
    case 4: return row_bcast<4>(x);
    case 5: return row_bcast<5>(x);
    case 6: return row_bcast<6>(x);
    case 7: return row_bcast<7>(x);
    case 8: return row_bcast<8>(x);
    case 9: return row_bcast<9>(x);
    case 10: return row_bcast<10>(x);
    case 11: return row_bcast<11>(x);
    case 12: return row_bcast<12>(x);
    case 13: return row_bcast<13>(x);
    case 14: return row_bcast<14>(x);
    default: return row_bcast<15>(x);
  }
}


// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// Block = 8 waves x 32 queries (two waves per SIMD, one block per CU): every
// K / V tile copied into LDS serves 256 queries, which halves the LDS-DMA
// writes per MFMA against two 4-wave blocks per CU.
constexpr int kFwdWaves = 8;
constexpr int kFwdRows = 32 * kFwdWaves;
static_assert(kFwdRows == kQueryBlockRows, "the host sizes KV splits with kQueryBlockRows");
// Keys per tile = 64 * kFwdSub: fewer barriers, pipeline fills and rescale
// tests per key; the block's LDS holds two such K / V tiles.
constexpr int kFwdSub = 2;
// KSTEPS = ceil(D/16) k-steps of the S contraction; DBLK = ceil(D/32) row
// blocks of O^T (DP = 32*DBLK >= 16*KSTEPS).  Block = kFwdWaves waves x 32 queries;
// 64*kFwdSub-key tiles (kFwdSub 64-row LDS sub-tiles).
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(64 * kFwdWaves, 1) void fwd_kernel(FwdParams p) {
  constexpr int DP = DBLK * 32;
  // At 5 k-steps (head dims 72 and 80) the last d block of O^T is 16 wide:
  // 16 x 16 x 32 MFMAs over d 64-79, as in dkdv_kernel and dq_kernel.
  constexpr bool kTail = KSTEPS == 5 && DBLK == 3;
  constexpr int DBF = kTail ? DBLK - 1 : DBLK;  // 32-wide d blocks
  constexpr int DPE = kTail ? 80 : DP;          // d columns the tiles and outputs hold
  // Head dims <= 64: a tile's 128 K (V) rows share one LDS tile in the
  // pair layout (DirectLoader), half the LDS and half the copy instructions,
  // and three buffers let each tile's copies be issued two tiles ahead
  // instead of one: at these head dims a tile's MFMA work is short against
  // the copies' memory latency.
  constexpr bool kPair = DPE <= 64;
  using GK = XorTile<kPair ? 128 : DPE>;  // K: row fragments only
  using GV = XorTile<kPair ? 128 : DPE>;  // V: transposed fragments
  constexpr float kTauExp = 256.f;  // lazy-rescale threshold: a lane's tile sum of P above 2^8
  constexpr int TK = 64 * kFwdSub, KB = TK / 32;  // keys and 32-key blocks per tile
  constexpr int NS = kPair ? 1 : kFwdSub;         // LDS tiles (64 rows, or 128 paired) per buffer
  constexpr int NB = kPair ? 3 : 2;               // buffers
  __shared__ __attribute__((aligned(16))) bf16 Ks[NB][NS][GK::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Vs[NB][NS][GV::ELEMS];

  // the wave index is wave-uniform; readfirstlane lets the compiler keep it in an SGPR
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  int qt, h, b;
  decode_block((p.T + kFwdRows - 1) / kFwdRows, p.H, qt, h, b);
  const KvSplit sp = kv_split(p.ct.n);
  const int qi = qt * kFwdRows + wave * 32 + l32;
  const bool q_ok = qi < p.T;
  const float c2 = p.scale * kLog2e;

  bf16x8 qf[KSTEPS];
  {
    const bf16* qrow = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh + (int64_t)qi * p.sqt;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int d0 = ks * 16 + g * 8;
      qf[ks] = (q_ok && d0 < p.D) ? *(const bf16x8*)(qrow + d0) : zero8();
    }
  }
  XorLanes<DPE, KSTEPS> klo;
  klo.init_rows_lean(lane);
  XorLanes<kPair ? 128 : DPE, KSTEPS> vlo;  // paired: d blocks 2-3 address rows 64-127
  vlo.init(lane, false);
  // V^T tail fragments (A operands of the tail MFMAs): lane group G = lane /
  // 16 takes keys 16 (1 - G % 2) + 4 (G / 2) + {0..3, 8..11} of a 32-key
  // block, the order v_permlane16_swap leaves the P^T B operands in, row d =
  // 64 + lane % 16 (as dq_kernel's K^T tail)
  int tail_off[2] = {0, 0};
  if constexpr (kTail) {
    const int G = lane >> 4, j = lane & 15;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 16 * (1 - (G & 1)) + 8 * hh + 4 * (G >> 1) + (j >> 2);
      tail_off[hh] = row * GV::W + (((8 + ((j & 3) >> 1)) ^ swz(row)) << 3) + 4 * (j & 1);
    }
  }
  using LK = DirectLoader<GK, kFwdWaves, kPair>;
  using LV = DirectLoader<GV, kFwdWaves, kPair>;
  static_assert(!kPair || (LK::kInstTot % kFwdWaves == 0 && LV::kInstTot % kFwdWaves == 0),
                "every wave issues the same number of copies (the paired wait counts them)");
  LK kld;
  kld.init(p.skt, p.D, wave, lane);
  LV vld;
  vld.init(p.skt, p.D, wave, lane);

  f32x16 o[DBF];
#pragma unroll
  for (int i = 0; i < DBF; ++i) o[i] = zero16();
  // the 16-wide tail (kTail): d 64-79 x queries 16 u .. 16 u + 15 of the
  // wave's 32, 16 x 16 C layout (column = query 16 u + lane % 16, rows d =
  // 64 + 4 (lane / 16) + i): a lane's tail values belong to another lane's
  // query, whose statistics it fetches (__shfl) when it scales them
  f32x4 ot[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) ot[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // reference point of P (log2 domain): the first keys of a row overflow
  // their exps against -FLT_MAX, which makes the tile rescale
  float m_ref = -__FLT_MAX__;
  float l_run = 0.f;  // this lane-half's partial sum of exp2(s*c2 - m_ref)

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  auto issue = [&](const KvCursor& t, int bf) {
#pragma unroll
    for (int sb = 0; sb < NS; ++sb) {
      const int r0 = t.k0 + 64 * sb, rows = t.len - r0;
      kld.load(rows_rsrc(t.k, p.skt, r0, rows), Ks[bf][sb]);
      vld.load(rows_rsrc(t.v, p.skt, r0, rows), Vs[bf][sb]);
    }
  };
  // Inside the loop the next tile's copies are issued spread over the S^T
  // MFMA steps (slot j at step j * kSlotStride) rather than in one burst
  // after the barrier: a burst fills the texture unit's FIFOs, and a wave
  // stalled on issuing a copy cannot issue MFMAs.  Slot j: sub-tile
  // j / kSlotsPerSub, K copies first, then V copies.
  constexpr int kSlotsK = LK::kInst, kSlotsV = LV::kInst;
  constexpr int kSlotsPerSub = kSlotsK + kSlotsV, kDmaSlots = NS * kSlotsPerSub;
  constexpr int kSSteps = KB * KSTEPS, kSlotStride = kSSteps / kDmaSlots > 0 ? kSSteps / kDmaSlots : 1;
  constexpr int kSlotsPerStep = (kDmaSlots + kSSteps - 1) / kSSteps;
  rsrc_t nk_rs[NS], nv_rs[NS];
  auto dma_slot = [&](int j, int bf) {
    const int sb = j / kSlotsPerSub, k = j % kSlotsPerSub;
    if (k < kSlotsK) kld.load_one(nk_rs[sb], Ks[bf][sb], k);
    else vld.load_one(nv_rs[sb], Vs[bf][sb], k - kSlotsK);
  };
  KvCursor cur;
  kv_enter(p.ct, kvo, sp.begin, sp.end, cur);
  int buf = 0;
  if (cur.step < sp.end) issue(cur, 0);
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) settle(qf[ks]);
  // kPair: the tile after cur, whose copies are in flight while cur runs
  KvCursor nx1 = cur;
  if constexpr (kPair) {
    nx1 = kv_next(p.ct, kvo, cur, TK, sp.end);
    if (nx1.step < sp.end) issue(nx1, 1);
  }
#pragma unroll 1
  while (cur.step < sp.end) {
    const int kv_left = cur.len - cur.k0;
    const KvCursor nxt = kPair ? nx1 : kv_next(p.ct, kvo, cur, TK, sp.end);
    // the tile whose copies this one issues (nxt, or the one after it) and its buffer
    const KvCursor pre = kPair ? kv_next(p.ct, kvo, nxt, TK, sp.end) : nxt;
    const int pbuf = kPair ? (buf == 0 ? 2 : buf - 1) : (buf ^ 1);
    if (kPair && nxt.step < sp.end) wait_lds_loads_but<kDmaSlots>();  // nxt's copies may stay in flight
    else wait_lds_loads();
    __syncthreads();
    const bool has_next = pre.step < sp.end;
    if (has_next) {
#pragma unroll
      for (int sb = 0; sb < NS; ++sb) {
        const int r0 = pre.k0 + 64 * sb, rows = pre.len - r0;
        nk_rs[sb] = rows_rsrc(pre.k, p.skt, r0, rows);
        nv_rs[sb] = rows_rsrc(pre.v, p.skt, r0, rows);
      }
    }
    prio<3>();
    // S^T (keys x queries), KB 32-key blocks; step i = (ks = i / KB, kb = i % KB)
    f32x16 s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s[kb] = zero16();
    pipelined<KB * KSTEPS, 2>([&](int i) {
                                if constexpr (kPair)  // rows 64-127 at k-steps 4-7 of the paired tile
                                  return klo.row_frag_lean(Ks[buf][0], i & 1, i / KB + 4 * ((i % KB) / 2));
                                else
                                  return klo.row_frag_lean(Ks[buf][(i % KB) / 2], i & 1, i / KB);
                              },
                              [&](int i, const bf16x8& a) {
                                s[i % KB] = mfma32x32x16(a, qf[i / KB], s[i % KB]);
                                if (has_next && i % kSlotStride == 0) {
#pragma unroll
                                  for (int u = 0; u < kSlotsPerStep; ++u) {
                                    const int j = (i / kSlotStride) * kSlotsPerStep + u;
                                    if (j < kDmaSlots) dma_slot(j, pbuf);
                                  }
                                }
                              });
    if (kv_left < TK) {  // tail tile of a chunk: mask keys past its valid length
      // a side-effecting (empty) asm keeps this a real uniform branch instead
      // of selects that would run on every tile
      asm volatile("");
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb * 32 + c_row(r, g) >= kv_left) s[kb][r] = -INFINITY;
    }

    prio<2>();
    // online softmax, lane = query: the exps run against the current
    // reference point at once, and the test looks at their sum.  A lane
    // whose tile sum passes 2^8 (some exp above it, or overflowed) makes the
    // wave move its reference points up to the tile's row maxima, rescale O
    // and l, and compute the tile's exps again; otherwise every exp is at
    // most 2^8.  No max / compare chain runs before the exps.
    bf16x8 pf[2 * KB];
    auto tile_exps = [&]() {
      float bs = 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float e = fast_exp2(__builtin_fmaf(s[kb][hf * 8 + j], c2, -m_ref));
            bs += e;
            pf[kb * 2 + hf][j] = (bf16)e;
          }
      return bs;
    };
    float bs = tile_exps();
    if (__any(bs > kTauExp)) {  // rare: the first tile of a row, or a jump of the row max
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      const float m_new = fmaxf(m_ref, wave_half_max(mx) * c2);
      const float corr = fast_exp2(m_ref - m_new);
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < DBF; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= corr;
      if constexpr (kTail) {
#pragma unroll
        for (int u = 0; u < 2; ++u) ot[u] *= __shfl(corr, 16 * u + (lane & 15));
      }
      m_ref = m_new;
      bs = tile_exps();
    }
    l_run += bs;

    prio<1>();
    // O^T += V^T P^T; step i = (ks2 = i / DBF, db = i % DBF), 16 keys per ks2
    pipelined<2 * KB * DBF, 2>(
        [&](int i) {
          if constexpr (kPair)  // rows 64-127 at d blocks 2-3 of the paired tile
            return vlo.tr_frag(Vs[buf][0], ((i / DBF) % 4) * 16, i % DBF + 2 * ((i / DBF) / 4));
          else
            return vlo.tr_frag(Vs[buf][(i / DBF) / 4], ((i / DBF) % 4) * 16, i % DBF);
        },
        [&](int i, const bf16x8& a) { o[i % DBF] = mfma32x32x16(a, pf[i / DBF], o[i % DBF]); });
    if constexpr (kTail) {
      // per 32-key block: P^T as 16 x 16 x 32 B operands (one swap per
      // dword: pf[2 kb + 1] then serves queries 0-15, pf[2 kb] 16-31)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const bf16* vt = Vs[buf][kb / 2] + (kb & 1) * 32 * GV::W;
        const bf16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vt + tail_off[0]));
        const bf16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vt + tail_off[1]));
        bf16x8 a;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = lo4[i];
          a[i + 4] = hi4[i];
        }
        permlane16_swap(pf[2 * kb + 1], pf[2 * kb]);
        ot[0] = mfma16x16x32(a, pf[2 * kb + 1], ot[0]);
        ot[1] = mfma16x16x32(a, pf[2 * kb], ot[1]);
      }
    }

    prio<0>();
    buf = kPair ? (buf == 2 ? 0 : buf + 1) : (buf ^ 1);
    cur = nxt;
    nx1 = pre;
  }

  // m = the reference point (a row without keys: m = -inf, l = 0), l relative to it
  const float l_tot = wave_half_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  const float m_out = (l_tot > 0.f) ? m_ref : -INFINITY;
  // lane-dependent indices again, from a fresh lane id (nothing kept live
  // across the loop for them)
  const int lane_e = lane_id_fresh(), g_e = lane_e >> 5;
  const int qi_e = qt * kFwdRows + wave * 32 + (lane_e & 31);
  using E = cq_epi::QRows<DPE>;
  if constexpr (E::kHalfBytes <= (int)sizeof(Ks) && E::kHalfBytes <= (int)sizeof(Vs)) {
    // O / l staged through LDS (cq_epilogue.h: waves 0-3 in the K tiles,
    // 4-7 in the V tiles), then every query row stored as contiguous
    // 16-byte pieces instead of one element per lane and store
    float* const st = (float*)(cq_epi::half(wave) ? &Vs[0][0][0] : &Ks[0][0][0]) + E::stage_base(wave);
    __syncthreads();  // every wave is done with the loop's K / V tiles
#pragma unroll
    for (int db = 0; db < DBF; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 x = {o[db][4 * i] * inv, o[db][4 * i + 1] * inv, o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv};
        *(f32x4*)(st + E::stage_write(db, i, lane_e)) = x;
      }
    if constexpr (kTail) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        *(f32x4*)(st + E::stage_write_tail(u, lane_e)) = ot[u] * __shfl(inv, 16 * u + (lane_e & 15));
    }
    __syncthreads();
    float* const ob = p.out + sp.index * p.split_o + (int64_t)b * p.sob + (int64_t)h * p.soh;
    const int q0 = qt * kFwdRows + wave * 32;
#pragma unroll
    for (int it0 = 0; it0 < E::kIters; it0 += 4) {
      f32x4 x[4];  // four chunks read back before any is stored: one LDS latency
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (it0 + j < E::kIters) x[j] = *(const f32x4*)(st + E::stage_read(it0 + j, lane_e));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (it0 + j >= E::kIters) break;  // a last group of fewer than four (16-wide d tail)
        const int qi = q0 + E::read_row(it0 + j, lane_e), ch = E::read_chunk(it0 + j, lane_e);
        if (qi >= p.T || 4 * ch >= p.D) continue;
        float* const o4 = ob + (int64_t)qi * p.sot + 4 * ch;
        o4[0] = x[j].x;
        o4[1] = x[j].y;
        o4[2] = x[j].z;
        o4[3] = x[j].w;
      }
    }
  } else if (qi_e < p.T) {
    static_assert(!kTail, "the tail variant always fits the staged epilogue");
    float* orow = p.out + sp.index * p.split_o + (int64_t)b * p.sob + (int64_t)h * p.soh + (int64_t)qi_e * p.sot;
#pragma unroll
    for (int db = 0; db < DBF; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = db * 32 + c_row(r, g_e);
        if (d < p.D) orow[d] = o[db][r] * inv;
      }
  }
  if (qi_e < p.T && g_e == 0) {
    const int64_t si = sp.index * p.split_ml + ((int64_t)b * p.H + h) * p.T + qi_e;
    const float m_nat = m_out * kLn2;
    if (p.m_bf16) {
      const bf16 mh = (bf16)m_nat;
      const float mhf = (float)mh;
      const float l_adj = (l_tot > 0.f) ? l_tot * __expf(m_nat - mhf) : 0.f;
      ((bf16*)p.m)[si] = mh;
      p.l[si] = l_adj;
    } else {
      ((float*)p.m)[si] = m_nat;
      p.l[si] = l_tot;
    }
  }
}

// ---------------------------------------------------------------------------
// D = rowsum(dO * O): 16 lanes per row, 8 elements per lane
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void delta_kernel(DeltaParams p) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  float acc = 0.f;
  if (row < rows) {
    const int t = (int)(row % p.T);
    const int64_t bh = row / p.T;
    const int h = (int)(bh % p.H), b = (int)(bh / p.H);
    const int d0 = sub * 8;
    if (d0 < p.D) {
      const bf16x8 g8 = *(const bf16x8*)(p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh + (int64_t)t * p.sdt + d0);
      const float* orow = p.out + (int64_t)b * p.sob + (int64_t)h * p.soh + (int64_t)t * p.sot + d0;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += (float)g8[j] * orow[j];
    }
  }
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// Backward statistics, in the form both backward kernels use: plane 0 =
// -(m + ln l) / scale per query (-inf for a row with l <= 0, which then gets
// P = 0), plane 1 = -D.  With S' = Q K^T + plane 0 and dP' = dO V^T + plane 1,
// P = exp2(S' c) and dS = P dP'.  The dQ kernel, launched first, computes
// them for its rows (bwd_stat_lse) and writes the planes the dK/dV kernel
// reads, so the backward needs no launch of its own for them.
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Backward dQ (Q-stationary): dQ = scale * sum_c dS_c K_c
// ---------------------------------------------------------------------------
// Block = 8 waves x 32 queries (two waves per SIMD, one block per CU), for
// the same reason as the forward: each K / V tile in LDS serves 256 queries.
constexpr int kDqWaves = 8;
constexpr int kDqRows = 32 * kDqWaves;
static_assert(kDqRows == kQueryBlockRows, "the host sizes KV splits with kQueryBlockRows");
// Keys per barrier interval = 64 * kDqSub (kDqSub 64-row LDS sub-tiles per
// buffer).  Within an interval the 32-key blocks j = 0 .. 2*kDqSub-1 run as
// one software pipeline: A(j) = S^T, dP^T of block j; B(j) = its dS^T (VALU);
// C(j) = dQ^T += K_j^T dS_j^T.  Order A(0), A(1)|B(0), C(0), A(2)|B(1), C(1),
// ..., B(last), C(last), where X|Y places Y's VALU instructions between X's
// MFMAs, so only one block's softmax per interval is exposed.
constexpr int kDqSub = 2;
constexpr int kDqPfA = 1;  // S^T / dP^T fragments issued this many steps ahead
// Pad keys need no mask here: their K / V rows load as zero, so s = 0 and
// dS^T = -P D, which dQ^T = K^T dS^T multiplies by the zero K row.  P is
// clamped to [0, 1] (exact for every valid key, whose score never exceeds
// the row's LSE): unclamped, a pad key's P = exp2(-LSE2) overflows to inf for
// a row whose LSE is below about -88, and 0 * inf would turn dQ into NaN.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(64 * kDqWaves, 1) void dq_kernel(BwdParams p) {
  constexpr int DP = DBLK * 32;
  // At 5 k-steps (head dims 72 and 80) the last d block of dQ^T is 16 wide:
  // 16 x 16 x 32 MFMAs over d 64-79, as in dkdv_kernel.
  constexpr bool kTail = KSTEPS == 5 && DBLK == 3;
  constexpr int DBF = kTail ? DBLK - 1 : DBLK;  // 32-wide d blocks
  constexpr int DPE = kTail ? 80 : DP;          // d columns the tiles and outputs hold
  // head dims <= 64: paired K / V tiles, three buffers, copies two tiles
  // ahead (as in fwd_kernel)
  constexpr bool kPair = DPE <= 64;
  using GK = XorTile<kPair ? 128 : DPE>;  // K: row and transposed fragments
  using GV = XorTile<kPair ? 128 : DPE>;  // V: row fragments only
  constexpr int TK = 64 * kDqSub, KB = TK / 32;  // keys and 32-key blocks per tile
  constexpr int NS = kPair ? 1 : kDqSub;         // LDS tiles (64 rows, or 128 paired) per buffer
  constexpr int NB = kPair ? 3 : 2;              // buffers
  __shared__ __attribute__((aligned(16))) bf16 Ks[NB][NS][GK::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Vs[NB][NS][GV::ELEMS];

  // the wave index is wave-uniform; readfirstlane lets the compiler keep it in an SGPR
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  int qt, h, b;
  decode_block((p.T + kDqRows - 1) / kDqRows, p.H, qt, h, b);
  const KvSplit sp = kv_split(p.ct.n);
  const int qi = qt * kDqRows + wave * 32 + l32;
  const bool q_ok = qi < p.T;
  const float c2 = p.scale * kLog2e;

  bf16x8 qf[KSTEPS], gf[KSTEPS];
  {
    const bf16* qrow = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh + (int64_t)qi * p.sqt;
    const bf16* grow = p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh + (int64_t)qi * p.sdt;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int d0 = ks * 16 + g * 8;
      const bool ok = q_ok && d0 < p.D;
      qf[ks] = ok ? *(const bf16x8*)(qrow + d0) : zero8();
      gf[ks] = ok ? *(const bf16x8*)(grow + d0) : zero8();
    }
  }
  const int64_t si = ((int64_t)b * p.H + h) * p.T + qi;
  const int64_t nrows = (int64_t)p.B * p.H * p.T;
  // the row's statistics (bwd_stat_lse), written once for the dK/dV kernel;
  // LSE2 = -c * plane 0 (+inf for a row without keys); D = -plane 1
  const float st0 = q_ok ? bwd_stat_lse(p, si) : 0.f;
  const float st1 = q_ok ? -p.delta[si] : 0.f;
  if (q_ok && g == 0 && sp.index == 0) {
    p.stats[si] = st0;
    p.stats[nrows + si] = st1;
  }
  const float lse2 = q_ok ? -st0 * c2 : INFINITY;
  const float dlt = q_ok ? -st1 : 0.f;
  XorLanes<kPair ? 128 : DPE, KSTEPS> klo;  // paired: d blocks 2-3 address rows 64-127
  klo.init_rows_lean(lane);
  klo.init_tr_lean(lane);
  XorLanes<DPE, KSTEPS> vlo;
  vlo.init_rows_lean(lane);
  using LK = DirectLoader<GK, kDqWaves, kPair>;
  using LV = DirectLoader<GV, kDqWaves, kPair>;
  static_assert(!kPair || (LK::kInstTot % kDqWaves == 0 && LV::kInstTot % kDqWaves == 0),
                "every wave issues the same number of copies (the paired wait counts them)");
  LK kld;
  kld.init(p.skt, p.D, wave, lane);
  LV vld;
  vld.init(p.skt, p.D, wave, lane);

  f32x16 dq[DBF];
#pragma unroll
  for (int i = 0; i < DBF; ++i) dq[i] = zero16();
  // the 16-wide tail (kTail): d 64-79 x queries 16 u .. 16 u + 15 of the
  // wave's 32, 16 x 16 C layout (column = query, rows d = 64 + 4 (lane / 16) + i)
  f32x4 dqt[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) dqt[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // K^T tail fragments (A operands of those MFMAs): lane group G = lane / 16
  // takes keys 16 (1 - G % 2) + 4 (G / 2) + {0..3, 8..11} of a 32-key block,
  // the order v_permlane16_swap leaves the dS^T B operands in, row d = 64 +
  // lane % 16 (lane j of a group addresses key row j / 4, the 8 bytes at
  // column 64 + 4 (j % 4))
  int tail_off[2] = {0, 0};
  if constexpr (kTail) {
    const int G = lane >> 4, j = lane & 15;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 16 * (1 - (G & 1)) + 8 * hh + 4 * (G >> 1) + (j >> 2);
      tail_off[hh] = row * GK::W + (((8 + ((j & 3) >> 1)) ^ swz(row)) << 3) + 4 * (j & 1);
    }
  }

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  auto issue = [&](const KvCursor& t, int bf) {
#pragma unroll
    for (int sb = 0; sb < NS; ++sb) {
      const int r0 = t.k0 + 64 * sb, rows = t.len - r0;
      kld.load(rows_rsrc(t.k, p.skt, r0, rows), Ks[bf][sb]);
      vld.load(rows_rsrc(t.v, p.skt, r0, rows), Vs[bf][sb]);
    }
  };
  // The next tile's copies are issued one instruction per MFMA step of the
  // first two S^T / dP^T phases instead of in one burst after the barrier:
  // a burst of ~80 one-KiB copies per CU keeps the texture unit's FIFOs
  // full for ~1000 cycles, and a wave stalled on issuing a copy cannot issue
  // MFMAs either.  Slot j < kDmaSlots: sub-tile j / kSlotsPerSub, K copies
  // first, then V copies.
  constexpr int kSlotsK = LK::kInst, kSlotsV = LV::kInst;
  constexpr int kSlotsPerSub = kSlotsK + kSlotsV, kDmaSlots = NS * kSlotsPerSub;
  constexpr int kSlotsPerStep = (kDmaSlots + 2 * KSTEPS - 1) / (2 * KSTEPS);
  rsrc_t nk_rs[NS], nv_rs[NS];
  auto prepare = [&](const KvCursor& t) {
#pragma unroll
    for (int sb = 0; sb < NS; ++sb) {
      const int r0 = t.k0 + 64 * sb, rows = t.len - r0;
      nk_rs[sb] = rows_rsrc(t.k, p.skt, r0, rows);
      nv_rs[sb] = rows_rsrc(t.v, p.skt, r0, rows);
    }
  };
  auto dma_slot = [&](int j, int bf) {
    const int sb = j / kSlotsPerSub, k = j % kSlotsPerSub;
    if (k < kSlotsK) kld.load_one(nk_rs[sb], Ks[bf][sb], k);
    else vld.load_one(nv_rs[sb], Vs[bf][sb], k - kSlotsK);
  };
  KvCursor cur;
  kv_enter(p.ct, kvo, sp.begin, sp.end, cur);
  int buf = 0;
  if (cur.step < sp.end) issue(cur, 0);
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    settle(qf[ks]);
    settle(gf[ks]);
  }
  float lse2_s = lse2, dlt_s = dlt;
  settle(lse2_s);
  settle(dlt_s);
  // -D, the dP^T accumulators' initial value (one value per lane: its
  // query), so dP - D comes out of the MFMAs and dS costs one multiply;
  // at four d blocks its 16 registers do not fit beside the rest, and dS
  // subtracts D instead
  constexpr bool kDInit = DBLK <= 3;
  f32x16 neg_d;
#pragma unroll
  for (int r = 0; r < 16; ++r) neg_d[r] = kDInit ? -dlt_s : 0.f;
  // kPair: the tile after cur, whose copies are in flight while cur runs
  KvCursor nx1 = cur;
  if constexpr (kPair) {
    nx1 = kv_next(p.ct, kvo, cur, TK, sp.end);
    if (nx1.step < sp.end) issue(nx1, 1);
  }
#pragma unroll 1
  while (cur.step < sp.end) {
    const KvCursor nxt = kPair ? nx1 : kv_next(p.ct, kvo, cur, TK, sp.end);
    // the tile whose copies this one issues (nxt, or the one after it) and its buffer
    const KvCursor pre = kPair ? kv_next(p.ct, kvo, nxt, TK, sp.end) : nxt;
    const int pbuf = kPair ? (buf == 0 ? 2 : buf - 1) : (buf ^ 1);
    if (kPair && nxt.step < sp.end) wait_lds_loads_but<kDmaSlots>();  // nxt's copies may stay in flight
    else wait_lds_loads();
    __syncthreads();
    const bool has_next = pre.step < sp.end;
    if (has_next) prepare(pre);

    // S^T / dP^T of two 32-key blocks in flight (block j in slot j & 1) and
    // the bf16 dS^T of the block whose dQ product is next
    f32x16 s[2], dp[2];
    bf16x8 dsf[2][2];
    // B(j), rows r0 .. r0+NR-1: dS^T = P^T (dP^T - D), P^T = exp2(S^T c2 - LSE2)
    // (the dP^T accumulators start at -D)
    auto softmax_rows = [&](int j, int r0, int nr) {
#pragma unroll
      for (int r = r0; r < r0 + nr; ++r) {
        const float pv = exp2_unit(__builtin_fmaf(s[j & 1][r], c2, -lse2_s));
        dsf[j & 1][r >> 3][r & 7] = (bf16)(pv * (kDInit ? dp[j & 1][r] : dp[j & 1][r] - dlt_s));
      }
    };
    // A(j), with B(jb) spread over its KSTEPS steps (jb < 0: none)
    auto phase_a = [&](auto J, auto JB) {
      constexpr int j = decltype(J)::value, jb = decltype(JB)::value;
      // paired: block j's rows at k-step offset 4 (j / 2) of the one tile
      const bf16* K = Ks[buf][kPair ? 0 : j / 2];
      const bf16* V = Vs[buf][kPair ? 0 : j / 2];
      constexpr int kso = kPair ? 4 * (j / 2) : 0;
      s[j & 1] = zero16();
      dp[j & 1] = kDInit ? neg_d : zero16();
      constexpr int kRowsPerStep = (16 + KSTEPS - 1) / KSTEPS;
      pipelined<KSTEPS, kDqPfA>(
          [&](int ks) { return Frag2{klo.row_frag_lean(K, j & 1, ks + kso), vlo.row_frag_lean(V, j & 1, ks + kso)}; },
          [&](int ks, const Frag2& f) {
            s[j & 1] = mfma32x32x16(f.a, qf[ks], s[j & 1]);
            if constexpr (j < 2) {
              if (has_next) {
#pragma unroll
                for (int u = 0; u < kSlotsPerStep; ++u) {
                  const int slot = (j * KSTEPS + ks) * kSlotsPerStep + u;
                  if (slot < kDmaSlots) dma_slot(slot, pbuf);
                }
              }
            }
            dp[j & 1] = mfma32x32x16(f.b, gf[ks], dp[j & 1]);
            if constexpr (jb >= 0) {
              const int r0 = ks * kRowsPerStep;
              if (r0 < 16) softmax_rows(jb, r0, (16 - r0 < kRowsPerStep) ? 16 - r0 : kRowsPerStep);
            }
          });
    };
    // C(j): dQ^T += K_j^T dS_j^T; step i = (16-key half i / DBF, d block i % DBF)
    auto phase_c = [&](auto J) {
      constexpr int j = decltype(J)::value;
      const bf16* K = Ks[buf][kPair ? 0 : j / 2];
      constexpr int dbo = kPair ? 2 * (j / 2) : 0;  // paired: block j's rows at d block offset 2 (j / 2)
      pipelined<2 * DBF, 2>(
          [&](int i) { return klo.tr_frag_lean(K, (j & 1) * 32 + (i / DBF) * 16, i % DBF + dbo); },
          [&](int i, const bf16x8& a) { dq[i % DBF] = mfma32x32x16(a, dsf[j & 1][i / DBF], dq[i % DBF]); });
      if constexpr (kTail) {
        // dS^T as 16 x 16 x 32 B operands (query columns 16 u + lane % 16,
        // 32 keys): one swap per dword, dsf[.][1] then serving queries 0-15
        // and dsf[.][0] queries 16-31
        const bf16* kt = K + (j & 1) * 32 * GK::W;
        const bf16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(kt + tail_off[0]));
        const bf16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(kt + tail_off[1]));
        bf16x8 a;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = lo4[i];
          a[i + 4] = hi4[i];
        }
        permlane16_swap(dsf[j & 1][1], dsf[j & 1][0]);
        dqt[0] = mfma16x16x32(a, dsf[j & 1][1], dqt[0]);
        dqt[1] = mfma16x16x32(a, dsf[j & 1][0], dqt[1]);
      }
    };
    prio<3>();
    phase_a(Int<0>{}, Int<-1>{});
    phase_a(Int<1>{}, Int<0>{});
    phase_c(Int<0>{});
    if constexpr (KB > 2) {
      prio<2>();
      phase_a(Int<2>{}, Int<1>{});
      phase_c(Int<1>{});
      prio<1>();
      phase_a(Int<3>{}, Int<2>{});
      phase_c(Int<2>{});
    }
    // s_setprio also fences the scheduler: the repeated level-0 calls keep the
    // last block's softmax and its dQ product as separate scheduling regions
    prio<0>();
    softmax_rows(KB - 1, 0, 16);
    prio<0>();
    phase_c(Int<KB - 1>{});
    prio<0>();

    buf = kPair ? (buf == 2 ? 0 : buf + 1) : (buf ^ 1);
    cur = nxt;
    nx1 = pre;
  }

  const int lane_e = lane_id_fresh(), g_e = lane_e >> 5;  // as in the forward's epilogue
  const int qi_e = qt * kDqRows + wave * 32 + (lane_e & 31);
  using E = cq_epi::QRows<DPE>;
  if constexpr (E::kHalfBytes <= (int)sizeof(Ks) && E::kHalfBytes <= (int)sizeof(Vs)) {
    // dQ staged through LDS as in the forward (cq_epilogue.h)
    float* const st = (float*)(cq_epi::half(wave) ? &Vs[0][0][0] : &Ks[0][0][0]) + E::stage_base(wave);
    __syncthreads();  // every wave is done with the loop's K / V tiles
#pragma unroll
    for (int db = 0; db < DBF; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 x = {dq[db][4 * i] * p.scale, dq[db][4 * i + 1] * p.scale, dq[db][4 * i + 2] * p.scale,
                         dq[db][4 * i + 3] * p.scale};
        *(f32x4*)(st + E::stage_write(db, i, lane_e)) = x;
      }
    if constexpr (kTail) {
#pragma unroll
      for (int u = 0; u < 2; ++u) *(f32x4*)(st + E::stage_write_tail(u, lane_e)) = dqt[u] * p.scale;
    }
    __syncthreads();
    const int64_t bh = sp.index * p.split_dq + (int64_t)b * p.sdqb + (int64_t)h * p.sdqh;
    const int q0 = qt * kDqRows + wave * 32;
    // bf16 rows go out 8 bytes per lane when the view is 8-byte aligned,
    // else one element per lane and store
    const bool wide = p.dq_f32 || ((((uintptr_t)p.dq & 7u) == 0) && ((p.sdqb | p.sdqh | p.sdqt) & 3) == 0);
    if (wide) {
#pragma unroll
      for (int it0 = 0; it0 < E::kIters; it0 += 4) {
        f32x4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (it0 + j < E::kIters) x[j] = *(const f32x4*)(st + E::stage_read(it0 + j, lane_e));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (it0 + j >= E::kIters) break;  // a last group of fewer than four (16-wide d tail)
          const int qi = q0 + E::read_row(it0 + j, lane_e), ch = E::read_chunk(it0 + j, lane_e);
          if (qi >= p.T || 4 * ch >= p.D) continue;
          const int64_t e = bh + (int64_t)qi * p.sdqt + 4 * ch;
          if (p.dq_f32) {
            float* const o4 = (float*)p.dq + e;
            o4[0] = x[j].x;
            o4[1] = x[j].y;
            o4[2] = x[j].z;
            o4[3] = x[j].w;
          } else {
            *(bf16x4*)((bf16*)p.dq + e) = __builtin_convertvector(x[j], bf16x4);
          }
        }
      }
    } else {
#pragma unroll 4
      for (int it = 0; it < E::kElemIters; ++it) {
        const int qi = q0 + E::elem_row(it, lane_e), col = E::elem_col(it, lane_e);
        const float x = st[E::stage_elem(it, lane_e)];
        if (qi < p.T && col < p.D) ((bf16*)p.dq)[bh + (int64_t)qi * p.sdqt + col] = (bf16)x;
      }
    }
  } else if (qi_e < p.T) {
    static_assert(!kTail, "the tail variant always fits the staged epilogue");
    char* drow = (char*)p.dq + ((sp.index * p.split_dq + (int64_t)b * p.sdqb + (int64_t)h * p.sdqh +
                                 (int64_t)qi_e * p.sdqt) << (p.dq_f32 ? 2 : 1));
#pragma unroll
    for (int db = 0; db < DBF; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = db * 32 + c_row(r, g_e);
        if (d < p.D) {
          const float v = dq[db][r] * p.scale;
          if (p.dq_f32) ((float*)drow)[d] = v;
          else ((bf16*)drow)[d] = (bf16)v;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Backward dK/dV (KV-stationary, as ring_attn.cpp:2723-2816)
// ---------------------------------------------------------------------------
// Block = 8 waves x 32 keys (256 keys; two waves per SIMD, one block per CU).
// Each wave keeps its 32 K rows (and up to head dim 96 its 32 V rows) as
// MFMA B operands in registers, read once from the block's LDS copies, and
// otherwise reads its V rows from the block's LDS copy per query tile; dK,
// dV accumulate in fp32 VGPRs over every query.  Queries stream in 64-row tiles (Q, dO, per-row statistics)
// through double-buffered LDS; per 32-query half:
//   A: S' = Q K^T - LSE2 / c, dP' = dO V^T - D   (C row = query, col = key;
//      the per-row terms are the accumulators' initial values, read from
//      LDS, so the softmax needs no per-row broadcast)
//   B: P = exp2(S' c), dS = P dP'
//   C: dV += P^T dO, dK += dS^T Q  (P / dS straight from the accumulator
//      layout as A operands; dO^T, Q^T by transposed LDS reads)
// Two waves per SIMD hide each other's VALU and LDS latency, and one LDS
// wave can only keep ~16 reads in flight: at two waves a SIMD gets ~1.5x the
// LDS read throughput of one.  Each Q / dO tile in LDS serves 256 keys.
// Pad keys (past the chunk's valid length) are written as zero at the end
// instead of being masked per tile: a key's P / dS only reach its own dK / dV.
// P is clamped to [0, 1] as in the dQ kernel, so even a pad key's values stay
// finite.
constexpr int kDkWaves = kDkdvBlockKeys / 32;
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(64 * kDkWaves, 1) void dkdv_kernel(BwdParams p) {
  constexpr int DP = DBLK * 32;
  // At 5 k-steps (head dims 72 and 80) the last d block of dK / dV is 16 wide:
  // 16 x 16 x 32 MFMAs over d 64-79 instead of 32 x 32 x 16 ones over 64-95.
  constexpr bool kTail = KSTEPS == 5 && DBLK == 3;
  constexpr int DBF = kTail ? DBLK - 1 : DBLK;  // 32-wide d blocks
  constexpr int DPE = kTail ? 80 : DP;          // d columns the tiles and outputs hold
  using GV = PadTile<DPE>;  // the block's V rows: row fragments only
  using GQ = XorTile<DPE>;  // Q / dO tiles: row and transposed fragments
  constexpr int NVT = kDkdvBlockKeys / 64;  // 64-row V tiles of the block
  __shared__ __attribute__((aligned(16))) bf16 Vb[NVT][GV::ELEMS];
  // two Q / dO buffers; before the loop they hold the block's K rows (as
  // NVT XorTiles) while each wave copies its K fragments into registers
  __shared__ __attribute__((aligned(16))) bf16 QG[2][2][GQ::ELEMS];  // [buffer][Q, dO]
  // per query of a tile: the initial values of the S' and dP' accumulators
  // (the prepared planes: -LSE2 / c and -D), [buffer][S', dP'][query]
  __shared__ __attribute__((aligned(16))) float St[2][2][64];
  static_assert(NVT <= 4, "K staging uses the four Q / dO tile slots");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  int kt, h, b;
  decode_block(p.n_key_tiles, p.H, kt, h, b);
  int c = 0;
#pragma unroll 1
  for (int i = 1; i < p.ct.n; ++i)
    if (kt >= p.ct.tile0[i]) c = i;
  const int kblk0 = (kt - p.ct.tile0[c]) * kDkdvBlockKeys;
  const int key0 = kblk0 + wave * 32;
  const int len = p.ct.len[c];
  const float c2 = p.scale * kLog2e;


  f32x16 dk[DBF], dv[DBF];
#pragma unroll
  for (int i = 0; i < DBF; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }
  // the 16-wide tail (kTail): keys 16 t .. 16 t + 15 of the wave's 32, d 64-79,
  // 16 x 16 C layout (column d = 64 + lane % 16, rows 4 (lane / 16) .. + 3)
  f32x4 dkt[2], dvt[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) dkt[t] = dvt[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (kblk0 < len) {  // block has at least one valid key (block-uniform)
    XorLanes<DPE, KSTEPS> lo;
    lo.init_rows_lean(lane);
    lo.init_tr_lean(lane);
    // transposed tail fragments (B operands of the 16 x 16 x 32 MFMAs): lane
    // group G = lane / 16 takes queries 16 (1 - G % 2) + 4 (G / 2) + {0..3,
    // 8..11} of a 32-query half, the order in which v_permlane16_swap leaves
    // the P / dS A operands, column d = 64 + lane % 16 (lane j of a group
    // addresses row j / 4, the 8 bytes at column 64 + 4 (j % 4))
    int tail_off[2];
    if constexpr (kTail) {
      const int G = lane >> 4, j = lane & 15;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = 16 * (1 - (G & 1)) + 8 * hh + 4 * (G >> 1) + (j >> 2);
        tail_off[hh] = row * GQ::W + (((8 + ((j & 3) >> 1)) ^ swz(row)) << 3) + 4 * (j & 1);
      }
    }
    auto tail_frag = [&](const bf16* t, int qb) {
      const bf16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + qb * 32 * GQ::W + tail_off[0]));
      const bf16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + qb * 32 * GQ::W + tail_off[1]));
      bf16x8 r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[i] = lo4[i];
        r[i + 4] = hi4[i];
      }
      return r;
    };
    PadRows<DPE> vlo;
    vlo.init(lane);
    DirectLoader<GQ, kDkWaves> qld, gld;
    qld.init(p.sqt, p.D, wave, lane);
    gld.init(p.sdt, p.D, wave, lane);
    const bf16* qb_ = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
    const bf16* gb_ = p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh;
    const int64_t sbase = ((int64_t)b * p.H + h) * p.T;
    const int64_t nrows = (int64_t)p.B * p.H * p.T;

    // Per-query statistics of a tile (the two prepared planes, 64 rows each)
    // go global -> LDS by two dword copies of wave 0.  Rows past T read as 0:
    // their Q and dO rows are zero too, so P dO and dS = P dP' vanish.
    auto issue_stats = [&](int q0, int bf) {
      if (wave == 0) {
        const uint32_t voff = (uint32_t)lane * 4u;
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) {
          const rsrc_t rs = make_rsrc(p.stats + pl * nrows + sbase + q0, (uint32_t)(p.T - q0) * 4u);
          lds_dma_b32(rs, (uint32_t)(uintptr_t)(lds_void*)&St[bf][pl][0], voff);
        }
      }
    };
    auto issue = [&](int q0, int bf) {
      qld.load(rows_rsrc(qb_, p.sqt, q0, p.T - q0), QG[bf][0]);
      gld.load(rows_rsrc(gb_, p.sdt, q0, p.T - q0), QG[bf][1]);
      issue_stats(q0, bf);
    };
    // Inside the loop the next tile's copies are issued one instruction per
    // MFMA step of the first S / dP phase rather than in one burst after
    // the barrier (a burst fills the texture unit's FIFOs, and a wave
    // stalled on issuing a copy cannot issue MFMAs); the statistics loads
    // follow the copies.  Slot j: Q copies, then dO copies.
    constexpr int kSlotsQ = DirectLoader<GQ, kDkWaves>::kInst, kDmaSlots = 2 * kSlotsQ;
    constexpr int kSlotsPerStep = (kDmaSlots + KSTEPS - 1) / KSTEPS;
    rsrc_t nq_rs, ng_rs;

    // V fragments in registers up to 6 k-steps (head dims <= 96); at 8 the
    // kernel has no registers left for them and reads them per query tile
    constexpr bool kVRegs = KSTEPS <= 6;
    bf16x8 kf[KSTEPS], vf[KSTEPS];
    {
      const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
      DirectLoader<GQ, kDkWaves> kld;
      kld.init(p.skt, p.D, wave, lane);
      DirectLoader<GV, kDkWaves> vld;
      vld.init(p.skt, p.D, wave, lane);
      bf16* kstage = &QG[0][0][0];
#pragma unroll
      for (int t = 0; t < NVT; ++t) {
        const int r0 = kblk0 + 64 * t;
        kld.load(rows_rsrc(p.ct.k[c] + kvo, p.skt, r0, len - r0), kstage + t * GQ::ELEMS);
        vld.load(rows_rsrc(p.ct.v[c] + kvo, p.skt, r0, len - r0), Vb[t]);
      }
      wait_lds_loads();
      __syncthreads();
      // this wave's 32 K rows: XorTile wave / 2, 32-row block wave % 2;
      // (kVRegs) its 32 V rows, the B operands of dP' = dO V^T, from the
      // block's V tile the same way: every query tile reuses them
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        kf[ks] = lo.row_frag_lean(kstage + (wave >> 1) * GQ::ELEMS, wave & 1, ks);
        if constexpr (kVRegs) vf[ks] = vlo.frag(Vb[wave >> 1], wave & 1, ks);
      }
      __syncthreads();  // every wave has its K fragments: the staging may be overwritten
    }
    const bf16* Vw = Vb[wave >> 1];
    const int vrb = wave & 1;
    issue(0, 0);

    // Initial accumulator of half qb from LDS row values: register 4j + i of
    // lane-half g holds row c_row(4j + i, g) = 8j + 4g + i, so four 16-byte
    // reads (the same address for all 32 lanes of a half) fill the tile.
    auto init_rows = [&](const float* col, int qb) {
      f32x16 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = *(const f32x4*)(col + qb * 32 + 8 * j + 4 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * j + i] = v[i];
      }
      return x;
    };
    const int n_tiles = (p.T + 63) >> 6;
    int buf = 0;
#pragma unroll 1
    for (int t = 0; t < n_tiles; ++t) {
      wait_lds_loads();
      __syncthreads();  // tile t published; every wave is done with tile t-1
      const bool has_next = t + 1 < n_tiles;
      const int nq0 = (t + 1) * 64;
      if (has_next) {
        nq_rs = rows_rsrc(qb_, p.sqt, nq0, p.T - nq0);
        ng_rs = rows_rsrc(gb_, p.sdt, nq0, p.T - nq0);
      }
      const bf16* Q = QG[buf][0];
      const bf16* Gd = QG[buf][1];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        if (qb == 0) prio<3>();
        else prio<1>();
        f32x16 s = init_rows(St[buf][0], qb), dp = init_rows(St[buf][1], qb);
        pipelined<KSTEPS, 1>(
            [&](int ks) {
              Frag3 f{lo.row_frag_lean(Q, qb, ks), lo.row_frag_lean(Gd, qb, ks), {}};
              if constexpr (!kVRegs) f.c = vlo.frag(Vw, vrb, ks);
              return f;
            },
            [&](int ks, const Frag3& f) {
              s = mfma32x32x16(f.a, kf[ks], s);
              if (qb == 0 && has_next) {
#pragma unroll
                for (int u = 0; u < kSlotsPerStep; ++u) {
                  const int j = ks * kSlotsPerStep + u;
                  if (j < kSlotsQ) qld.load_one(nq_rs, QG[buf ^ 1][0], j);
                  else if (j < kDmaSlots) gld.load_one(ng_rs, QG[buf ^ 1][1], j - kSlotsQ);
                }
                if (ks == KSTEPS - 1) issue_stats(nq0, buf ^ 1);
              }
              dp = mfma32x32x16(f.b, kVRegs ? vf[ks] : f.c, dp);
            });
        if (qb == 0) prio<3>();
        else prio<1>();
        bf16x8 pf[2], dsf[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = exp2_unit(s[r] * c2);
          pf[r >> 3][r & 7] = (bf16)pv;
          dsf[r >> 3][r & 7] = (bf16)(pv * dp[r]);
        }
        if (qb == 0) prio<2>();
        else prio<0>();
        // dV += P^T dO ; dK += dS^T Q (M = keys, N = d, K = the 32 queries of
        // this half); step s2 = (h2 = s2 / DBF, db = s2 % DBF)
        pipelined<2 * DBF, 1>(
            [&](int s2) {
              const int r0 = qb * 32 + (s2 / DBF) * 16;
              return Frag2{lo.tr_frag_lean(Gd, r0, s2 % DBF), lo.tr_frag_lean(Q, r0, s2 % DBF)};
            },
            [&](int s2, const Frag2& f) {
              const int h2 = s2 / DBF, db = s2 % DBF;
              dv[db] = mfma32x32x16(pf[h2], f.a, dv[db]);
              dk[db] = mfma32x32x16(dsf[h2], f.b, dk[db]);
            });
        if constexpr (kTail) {
          // P / dS as 16 x 16 x 32 A operands (key rows 16 t + lane % 16,
          // 32 queries): lane l holds key l % 32 with queries c_row(8 h2 + i,
          // l / 32) in pf[h2]; one swap per dword brings every 16-lane group
          // the right keys, pf[1] then serving keys 0-15 and pf[0] keys 16-31
          const bf16x8 gt = tail_frag(Gd, qb), qt = tail_frag(Q, qb);
          permlane16_swap(pf[1], pf[0]);
          permlane16_swap(dsf[1], dsf[0]);
          dvt[0] = mfma16x16x32(pf[1], gt, dvt[0]);
          dvt[1] = mfma16x16x32(pf[0], gt, dvt[1]);
          dkt[0] = mfma16x16x32(dsf[1], qt, dkt[0]);
          dkt[1] = mfma16x16x32(dsf[0], qt, dkt[1]);
        }
      }
      prio<0>();
      buf ^= 1;
    }
  }

  // store: C layout row = key key0 + c_row(r,g), col = d = db*32 + l32;
  // keys past the valid length (pads) get zero
  const int64_t base = (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
  const int lane_e = lane_id_fresh(), g_e = lane_e >> 5;  // as in the forward's epilogue
  using E = cq_epi::KRows<DPE>;
  if constexpr (E::kHalfBytes <= (int)sizeof(QG) && E::kHalfBytes <= (int)sizeof(Vb)) {
    // dK, then dV, staged through LDS (cq_epilogue.h: waves 0-3 in the Q / dO
    // buffers, 4-7 in the V tiles) and stored as contiguous row pieces
    float* const st = (float*)(cq_epi::half(wave) ? (void*)&Vb[0][0] : (void*)&QG[0][0][0]) + E::stage_base(wave);
    const int rows_c = p.ct_rows[c];
    // bf16 rows 8 bytes per lane when both views are 8-byte aligned, else one
    // element per lane and store
    const bool wide = p.dkv_f32 || (((((uintptr_t)p.ct.dk[c]) | ((uintptr_t)p.ct.dv[c])) & 7u) == 0 &&
                                    ((p.sdkb | p.sdkh | p.sdkt) & 3) == 0);
    __syncthreads();  // every wave is done with the loop's LDS
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
      const float sc = tn == 0 ? p.scale : 1.f;
#pragma unroll
      for (int db = 0; db < DBF; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st[E::stage_write(db, r, lane_e)] = (tn == 0 ? dk[db][r] : dv[db][r]) * sc;
      if constexpr (kTail) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[E::stage_write_tail(t, i, lane_e)] = (tn == 0 ? dkt[t][i] : dvt[t][i]) * sc;
      }
      __syncthreads();
      void* const outp = tn == 0 ? (void*)p.ct.dk[c] : (void*)p.ct.dv[c];
      if (wide) {
#pragma unroll
        for (int it0 = 0; it0 < E::kIters; it0 += 4) {
          f32x4 x[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (it0 + j < E::kIters) x[j] = *(const f32x4*)(st + E::stage_read(it0 + j, lane_e));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (it0 + j >= E::kIters) break;  // a last group of fewer than four (16-wide d tail)
            const int kk = key0 + E::read_row(it0 + j, lane_e), ch = E::read_chunk(it0 + j, lane_e);
            if (kk >= rows_c || 4 * ch >= p.D) continue;
            const f32x4 y = kk < len ? x[j] : f32x4{0.f, 0.f, 0.f, 0.f};
            const int64_t e = base + (int64_t)kk * p.sdkt + 4 * ch;
            if (p.dkv_f32) {
              float* const o4 = (float*)outp + e;
              o4[0] = y.x;
              o4[1] = y.y;
              o4[2] = y.z;
              o4[3] = y.w;
            } else {
              *(bf16x4*)((bf16*)outp + e) = __builtin_convertvector(y, bf16x4);
            }
          }
        }
      } else {
#pragma unroll 4
        for (int it = 0; it < E::kElemIters; ++it) {
          const int kk = key0 + E::elem_row(it, lane_e), col = E::elem_col(it, lane_e);
          const float x = st[E::stage_elem(it, lane_e)];
          if (kk < rows_c && col < p.D) ((bf16*)outp)[base + (int64_t)kk * p.sdkt + col] = (bf16)(kk < len ? x : 0.f);
        }
      }
      __syncthreads();  // the staging rows are rewritten with dV
    }
  } else {
    static_assert(!kTail, "the tail variant always fits the staged epilogue");
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
      const int d = db * 32 + (lane_e & 31);
      if (d >= p.D) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = key0 + c_row(r, g_e);
        if (kk >= p.ct_rows[c]) continue;
        const int64_t e = base + (int64_t)kk * p.sdkt + d;
        const bool valid = kk < len;
        const float vk = valid ? dk[db][r] * p.scale : 0.f, vv = valid ? dv[db][r] : 0.f;
        if (p.dkv_f32) {
          ((float*)p.ct.dk[c])[e] = vk;
          ((float*)p.ct.dv[c])[e] = vv;
        } else {
          p.ct.dk[c][e] = (bf16)vk;
          p.ct.dv[c][e] = (bf16)vv;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// KV-split merges: LPR lanes per query row (16, or 8 when D <= 64), 8
// elements of D per lane.  The splits are read G at a time (G = the split
// count up to 8), all loads of a group issued before any is used (an index
// past the last split reads the last one again and is given no weight), so a
// merge of n splits waits for ceil(n / 8) load latencies instead of n.
// ---------------------------------------------------------------------------
template <int G, int LPR>
__global__ __launch_bounds__(256) void fwd_merge_kernel(FwdMergeParams p) {
  constexpr int kRowsPerBlock = 256 / LPR;
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x / LPR);
  const int sub = threadIdx.x % LPR, d0 = sub * 8;
  if (row >= rows) return;  // whole LPR-lane groups
  const bool has_d = d0 < p.D;
  const int dr = has_d ? d0 : 0;  // lanes past D read (and drop) elements 0..7
  float ms[G], ls[G], o[G][8];
  // splits s0 .. s0 + G - 1 (an index past the last split reads the last one again)
  auto load_group = [&](int s0) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int64_t sr = min(s0 + u, p.n_split - 1) * rows + row;
      ms[u] = p.part_m[sr];
      ls[u] = p.part_l[sr];
      const float* op = p.part_o + sr * p.D + dr;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[u][j] = op[j];
    }
  };
  float mx = -INFINITY, l = 0.f, acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  auto add_group = [&](int s0) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (s0 + u >= p.n_split) break;  // a repeated split gets no weight
      // a split without keys (l = 0) adds nothing; NaN statistics propagate
      const float w = (ls[u] == 0.f) ? 0.f : ls[u] * __expf(ms[u] - mx);
      l += w;
      if (w != 0.f) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += w * o[u][j];
      }
    }
  };
  if (p.n_split <= G) {  // up to 8 splits: one round of loads, the maximum over the loaded m
    load_group(0);
#pragma unroll
    for (int u = 0; u < G; ++u) mx = fmaxf(mx, ms[u]);  // a repeated split changes no maximum
    add_group(0);
  } else {  // more: the maximum first, then the groups again
    for (int s0 = 0; s0 < p.n_split; s0 += G) {
#pragma unroll
      for (int u = 0; u < G; ++u) mx = fmaxf(mx, p.part_m[min(s0 + u, p.n_split - 1) * rows + row]);
    }
    for (int s0 = 0; s0 < p.n_split; s0 += G) {
      load_group(s0);
      add_group(s0);
    }
  }
  const int t = (int)(row % p.T);
  const int64_t bh = row / p.T;
  const int h = (int)(bh % p.H), b = (int)(bh / p.H);
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  if (has_d) {
    float* orow = p.out + (int64_t)b * p.sob + (int64_t)h * p.soh + (int64_t)t * p.sot + d0;
#pragma unroll
    for (int j = 0; j < 8; ++j) orow[j] = acc[j] * inv;
  }
  if (sub == 0) {  // statistics as the forward kernel writes them
    if (p.m_bf16) {
      const bf16 mh = (bf16)mx;
      const float mhf = (float)mh;
      ((bf16*)p.m)[row] = mh;
      p.l[row] = (l > 0.f) ? l * __expf(mx - mhf) : 0.f;
    } else {
      ((float*)p.m)[row] = mx;
      p.l[row] = l;
    }
  }
}

template <int G, int LPR>
__global__ __launch_bounds__(256) void dq_merge_kernel(DqMergeParams p) {
  constexpr int kRowsPerBlock = 256 / LPR;
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x / LPR);
  const int d0 = (threadIdx.x % LPR) * 8;
  if (row >= rows || d0 >= p.D) return;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  for (int s0 = 0; s0 < p.n_split; s0 += G) {
    float o[G][8];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const float* op = p.part + (min(s0 + u, p.n_split - 1) * rows + row) * p.D + d0;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[u][j] = op[j];
    }
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (s0 + u >= p.n_split) break;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += o[u][j];
    }
  }
  const int t = (int)(row % p.T);
  const int64_t bh = row / p.T;
  const int h = (int)(bh % p.H), b = (int)(bh / p.H);
  const int64_t e = (int64_t)b * p.sdqb + (int64_t)h * p.sdqh + (int64_t)t * p.sdqt + d0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (p.dq_f32) ((float*)p.dq)[e + j] = acc[j];
    else ((bf16*)p.dq)[e + j] = (bf16)acc[j];
  }
}

namespace {

// The merge instance for this split count and head dim: group = splits (2..8;
// more splits go 8 at a time), 8 lanes per row when D <= 64 (16 otherwise).
template <template <int, int> class K, class P>
hipError_t launch_merge(const P& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  const bool narrow = p.D <= 64;
  const int rpb = narrow ? 32 : 16;
  const dim3 grid((unsigned)((rows + rpb - 1) / rpb)), block(256);
  const int g = p.n_split < 2 ? 2 : (p.n_split > 8 ? 8 : p.n_split);
#define HARP_MERGE_CASE(G)                                                         \
  case G:                                                                          \
    if (narrow) hipLaunchKernelGGL((K<G, 8>::kernel), grid, block, 0, st, p);     \
    else hipLaunchKernelGGL((K<G, 16>::kernel), grid, block, 0, st, p);           \
    break;
  switch (g) {
    HARP_MERGE_CASE(2)
    HARP_MERGE_CASE(3)
    HARP_MERGE_CASE(4)
    HARP_MERGE_CASE(5)
    HARP_MERGE_CASE(6)
    HARP_MERGE_CASE(7)
    default: HARP_MERGE_CASE(8)
  }
#undef HARP_MERGE_CASE
  return hipGetLastError();
}
template <int G, int LPR>
struct FwdMergeK {
  static constexpr auto kernel = fwd_merge_kernel<G, LPR>;
};
template <int G, int LPR>
struct DqMergeK {
  static constexpr auto kernel = dq_merge_kernel<G, LPR>;
};

}  // namespace

hipError_t launch_fwd_merge(const FwdMergeParams& p, hipStream_t st) { return launch_merge<FwdMergeK>(p, st); }
hipError_t launch_dq_merge(const DqMergeParams& p, hipStream_t st) { return launch_merge<DqMergeK>(p, st); }

// Every (KSTEPS, DBLK) variant the launchers dispatch to, instantiated
// explicitly: with lambdas in the kernel bodies the host pass otherwise
// emits launch stubs for only some of the implicitly instantiated kernels.
#define HARP_RA_INSTANTIATE(KS, DB)                             \
  template __global__ void fwd_kernel<KS, DB>(FwdParams);       \
  template __global__ void dq_kernel<KS, DB>(BwdParams);        \
  template __global__ void dkdv_kernel<KS, DB>(BwdParams);
HARP_RA_INSTANTIATE(2, 1)
HARP_RA_INSTANTIATE(4, 2)
HARP_RA_INSTANTIATE(5, 3)
HARP_RA_INSTANTIATE(6, 3)
HARP_RA_INSTANTIATE(8, 4)
#undef HARP_RA_INSTANTIATE

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------
template <int KSTEPS, int DBLK>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t st) {
  const int n = ((p.T + kFwdRows - 1) / kFwdRows) * p.H * p.B;
  hipLaunchKernelGGL((fwd_kernel<KSTEPS, DBLK>), dim3(n, p.n_split), dim3(64 * kFwdWaves), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dq_t(const BwdParams& p, hipStream_t st) {
  const int n = ((p.T + kDqRows - 1) / kDqRows) * p.H * p.B;
  hipLaunchKernelGGL((dq_kernel<KSTEPS, DBLK>), dim3(n, p.n_split), dim3(64 * kDqWaves), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dkdv_t(const BwdParams& p, hipStream_t st) {
  const int n = p.n_key_tiles * p.H * p.B;
  hipLaunchKernelGGL((dkdv_kernel<KSTEPS, DBLK>), dim3(n), dim3(64 * kDkWaves), 0, st, p);
  return hipGetLastError();
}

#define HARP_RA_DISPATCH_D(D_, FN, ...)                                 \
  switch (D_) {                                                         \
    case 64: return FN<4, 2>(__VA_ARGS__);                              \
    case 72: return FN<5, 3>(__VA_ARGS__);                              \
    case 128: return FN<8, 4>(__VA_ARGS__);                             \
    default: break;                                                     \
  }                                                                     \
  if ((D_) <= 32) return FN<2, 1>(__VA_ARGS__);                         \
  if ((D_) <= 64) return FN<4, 2>(__VA_ARGS__);                         \
  if ((D_) <= 96) return FN<6, 3>(__VA_ARGS__);                         \
  return FN<8, 4>(__VA_ARGS__);

hipError_t launch_fwd(const FwdParams& p, hipStream_t st) {
  if (fwd_asm_applies(p)) return launch_fwd_asm(p, st);
  HARP_RA_DISPATCH_D(p.D, launch_fwd_t, p, st)
}
hipError_t launch_delta(const DeltaParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  dim3 grid((unsigned)((rows + 15) / 16));
  hipLaunchKernelGGL(delta_kernel, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
hipError_t launch_dq(const BwdParams& p, hipStream_t st) {
  if (dq_asm_applies(p)) return launch_dq_asm(p, st);
  HARP_RA_DISPATCH_D(p.D, launch_dq_t, p, st)
}
hipError_t launch_dkdv(const BwdParams& p, hipStream_t st) {
  if (dkdv_asm_applies(p)) return launch_dkdv_asm(p, st);
  HARP_RA_DISPATCH_D(p.D, launch_dkdv_t, p, st)
}

}  // namespace harp_ra
