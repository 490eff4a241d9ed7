// gfx950 kernels for the ring-attention block, forward and backward.
//
// Reference math: gemm/ring_attention/ring_attn.cpp
//   forward  ring_attention_forward   :2412-2575  (Q-stationary online softmax over KV chunks)
//   backward ring_attention_backward  :2577-2829  (S/dP recompute, P = exp(S-m)/l, dS, dQ/dK/dV)
// D = rowsum(dO * O) is the caller's preprocess (src/models/z_image/module/attn.py:41).
//
// Work split on one GPU (one rank's share, all ring steps in one launch each):
//   fwd_kernel    per 128-query tile: S^T = K Q^T -> online softmax (lane = query)
//                 -> O^T += V^T P^T, over every 64-key tile of every chunk in ring order.
//   delta_kernel  D = rowsum(dO * O) (fp32).
//   dq_kernel     per 128-query tile: recompute S^T, dP^T, dS^T; dQ^T += K^T dS^T.
//   dkdv_kernel   per 128-key tile (KV-stationary like the reference): per 64-query
//                 tile recompute S, dP; dV += P^T dO, dK += dS^T Q.
//
// Memory path: every streamed 64-row tile is fetched with buffer loads (the
// hardware range check zero-fills rows past a chunk's valid length and
// columns past D), staged in registers while the current tile computes, and
// written to one of two LDS buffers (one barrier per tile).  LDS rows are
// stored with an XOR swizzle of their 16-byte chunks, chunk c of row r at
// position c ^ swz(r), which keeps both access patterns below free of bank
// conflicts:
//   * row reads (ds_read_b128, MFMA operand rows: 8 consecutive rows, one
//     chunk) and
//   * transposed reads (ds_read_b64_tr_b16, MFMA operands that need the tile
//     transposed: V^T, K^T, dO^T, Q^T — 4 rows x 2 chunks per 16 lanes).
// Accumulation is fp32 in registers; P and dS are rounded to bf16 only as
// MFMA operands; exp is v_exp_f32 (exp2) with log2(e) folded into the scale.
#include "ra_common.h"
#include "ra_kernels.h"

namespace harp_ra {

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every valid range: loads 0

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// 64-row LDS tile of DP (>= D) bf16 columns, row width W, swizzled chunks.
template <int DP>
struct Tile {
  static constexpr int W = DP <= 64 ? 64 : 128;
  static constexpr int NCH = DP / 8;  // 16-byte data chunks per row
  static constexpr int ELEMS = 64 * W;
  static __device__ __forceinline__ int off(int r, int c) { return r * W + ((c ^ swz(r)) << 3); }
};

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ bf16x8 buf_load16(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// Per-thread share of a 64-row tile: which 16-byte chunks this thread moves
// (byte offsets relative to the tile's first row, and LDS element offsets).
template <int DP, int NTHR>
struct TileMap {
  using G = Tile<DP>;
  static constexpr int kTot = 64 * G::NCH;
  static constexpr int kN = (kTot + NTHR - 1) / NTHR;
  uint32_t voff[kN];
  int loff[kN];
  __device__ __forceinline__ void init(int64_t row_stride, int D, int tid) {
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int idx = tid + i * NTHR;
      const int r = idx / G::NCH, c = idx % G::NCH;
      const bool in_tile = (kTot % NTHR == 0) || idx < kTot;
      voff[i] = (in_tile && c * 8 < D) ? (uint32_t)(r * row_stride * 2 + c * 16) : kOOB;
      loff[i] = in_tile ? G::off(r, c) : -1;
    }
  }
};

template <int DP, int NTHR>
struct TileRegs {
  using M = TileMap<DP, NTHR>;
  bf16x8 v[M::kN];
  __device__ __forceinline__ void load(const M& m, rsrc_t r) {
#pragma unroll
    for (int i = 0; i < M::kN; ++i) v[i] = buf_load16(r, m.voff[i]);
  }
  __device__ __forceinline__ void store(const M& m, bf16* lds) const {
#pragma unroll
    for (int i = 0; i < M::kN; ++i)
      if ((M::kTot % NTHR == 0) || m.loff[i] >= 0) *(bf16x8*)(lds + m.loff[i]) = v[i];
  }
};

// Buffer resource over rows [row0, row0 + rows) of a [rows][stride] bf16 view.
__device__ __forceinline__ rsrc_t rows_rsrc(const bf16* base, int64_t stride, int row0, int rows) {
  return make_rsrc(base + (int64_t)row0 * stride, (uint32_t)((int64_t)(rows > 0 ? rows : 0) * stride * 2));
}

// Lane offsets for the two LDS read patterns of a Tile<DP>.
template <int DP>
struct LaneOffsets {
  using G = Tile<DP>;
  static constexpr int NDB = DP / 32;
  // row reads: row = rb*32 + l32, chunk = 2*ks + g  ->  rb*32*W + row_off[ks&3] + (ks>>2)*64
  int row_off[4];
  // transposed reads: rows r0 + 4g + s (+8), columns c0 + l32 with c0 = 32*db
  //   ->  r0*W + tr_off[db]  (second half: + 8*W)
  int tr_off[NDB];
  __device__ __forceinline__ void init(int lane) {
    const int l32 = lane & 31, g = lane >> 5;
    const int y = g ^ swz(l32);
#pragma unroll
    for (int b = 0; b < 4; ++b) row_off[b] = l32 * G::W + (((2 * b) ^ y) << 3);
    const int j = lane >> 4, s = (lane >> 2) & 3, m = lane & 3;
    const int row = 4 * g + s;
    const int cl = 2 * (j & 1) + (m >> 1);
#pragma unroll
    for (int db = 0; db < NDB; ++db) tr_off[db] = row * G::W + (((4 * db + cl) ^ swz(row)) << 3) + 4 * (m & 1);
  }
  // A/B operand row fragment: T[rb*32 + l32][16*ks + 8*g .. +7]
  __device__ __forceinline__ bf16x8 row_frag(const bf16* t, int rb, int ks) const {
    return *(const bf16x8*)(t + rb * 32 * G::W + row_off[ks & 3] + (ks >> 2) * 64);
  }
  // k-operand fragment read transposed: T[r0 + {4g+0..3, 8+4g+0..3}][32*db + l32]
  // ds_read_b64_tr_b16: in each 16-lane group, lane i slot s' receives element
  // i%4 of the 8 bytes addressed by lane 4s' + i/4 of that group.
  __device__ __forceinline__ bf16x8 tr_frag(const bf16* t, int r0, int db) const {
    const bf16* p0 = t + r0 * G::W + tr_off[db];
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p0);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 8 * G::W));
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = lo[i];
      r[i + 4] = hi[i];
    }
    return r;
  }
};

// Register-class pins (emit no instructions): long-lived MFMA accumulators
// stay in AGPRs, values the VALU consumes stay in VGPRs, so the allocator does
// not shuttle them between the two files inside the main loops.
__device__ __forceinline__ void pin_agpr(f32x16& x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void pin_vgpr(f32x16& x) { asm volatile("" : "+v"(x)); }

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

// Next (ring step, key tile) after (step, k0), skipping empty chunks.
__device__ __forceinline__ void next_tile(const ChunkTable& ct, int step, int k0, int& nstep, int& nk0) {
  nstep = step;
  nk0 = k0 + 64;
  while (nstep < ct.n && nk0 >= ct.len[ct.order[nstep]]) {
    ++nstep;
    nk0 = 0;
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// KSTEPS = ceil(D/16) k-steps of the S contraction; DBLK = ceil(D/32) row
// blocks of O^T (DP = 32*DBLK >= 16*KSTEPS).  Block = 4 waves x 32 queries;
// 64-key tiles.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 2) void fwd_kernel(FwdParams p) {
  constexpr int DP = DBLK * 32;
  using G = Tile<DP>;
  constexpr float kTau = 8.f;  // lazy-rescale threshold (log2 units): P <= 2^8
  __shared__ __attribute__((aligned(16))) bf16 Ks[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Vs[2][G::ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  int qt, h, b;
  decode_block((p.T + 127) / 128, p.H, qt, h, b);
  const int qi = qt * 128 + wave * 32 + l32;
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
  LaneOffsets<DP> lo;
  lo.init(lane);
  TileMap<DP, 256> tm;
  tm.init(p.skt, p.D, tid);

  f32x16 o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) o[i] = zero16();
  float m_ref = -INFINITY;  // reference point of P (log2 domain), lags the max by < kTau
  float m_max = -INFINITY;  // exact running max of s*c2
  float l_run = 0.f;        // this lane-half's partial sum of exp2(s*c2 - m_ref)

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  int step = 0, k0 = 0;
  while (step < p.ct.n && p.ct.len[p.ct.order[step]] == 0) ++step;
  TileRegs<DP, 256> kr, vr;
  int buf = 0;
  if (step < p.ct.n) {
    const int c = p.ct.order[step];
    kr.load(tm, rows_rsrc(p.ct.k[c] + kvo, p.skt, 0, p.ct.len[c]));
    vr.load(tm, rows_rsrc(p.ct.v[c] + kvo, p.skt, 0, p.ct.len[c]));
    kr.store(tm, Ks[0]);
    vr.store(tm, Vs[0]);
  }
#pragma unroll 1
  while (step < p.ct.n) {
    const int kv_left = p.ct.len[p.ct.order[step]] - k0;
    int nstep, nk0;
    next_tile(p.ct, step, k0, nstep, nk0);
    const bool has_next = nstep < p.ct.n;
    if (has_next) {
      const int c = p.ct.order[nstep];
      const int rows = p.ct.len[c] - nk0;
      kr.load(tm, rows_rsrc(p.ct.k[c] + kvo, p.skt, nk0, rows));
      vr.load(tm, rows_rsrc(p.ct.v[c] + kvo, p.skt, nk0, rows));
    }
    __syncthreads();
    const bf16* K = Ks[buf];
    const bf16* V = Vs[buf];

    // S^T (keys x queries), two 32-key blocks
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[kb] = zero16();
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s[kb] = mfma32x32x16(lo.row_frag(K, kb, ks), qf[ks], s[kb]);
    if (kv_left < 64) {  // tail tile of a chunk: mask keys past its valid length
      // a side-effecting (empty) asm keeps this a real uniform branch instead
      // of selects that would run on every tile
      asm volatile("");
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb * 32 + c_row(r, g) >= kv_left) s[kb][r] = -INFINITY;
    }

    // online softmax, lane = query
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = wave_half_max(mx) * c2;
    m_max = fmaxf(m_max, mx);
    if (__any(mx > m_ref + kTau)) {
      const float m_new = fmaxf(m_ref, mx);
      const float corr = fast_exp2(m_ref - (m_new == -INFINITY ? 0.f : m_new));
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < DBLK; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= corr;
      m_ref = m_new;
    }
    const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;

    bf16x8 pf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float e = fast_exp2(__builtin_fmaf(s[kb][hf * 8 + j], c2, -m_use));
          l_run += e;
          pf[kb * 2 + hf][j] = (bf16)e;
        }

    // O^T += V^T P^T
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2)
#pragma unroll
      for (int db = 0; db < DBLK; ++db) o[db] = mfma32x32x16(lo.tr_frag(V, ks2 * 16, db), pf[ks2], o[db]);

    if (!has_next) break;
    kr.store(tm, Ks[buf ^ 1]);
    vr.store(tm, Vs[buf ^ 1]);
    buf ^= 1;
    step = nstep;
    k0 = nk0;
  }

  // l relative to the exact max: l * 2^(m_ref - m_max)
  float l_tot = wave_half_sum(l_run);
  const float shift = (m_max == -INFINITY) ? 1.f : fast_exp2(m_ref - m_max);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  l_tot *= shift;
  if (!q_ok) return;
  float* orow = p.out + (int64_t)b * p.sob + (int64_t)h * p.soh + (int64_t)qi * p.sot;
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = db * 32 + c_row(r, g);
      if (d < p.D) orow[d] = o[db][r] * inv;
    }
  if (g == 0) {
    const int64_t si = ((int64_t)b * p.H + h) * p.T + qi;
    const float m_nat = m_max * kLn2;
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

// Per-query log2-domain LSE from the forward's (m, l): (m + ln l) * log2(e).
// Rows with l <= 0 (no valid key) get +inf so that P = exp2(s - inf) = 0.
__device__ __forceinline__ float lse2_of(const void* m, int m_bf16, const float* l, int64_t i) {
  const float mm = m_bf16 ? (float)((const bf16*)m)[i] : ((const float*)m)[i];
  const float ll = l[i];
  return (ll > 0.f) ? (mm + __logf(ll)) * kLog2e : INFINITY;
}

// ---------------------------------------------------------------------------
// Backward dQ (Q-stationary): dQ = scale * sum_c dS_c K_c
// ---------------------------------------------------------------------------
// Pad keys need no mask here: their K/V rows load as zero, so their dS has
// no effect on dQ^T = K^T dS^T.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 2) void dq_kernel(BwdParams p) {
  constexpr int DP = DBLK * 32;
  using G = Tile<DP>;
  __shared__ __attribute__((aligned(16))) bf16 Ks[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Vs[2][G::ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  int qt, h, b;
  decode_block((p.T + 127) / 128, p.H, qt, h, b);
  const int qi = qt * 128 + wave * 32 + l32;
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
  const float lse2 = q_ok ? lse2_of(p.m, p.m_bf16, p.l, si) : INFINITY;
  const float dlt = q_ok ? p.delta[si] : 0.f;
  LaneOffsets<DP> lo;
  lo.init(lane);
  TileMap<DP, 256> tm;
  tm.init(p.skt, p.D, tid);

  f32x16 dq[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) dq[i] = zero16();

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  int step = 0, k0 = 0;
  while (step < p.ct.n && p.ct.len[p.ct.order[step]] == 0) ++step;
  TileRegs<DP, 256> kr, vr;
  int buf = 0;
  if (step < p.ct.n) {
    const int c = p.ct.order[step];
    kr.load(tm, rows_rsrc(p.ct.k[c] + kvo, p.skt, 0, p.ct.len[c]));
    vr.load(tm, rows_rsrc(p.ct.v[c] + kvo, p.skt, 0, p.ct.len[c]));
    kr.store(tm, Ks[0]);
    vr.store(tm, Vs[0]);
  }
#pragma unroll 1
  while (step < p.ct.n) {
    int nstep, nk0;
    next_tile(p.ct, step, k0, nstep, nk0);
    const bool has_next = nstep < p.ct.n;
    if (has_next) {
      const int c = p.ct.order[nstep];
      const int rows = p.ct.len[c] - nk0;
      kr.load(tm, rows_rsrc(p.ct.k[c] + kvo, p.skt, nk0, rows));
      vr.load(tm, rows_rsrc(p.ct.v[c] + kvo, p.skt, nk0, rows));
    }
    __syncthreads();
    const bf16* K = Ks[buf];
    const bf16* V = Vs[buf];

    f32x16 s[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = zero16();
      dp[kb] = zero16();
    }
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = mfma32x32x16(lo.row_frag(K, kb, ks), qf[ks], s[kb]);
        dp[kb] = mfma32x32x16(lo.row_frag(V, kb, ks), gf[ks], dp[kb]);
      }
    bf16x8 dsf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fast_exp2(__builtin_fmaf(s[kb][r], c2, -lse2));
        dsf[kb * 2 + (r >> 3)][r & 7] = (bf16)(pv * (dp[kb][r] - dlt));
      }

    // dQ^T += K^T dS^T
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2)
#pragma unroll
      for (int db = 0; db < DBLK; ++db) dq[db] = mfma32x32x16(lo.tr_frag(K, ks2 * 16, db), dsf[ks2], dq[db]);

    if (!has_next) break;
    kr.store(tm, Ks[buf ^ 1]);
    vr.store(tm, Vs[buf ^ 1]);
    buf ^= 1;
    step = nstep;
    k0 = nk0;
  }

  if (!q_ok) return;
  char* drow = (char*)p.dq + (((int64_t)b * p.sdqb + (int64_t)h * p.sdqh + (int64_t)qi * p.sdqt) << (p.dq_f32 ? 2 : 1));
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = db * 32 + c_row(r, g);
      if (d < p.D) {
        const float v = dq[db][r] * p.scale;
        if (p.dq_f32) ((float*)drow)[d] = v;
        else ((bf16*)drow)[d] = (bf16)v;
      }
    }
}

// ---------------------------------------------------------------------------
// Backward dK/dV (KV-stationary, as ring_attn.cpp:2723-2816)
// ---------------------------------------------------------------------------
// Block = 4 waves x 32 keys.  The block's 128 K and V rows stay in LDS for the
// whole kernel (both are MFMA row operands there); the loop streams 64-query
// tiles of Q / dO (+ LSE, D) through double-buffered LDS and handles each tile
// as two 32-query halves.  Pad keys (past the chunk's valid length) are
// written as zero at the end instead of being masked per tile: in this layout
// a key's P / dS only reach its own dK / dV rows.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 1) void dkdv_kernel(BwdParams p) {
  constexpr int DP = DBLK * 32;
  using G = Tile<DP>;
  __shared__ __attribute__((aligned(16))) bf16 Kb[2 * G::ELEMS];  // 128 key rows
  __shared__ __attribute__((aligned(16))) bf16 Vb[2 * G::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Qs[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 Gs[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) float Ls[2][64];
  __shared__ __attribute__((aligned(16))) float Dls[2][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  int kt, h, b;
  decode_block(p.n_key_tiles, p.H, kt, h, b);
  int c = 0;
#pragma unroll 1
  for (int i = 1; i < p.ct.n; ++i)
    if (kt >= p.ct.tile0[i]) c = i;
  const int kblk0 = (kt - p.ct.tile0[c]) * 128;
  const int key0 = kblk0 + wave * 32;
  const int len = p.ct.len[c];
  const float c2 = p.scale * kLog2e;

  f32x16 dk[DBLK], dv[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
    pin_agpr(dk[i]);
    pin_agpr(dv[i]);
  }

  if (kblk0 < len) {  // block has at least one valid key (block-uniform)
    LaneOffsets<DP> lo;
    lo.init(lane);
    {
      TileMap<DP, 256> tmk;
      tmk.init(p.skt, p.D, tid);
      const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
      TileRegs<DP, 256> t;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r0 = kblk0 + 64 * half;
        t.load(tmk, rows_rsrc(p.ct.k[c] + kvo, p.skt, r0, len - r0));
        t.store(tmk, Kb + half * G::ELEMS);
        t.load(tmk, rows_rsrc(p.ct.v[c] + kvo, p.skt, r0, len - r0));
        t.store(tmk, Vb + half * G::ELEMS);
      }
    }
    TileMap<DP, 256> tmq, tmg;
    tmq.init(p.sqt, p.D, tid);
    tmg.init(p.sdt, p.D, tid);
    const bf16* qb_ = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
    const bf16* gb_ = p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh;
    const int64_t sbase = ((int64_t)b * p.H + h) * p.T;

    TileRegs<DP, 256> qr, gr;
    float lse_r = INFINITY, dl_r = 0.f;
    auto load_q = [&](int q0) {
      qr.load(tmq, rows_rsrc(qb_, p.sqt, q0, p.T - q0));
      gr.load(tmg, rows_rsrc(gb_, p.sdt, q0, p.T - q0));
      if (tid < 64) {
        const int qq = q0 + tid;
        lse_r = (qq < p.T) ? lse2_of(p.m, p.m_bf16, p.l, sbase + qq) : INFINITY;
        dl_r = (qq < p.T) ? p.delta[sbase + qq] : 0.f;
      }
    };
    auto store_q = [&](int bf) {
      qr.store(tmq, Qs[bf]);
      gr.store(tmg, Gs[bf]);
      if (tid < 64) {
        Ls[bf][tid] = lse_r;
        Dls[bf][tid] = dl_r;
      }
    };
    load_q(0);
    store_q(0);
    int buf = 0;
#pragma unroll 1
    for (int q0 = 0; q0 < p.T; q0 += 64) {
      const bool has_next = q0 + 64 < p.T;
      if (has_next) load_q(q0 + 64);
      __syncthreads();
      const bf16* Q = Qs[buf];
      const bf16* Gd = Gs[buf];
#pragma unroll
      for (int i = 0; i < DBLK; ++i) {
        pin_agpr(dk[i]);
        pin_agpr(dv[i]);
      }

      // per 32-query half: S = Q K^T, dP = dO V^T (C row = query, col = key),
      // then P, dS and the dV / dK updates of that half
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          s = mfma32x32x16(lo.row_frag(Q, qb, ks), lo.row_frag(Kb, wave, ks), s);
          dp = mfma32x32x16(lo.row_frag(Gd, qb, ks), lo.row_frag(Vb, wave, ks), dp);
        }
        bf16x8 pf[2], dsf[2];
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x4 lse4 = *(const f32x4*)(&Ls[buf][qb * 32 + 8 * i4 + 4 * g]);
          const f32x4 dl4 = *(const f32x4*)(&Dls[buf][qb * 32 + 8 * i4 + 4 * g]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = i4 * 4 + t;
            const float pv = fast_exp2(__builtin_fmaf(s[r], c2, -lse4[t]));
            pf[r >> 3][r & 7] = (bf16)pv;
            dsf[r >> 3][r & 7] = (bf16)(pv * (dp[r] - dl4[t]));
          }
        }
        // dV += P^T dO ; dK += dS^T Q   (M = keys, N = d, K = the 32 queries of this half)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int db = 0; db < DBLK; ++db) {
            const int r0 = qb * 32 + h2 * 16;
            dv[db] = mfma32x32x16(pf[h2], lo.tr_frag(Gd, r0, db), dv[db]);
            dk[db] = mfma32x32x16(dsf[h2], lo.tr_frag(Q, r0, db), dk[db]);
          }
      }

#pragma unroll
      for (int i = 0; i < DBLK; ++i) {
        pin_agpr(dk[i]);
        pin_agpr(dv[i]);
      }
      if (!has_next) break;
      store_q(buf ^ 1);
      buf ^= 1;
    }
  }

  // store: C layout row = key key0 + c_row(r,g), col = d = db*32 + l32;
  // keys past the valid length (pads) get zero
  const int64_t base = (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
#pragma unroll
  for (int db = 0; db < DBLK; ++db) {
    const int d = db * 32 + l32;
    if (d >= p.D) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = key0 + c_row(r, g);
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

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------
template <int KSTEPS, int DBLK>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t st) {
  const int n = ((p.T + 127) / 128) * p.H * p.B;
  hipLaunchKernelGGL((fwd_kernel<KSTEPS, DBLK>), dim3(n), dim3(256), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dq_t(const BwdParams& p, hipStream_t st) {
  const int n = ((p.T + 127) / 128) * p.H * p.B;
  hipLaunchKernelGGL((dq_kernel<KSTEPS, DBLK>), dim3(n), dim3(256), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dkdv_t(const BwdParams& p, hipStream_t st) {
  const int n = p.n_key_tiles * p.H * p.B;
  hipLaunchKernelGGL((dkdv_kernel<KSTEPS, DBLK>), dim3(n), dim3(256), 0, st, p);
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

hipError_t launch_fwd(const FwdParams& p, hipStream_t st) { HARP_RA_DISPATCH_D(p.D, launch_fwd_t, p, st) }
hipError_t launch_delta(const DeltaParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  dim3 grid((unsigned)((rows + 15) / 16));
  hipLaunchKernelGGL(delta_kernel, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
hipError_t launch_dq(const BwdParams& p, hipStream_t st) { HARP_RA_DISPATCH_D(p.D, launch_dq_t, p, st) }
hipError_t launch_dkdv(const BwdParams& p, hipStream_t st) { HARP_RA_DISPATCH_D(p.D, launch_dkdv_t, p, st) }

}  // namespace harp_ra
