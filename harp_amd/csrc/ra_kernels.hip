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
// Every streamed tile is staged global -> registers -> LDS (row-major, padded
// rows) with the next tile's loads in flight during the current tile's MFMA
// work (two LDS buffers, one barrier per tile).  Operands that the MFMA wants
// transposed (V^T, K^T, dO^T, Q^T) are read from the same row-major tiles with
// ds_read_b64_tr_b16.  Accumulation is fp32 in registers; P and dS are
// rounded to bf16 only as MFMA operands; exp is v_exp_f32 (exp2) with
// log2(e) folded into the softmax scale.
#include "ra_common.h"
#include "ra_kernels.h"

namespace harp_ra {

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// k-operand fragment read transposed from a row-major LDS tile T[rows][ld]:
// lane l gets T[r0 + {4g+0..3, 8+4g+0..3}][c0 + l%32] (g = l/32), the k-set a
// 32x32 C-layout accumulator holds, so it pairs with a C-layout operand.
// ds_read_b64_tr_b16: in each 16-lane group, lane i slot s receives element
// i%4 of the 8 bytes addressed by lane 4s + i/4 of that group.
__device__ __forceinline__ bf16x8 tr_kset(const bf16* tile, int ld, int r0, int c0, int lane) {
  const int j = lane >> 4, s = (lane >> 2) & 3, m = lane & 3, g = lane >> 5;
  const bf16* p0 = tile + (r0 + 4 * g + s) * ld + c0 + 16 * (j & 1) + 4 * m;
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p0);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 8 * ld));
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = lo[i];
    r[i + 4] = hi[i];
  }
  return r;
}

__device__ __forceinline__ float wave_half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 64-row tile of NCH 16-byte chunks per row, staged through registers.
template <int NCH, int NTHR>
struct TileRegs {
  static constexpr int kN = (64 * NCH + NTHR - 1) / NTHR;
  bf16x8 v[kN];

  // rows >= rows_valid or columns >= cols_valid load as zero
  __device__ __forceinline__ void load(const bf16* base, int64_t rs, int rows_valid, int cols_valid, int tid) {
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int idx = tid + i * NTHR;
      const int r = idx / NCH, c = (idx % NCH) * 8;
      const bool ok = (64 * NCH % NTHR == 0 || idx < 64 * NCH) && r < rows_valid && c < cols_valid;
      v[i] = ok ? *(const bf16x8*)(base + (int64_t)r * rs + c) : zero8();
    }
  }
  __device__ __forceinline__ void store(bf16* lds, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int idx = tid + i * NTHR;
      if (64 * NCH % NTHR == 0 || idx < 64 * NCH) {
        const int r = idx / NCH, c = (idx % NCH) * 8;
        *(bf16x8*)(lds + r * ld + c) = v[i];
      }
    }
  }
};

// Block index -> (tile, head, batch) with all tiles of one (b, h) kept on one
// XCD (workgroups are dealt to the 8 XCDs round-robin), so a head's K/V
// stream is fetched into that XCD's L2 once for all of its query tiles.
__device__ __forceinline__ void decode_block(int n_tiles, int H, int& tile, int& h, int& b) {
  const int total = (int)gridDim.x;
  int lin = (int)blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  tile = lin % n_tiles;
  const int bh = lin / n_tiles;
  h = bh % H;
  b = bh / H;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// KSTEPS = ceil(D/16) k-steps of the S contraction; DBLK = ceil(D/32) row
// blocks of O^T (DP = 32*DBLK >= KD = 16*KSTEPS).  Block = 4 waves x 32
// queries; 64-key tiles.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 2) void fwd_kernel(FwdParams p) {
  constexpr int BN = 64;
  constexpr int DP = DBLK * 32;
  constexpr int LD = DP + 8;  // padded LDS row (bf16 elements)
  constexpr int NCH = DP / 8;
  constexpr float kTau = 8.f;  // lazy-rescale threshold (log2 units): P <= 2^8
  __shared__ __attribute__((aligned(16))) bf16 Ks[2][BN * LD];
  __shared__ __attribute__((aligned(16))) bf16 Vs[2][BN * LD];

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

  f32x16 o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) o[i] = zero16();
  float m_ref = -INFINITY;  // reference point of P (log2 domain), lags the max by < kTau
  float m_max = -INFINITY;  // exact running max of s*c2
  float l_run = 0.f;        // this lane-half's partial sum of exp2(s*c2 - m_ref)

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  // flattened (ring step, key tile) schedule
  int step = 0, k0 = 0;
  while (step < p.ct.n && p.ct.len[p.ct.order[step]] == 0) ++step;
  TileRegs<NCH, 256> kr, vr;
  int buf = 0;
  if (step < p.ct.n) {
    const int c = p.ct.order[step];
    kr.load(p.ct.k[c] + kvo, p.skt, p.ct.len[c], p.D, tid);
    vr.load(p.ct.v[c] + kvo, p.skt, p.ct.len[c], p.D, tid);
    kr.store(Ks[0], LD, tid);
    vr.store(Vs[0], LD, tid);
  }
#pragma unroll 1
  while (step < p.ct.n) {
    const int len = p.ct.len[p.ct.order[step]];
    int nstep = step, nk0 = k0 + BN;
    while (nstep < p.ct.n && nk0 >= p.ct.len[p.ct.order[nstep]]) {
      ++nstep;
      nk0 = 0;
    }
    const bool has_next = nstep < p.ct.n;
    if (has_next) {
      const int c = p.ct.order[nstep];
      const int64_t off = kvo + (int64_t)nk0 * p.skt;
      kr.load(p.ct.k[c] + off, p.skt, p.ct.len[c] - nk0, p.D, tid);
      vr.load(p.ct.v[c] + off, p.skt, p.ct.len[c] - nk0, p.D, tid);
    }
    __syncthreads();
    const bf16* K = Ks[buf];
    const bf16* V = Vs[buf];

    // S^T (keys x queries), two 32-key blocks
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = zero16();
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const bf16x8 a = *(const bf16x8*)(K + (kb * 32 + l32) * LD + ks * 16 + g * 8);
        s[kb] = mfma32x32x16(a, qf[ks], s[kb]);
      }
    }
    const int kv_left = len - k0;
    if (kv_left < BN) {
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
      for (int db = 0; db < DBLK; ++db) {
        const bf16x8 a = tr_kset(V, LD, ks2 * 16, db * 32, lane);
        o[db] = mfma32x32x16(a, pf[ks2], o[db]);
      }

    if (!has_next) break;
    kr.store(Ks[buf ^ 1], LD, tid);
    vr.store(Vs[buf ^ 1], LD, tid);
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
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 2) void dq_kernel(BwdParams p) {
  constexpr int BN = 64;
  constexpr int DP = DBLK * 32;
  constexpr int LD = DP + 8;
  constexpr int NCH = DP / 8;
  __shared__ __attribute__((aligned(16))) bf16 Ks[2][BN * LD];
  __shared__ __attribute__((aligned(16))) bf16 Vs[2][BN * LD];

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

  f32x16 dq[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) dq[i] = zero16();

  const int64_t kvo = (int64_t)b * p.skb + (int64_t)h * p.skh;
  int step = 0, k0 = 0;
  while (step < p.ct.n && p.ct.len[p.ct.order[step]] == 0) ++step;
  TileRegs<NCH, 256> kr, vr;
  int buf = 0;
  if (step < p.ct.n) {
    const int c = p.ct.order[step];
    kr.load(p.ct.k[c] + kvo, p.skt, p.ct.len[c], p.D, tid);
    vr.load(p.ct.v[c] + kvo, p.skt, p.ct.len[c], p.D, tid);
    kr.store(Ks[0], LD, tid);
    vr.store(Vs[0], LD, tid);
  }
#pragma unroll 1
  while (step < p.ct.n) {
    const int len = p.ct.len[p.ct.order[step]];
    int nstep = step, nk0 = k0 + BN;
    while (nstep < p.ct.n && nk0 >= p.ct.len[p.ct.order[nstep]]) {
      ++nstep;
      nk0 = 0;
    }
    const bool has_next = nstep < p.ct.n;
    if (has_next) {
      const int c = p.ct.order[nstep];
      const int64_t off = kvo + (int64_t)nk0 * p.skt;
      kr.load(p.ct.k[c] + off, p.skt, p.ct.len[c] - nk0, p.D, tid);
      vr.load(p.ct.v[c] + off, p.skt, p.ct.len[c] - nk0, p.D, tid);
    }
    __syncthreads();
    const bf16* K = Ks[buf];
    const bf16* V = Vs[buf];
    const int kv_left = len - k0;

    bf16x8 dsf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const bf16x8 a = *(const bf16x8*)(K + (kb * 32 + l32) * LD + ks * 16 + g * 8);
        s = mfma32x32x16(a, qf[ks], s);
        const bf16x8 av = *(const bf16x8*)(V + (kb * 32 + l32) * LD + ks * 16 + g * 8);
        dp = mfma32x32x16(av, gf[ks], dp);
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = hf * 8 + j;
          float pv = fast_exp2(__builtin_fmaf(s[r], c2, -lse2));
          if (kv_left < BN && kb * 32 + c_row(r, g) >= kv_left) pv = 0.f;
          dsf[kb * 2 + hf][j] = (bf16)(pv * (dp[r] - dlt));
        }
    }

    // dQ^T += K^T dS^T
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2)
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const bf16x8 a = tr_kset(K, LD, ks2 * 16, db * 32, lane);
        dq[db] = mfma32x32x16(a, dsf[ks2], dq[db]);
      }

    if (!has_next) break;
    kr.store(Ks[buf ^ 1], LD, tid);
    vr.store(Vs[buf ^ 1], LD, tid);
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
// Block = 4 waves x 32 keys; loops over 64-query tiles of the local Q.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 1) void dkdv_kernel(BwdParams p) {
  constexpr int BMQ = 64;
  constexpr int DP = DBLK * 32;
  constexpr int LD = DP + 8;
  constexpr int NCH = DP / 8;
  __shared__ __attribute__((aligned(16))) bf16 Qs[2][BMQ * LD];
  __shared__ __attribute__((aligned(16))) bf16 Gs[2][BMQ * LD];
  __shared__ __attribute__((aligned(16))) float Ls[2][BMQ];
  __shared__ __attribute__((aligned(16))) float Dls[2][BMQ];

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
  const int key = key0 + l32;
  const bool k_ok = key < len;
  const float c2 = p.scale * kLog2e;

  f32x16 dk[DBLK], dv[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  if (kblk0 < len) {  // block has at least one valid key (block-uniform)
    bf16x8 kf[KSTEPS], vf[KSTEPS];
    {
      const int64_t ko = (int64_t)b * p.skb + (int64_t)h * p.skh + (int64_t)key * p.skt;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int d0 = ks * 16 + g * 8;
        const bool ok = k_ok && d0 < p.D;
        kf[ks] = ok ? *(const bf16x8*)(p.ct.k[c] + ko + d0) : zero8();
        vf[ks] = ok ? *(const bf16x8*)(p.ct.v[c] + ko + d0) : zero8();
      }
    }
    const bf16* qb_ = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
    const bf16* gb_ = p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh;
    const int64_t sbase = ((int64_t)b * p.H + h) * p.T;

    TileRegs<NCH, 256> qr, gr;
    float lse_r = INFINITY, dl_r = 0.f;
    auto load_q = [&](int q0) {
      qr.load(qb_ + (int64_t)q0 * p.sqt, p.sqt, p.T - q0, p.D, tid);
      gr.load(gb_ + (int64_t)q0 * p.sdt, p.sdt, p.T - q0, p.D, tid);
      if (tid < BMQ) {
        const int qq = q0 + tid;
        lse_r = (qq < p.T) ? lse2_of(p.m, p.m_bf16, p.l, sbase + qq) : INFINITY;
        dl_r = (qq < p.T) ? p.delta[sbase + qq] : 0.f;
      }
    };
    auto store_q = [&](int bf) {
      qr.store(Qs[bf], LD, tid);
      gr.store(Gs[bf], LD, tid);
      if (tid < BMQ) {
        Ls[bf][tid] = lse_r;
        Dls[bf][tid] = dl_r;
      }
    };
    load_q(0);
    store_q(0);
    int buf = 0;
#pragma unroll 1
    for (int q0 = 0; q0 < p.T; q0 += BMQ) {
      const bool has_next = q0 + BMQ < p.T;
      if (has_next) load_q(q0 + BMQ);
      __syncthreads();
      const bf16* Q = Qs[buf];
      const bf16* G = Gs[buf];

      bf16x8 pf[4], dsf[4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const bf16x8 aq = *(const bf16x8*)(Q + (qb * 32 + l32) * LD + ks * 16 + g * 8);
          s = mfma32x32x16(aq, kf[ks], s);
          const bf16x8 ag = *(const bf16x8*)(G + (qb * 32 + l32) * LD + ks * 16 + g * 8);
          dp = mfma32x32x16(ag, vf[ks], dp);
        }
        // C layout: row = query qb*32 + c_row(r,g), col = key (this lane)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x4 lse4 = *(const f32x4*)(&Ls[buf][qb * 32 + 8 * i4 + 4 * g]);
          const f32x4 dl4 = *(const f32x4*)(&Dls[buf][qb * 32 + 8 * i4 + 4 * g]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = i4 * 4 + t;
            float pv = fast_exp2(__builtin_fmaf(s[r], c2, -lse4[t]));
            if (!k_ok) pv = 0.f;
            const float ds = pv * (dp[r] - dl4[t]);
            pf[qb * 2 + (r >> 3)][r & 7] = (bf16)pv;
            dsf[qb * 2 + (r >> 3)][r & 7] = (bf16)ds;
          }
        }
      }

      // dV += P^T dO ; dK += dS^T Q   (M = keys, N = d, K = queries)
#pragma unroll
      for (int ks2 = 0; ks2 < 4; ++ks2)
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
          const bf16x8 bg = tr_kset(G, LD, ks2 * 16, db * 32, lane);
          dv[db] = mfma32x32x16(pf[ks2], bg, dv[db]);
          const bf16x8 bq = tr_kset(Q, LD, ks2 * 16, db * 32, lane);
          dk[db] = mfma32x32x16(dsf[ks2], bq, dk[db]);
        }

      if (!has_next) break;
      store_q(buf ^ 1);
      buf ^= 1;
    }
  }

  // store: C layout row = key key0 + c_row(r,g), col = d = db*32 + l32
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
      const float vk = dk[db][r] * p.scale, vv = dv[db][r];
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
