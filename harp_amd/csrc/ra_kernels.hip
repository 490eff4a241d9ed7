// gfx950 kernels for the ring-attention block, forward and backward.
//
// Reference math: gemm/ring_attention/ring_attn.cpp
//   forward  ring_attention_forward   :2412-2575  (Q-stationary online softmax over KV chunks)
//   backward ring_attention_backward  :2577-2829  (S/dP recompute, P = exp(S-m)/l, dS, dQ/dK/dV)
// D = rowsum(dO * O) is the caller's preprocess (src/models/z_image/module/attn.py:41).
//
// Work split on one GPU (one rank's share, all ring steps in one launch):
//   pack_t_kernel   transposes a [rows][D] operand into a zero-padded [DP][Lp]
//                   panel (the MFMA k-operand wants consecutive rows per lane);
//                   the GPU analogue of the reference's pack_b/pack_a panels.
//   fwd_kernel      per 128-query tile: S^T = K Q^T -> online softmax (lane = query)
//                   -> O^T += V^T P^T, looping over every KV tile of every chunk.
//   delta_kernel    D = rowsum(dO * O) (fp32).
//   dq_kernel       per 128-query tile: recompute S^T, dP^T, dS^T; dQ^T += K^T dS^T.
//   dkdv_kernel     per 128-key tile (KV-stationary like the reference):
//                   recompute S, dP per 64-query tile; dV += P^T dO, dK += dS^T Q.
// All accumulation is fp32 in registers; P and dS are rounded to bf16 only as
// MFMA operands.  exp uses v_exp_f32 (exp2) with log2(e) folded into the scale.
#include "ra_common.h"
#include "ra_kernels.h"

namespace harp_ra {

// ---------------------------------------------------------------------------
// Transposing pack: dst[b][h][d][off[c] + r] = src_c[b][h][r][d] (zero pad)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_t_kernel(PackParams p) {
  __shared__ bf16 tile[64][130];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  int c = 0;
#pragma unroll 1
  for (int i = 1; i < p.n; ++i)
    if ((int)blockIdx.x >= p.tile0[i]) c = i;
  const int r0 = ((int)blockIdx.x - p.tile0[c]) * 64;
  const int nvec = p.DP / 8;
  const bf16* src = p.src[c] + (int64_t)b * p.sb + (int64_t)h * p.sh;
  for (int idx = tid; idx < 64 * nvec; idx += 256) {
    const int r = idx / nvec, d0 = (idx % nvec) * 8;
    bf16x8 val = zero8();
    if (r0 + r < p.len[c] && d0 < p.D) val = *(const bf16x8*)(src + (int64_t)(r0 + r) * p.st + d0);
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[r][d0 + j] = val[j];
  }
  __syncthreads();
  bf16* dst = p.dst + ((int64_t)(b * p.H + h) * p.DP) * p.lp + p.off[c] + r0;
  for (int idx = tid; idx < p.DP * 8; idx += 256) {
    const int d = idx / 8, cv = (idx % 8) * 8;
    bf16x8 val;
#pragma unroll
    for (int j = 0; j < 8; ++j) val[j] = tile[cv + j][d];
    *(bf16x8*)(dst + (int64_t)d * p.lp + cv) = val;
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// KSTEPS = ceil(D/16) k-steps of the S contraction; DBLK = ceil(D/32) row
// blocks of O^T.  Block = 4 waves, 32 queries per wave, 64 keys per KV tile.
template <int KSTEPS, int DBLK>
__global__ __launch_bounds__(256, 1) void fwd_kernel(FwdParams p) {
  constexpr int BN = 64;
  constexpr int KD = KSTEPS * 16;
  constexpr int KS_LD = KD + 8;
  constexpr int DP = DBLK * 32;
  constexpr int VT_LD = BN + 8;
  __shared__ __attribute__((aligned(16))) bf16 Ks[BN * KS_LD];
  __shared__ __attribute__((aligned(16))) bf16 Vts[DP * VT_LD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qi = blockIdx.x * 128 + wave * 32 + l32;
  const bool q_ok = qi < p.T;
  const float c2 = p.scale * kLog2e;

  // Q^T columns (B operand of S^T = K Q^T): lane holds Q[qi][ks*16 + 8g .. +7].
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
  float m_run = -INFINITY;  // running max of s*c2 (log2 domain)
  float l_run = 0.f;        // this lane-half's partial row sum

  const bf16* vt_bh = p.vt + ((int64_t)(b * p.H + h) * DP) * p.ct.lp;
#pragma unroll 1
  for (int step = 0; step < p.ct.n; ++step) {
    const int c = p.ct.order[step];
    const int len = p.ct.len[c];
    const bf16* kc = p.ct.k[c] + (int64_t)b * p.skb + (int64_t)h * p.skh;
    const bf16* vtc = vt_bh + p.ct.off[c];
#pragma unroll 1
    for (int k0 = 0; k0 < len; k0 += BN) {
      __syncthreads();
      // K tile [BN][KD] (row-major, zero beyond len / D)
      for (int idx = tid; idx < BN * (KD / 8); idx += 256) {
        const int r = idx / (KD / 8), d0 = (idx % (KD / 8)) * 8;
        bf16x8 val = zero8();
        if (k0 + r < len && d0 < p.D) val = *(const bf16x8*)(kc + (int64_t)(k0 + r) * p.skt + d0);
        *(bf16x8*)(&Ks[r * KS_LD + d0]) = val;
      }
      // V^T tile [DP][BN] from the packed panel
      for (int idx = tid; idx < DP * (BN / 8); idx += 256) {
        const int r = idx / (BN / 8), c0 = (idx % (BN / 8)) * 8;
        *(bf16x8*)(&Vts[r * VT_LD + c0]) = *(const bf16x8*)(vtc + (int64_t)r * p.ct.lp + k0 + c0);
      }
      __syncthreads();

      // S^T (keys x queries), two 32-key blocks
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = zero16();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const bf16x8 a = *(const bf16x8*)(&Ks[(kb * 32 + l32) * KS_LD + ks * 16 + g * 8]);
          s[kb] = mfma32x32x16(a, qf[ks], s[kb]);
        }
      }
      if (k0 + BN > len) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (k0 + kb * 32 + c_row(r, g) >= len) s[kb][r] = -INFINITY;
      }

      // online softmax, lane = query
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx * c2);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float corr = fast_exp2(m_run - m_use);
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < DBLK; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= corr;
      m_run = m_new;

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
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
          const bf16* vrow = &Vts[(db * 32 + l32) * VT_LD + ks2 * 16 + 4 * g];
          const bf16x4 lo = *(const bf16x4*)vrow;
          const bf16x4 hi = *(const bf16x4*)(vrow + 8);
          bf16x8 a;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            a[j] = lo[j];
            a[j + 4] = hi[j];
          }
          o[db] = mfma32x32x16(a, pf[ks2], o[db]);
        }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!q_ok) return;
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
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
    const float m_nat = m_run * kLn2;
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
__global__ __launch_bounds__(256, 1) void dq_kernel(BwdParams p) {
  constexpr int BN = 64;
  constexpr int KD = KSTEPS * 16;
  constexpr int KS_LD = KD + 8;
  constexpr int DP = DBLK * 32;
  constexpr int VT_LD = BN + 8;
  __shared__ __attribute__((aligned(16))) bf16 Ks[BN * KS_LD];
  __shared__ __attribute__((aligned(16))) bf16 Vs[BN * KS_LD];
  __shared__ __attribute__((aligned(16))) bf16 Kts[DP * VT_LD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qi = blockIdx.x * 128 + wave * 32 + l32;
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

  const bf16* kt_bh = p.kt + ((int64_t)(b * p.H + h) * DP) * p.ct.lp;
#pragma unroll 1
  for (int step = 0; step < p.ct.n; ++step) {
    const int c = p.ct.order[step];
    const int len = p.ct.len[c];
    const bf16* kc = p.ct.k[c] + (int64_t)b * p.skb + (int64_t)h * p.skh;
    const bf16* vc = p.ct.v[c] + (int64_t)b * p.skb + (int64_t)h * p.skh;
    const bf16* ktc = kt_bh + p.ct.off[c];
#pragma unroll 1
    for (int k0 = 0; k0 < len; k0 += BN) {
      __syncthreads();
      for (int idx = tid; idx < BN * (KD / 8); idx += 256) {
        const int r = idx / (KD / 8), d0 = (idx % (KD / 8)) * 8;
        bf16x8 kv = zero8(), vv = zero8();
        if (k0 + r < len && d0 < p.D) {
          kv = *(const bf16x8*)(kc + (int64_t)(k0 + r) * p.skt + d0);
          vv = *(const bf16x8*)(vc + (int64_t)(k0 + r) * p.skt + d0);
        }
        *(bf16x8*)(&Ks[r * KS_LD + d0]) = kv;
        *(bf16x8*)(&Vs[r * KS_LD + d0]) = vv;
      }
      for (int idx = tid; idx < DP * (BN / 8); idx += 256) {
        const int r = idx / (BN / 8), c0 = (idx % (BN / 8)) * 8;
        *(bf16x8*)(&Kts[r * VT_LD + c0]) = *(const bf16x8*)(ktc + (int64_t)r * p.ct.lp + k0 + c0);
      }
      __syncthreads();

      bf16x8 dsf[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const bf16x8 a = *(const bf16x8*)(&Ks[(kb * 32 + l32) * KS_LD + ks * 16 + g * 8]);
          s = mfma32x32x16(a, qf[ks], s);
          const bf16x8 av = *(const bf16x8*)(&Vs[(kb * 32 + l32) * KS_LD + ks * 16 + g * 8]);
          dp = mfma32x32x16(av, gf[ks], dp);
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int r = hf * 8 + j;
            float pv = fast_exp2(__builtin_fmaf(s[r], c2, -lse2));
            if (k0 + kb * 32 + c_row(r, g) >= len) pv = 0.f;
            dsf[kb * 2 + hf][j] = (bf16)(pv * (dp[r] - dlt));
          }
      }

#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
          const bf16* krow = &Kts[(db * 32 + l32) * VT_LD + ks2 * 16 + 4 * g];
          const bf16x4 lo = *(const bf16x4*)krow;
          const bf16x4 hi = *(const bf16x4*)(krow + 8);
          bf16x8 a;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            a[j] = lo[j];
            a[j + 4] = hi[j];
          }
          dq[db] = mfma32x32x16(a, dsf[ks2], dq[db]);
        }
    }
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
  constexpr int KD = KSTEPS * 16;
  constexpr int KS_LD = KD + 8;
  constexpr int DP = DBLK * 32;
  constexpr int T_LD = BMQ + 8;
  __shared__ __attribute__((aligned(16))) bf16 Qs[BMQ * KS_LD];
  __shared__ __attribute__((aligned(16))) bf16 Gs[BMQ * KS_LD];
  __shared__ __attribute__((aligned(16))) bf16 Qts[DP * T_LD];
  __shared__ __attribute__((aligned(16))) bf16 Gts[DP * T_LD];
  __shared__ __attribute__((aligned(16))) float Ls[BMQ];
  __shared__ __attribute__((aligned(16))) float Dls[BMQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int b = blockIdx.z, h = blockIdx.y;
  int c = 0;
#pragma unroll 1
  for (int i = 1; i < p.ct.n; ++i)
    if ((int)blockIdx.x >= p.ct.tile0[i]) c = i;
  const int key0 = ((int)blockIdx.x - p.ct.tile0[c]) * 128 + wave * 32;
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

  if (key0 - wave * 32 < len) {  // block has at least one valid key
    // K, V rows of this lane's key (B operands of S = Q K^T and dP = dO V^T)
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
    const bf16* qt_bh = p.qt + ((int64_t)(b * p.H + h) * DP) * p.tp;
    const bf16* gt_bh = p.gt + ((int64_t)(b * p.H + h) * DP) * p.tp;
    const bf16* qb_ = p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
    const bf16* gb_ = p.dout + (int64_t)b * p.sdb + (int64_t)h * p.sdh;
    const int64_t sbase = ((int64_t)b * p.H + h) * p.T;

#pragma unroll 1
    for (int q0 = 0; q0 < p.T; q0 += BMQ) {
      __syncthreads();
      for (int idx = tid; idx < BMQ * (KD / 8); idx += 256) {
        const int r = idx / (KD / 8), d0 = (idx % (KD / 8)) * 8;
        bf16x8 qv = zero8(), gv = zero8();
        if (q0 + r < p.T && d0 < p.D) {
          qv = *(const bf16x8*)(qb_ + (int64_t)(q0 + r) * p.sqt + d0);
          gv = *(const bf16x8*)(gb_ + (int64_t)(q0 + r) * p.sdt + d0);
        }
        *(bf16x8*)(&Qs[r * KS_LD + d0]) = qv;
        *(bf16x8*)(&Gs[r * KS_LD + d0]) = gv;
      }
      for (int idx = tid; idx < DP * (BMQ / 8); idx += 256) {
        const int r = idx / (BMQ / 8), c0 = (idx % (BMQ / 8)) * 8;
        *(bf16x8*)(&Qts[r * T_LD + c0]) = *(const bf16x8*)(qt_bh + (int64_t)r * p.tp + q0 + c0);
        *(bf16x8*)(&Gts[r * T_LD + c0]) = *(const bf16x8*)(gt_bh + (int64_t)r * p.tp + q0 + c0);
      }
      if (tid < BMQ) {
        const int qq = q0 + tid;
        Ls[tid] = (qq < p.T) ? lse2_of(p.m, p.m_bf16, p.l, sbase + qq) : INFINITY;
        Dls[tid] = (qq < p.T) ? p.delta[sbase + qq] : 0.f;
      }
      __syncthreads();

      bf16x8 pf[4], dsf[4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const bf16x8 aq = *(const bf16x8*)(&Qs[(qb * 32 + l32) * KS_LD + ks * 16 + g * 8]);
          s = mfma32x32x16(aq, kf[ks], s);
          const bf16x8 ag = *(const bf16x8*)(&Gs[(qb * 32 + l32) * KS_LD + ks * 16 + g * 8]);
          dp = mfma32x32x16(ag, vf[ks], dp);
        }
        // C layout: row = query qb*32 + c_row(r,g), col = key (this lane)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x4 lse4 = *(const f32x4*)(&Ls[qb * 32 + 8 * i4 + 4 * g]);
          const f32x4 dl4 = *(const f32x4*)(&Dls[qb * 32 + 8 * i4 + 4 * g]);
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
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
          const bf16* grow = &Gts[(db * 32 + l32) * T_LD + ks2 * 16 + 4 * g];
          const bf16* qrow = &Qts[(db * 32 + l32) * T_LD + ks2 * 16 + 4 * g];
          const bf16x4 glo = *(const bf16x4*)grow, ghi = *(const bf16x4*)(grow + 8);
          const bf16x4 qlo = *(const bf16x4*)qrow, qhi = *(const bf16x4*)(qrow + 8);
          bf16x8 bg, bq;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            bg[j] = glo[j];
            bg[j + 4] = ghi[j];
            bq[j] = qlo[j];
            bq[j + 4] = qhi[j];
          }
          dv[db] = mfma32x32x16(pf[ks2], bg, dv[db]);
          dk[db] = mfma32x32x16(dsf[ks2], bq, dk[db]);
        }
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
  dim3 grid((p.T + 127) / 128, p.H, p.B);
  hipLaunchKernelGGL((fwd_kernel<KSTEPS, DBLK>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dq_t(const BwdParams& p, hipStream_t st) {
  dim3 grid((p.T + 127) / 128, p.H, p.B);
  hipLaunchKernelGGL((dq_kernel<KSTEPS, DBLK>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
template <int KSTEPS, int DBLK>
static hipError_t launch_dkdv_t(const BwdParams& p, int n_key_tiles, hipStream_t st) {
  dim3 grid(n_key_tiles, p.H, p.B);
  hipLaunchKernelGGL((dkdv_kernel<KSTEPS, DBLK>), grid, dim3(256), 0, st, p);
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

hipError_t launch_pack_t(const PackParams& p, int n_tiles, hipStream_t st) {
  dim3 grid(n_tiles, p.H, p.B);
  hipLaunchKernelGGL(pack_t_kernel, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
hipError_t launch_fwd(const FwdParams& p, hipStream_t st) { HARP_RA_DISPATCH_D(p.D, launch_fwd_t, p, st) }
hipError_t launch_delta(const DeltaParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  dim3 grid((unsigned)((rows + 15) / 16));
  hipLaunchKernelGGL(delta_kernel, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
hipError_t launch_dq(const BwdParams& p, hipStream_t st) { HARP_RA_DISPATCH_D(p.D, launch_dq_t, p, st) }
hipError_t launch_dkdv(const BwdParams& p, int n_key_tiles, hipStream_t st) {
  HARP_RA_DISPATCH_D(p.D, launch_dkdv_t, p, n_key_tiles, st)
}

int padded_d(int D) { return ((D + 31) / 32) * 32; }

}  // namespace harp_ra
