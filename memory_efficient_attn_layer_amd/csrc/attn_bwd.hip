// Causal flash attention backward on gfx950 MFMA, fused with the backward of
// the per-head q/k RMSNorm and rotary and with the input-RMSNorm row scale.
//
// Replaces aten._scaled_dot_product_flash_attention_backward
// (fast_triton_attn.py:586-596) and the q/k gradient chain after it
// (:603-634). The chain is computed exactly for any rotary table with
// invertible 2x2 pair blocks, instead of the reference's rotated-space
// shortcut, which is exact only for orthonormal tables:
//   q = R qh with R the per-pair block [[f1[2i], f2[2i]], [f2[2i+1], f1[2i+1]]]
//   dqh = R^T dq
//   da_q = rq * (dqh - qh * (dqh . qh) / N)
//   df1[t, n] += dq[n] qh[n],  df2[t, n] += dq[n] qh[n^1]
// qh is recovered from the stored rotated q by inverting R per pair, so the
// recompute pass does not have to keep the pre-rotation values.
//
// Two kernels (deterministic, no atomics on dQ):
//   dq kernel   : one workgroup per (b, h, 128 queries), streams key tiles.
//                 S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - delta),
//                 dQ^T += K^T dS^T.
//   dkdv kernel : one workgroup per (b, h, 128 keys), streams query tiles.
//                 S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.
// Operands that reduce over a sequence index (K^T, Q^T, dO^T) are written
// into LDS transposed, as 32-bit pairs of adjacent rows.
#include "common.cuh"
#include "kernels.h"

namespace mea {

// Row-wise tail for one wave: 32 staged rows of fp32 gradient (pitch FP)
// for sequence positions t0 .. t0+31 of head (b, h).
//   rotary != 0 : head RMSNorm + rotary backward of q or k (xrot = q or k).
//   rotary == 0 : plain copy (v).
// Output row t goes to out[(b*T + t)*HN + h*N ...], scaled by rx[b*T + t].
template <int N>
__device__ __forceinline__ void head_row_bwd(const float* stg, int FP, int t0, const AttnBwdParams& p,
                                             int b, int h, bool rotary, const bf16_bits* xrot,
                                             const float* rstat, bf16_bits* out) {
  constexpr int CPR = N / 8, RPP = 64 / CPR;
  const int lane = threadIdx.x & 63;
  const int T = p.T, H = p.H;
  const size_t HN = (size_t)H * N;
  const size_t bh = (size_t)b * H + h;
#pragma unroll 1
  for (int pass = 0; pass < 32 / RPP; ++pass) {
    const int row = pass * RPP + lane / CPR, dc = lane % CPR;
    const int t = t0 + row;
    const bool valid = t < T;
    const int tc = valid ? t : T - 1;
    float dv[8];
    {
      const f32x4 a = *reinterpret_cast<const f32x4*>(stg + row * FP + dc * 8);
      const f32x4 c = *reinterpret_cast<const f32x4*>(stg + row * FP + dc * 8 + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { dv[i] = a[i]; dv[4 + i] = c[i]; }
    }
    const float rxv = p.rx[(size_t)b * T + tc];
    float res[8];
    if (rotary) {
      float xv[8], a1[8], a2[8];
      unpack8(ld16(xrot + (bh * T + tc) * N + dc * 8), xv);
      const float* f1r = p.f1 + (size_t)tc * N + dc * 8;
      const float* f2r = p.f2 + (size_t)tc * N + dc * 8;
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(f1r + i);
        const f32x4 w = *reinterpret_cast<const f32x4*>(f2r + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) { a1[i + e] = u[e]; a2[i + e] = w[e]; }
      }
      float xh[8], dh[8], dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const float det = a1[i] * a1[i + 1] - a2[i] * a2[i + 1];
        const float inv = 1.0f / det;
        xh[i] = (a1[i + 1] * xv[i] - a2[i] * xv[i + 1]) * inv;
        xh[i + 1] = (a1[i] * xv[i + 1] - a2[i + 1] * xv[i]) * inv;
        dh[i] = a1[i] * dv[i] + a2[i + 1] * dv[i + 1];
        dh[i + 1] = a1[i + 1] * dv[i + 1] + a2[i] * dv[i];
        dot += dh[i] * xh[i] + dh[i + 1] * xh[i + 1];
      }
      // Reduce the dot product over the CPR lanes of this row.
      dot += xor1(dot);
      dot += xor2(dot);
      dot += shfl_xor(dot, 4);
      if (CPR == 16) dot += shfl_xor(dot, 8);
      const float rr = rstat[bh * T + tc];
      const float sc = rxv * rr, cf = dot / (float)N;
#pragma unroll
      for (int i = 0; i < 8; ++i) res[i] = sc * (dh[i] - xh[i] * cf);
      if (p.df1 != nullptr && valid) {
        float* d1 = p.df1 + (size_t)t * N + dc * 8;
        float* d2 = p.df2 + (size_t)t * N + dc * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          atomicAdd(d1 + i, dv[i] * xh[i]);
          atomicAdd(d2 + i, dv[i] * xh[i ^ 1]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) res[i] = rxv * dv[i];
    }
    if (valid) st16(out + ((size_t)b * T + t) * HN + (size_t)h * N + dc * 8, pack8(res));
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnBwdParams p) {
  constexpr int BQ = 128, BKV = 64, QW = 32;
  constexpr int KP = N + 8, TP = BKV + 8;
  constexpr int NS = N / 32, DB = N / 16, FP = N + 4;
  constexpr int SM_LOOP = (2 * BKV * KP + N * TP) * 2;  // bytes
  constexpr int SM_OUT = 4 * QW * FP * 4;
  constexpr int SMEM = SM_LOOP > SM_OUT ? SM_LOOP : SM_OUT;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  bf16_bits* Ks = reinterpret_cast<bf16_bits*>(smem);
  bf16_bits* Vs = Ks + BKV * KP;
  bf16_bits* Kt = Vs + BKV * KP;

  const int T = p.T, H = p.H, BH = p.B * p.H;
  const int nqb = (T + BQ - 1) / BQ;
  const int L = blockIdx.x;
  const int bh = L % BH, qi = nqb - 1 - L / BH;
  const int b = bh / H, h = bh % H;
  const int q0 = qi * BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int qw0 = q0 + wave * QW;
  const size_t head_off = (size_t)bh * T * N;
  const bf16_bits* kg = p.k + head_off;
  const bf16_bits* vg = p.v + head_off;

  bf16x8 qf[2][NS], df[2][NS];
  float lse2[2], dlt[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int t = qw0 + qb * 16 + c16;
    const bool ok = t < T;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const size_t off = head_off + (size_t)t * N + s * 32 + 8 * g;
      qf[qb][s] = as_frag(ok ? ld16(p.q + off) : u32x4{0u, 0u, 0u, 0u});
      df[qb][s] = as_frag(ok ? ld16(p.dO + off) : u32x4{0u, 0u, 0u, 0u});
    }
    lse2[qb] = ok ? p.lse[(size_t)bh * T + t] * kLog2e : 0.f;
    dlt[qb] = ok ? p.delta[(size_t)bh * T + t] : 0.f;
  }

  constexpr int KCH = BKV * N / 8 / 256;          // row chunks per thread
  constexpr int PCH = (BKV / 2) * (N / 8) / 256;  // row-pair chunks per thread
  u32x4 rk[KCH], rv[KCH], rp0[PCH], rp1[PCH];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int id = tid + 256 * i, row = id / (N / 8), dc = id % (N / 8);
      const int t = j0 + row;
      rk[i] = t < T ? ld16(kg + (size_t)t * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
      rv[i] = t < T ? ld16(vg + (size_t)t * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      const int t = j0 + 2 * rp;
      rp0[i] = t < T ? ld16(kg + (size_t)t * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
      rp1[i] = t + 1 < T ? ld16(kg + (size_t)(t + 1) * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int id = tid + 256 * i, row = id / (N / 8), dc = id % (N / 8);
      st16(Ks + row * KP + dc * 8, rk[i]);
      st16(Vs + row * KP + dc * 8, rv[i]);
    }
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      uint32_t* dst = reinterpret_cast<uint32_t*>(Kt + (dc * 8) * TP + 2 * rp);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t a = rp0[i][e], c = rp1[i][e];
        dst[(2 * e) * TP / 2] = (a & 0xffffu) | (c << 16);
        dst[(2 * e + 1) * TP / 2] = (a >> 16) | (c & 0xffff0000u);
      }
    }
  };

  f32x4 dq[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db][0] = dq[db][1] = zero4();

  const int kv_end = min(T, q0 + BQ);
  const int nkv = (kv_end + BKV - 1) / BKV;
  fetch(0);
  for (int j = 0; j < nkv; ++j) {
    store();
    __syncthreads();
    if (j + 1 < nkv) fetch((j + 1) * BKV);
    const int j0 = j * BKV;
    if (j0 <= qw0 + QW - 1) {
      f32x4 sa[4][2], pa[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sa[kb][0] = sa[kb][1] = pa[kb][0] = pa[kb][1] = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x8 kf = as_frag(*reinterpret_cast<const u32x4*>(Ks + (kb * 16 + c16) * KP + s * 32 + 8 * g));
          const bf16x8 vf = as_frag(*reinterpret_cast<const u32x4*>(Vs + (kb * 16 + c16) * KP + s * 32 + 8 * g));
          sa[kb][0] = mfma(kf, qf[0][s], sa[kb][0]);
          sa[kb][1] = mfma(kf, qf[1][s], sa[kb][1]);
          pa[kb][0] = mfma(vf, df[0][s], pa[kb][0]);
          pa[kb][1] = mfma(vf, df[1][s], pa[kb][1]);
        }
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qq = qw0 + qb * 16 + c16;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = j0 + kb * 16 + 4 * g + r;
            float pv = fast_exp2(sa[kb][qb][r] * p.sl2e - lse2[qb]);
            if (key > qq || key >= T) pv = 0.f;
            sa[kb][qb][r] = pv * (pa[kb][qb][r] - dlt[qb]);
          }
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        bf16x8 sf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          u32x4 w;
          w[0] = pack2(sa[2 * s2][qb][0], sa[2 * s2][qb][1]);
          w[1] = pack2(sa[2 * s2][qb][2], sa[2 * s2][qb][3]);
          w[2] = pack2(sa[2 * s2 + 1][qb][0], sa[2 * s2 + 1][qb][1]);
          w[3] = pack2(sa[2 * s2 + 1][qb][2], sa[2 * s2 + 1][qb][3]);
          sf[qb] = as_frag(w);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16_bits* kr = Kt + (db * 16 + c16) * TP + s2 * 32 + 4 * g;
          const bf16x8 kt = frag_from2(*reinterpret_cast<const u32x2*>(kr), *reinterpret_cast<const u32x2*>(kr + 16));
          dq[db][0] = mfma(kt, sf[0], dq[db][0]);
          dq[db][1] = mfma(kt, sf[1], dq[db][1]);
        }
      }
    }
    __syncthreads();
  }

  // Stage dQ (times the softmax scale) as fp32 rows, then the q chain.
  float* stg = reinterpret_cast<float*>(smem) + wave * QW * FP;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<f32x4*>(stg + (qb * 16 + c16) * FP + db * 16 + 4 * g) = dq[db][qb] * p.scale;
  __syncthreads();
  head_row_bwd<N>(stg, FP, qw0, p, b, h, true, p.q, p.rq, p.daq);
}

// ---------------------------------------------------------------------------
// dK, dV
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnBwdParams p) {
  constexpr int BKV = 128, KW = 32, BQ = 64;
  constexpr int QP = N + 8, TP = BQ + 8;
  constexpr int NS = N / 32, DB = N / 16, FP = N + 4;
  constexpr int SM_LOOP = (2 * BQ * QP + 2 * N * TP) * 2 + 2 * BQ * 4;
  constexpr int SM_OUT = 4 * KW * FP * 4;
  constexpr int SMEM = SM_LOOP > SM_OUT ? SM_LOOP : SM_OUT;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  bf16_bits* Qs = reinterpret_cast<bf16_bits*>(smem);
  bf16_bits* Ds = Qs + BQ * QP;
  bf16_bits* Qt = Ds + BQ * QP;
  bf16_bits* Dt = Qt + N * TP;
  float* lse_s = reinterpret_cast<float*>(Dt + N * TP);
  float* dlt_s = lse_s + BQ;

  const int T = p.T, H = p.H, BH = p.B * p.H;
  const int nkb = (T + BKV - 1) / BKV;
  // Key blocks near the start of the sequence see the most queries: first.
  const int L = blockIdx.x;
  const int bh = L % BH, ki = L / BH;
  const int b = bh / H, h = bh % H;
  const int k0 = ki * BKV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int kw0 = k0 + wave * KW;
  const size_t head_off = (size_t)bh * T * N;
  const bf16_bits* qg = p.q + head_off;
  const bf16_bits* dg = p.dO + head_off;
  (void)nkb;

  bf16x8 kf[2][NS], vf[2][NS];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int t = kw0 + kb * 16 + c16;
    const bool ok = t < T;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const size_t off = head_off + (size_t)t * N + s * 32 + 8 * g;
      kf[kb][s] = as_frag(ok ? ld16(p.k + off) : u32x4{0u, 0u, 0u, 0u});
      vf[kb][s] = as_frag(ok ? ld16(p.v + off) : u32x4{0u, 0u, 0u, 0u});
    }
  }

  constexpr int PCH = (BQ / 2) * (N / 8) / 256;  // row-pair chunks per thread
  u32x4 rq0[PCH], rq1[PCH], rd0[PCH], rd1[PCH];
  float rstat = 0.f;
  auto fetch = [&](int i0) {
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      const int t = i0 + 2 * rp;
      const u32x4 z = {0u, 0u, 0u, 0u};
      rq0[i] = t < T ? ld16(qg + (size_t)t * N + dc * 8) : z;
      rq1[i] = t + 1 < T ? ld16(qg + (size_t)(t + 1) * N + dc * 8) : z;
      rd0[i] = t < T ? ld16(dg + (size_t)t * N + dc * 8) : z;
      rd1[i] = t + 1 < T ? ld16(dg + (size_t)(t + 1) * N + dc * 8) : z;
    }
    if (tid < 2 * BQ) {
      const int t = i0 + (tid & (BQ - 1));
      rstat = t < T ? (tid < BQ ? p.lse[(size_t)bh * T + t] * kLog2e : p.delta[(size_t)bh * T + t]) : 0.f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      st16(Qs + (2 * rp) * QP + dc * 8, rq0[i]);
      st16(Qs + (2 * rp + 1) * QP + dc * 8, rq1[i]);
      st16(Ds + (2 * rp) * QP + dc * 8, rd0[i]);
      st16(Ds + (2 * rp + 1) * QP + dc * 8, rd1[i]);
      uint32_t* dq_ = reinterpret_cast<uint32_t*>(Qt + (dc * 8) * TP + 2 * rp);
      uint32_t* dd_ = reinterpret_cast<uint32_t*>(Dt + (dc * 8) * TP + 2 * rp);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t a = rq0[i][e], c = rq1[i][e];
        dq_[(2 * e) * TP / 2] = (a & 0xffffu) | (c << 16);
        dq_[(2 * e + 1) * TP / 2] = (a >> 16) | (c & 0xffff0000u);
        a = rd0[i][e];
        c = rd1[i][e];
        dd_[(2 * e) * TP / 2] = (a & 0xffffu) | (c << 16);
        dd_[(2 * e + 1) * TP / 2] = (a >> 16) | (c & 0xffff0000u);
      }
    }
    if (tid < 2 * BQ) lse_s[tid] = rstat;  // lse_s and dlt_s are contiguous
  };

  f32x4 dk[DB][2], dv[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) dk[db][0] = dk[db][1] = dv[db][0] = dv[db][1] = zero4();

  const int nq = k0 < T ? (T - k0 + BQ - 1) / BQ : 0;
  if (nq > 0) fetch(k0);
  for (int i = 0; i < nq; ++i) {
    store();
    __syncthreads();
    const int i0 = k0 + i * BQ;
    if (i + 1 < nq) fetch(i0 + BQ);
    if (i0 + BQ - 1 >= kw0) {
      f32x4 sa[4][2], pa[4][2];
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) {
        sa[qb][0] = sa[qb][1] = pa[qb][0] = pa[qb][1] = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x8 qa = as_frag(*reinterpret_cast<const u32x4*>(Qs + (qb * 16 + c16) * QP + s * 32 + 8 * g));
          const bf16x8 da = as_frag(*reinterpret_cast<const u32x4*>(Ds + (qb * 16 + c16) * QP + s * 32 + 8 * g));
          sa[qb][0] = mfma(qa, kf[0][s], sa[qb][0]);
          sa[qb][1] = mfma(qa, kf[1][s], sa[qb][1]);
          pa[qb][0] = mfma(da, vf[0][s], pa[qb][0]);
          pa[qb][1] = mfma(da, vf[1][s], pa[qb][1]);
        }
      }
      // sa <- P, pa <- dS.
#pragma unroll
      for (int qb = 0; qb < 4; ++qb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ql = qb * 16 + 4 * g + r;
          const int qq = i0 + ql;
          const float l2 = lse_s[ql], dl = dlt_s[ql];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            const int key = kw0 + kb * 16 + c16;
            float pv = fast_exp2(sa[qb][kb][r] * p.sl2e - l2);
            if (key > qq || qq >= T) pv = 0.f;
            sa[qb][kb][r] = pv;
            pa[qb][kb][r] = pv * (pa[qb][kb][r] - dl);
          }
        }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        bf16x8 pf[2], sf[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          u32x4 w, u;
          w[0] = pack2(sa[2 * s2][kb][0], sa[2 * s2][kb][1]);
          w[1] = pack2(sa[2 * s2][kb][2], sa[2 * s2][kb][3]);
          w[2] = pack2(sa[2 * s2 + 1][kb][0], sa[2 * s2 + 1][kb][1]);
          w[3] = pack2(sa[2 * s2 + 1][kb][2], sa[2 * s2 + 1][kb][3]);
          u[0] = pack2(pa[2 * s2][kb][0], pa[2 * s2][kb][1]);
          u[1] = pack2(pa[2 * s2][kb][2], pa[2 * s2][kb][3]);
          u[2] = pack2(pa[2 * s2 + 1][kb][0], pa[2 * s2 + 1][kb][1]);
          u[3] = pack2(pa[2 * s2 + 1][kb][2], pa[2 * s2 + 1][kb][3]);
          pf[kb] = as_frag(w);
          sf[kb] = as_frag(u);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16_bits* dr = Dt + (db * 16 + c16) * TP + s2 * 32 + 4 * g;
          const bf16_bits* qr = Qt + (db * 16 + c16) * TP + s2 * 32 + 4 * g;
          const bf16x8 dt = frag_from2(*reinterpret_cast<const u32x2*>(dr), *reinterpret_cast<const u32x2*>(dr + 16));
          const bf16x8 qt = frag_from2(*reinterpret_cast<const u32x2*>(qr), *reinterpret_cast<const u32x2*>(qr + 16));
          dv[db][0] = mfma(dt, pf[0], dv[db][0]);
          dv[db][1] = mfma(dt, pf[1], dv[db][1]);
          dk[db][0] = mfma(qt, sf[0], dk[db][0]);
          dk[db][1] = mfma(qt, sf[1], dk[db][1]);
        }
      }
    }
    __syncthreads();
  }

  // dV tail, then dK tail (shared staging).
  float* stg = reinterpret_cast<float*>(smem) + wave * KW * FP;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<f32x4*>(stg + (kb * 16 + c16) * FP + db * 16 + 4 * g) = dv[db][kb];
  __syncthreads();
  head_row_bwd<N>(stg, FP, kw0, p, b, h, false, nullptr, nullptr, p.dav);
  __syncthreads();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<f32x4*>(stg + (kb * 16 + c16) * FP + db * 16 + 4 * g) = dk[db][kb] * p.scale;
  __syncthreads();
  head_row_bwd<N>(stg, FP, kw0, p, b, h, true, p.k, p.rk, p.dak);
}

hipError_t launch_attn_bwd_dq(const AttnBwdParams& p, int N, hipStream_t s) {
  const int G = p.B * p.H * ((p.T + 127) / 128);
  if (N == 64)
    hipLaunchKernelGGL(attn_bwd_dq_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_bwd_dq_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_attn_bwd_dkdv(const AttnBwdParams& p, int N, hipStream_t s) {
  const int G = p.B * p.H * ((p.T + 127) / 128);
  if (N == 64)
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
