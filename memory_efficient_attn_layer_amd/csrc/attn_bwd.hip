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
#include <type_traits>

#include "common.cuh"
#include "kernels.h"

namespace mea {

// Row-wise tail for one wave: 32 staged rows of fp32 gradient (pitch FP)
// for sequence positions t0 .. t0+31 of head (b, h).
//   rotary != 0 : head RMSNorm + rotary backward of q or k (xrot = q or k
//                 as stored, xrot * xscale the rotated rows themselves).
//   rotary == 0 : plain copy (v).
// Output row t goes to out[(b*T + t)*ld_da + h*N ...], scaled by rx[b*T + t].
template <int N>
__device__ __forceinline__ void head_row_bwd(const float* stg, int FP, int t0, const AttnBwdParams& p,
                                             int b, int h, bool rotary, const bf16_bits* xrot, float xscale,
                                             const float* rstat, bf16_bits* out) {
  constexpr int CPR = N / 8, RPP = 64 / CPR;
  const int lane = threadIdx.x & 63;
  const int T = p.T, H = p.H;
  const size_t ld = (size_t)p.ld_da;
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
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] *= xscale;
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
    if (valid) st16(out + ((size_t)b * T + t) * ld + (size_t)h * N + dc * 8, pack8(res));
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
  head_row_bwd<N>(stg, FP, qw0, p, b, h, true, p.q, 1.0f / p.qscale, p.rq, p.daq);
}

// ---------------------------------------------------------------------------
// dK, dV
//
// One workgroup = one (batch, head) and BKV = 4*KW keys; wave w owns KW
// consecutive keys (KW = 64 for N = 64, 32 for N = 128) whose K and V rows
// stay in registers as the B operands of
//   S  = Q K^T   and   dP = dO V^T        (A = Q, dO rows from LDS)
// on v_mfma_f32_32x32x16_bf16. The key index sits on the lane, so P and
// dS = P (dP - delta) are already the B operands (k = query) of
//   dV^T += dO^T P   and   dK^T += Q^T dS
// whose A operands dO^T, Q^T are read from the same row-major LDS tiles with
// the transposing ds_read_b64_tr_b16. Query tiles of 64 stream through LDS
// (global_load_lds, double-buffered, one barrier per tile), starting at the
// block's first key (causal).
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnBwdParams p) {
  constexpr int KW = N == 64 ? 64 : 32;  // keys per wave
  constexpr int KB = KW / 32;            // 32-key MFMA blocks per wave
  constexpr int BKV = 4 * KW;            // keys per workgroup
  constexpr int BQ = 64;                 // queries per LDS tile
  constexpr int CH = N / 8, KS = N / 16, DB = N / 32;
  constexpr int TILE = BQ * N;
  constexpr int LOADS = TILE / 8 / 256;
  constexpr int FP = N + 4;  // fp32 staging pitch
  constexpr int SM_LOOP = 2 * 2 * TILE * 2 + 2 * 2 * BQ * 4;  // bytes
  constexpr int SM_OUT = 4 * 32 * FP * 4;
  constexpr int SMEM = SM_LOOP > SM_OUT ? SM_LOOP : SM_OUT;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  bf16_bits* tiles = reinterpret_cast<bf16_bits*>(smem);           // [stage][Q | dO]
  float* stats = reinterpret_cast<float*>(smem + 2 * 2 * TILE * 2);  // [stage][lse*log2e | delta]

  const int T = p.T, BH = p.B * p.H;
  const int nkb = (T + BKV - 1) / BKV;
  // Each XCD walks whole heads, the key block that sees the most queries
  // first, so the Q/dO tiles of a head are shared in one L2.
  const int lid = xcd_remap(blockIdx.x, BH * nkb);
  const int bh = lid / nkb, ki = lid % nkb;
  const int b = bh / p.H, hd = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, h = lane >> 5;
  const int k0 = ki * BKV, kw0 = k0 + wave * KW;
  const size_t head_off = (size_t)bh * T * N;
  const bf16_bits* qg = p.q + head_off;
  const bf16_bits* dg = p.dO + head_off;

  // K^T, V^T fragments (B operands): lane holds key kw0 + 32kb + c, d = 16ks + 8h.
  bf16x8 kf[KB][KS], vf[KB][KS];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const size_t row = head_off + (size_t)min(kw0 + 32 * kb + c, T - 1) * N;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[kb][ks] = as_frag(ld16(p.k + row + 16 * ks + 8 * h));
      vf[kb][ks] = as_frag(ld16(p.v + row + 16 * ks + 8 * h));
    }
  }

  float st_reg = 0.f;
  auto issue_tile = [&](int q0, int stage) {
    bf16_bits* qt = tiles + stage * 2 * TILE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int slot = (u * 4 + wave) * 64 + lane;
      const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
      const size_t off = (size_t)min(q0 + row, T - 1) * N + cc * 8;
      g2lds16(qg + off, qt + (u * 4 + wave) * 512);
      g2lds16(dg + off, qt + TILE + (u * 4 + wave) * 512);
    }
    if (tid < 2 * BQ) {
      const size_t t = (size_t)bh * T + min(q0 + (tid & (BQ - 1)), T - 1);
      st_reg = tid < BQ ? p.lse[t] : p.delta[t];
    }
  };
  // Called after wait_vmcnt0(): st_reg is consumed only once every load of
  // the tile has landed, so no wait is placed inside the prefetch.
  auto publish_stats = [&](int stage) {
    if (tid < 2 * BQ) stats[stage * 2 * BQ + tid] = tid < BQ ? st_reg * kLog2e : st_reg;
  };

  f32x16 dv[KB][DB], dk[KB][DB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int db = 0; db < DB; ++db) dv[kb][db] = dk[kb][db] = zero16();

  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * h + (i16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

  const int nq = (T - k0 + BQ - 1) / BQ;
  issue_tile(k0, 0);
  wait_vmcnt0();
  publish_stats(0);
  __syncthreads();
  for (int it = 0; it < nq; ++it) {
    const int q0 = k0 + it * BQ;
    if (it + 1 < nq) issue_tile(q0 + BQ, (it + 1) & 1);
    const bf16_bits* qt = tiles + (it & 1) * 2 * TILE;
    const bf16_bits* dt = qt + TILE;
    const float* ls = stats + (it & 1) * 2 * BQ;
    const float* dls = ls + BQ;
    // One 32-query step; DIAG steps mask key > query and query >= T with
    // selects, the others run without any per-element test. Each variant is
    // one basic block, so the scheduler can overlap the MFMAs of one key
    // block with the exp/convert work of the other.
    auto step = [&](int sub, auto diag_tag) {
      constexpr bool DIAG = decltype(diag_tag)::value;
      const int qs0 = q0 + 32 * sub;
      bf16x8 qa[KS], da[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = swz_off<CH>(32 * sub + c, 16 * ks + 8 * h);
        qa[ks] = as_frag(*reinterpret_cast<const u32x4*>(qt + off));
        da[ks] = as_frag(*reinterpret_cast<const u32x4*>(dt + off));
      }
      // Statistics of the queries held by accumulator register 4*r4 + e:
      // query qs0 + 8*r4 + 4h + e.
      f32x4 l4[4], d4[4];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        l4[r4] = *reinterpret_cast<const f32x4*>(ls + 32 * sub + 8 * r4 + 4 * h);
        d4[r4] = *reinterpret_cast<const f32x4*>(dls + 32 * sub + 8 * r4 + 4 * h);
      }
      bf16x8 pb[KB][2], sb[KB][2];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = mfma32(qa[ks], kf[kb][ks], s);
          dp = mfma32(da[ks], vf[kb][ks], dp);
        }
        const int key = kw0 + 32 * kb + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r4 = i >> 2, e = i & 3;
          float pv = fast_exp2(__builtin_fmaf(s[i], p.sl2e, -l4[r4][e]));
          if (DIAG) {
            const int q = qs0 + 8 * r4 + 4 * h + e;
            pv = (key > q || q >= T) ? 0.f : pv;
          }
          s[i] = pv;
          dp[i] = pv * (dp[i] - d4[r4][e]);
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
          u32x4 w, u;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[e] = pack2(s[8 * kst + 2 * e], s[8 * kst + 2 * e + 1]);
            u[e] = pack2(dp[8 * kst + 2 * e], dp[8 * kst + 2 * e + 1]);
          }
          pb[kb][kst] = as_frag(w);
          sb[kb][kst] = as_frag(u);
        }
      }
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int r = 32 * sub + 16 * kst + tr_row, col = 32 * db + tr_col;
          const int o0 = swz_off<CH>(r, col), o1 = swz_off<CH>(r + 8, col);
          const bf16x8 dT = frag_from2(lds_read_tr4(dt + o0), lds_read_tr4(dt + o1));
          const bf16x8 qT = frag_from2(lds_read_tr4(qt + o0), lds_read_tr4(qt + o1));
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            dv[kb][db] = mfma32(dT, pb[kb][kst], dv[kb][db]);
            dk[kb][db] = mfma32(qT, sb[kb][kst], dk[kb][db]);
          }
        }
      }
    };
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int qs0 = q0 + 32 * sub;
      if (qs0 + 31 < kw0 || qs0 >= T) continue;  // wave-uniform: nothing to add
      if (qs0 < kw0 + KW - 1 || qs0 + 31 >= T)
        step(sub, std::true_type{});
      else
        step(sub, std::false_type{});
    }
    wait_vmcnt0();
    if (it + 1 < nq) publish_stats((it + 1) & 1);
    __syncthreads();
  }

  // Epilogue per 32-key block: stage dV (then dK * scale) as fp32 rows and run
  // the row-wise tails (rx scale; k RMSNorm + rotary backward for dK).
  float* stg = reinterpret_cast<float*>(smem) + wave * 32 * FP;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 v = {dv[kb][db][4 * r4], dv[kb][db][4 * r4 + 1], dv[kb][db][4 * r4 + 2], dv[kb][db][4 * r4 + 3]};
        *reinterpret_cast<f32x4*>(stg + c * FP + 32 * db + 8 * r4 + 4 * h) = v;
      }
    __syncthreads();
    head_row_bwd<N>(stg, FP, kw0 + 32 * kb, p, b, hd, false, nullptr, 1.0f, nullptr, p.dav);
    __syncthreads();
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 v = {dk[kb][db][4 * r4], dk[kb][db][4 * r4 + 1], dk[kb][db][4 * r4 + 2], dk[kb][db][4 * r4 + 3]};
        *reinterpret_cast<f32x4*>(stg + c * FP + 32 * db + 8 * r4 + 4 * h) = v * (p.scale / p.qscale);
      }
    __syncthreads();
    head_row_bwd<N>(stg, FP, kw0 + 32 * kb, p, b, hd, true, p.k, 1.0f, p.rk, p.dak);
    __syncthreads();
  }
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
  const int BKV = N == 64 ? 256 : 128;
  const int G = p.B * p.H * ((p.T + BKV - 1) / BKV);
  if (N == 64)
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
