// Causal flash attention forward on gfx950 MFMA.
//
// Replaces the aten._scaled_dot_product_flash_attention call of the
// reference (fast_triton_attn.py:425-444): softmax(q k^T * scale) v with
// scale = 1/sqrt(N) (:426), causal, no dropout, returning the output and the
// natural-log row normaliser (lse).
//
// One workgroup = one (batch, head) and BQ = 128 queries; wave w owns
// queries 32w .. 32w+31. Keys stream through LDS in tiles of 64.
// Scores are computed transposed, S^T = K Q^T, so that the query index sits
// on the lane (c) and the key index on the accumulator registers: the
// softmax statistics are then per-lane values, and the probability tile is
// already laid out as the B operand of O^T = V^T P^T (keys 4g..4g+3 and
// 16+4g..16+4g+3 of each 32-key step, matched by the V^T fragment reads).
// Output is written straight into the (B, T, H*N) layout the output
// projection reads (the reference's gate_repack layout, :171-176).
#include "common.cuh"
#include "kernels.h"

namespace mea {

template <int N>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnFwdParams p) {
  constexpr int BQ = 128, BKV = 64, QW = 32;
  constexpr int KP = N + 8;     // K tile pitch
  constexpr int VP = BKV + 8;   // V^T tile pitch
  constexpr int NS = N / 32;    // MFMA k-steps over the head dim
  constexpr int DB = N / 16;    // output d-blocks
  constexpr int OP = N + 8;     // output staging pitch
  constexpr int SM_LOOP = BKV * KP + N * VP, SM_OUT = 4 * QW * OP;
  constexpr int SMEM = SM_LOOP > SM_OUT ? SM_LOOP : SM_OUT;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SMEM];
  bf16_bits* Ks = smem;
  bf16_bits* Vt = smem + BKV * KP;

  const int T = p.T, H = p.H, BH = p.B * p.H;
  const int nqb = (T + BQ - 1) / BQ;
  // Heaviest (last) query blocks first; consecutive ids walk (b, h) so all
  // blocks of one head land on one XCD when B*H is a multiple of 8.
  const int L = blockIdx.x;
  const int bh = L % BH, qi = nqb - 1 - L / BH;
  const int b = bh / H, h = bh % H;
  const int q0 = qi * BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int qw0 = q0 + wave * QW;
  const size_t head_off = (size_t)bh * T * N;
  const bf16_bits* qg = p.q + head_off;
  const bf16_bits* kg = p.k + head_off;
  const bf16_bits* vg = p.v + head_off;

  // Q fragments (B operand of S^T): lane holds query c of block qb, d = 32s+8g..
  bf16x8 qf[2][NS];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int t = qw0 + qb * 16 + c16;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (t < T) v = ld16(qg + (size_t)t * N + s * 32 + 8 * g);
      qf[qb][s] = as_frag(v);
    }
  }

  // Cooperative tile loads: K rows as 16-byte chunks, V as row pairs that are
  // interleaved into 32-bit words of the transposed tile.
  constexpr int KCH = BKV * N / 8 / 256;        // K chunks per thread
  constexpr int VCH = (BKV / 2) * (N / 8) / 256;  // V row-pair chunks per thread
  u32x4 rk[KCH], rv0[VCH], rv1[VCH];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int id = tid + 256 * i, row = id / (N / 8), dc = id % (N / 8);
      const int t = j0 + row;
      rk[i] = t < T ? ld16(kg + (size_t)t * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      const int t = j0 + 2 * rp;
      rv0[i] = t < T ? ld16(vg + (size_t)t * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
      rv1[i] = t + 1 < T ? ld16(vg + (size_t)(t + 1) * N + dc * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int id = tid + 256 * i, row = id / (N / 8), dc = id % (N / 8);
      st16(Ks + row * KP + dc * 8, rk[i]);
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int id = tid + 256 * i, rp = id / (N / 8), dc = id % (N / 8);
      uint32_t* dst = reinterpret_cast<uint32_t*>(Vt + (dc * 8) * VP + 2 * rp);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t a = rv0[i][e], c = rv1[i][e];
        dst[(2 * e) * VP / 2] = (a & 0xffffu) | (c << 16);
        dst[(2 * e + 1) * VP / 2] = (a >> 16) | (c & 0xffff0000u);
      }
    }
  };

  const int kv_end = min(T, q0 + BQ);
  const int nkv = (kv_end + BKV - 1) / BKV;
  float m_i[2] = {-INFINITY, -INFINITY}, l_i[2] = {0.f, 0.f};
  f32x4 oacc[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db][0] = oacc[db][1] = zero4();

  fetch(0);
  for (int j = 0; j < nkv; ++j) {
    store();
    __syncthreads();
    if (j + 1 < nkv) fetch((j + 1) * BKV);
    const int j0 = j * BKV;
    if (j0 <= qw0 + QW - 1) {
      f32x4 sacc[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sacc[kb][0] = sacc[kb][1] = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x8 kf = as_frag(*reinterpret_cast<const u32x4*>(Ks + (kb * 16 + c16) * KP + s * 32 + 8 * g));
          sacc[kb][0] = mfma(kf, qf[0][s], sacc[kb][0]);
          sacc[kb][1] = mfma(kf, qf[1][s], sacc[kb][1]);
        }
      }
      const bool need_mask = (j0 + BKV - 1 > qw0) || (j0 + BKV > T);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qq = qw0 + qb * 16 + c16;
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = sacc[kb][qb][r] * p.sl2e;
            if (need_mask) {
              const int key = j0 + kb * 16 + 4 * g + r;
              if (key > qq || key >= T) v = -INFINITY;
            }
            sacc[kb][qb][r] = v;
            mx = fmaxf(mx, v);
          }
        mx = max_g(mx);
        const float mnew = fmaxf(m_i[qb], mx);
        const float moff = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = fast_exp2(m_i[qb] - moff);
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float e = fast_exp2(sacc[kb][qb][r] - moff);
            sacc[kb][qb][r] = e;
            ls += e;
          }
        l_i[qb] = l_i[qb] * alpha + ls;
        m_i[qb] = mnew;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db][qb] *= alpha;
      }
      // O^T += V^T P^T over two 32-key steps.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        bf16x8 pf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          u32x4 w;
          w[0] = pack2(sacc[2 * s2][qb][0], sacc[2 * s2][qb][1]);
          w[1] = pack2(sacc[2 * s2][qb][2], sacc[2 * s2][qb][3]);
          w[2] = pack2(sacc[2 * s2 + 1][qb][0], sacc[2 * s2 + 1][qb][1]);
          w[3] = pack2(sacc[2 * s2 + 1][qb][2], sacc[2 * s2 + 1][qb][3]);
          pf[qb] = as_frag(w);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16_bits* vrow = Vt + (db * 16 + c16) * VP + s2 * 32 + 4 * g;
          const bf16x8 vf = frag_from2(*reinterpret_cast<const u32x2*>(vrow),
                                       *reinterpret_cast<const u32x2*>(vrow + 16));
          oacc[db][0] = mfma(vf, pf[0], oacc[db][0]);
          oacc[db][1] = mfma(vf, pf[1], oacc[db][1]);
        }
      }
    }
    __syncthreads();
  }

  // Normalise, write lse and stage O for row-contiguous stores.
  bf16_bits* stg = smem + wave * QW * OP;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l = sum_g(l_i[qb]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const int qq = qw0 + qb * 16 + c16;
    if (p.lse != nullptr && g == 0 && qq < T)
      p.lse[(size_t)bh * T + qq] = (m_i[qb] + __log2f(l)) * kLn2;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const f32x4 o = oacc[db][qb] * inv;
      u32x2 w = {pack2(o[0], o[1]), pack2(o[2], o[3])};
      *reinterpret_cast<u32x2*>(stg + (qb * 16 + c16) * OP + db * 16 + 4 * g) = w;
    }
  }
  __syncthreads();
  constexpr int CPR = N / 8;
  const size_t HN = (size_t)H * N;
#pragma unroll
  for (int it = 0; it < QW * CPR / 64; ++it) {
    const int id = lane + 64 * it, row = id / CPR, dc = id % CPR;
    const int t = qw0 + row;
    if (t < T) {
      const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * OP + dc * 8);
      st16(p.o + ((size_t)b * T + t) * HN + (size_t)h * N + dc * 8, val);
    }
  }
}

hipError_t launch_attn_fwd(const AttnFwdParams& p, int N, hipStream_t s) {
  const int G = p.B * p.H * ((p.T + 127) / 128);
  if (N == 64)
    hipLaunchKernelGGL(attn_fwd_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
