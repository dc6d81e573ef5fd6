// Input RMSNorm + q/k/v/g projection + per-head q/k RMSNorm + rotary +
// sigmoid, as one MFMA GEMM with a fused prologue and epilogue.
//
// Replaces rms_norm_kernel (fast_triton_attn.py:12-34) and
// fused_qkvg_norm_rope_kernel (:36-144), and their backward-recompute
// variants (:181-332) when rx/rq/rk are requested.
//
// The product is computed transposed, D^T = W x^T: the A operand is a slice
// of the stacked weights [Wq_h; Wk_h; Wv_h; Wg_h] of one head h (features),
// the B operand a tile of x rows (tokens). In the 16x16 accumulator layout a
// lane then holds one token and 4 consecutive features, so the head RMSNorm
// is an in-lane sum plus two lane exchanges, both members of every rotary
// pair (n, n^1) sit in one lane, and results leave as 8-byte stores.
//
// Tile: 256 features x 256 tokens, k-slabs of 64 double-buffered in LDS and
// filled by direct global->LDS loads (one barrier per slab). Four waves, each
// 128 features x 128 tokens (64 accumulators of 16x16).
//
// The input RMSNorm is never materialised: diag(1/rms(x)) commutes with the
// GEMM. The waves sum the squares of the x fragments they read anyway (the two
// waves sharing a token half split the rows) and the row scale multiplies the
// fp32 accumulator.
#include "kernels.h"
#include "slab.cuh"

namespace mea {

template <int N>
__global__ __launch_bounds__(256, 1) void qkvg_proj_kernel(ProjParams p) {
  constexpr int BT = 256;              // tokens per tile
  constexpr int BF = 256;              // stacked-weight rows per tile
  constexpr int NFT = 4 * N / BF;      // feature tiles per head
  constexpr int STAGE = (BF + BT) * kSlabK;
  constexpr int GF = N / 16;           // 16-feature blocks per projection
  constexpr int NG = 8 / GF;           // projections per wave
  __shared__ __attribute__((aligned(16))) bf16_bits smem[2 * STAGE];
  __shared__ float ssq_s[BT];

  // Locals, not captures of the argument block: a lambda holding &p would
  // force the block into scratch memory.
  const bf16_bits* __restrict__ xg = p.x;
  const bf16_bits *wq = p.wq, *wk = p.wk, *wv = p.wv, *wg = p.wg;
  const int M = p.M, C = p.C, H = p.H, T = p.T, HN = H * N;

  const int ntt = (M + BT - 1) / BT;
  const int L = xcd_remap(blockIdx.x, ntt * H * NFT);
  const int tt = L / (H * NFT), rem = L - tt * (H * NFT);
  const int h = rem / NFT, f0 = (rem % NFT) * BF;
  const int m0 = tt * BT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int wf = wave >> 1, wt = wave & 1;

  // Source matrix of each N-row segment of the stacked-weight slab.
  constexpr int NSEG = BF / N;
  const bf16_bits* wseg[NSEG];
  if (NSEG == 4) {
    wseg[0] = wq;
    wseg[NSEG > 1 ? 1 : 0] = wk;
    wseg[NSEG > 2 ? 2 : 0] = wv;
    wseg[NSEG > 3 ? 3 : 0] = wg;
  } else {
    wseg[0] = f0 == 0 ? wq : wv;
    wseg[NSEG > 1 ? 1 : 0] = f0 == 0 ? wk : wg;
  }

  auto issue = [&](int ks, int st) {
    bf16_bits* base = smem + st * STAGE;
    const int k0 = ks * kSlabK;
    slab_issue<BF>(base, [&](int r, int u) {
      const int seg = (32 * u) / N;  // compile-time after unrolling
      return wseg[seg] + (size_t)(h * N + r - seg * N) * C + k0;
    });
    slab_issue<BT>(base + BF * kSlabK, [&](int r, int) { return xg + (size_t)min(m0 + r, M - 1) * C + k0; });
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int fb = 0; fb < 8; ++fb)
#pragma unroll
    for (int tb = 0; tb < 8; ++tb) acc[fb][tb] = zero4();
  float ss[4] = {0.f, 0.f, 0.f, 0.f};

  const int nk = C / kSlabK;
  issue(0, 0);
  for (int ks = 0; ks < nk; ++ks) {
    wait_vmcnt0();
    __syncthreads();
    if (ks + 1 < nk) issue(ks + 1, (ks + 1) & 1);
    const bf16_bits* As = smem + (ks & 1) * STAGE;
    const bf16_bits* Bs = As + BF * kSlabK;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 af[8], bfr[8];
#pragma unroll
      for (int fb = 0; fb < 8; ++fb) af[fb] = as_frag(slab_read(As, wf * 128 + fb * 16 + c16, 4 * kk + g));
#pragma unroll
      for (int tb = 0; tb < 8; ++tb) {
        const u32x4 v = slab_read(Bs, wt * 128 + tb * 16 + c16, 4 * kk + g);
        bfr[tb] = as_frag(v);
        if ((tb >> 2) == wf) ss[tb & 3] = sumsq8(v, ss[tb & 3]);
      }
#pragma unroll
      for (int fb = 0; fb < 8; ++fb)
#pragma unroll
        for (int tb = 0; tb < 8; ++tb) acc[fb][tb] = mfma(af[fb], bfr[tb], acc[fb][tb]);
    }
  }

  // Sum of squares of each token row: lane (g, c16) holds the k chunks g and
  // 4+g of every slab.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = ss[i];
    s += shfl_xor(s, 16);
    s += shfl_xor(s, 32);
    if (g == 0) ssq_s[wt * 128 + (4 * wf + i) * 16 + c16] = s;
  }
  __syncthreads();

  int mrow[8];
#pragma unroll
  for (int tb = 0; tb < 8; ++tb) {
    const int tl = wt * 128 + tb * 16 + c16;
    mrow[tb] = m0 + tl;
    const float rx = rsqrtf(ssq_s[tl] / (float)C + p.eps);
    if (p.rx != nullptr && h == 0 && f0 == 0 && wf == 0 && g == 0 && mrow[tb] < M) p.rx[mrow[tb]] = rx;
#pragma unroll
    for (int fb = 0; fb < 8; ++fb) acc[fb][tb] *= rx;
  }

  const int v0 = f0 + wf * 128;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int pj = v0 / N + gi;  // projection of this group (wave-uniform)
    if (pj < 2) {
      // Head RMSNorm over N (fast_triton_attn.py:102-106), then the rotary
      // from the bf16-rounded normalised values, the reference's rounding
      // point (:103, :140): out[n] = qh[n] f1[t,n] + qh[n^1] f2[t,n].
      float* rstat = pj == 0 ? p.rq : p.rk;
      bf16_bits* outp = pj == 0 ? p.q : p.k;
#pragma unroll
      for (int tb = 0; tb < 8; ++tb) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < GF; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) s += acc[gi * GF + j][tb][r] * acc[gi * GF + j][tb][r];
        s += shfl_xor(s, 16);
        s += shfl_xor(s, 32);
        const float rr = rsqrtf(s / (float)N + p.eps);
        const int m = mrow[tb];
        if (m < M) {
          const int b = m / T, t = m - b * T;
          const size_t hrow = ((size_t)b * H + h) * T + t;
          if (rstat != nullptr && g == 0) rstat[hrow] = rr;
          const float* f1r = p.f1 + (size_t)t * N;
          const float* f2r = p.f2 + (size_t)t * N;
#pragma unroll
          for (int j = 0; j < GF; ++j) {
            const int n = 16 * j + 4 * g;
            const f32x4 a1 = *reinterpret_cast<const f32x4*>(f1r + n);
            const f32x4 a2 = *reinterpret_cast<const f32x4*>(f2r + n);
            float qh[4], o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) qh[r] = bf2f(f2bf(acc[gi * GF + j][tb][r] * rr));
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = qh[r] * a1[r] + qh[r ^ 1] * a2[r];
            *reinterpret_cast<u32x2*>(outp + hrow * N + n) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
          }
        }
      }
    } else {
      const bool is_v = pj == 2;
#pragma unroll
      for (int tb = 0; tb < 8; ++tb) {
        const int m = mrow[tb];
        if (m >= M) continue;
        bf16_bits* dst;
        if (is_v) {
          const int b = m / T, t = m - b * T;
          dst = p.v + (((size_t)b * H + h) * T + t) * N;
        } else {
          dst = p.sig + (size_t)m * HN + h * N;
        }
#pragma unroll
        for (int j = 0; j < GF; ++j) {
          const f32x4& a = acc[gi * GF + j][tb];
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = is_v ? a[r] : sigmoidf(a[r]);
          *reinterpret_cast<u32x2*>(dst + 16 * j + 4 * g) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
        }
      }
    }
  }
}

hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s) {
  const int G = ((p.M + 255) / 256) * p.H * (4 * N / 256);
  if (N == 64)
    hipLaunchKernelGGL(qkvg_proj_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(qkvg_proj_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
