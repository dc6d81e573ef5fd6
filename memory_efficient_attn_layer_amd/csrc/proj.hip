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
// filled by direct global->LDS loads (one barrier per slab). Eight waves, two
// per SIMD, each owning one projection's features of its tokens: 64 features
// x 128 tokens for N = 64, 128 x 64 for N = 128 (32 accumulators of 16x16).
//
// The input RMSNorm is never materialised: diag(1/rms(x)) commutes with the
// GEMM, so the row scale multiplies the fp32 accumulator. The row sums of
// squares come from the matrix cores: the diagonal of the 16x16 Gram matrix
// X X^T of each 16-token block, one extra MFMA per block and k-step on the x
// fragments already in registers (the two waves sharing a token half split
// the blocks).
#include "kernels.h"
#include "slab.cuh"

namespace mea {

template <int N>
__global__ __launch_bounds__(512, 1) void qkvg_proj_kernel(ProjParams p) {
  constexpr int BT = 256;              // tokens per tile
  constexpr int BF = 256;              // stacked-weight rows per tile
  constexpr int NFT = 4 * N / BF;      // feature tiles per head
  constexpr int STAGE = (BF + BT) * kSlabK;
  constexpr int WF = BF / N;           // waves along features (one projection each)
  constexpr int WT = 8 / WF;           // waves along tokens
  constexpr int FB = N / 16;           // 16-feature blocks per wave
  constexpr int TB = BT / WT / 16;     // 16-token blocks per wave
  constexpr int GB = TB / WF;          // Gram blocks per wave
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
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave % WF, wt = wave / WF;

  // Source matrix of each N-row segment of the stacked-weight slab.
  const bf16_bits* wseg[WF];
  if (WF == 4) {
    wseg[0] = wq;
    wseg[WF > 1 ? 1 : 0] = wk;
    wseg[WF > 2 ? 2 : 0] = wv;
    wseg[WF > 3 ? 3 : 0] = wg;
  } else {
    wseg[0] = f0 == 0 ? wq : wv;
    wseg[WF > 1 ? 1 : 0] = f0 == 0 ? wk : wg;
  }

  auto issue = [&](int ks, int st) {
    bf16_bits* base = smem + st * STAGE;
    const int k0 = ks * kSlabK;
    slab_issue<BF, 8>(base, wave, [&](int r, int u) {
      const int seg = (64 * u) / N;  // compile-time after unrolling
      return wseg[seg] + (size_t)(h * N + r - seg * N) * C + k0;
    });
    slab_issue<BT, 8>(base + BF * kSlabK, wave,
                      [&](int r, int) { return xg + (size_t)min(m0 + r, M - 1) * C + k0; });
  };

  f32x4 acc[FB][TB];
#pragma unroll
  for (int fb = 0; fb < FB; ++fb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = zero4();
  f32x4 gram[GB];  // Gram blocks of token blocks GB*wf .. GB*wf+GB-1
#pragma unroll
  for (int i = 0; i < GB; ++i) gram[i] = zero4();

  // One k-slab from LDS stage st: 2 x (FB*TB + GB) MFMAs.
  auto compute = [&](int st) {
    const bf16_bits* As = smem + st * STAGE;
    const bf16_bits* Bs = As + BF * kSlabK;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 af[FB], bfr[TB];
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) af[fb] = as_frag(slab_read(As, wf * N + fb * 16 + c16, 4 * kk + g));
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) bfr[tb] = as_frag(slab_read(Bs, wt * (TB * 16) + tb * 16 + c16, 4 * kk + g));
#pragma unroll
      for (int fb = 0; fb < FB; ++fb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = mfma(af[fb], bfr[tb], acc[fb][tb]);
#pragma unroll
      for (int i = 0; i < GB; ++i) {
        bf16x8 xb = bfr[i];
#pragma unroll
        for (int j = 1; j < WF; ++j) xb = wf == j ? bfr[j * GB + i] : xb;
        gram[i] = mfma(xb, xb, gram[i]);
      }
    }
  };

  // Double-buffered main loop: one barrier per slab; the next slab's loads
  // are in flight while this one is multiplied.
  const int nk = C / kSlabK;
  issue(0, 0);
  for (int ks = 0; ks + 1 < nk; ++ks) {
    wait_vmcnt0();
    __syncthreads();
    issue(ks + 1, (ks + 1) & 1);
    compute(ks & 1);
  }
  wait_vmcnt0();
  __syncthreads();
  compute((nk - 1) & 1);

  // Diagonal of each Gram block: token c16 of the block sits in lane
  // (g = c16 / 4, c16), register c16 % 4.
#pragma unroll
  for (int i = 0; i < GB; ++i) {
    if (g == (c16 >> 2)) {
      const int r = c16 & 3;
      const float d = r == 0 ? gram[i][0] : r == 1 ? gram[i][1] : r == 2 ? gram[i][2] : gram[i][3];
      ssq_s[wt * (TB * 16) + (GB * wf + i) * 16 + c16] = d;
    }
  }
  __syncthreads();

  // Row coordinates. A tile that lies inside one sequence (the usual case:
  // T a multiple of 256) needs no per-row division or bounds checks.
  const float inv_c = 1.0f / (float)C, inv_n = 1.0f / (float)N, eps = p.eps;
  const int b0 = m0 / T, t0 = m0 - b0 * T;
  const bool whole = m0 + BT <= M && t0 + BT <= T;
  int trow[TB], brow[TB];
  bool ok[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int tl = wt * (TB * 16) + tb * 16 + c16, m = m0 + tl;
    if (whole) {
      brow[tb] = b0;
      trow[tb] = t0 + tl;
      ok[tb] = true;
    } else {
      brow[tb] = m / T;
      trow[tb] = m - brow[tb] * T;
      ok[tb] = m < M;
    }
    const float rx = rsqrtf(ssq_s[tl] * inv_c + eps);
    if (p.rx != nullptr && h == 0 && f0 == 0 && wf == 0 && g == 0 && ok[tb]) p.rx[m] = rx;
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) acc[fb][tb] *= rx;
  }

  const int pj = (f0 + wf * N) / N;  // this wave's projection (wave-uniform)
  if (pj < 2) {
    // Head RMSNorm over N (fast_triton_attn.py:102-106), then the rotary
    // from the bf16-rounded normalised values, the reference's rounding point
    // (:103, :140): out[n] = qh[n] f1[t,n] + qh[n^1] f2[t,n].
    float* rstat = pj == 0 ? p.rq : p.rk;
    bf16_bits* outp = pj == 0 ? p.q : p.k;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      float s = 0.f;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += acc[fb][tb][r] * acc[fb][tb][r];
      s += shfl_xor(s, 16);
      s += shfl_xor(s, 32);
      const float rr = rsqrtf(s * inv_n + eps);
      if (ok[tb]) {
        const int t = trow[tb];
        const size_t hrow = ((size_t)brow[tb] * H + h) * T + t;
        if (rstat != nullptr && g == 0) rstat[hrow] = rr;
        const float* f1r = p.f1 + (size_t)t * N;
        const float* f2r = p.f2 + (size_t)t * N;
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) {
          const int n = 16 * fb + 4 * g;
          const f32x4 a1 = *reinterpret_cast<const f32x4*>(f1r + n);
          const f32x4 a2 = *reinterpret_cast<const f32x4*>(f2r + n);
          float qh[4], o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) qh[r] = bf2f(f2bf(acc[fb][tb][r] * rr));
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = qh[r] * a1[r] + qh[r ^ 1] * a2[r];
          *reinterpret_cast<u32x2*>(outp + hrow * N + n) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
        }
      }
    }
  } else {
    const bool is_v = pj == 2;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      if (!ok[tb]) continue;
      bf16_bits* dst = is_v ? p.v + (((size_t)brow[tb] * H + h) * T + trow[tb]) * N
                            : p.sig + ((size_t)brow[tb] * T + trow[tb]) * HN + h * N;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        const f32x4& a = acc[fb][tb];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = is_v ? a[r] : fast_sigmoid(a[r]);
        *reinterpret_cast<u32x2*>(dst + 16 * fb + 4 * g) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
    }
  }
}

hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s) {
  const int G = ((p.M + 255) / 256) * p.H * (4 * N / 256);
  if (N == 64)
    hipLaunchKernelGGL(qkvg_proj_kernel<64>, dim3(G), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL(qkvg_proj_kernel<128>, dim3(G), dim3(512), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
