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

// Tile coordinates of logical tile L: token tile (head-minor order, so the
// tiles of one token tile are consecutive and share their x rows in L2).
struct ProjTile {
  int m0, h, f0;
};

template <int N>
__device__ __forceinline__ ProjTile proj_tile(int L, int H) {
  constexpr int NFT = 4 * N / 256;
  const int tt = L / (H * NFT), rem = L - tt * (H * NFT);
  return ProjTile{tt * 256, rem / NFT, (rem % NFT) * 256};
}

// Persistent: one workgroup per CU walks tiles; the first k-slab of its next
// tile is loaded while the current tile's epilogue runs. Workgroup w runs on
// XCD w % 8 and takes tiles from a contiguous range owned by that XCD, so the
// workgroups of one XCD work on neighbouring tiles at the same time.
template <int N>
__global__ __launch_bounds__(512, 1) void qkvg_proj_kernel(ProjParams p) {
  constexpr int BT = 256;              // tokens per tile
  constexpr int BF = 256;              // stacked-weight rows per tile
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
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave % WF, wt = wave / WF;

  // This workgroup's tiles: start + j, start + j + nj, ... (< start + cnt).
  const int ntiles = ((M + BT - 1) / BT) * H * (4 * N / BF);
  const int G = gridDim.x, xcd = blockIdx.x & 7, j0 = blockIdx.x >> 3;
  const int nj = (G - xcd + 7) >> 3;
  const int q8 = ntiles >> 3, r8 = ntiles & 7;
  const int start = xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8;
  const int cnt = xcd < r8 ? q8 + 1 : q8;

  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](const ProjTile& tl, int ks, int st) {
    const uint32_t lds = lds0 + (uint32_t)(st * STAGE) * 2u;
    const int k0 = ks * kSlabK;
    const bf16_bits* wseg[WF];
    if (WF == 4) {
      wseg[0] = wq;
      wseg[WF > 1 ? 1 : 0] = wk;
      wseg[WF > 2 ? 2 : 0] = wv;
      wseg[WF > 3 ? 3 : 0] = wg;
    } else {
      wseg[0] = tl.f0 == 0 ? wq : wv;
      wseg[WF > 1 ? 1 : 0] = tl.f0 == 0 ? wk : wg;
    }
    // Stacked-weight rows: group u (64 rows) lies inside one projection.
    slab_issue<BF, 8>(
        lds, wave, C,
        [&](int u) {
          const int seg = (64 * u) / N;  // compile-time after unrolling
          return wseg[seg] + (size_t)(tl.h * N + 64 * u - seg * N) * C + k0;
        },
        [](int, int i) { return i; });
    // x rows, clamped to the last token.
    slab_issue<BT, 8>(
        lds + BF * kSlabK * 2, wave, C,
        [&](int u) { return xg + (size_t)min(tl.m0 + 64 * u, M - 1) * C + k0; },
        [&](int u, int i) { return min(tl.m0 + 64 * u + i, M - 1) - min(tl.m0 + 64 * u, M - 1); });
  };

  f32x4 acc[FB][TB];
  f32x4 gram[GB];  // Gram blocks of token blocks GB*wf .. GB*wf+GB-1

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

  const int nk = C / kSlabK;
  if (j0 < cnt) issue(proj_tile<N>(start + j0, H), 0, 0);
  for (int jt = j0; jt < cnt; jt += nj) {
    const ProjTile tl = proj_tile<N>(start + jt, H);
    const bool has_next = jt + nj < cnt;
    const ProjTile nx = proj_tile<N>(start + (has_next ? jt + nj : jt), H);

#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = zero4();
#pragma unroll
    for (int i = 0; i < GB; ++i) gram[i] = zero4();

    // Double-buffered main loop: one barrier per slab; the next slab's loads
    // (after the last slab: the next tile's first) are in flight while this
    // one is multiplied. Slab ks lives in stage ks & 1 (nk is even).
    for (int ks = 0; ks + 1 < nk; ++ks) {
      wait_vmcnt0();
      __syncthreads();
      issue(tl, ks + 1, (ks + 1) & 1);
      compute(ks & 1);
    }
    wait_vmcnt0();
    __syncthreads();
    if (has_next) issue(nx, 0, 0);
    compute(1);

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

    // Row coordinates. A tile inside one sequence (the usual case: T a
    // multiple of 256) needs no per-row division or bounds checks.
    const int m0 = tl.m0, h = tl.h;
    const float inv_c = 1.0f / (float)C, inv_n = 1.0f / (float)N, eps = p.eps;
    const int b0 = m0 / T, t0 = m0 - b0 * T;
    const bool whole = m0 + BT <= M && t0 + BT <= T;
    int trow[TB], brow[TB];
    bool ok[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int tlr = wt * (TB * 16) + tb * 16 + c16, m = m0 + tlr;
      if (whole) {
        brow[tb] = b0;
        trow[tb] = t0 + tlr;
        ok[tb] = true;
      } else {
        brow[tb] = m / T;
        trow[tb] = m - brow[tb] * T;
        ok[tb] = m < M;
      }
      const float rx = rsqrtf(ssq_s[tlr] * inv_c + eps);
      if (p.rx != nullptr && h == 0 && tl.f0 == 0 && wf == 0 && g == 0 && ok[tb]) p.rx[m] = rx;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) acc[fb][tb] *= rx;
    }

    const int pj = (tl.f0 + wf * N) / N;  // this wave's projection (wave-uniform)
    if (pj < 2) {
      // Head RMSNorm over N (fast_triton_attn.py:102-106), then the rotary
      // from the bf16-rounded normalised values, the reference's rounding
      // point (:103, :140): out[n] = qh[n] f1[t,n] + qh[n^1] f2[t,n].
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
}

// Workgroups per device for the persistent kernels: one per CU.
int persistent_grid(int tiles) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return tiles < cus[dev] ? tiles : cus[dev];
}

hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s) {
  const int G = persistent_grid(((p.M + 255) / 256) * p.H * (4 * N / 256));
  if (N == 64)
    hipLaunchKernelGGL(qkvg_proj_kernel<64>, dim3(G), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL(qkvg_proj_kernel<128>, dim3(G), dim3(512), 0, s, p);
  return hipGetLastError();
}

}  // namespace mea
