// Input RMSNorm + q/k/v/g projection + per-head q/k RMSNorm + rotary +
// sigmoid, as one MFMA GEMM with a fused prologue and epilogue.
//
// Replaces rms_norm_kernel (fast_triton_attn.py:12-34) and
// fused_qkvg_norm_rope_kernel (:36-144), and their backward-recompute
// variants (:181-332) when rx/rq/rk are requested.
//
// Tile: one workgroup owns BM = 8192/N token rows and one head h; its four
// waves compute the four projections of that head (wave p -> W_p rows
// h*N .. h*N+N-1), so every head-local reduction of the epilogue stays inside
// one wave. The input RMSNorm is never materialised: diag(1/rms(x)) commutes
// with the GEMM, so each thread accumulates the sum of squares of the x
// chunks it streams and the row scale is applied to the fp32 accumulator.
#include "gemm_core.cuh"
#include "kernels.h"

namespace mea {

template <int N>
__global__ __launch_bounds__(256) void qkvg_proj_kernel(ProjParams p) {
  constexpr int BM = 8192 / N, BN = 4 * N;
  constexpr int MB = BM / 16, NB = N / 16;
  constexpr int SP = N + 8;  // staging pitch (elements)
  constexpr int SMEM_MAIN = NtSmem<BM, BN>::elems, SMEM_STG = 4 * BM * SP;
  constexpr int SMEM = SMEM_MAIN > SMEM_STG ? SMEM_MAIN : SMEM_STG;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SMEM];
  __shared__ float rxs[BM];

  const int M = p.M, C = p.C, H = p.H, T = p.T, HN = H * N;
  const int ntm = (M + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, ntm * H);
  const int h = L % H, m0 = (L / H) * BM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;

  // Locals, not captures of the argument block: a lambda holding &p would
  // force the block into scratch memory.
  const bf16_bits* __restrict__ xg = p.x;
  const bf16_bits *wq = p.wq, *wk = p.wk, *wv = p.wv, *wg = p.wg;
  bf16_bits *oq = p.q, *ok = p.k, *ov = p.v, *osig = p.sig;
  float *rq = p.rq, *rk = p.rk;

  // Sum of squares of the x rows this thread streams: rows (tid>>2) + 64*i.
  float ss0 = 0.f, ss1 = 0.f;
  auto load_a = [&](int row, int k0, int kc, int) -> u32x4 {
    const int m = m0 + row;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < M) {
      v = ld16(xg + (size_t)m * C + k0 + kc * 8);
      float f[8];
      unpack8(v, f);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s += f[i] * f[i];
      if (row >= 64) ss1 += s; else ss0 += s;
    }
    return v;
  };
  auto load_b = [&](int row, int k0, int kc, int i) -> u32x4 {
    const int pj = (64 * i) / N, n = row % N;  // row = (tid >> 2) + 64 i
    const bf16_bits* w = pj == 0 ? wq : pj == 1 ? wk : pj == 2 ? wv : wg;
    return ld16(w + (size_t)(h * N + n) * C + k0 + kc * 8);
  };

  f32x4 acc[MB][NB];
  mainloop_nt<BM, BN, 1, 4>(C, smem, load_a, load_b, acc);

  // Row scale 1/rms(x): reduce over the 4 threads that share a row.
  {
    constexpr int ASL = (BM * 4 + 255) / 256;
#pragma unroll
    for (int i = 0; i < ASL; ++i) {
      float s = i == 0 ? ss0 : ss1;
      s += xor1(s);
      s += xor2(s);
      const int row = (tid >> 2) + 64 * i;
      if ((tid & 3) == 0 && row < BM) {
        const float r = rsqrtf(s / (float)C + p.eps);
        rxs[row] = r;
        if (p.rx != nullptr && h == 0 && m0 + row < M) p.rx[m0 + row] = r;
      }
    }
  }
  __syncthreads();

  float rxv[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) rxv[mb][r] = rxs[mb * 16 + 4 * g + r];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mb][nb][r] *= rxv[mb][r];

  if (wave < 2) {
    // Head RMSNorm over N (fast_triton_attn.py:102-106). The rotary is applied
    // in the row-contiguous store below, from the bf16-rounded normalised
    // values, the same rounding point as the reference (:103, :140).
    float* rstat = wave == 0 ? rq : rk;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s = 0.f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s += acc[mb][nb][r] * acc[mb][nb][r];
        s = sum16(s);
        const float rr = rsqrtf(s / (float)N + p.eps);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb][r] *= rr;
        const int m = m0 + mb * 16 + 4 * g + r;
        if (rstat != nullptr && c16 == 0 && m < M) {
          const int b = m / T, t = m - b * T;
          rstat[((size_t)b * H + h) * T + t] = rr;
        }
      }
  } else if (wave == 3) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mb][nb][r] = sigmoidf(acc[mb][nb][r]);
  }

  // Stage the wave's BM x N tile as bf16 and store it with 16-byte rows.
  bf16_bits* stg = smem + wave * BM * SP;
  stage_acc_bf16<MB, NB, SP>(stg, 0, 0, acc, [](int, int, float v) { return v; });
  __syncthreads();
  constexpr int CPR = N / 8;  // 16-byte chunks per row
  bf16_bits* base = wave == 0 ? oq : wave == 1 ? ok : wave == 2 ? ov : osig;
#pragma unroll 4
  for (int it = 0; it < BM * CPR / 64; ++it) {
    const int id = lane + 64 * it, row = id / CPR, dc = id % CPR;
    const int m = m0 + row;
    if (m < M) {
      u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * SP + dc * 8);
      size_t off;
      if (wave < 3) {
        const int b = m / T, t = m - b * T;
        off = (((size_t)b * H + h) * T + t) * N + dc * 8;
        if (wave < 2) {
          // Adjacent-pair rotary out[n] = t[n]*f1[t,n] + t[n^1]*f2[t,n]
          // (fast_triton_attn.py:132-141); both pair members are in this chunk.
          const float* f1r = p.f1 + (size_t)t * N + dc * 8;
          const float* f2r = p.f2 + (size_t)t * N + dc * 8;
          float xh[8], o[8];
          unpack8(val, xh);
#pragma unroll
          for (int i = 0; i < 8; i += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(f1r + i);
            const f32x4 c = *reinterpret_cast<const f32x4*>(f2r + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[i + e] = xh[i + e] * a[e] + xh[(i + e) ^ 1] * c[e];
          }
          val = pack8(o);
        }
      } else {
        off = (size_t)m * HN + h * N + dc * 8;
      }
      st16(base + off, val);
    }
  }
}

hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s) {
  if (N == 64) {
    const int G = ((p.M + 127) / 128) * p.H;
    hipLaunchKernelGGL(qkvg_proj_kernel<64>, dim3(G), dim3(256), 0, s, p);
  } else {
    const int G = ((p.M + 63) / 64) * p.H;
    hipLaunchKernelGGL(qkvg_proj_kernel<128>, dim3(G), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace mea
