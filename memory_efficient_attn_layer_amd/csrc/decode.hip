// KV-cache decode step of the block on gfx950: one new token per sequence.
//
// The reference is a training kernel and has no decode path; this is the
// same block math (README.md:42-64) for the last row of a causal sequence
// whose earlier k / v rows are cached: the new token's q, k, v come from the
// projection epilogue (at rotary row pos[b]), which writes its k / v straight
// into cache row pos[b], and
//   O[b, h] = sum_{t <= pos[b]} 2^(q'.k_t - m) v_t / sum_{t <= pos[b]} 2^(q'.k_t - m)
// with q' = q * log2(e) / sqrt(N) as the projection stores it.
//
// One query row per (b, h) leaves nothing for the matrix cores: the step
// reads every cached k / v row once and is bound by HBM. The keys of a
// (b, h) are split over many waves (split-K, "flash decoding"); each wave
// streams its split with full 16-byte row loads, N / 8 lanes per row, so one
// load instruction covers 64 / (N / 8) consecutive rows, 1 KB contiguous.
// The N / 8 lanes of a row form the dot product from their 8 elements each
// and sum it across the group; the softmax runs online (running maximum in
// log2 units) and every wave leaves an fp32 partial (o[N], m, l) that a
// second kernel combines.
#include "kernels.h"
#include "tokgemm.cuh"

namespace mea {

namespace {

constexpr int kDecodeWaves = 4;     // waves (splits) per workgroup
constexpr int kTargetWaves = 4096;  // splits over all (b, h) to fill the GPU

__device__ __forceinline__ int clamp_pos(const DecodeParams& p, int b) {
  return min(max(p.pos[b], 0), p.Tc - 1);
}

template <int N>
__global__ __launch_bounds__(64 * kDecodeWaves) void attn_decode_kernel(DecodeParams p) {
  constexpr int KL = N / 8;     // lanes per key row
  constexpr int KPI = 64 / KL;  // rows per load instruction
  constexpr int NI = 8;         // load instructions per block
  constexpr int KB = NI * KPI;  // keys per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane / KL, c = lane % KL;
  const int bh = blockIdx.x, b = bh / p.H;
  const int s = blockIdx.y * kDecodeWaves + wave;
  const int L = clamp_pos(p, b) + 1;  // keys 0 .. pos[b]
  const int k_begin = s * p.chunk, k_end = min(k_begin + p.chunk, L);

  float qv[8];
  unpack8(ld16(p.q + (size_t)bh * N + 8 * c), qv);
  const bf16_bits* kc = p.k_cache + (size_t)bh * p.Tc * N + 8 * c;
  const bf16_bits* vc = p.v_cache + (size_t)bh * p.Tc * N + 8 * c;

  float m_run = -INFINITY, l_run = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;

  for (int k0 = k_begin; k0 < k_end; k0 += KB) {
    // The block's K and V rows are requested together (V does not depend on
    // the scores), so twice the bytes are in flight per wave.
    u32x4 kr[NI], vr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + i * KPI + j;
      kr[i] = key < k_end ? ld16(kc + (size_t)key * N) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + i * KPI + j;
      vr[i] = key < k_end ? ld16(vc + (size_t)key * N) : u32x4{0u, 0u, 0u, 0u};
    }
    float sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float kf[8];
      unpack8(kr[i], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = __builtin_fmaf(qv[e], kf[e], d);
#pragma unroll
      for (int off = 1; off < KL; off <<= 1) d += shfl_xor(d, off);
      sc[i] = k0 + i * KPI + j < k_end ? d : -INFINITY;
    }
    float mb = sc[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) mb = fmaxf(mb, sc[i]);
#pragma unroll
    for (int off = KL; off < 64; off <<= 1) mb = fmaxf(mb, shfl_xor(mb, off));
    // The block's first key is valid, so mb is finite.
    const float m_new = fmaxf(m_run, mb);
    const float alpha = exp2f(m_run - m_new);  // 0 on the first block
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= alpha;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float pv = exp2f(sc[i] - m_new);  // 0 for keys past the split
      l_run += pv;
      float vf[8];
      unpack8(vr[i], vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(pv, vf[e], o[e]);
    }
  }
  // Sum over the key slots (lanes with the same chunk c). Every lane of a
  // slot holds the slot's l, so the sum over slots is the wave's l.
#pragma unroll
  for (int off = KL; off < 64; off <<= 1) {
    l_run += shfl_xor(l_run, off);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += shfl_xor(o[e], off);
  }
  float* part = p.part + ((size_t)bh * p.S + s) * (N + 4);
  if (j == 0) {
    *reinterpret_cast<f32x4*>(part + 8 * c) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4*>(part + 8 * c + 4) = f32x4{o[4], o[5], o[6], o[7]};
  }
  if (lane == 0) *reinterpret_cast<f32x4*>(part + N) = f32x4{m_run, l_run, 0.f, 0.f};
}

// O[b, h, n] = sum_s 2^(m_s - M) o_s[n] / sum_s 2^(m_s - M) l_s. One
// workgroup of 256 threads per (b, h): 256 / N groups of N threads, group
// gi takes splits gi, gi + G, ...; thread n of a group accumulates element
// n (coalesced reads of each partial), and the groups' sums meet in LDS.
// Split 0 always holds key 0, so M is finite; empty splits carry m = -inf
// and weigh 0. (A last-workgroup-combines form inside the attention kernel
// needs a device-scope release per workgroup, an L2 write-back on this
// GPU; it made the attention 4x slower.)
template <int N>
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(DecodeParams p) {
  constexpr int G = 256 / N;
  __shared__ float red[256];
  __shared__ float num_s[G][N], den_s[G];
  const int bh = blockIdx.x, tid = threadIdx.x, gi = tid / N, n = tid % N;
  const float* part = p.part + (size_t)bh * p.S * (N + 4);
  float M = -INFINITY;
  for (int s = tid; s < p.S; s += 256) M = fmaxf(M, part[(size_t)s * (N + 4) + N]);
  red[tid] = M;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
    __syncthreads();
  }
  M = red[0];
  float num = 0.f, den = 0.f;
#pragma unroll 4
  for (int s = gi; s < p.S; s += G) {
    const float* ps = part + (size_t)s * (N + 4);
    const float w = exp2f(ps[N] - M);
    num = __builtin_fmaf(w, ps[n], num);
    den = __builtin_fmaf(w, ps[N + 1], den);
  }
  num_s[gi][n] = num;
  if (n == 0) den_s[gi] = den;
  __syncthreads();
  if (gi == 0) {
    float nt = 0.f, dt = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      nt += num_s[g][n];
      dt += den_s[g];
    }
    const int b = bh / p.H, h = bh - b * p.H;
    p.o[(size_t)b * p.H * N + h * N + n] = f2bf(nt / dt);
  }
}

// Few-token product, one workgroup per 16 output features and 64 tokens:
// D^T = W A^T on v_mfma_f32_16x16x32_bf16 (A operand = 16 weight rows, B
// operand = 16 tokens), so every weight element is read once over the grid
// and the K loop is spread over the four waves (slab ks goes to wave ks % 4),
// whose partial sums meet in LDS. Rows of A past M - 1 read row M - 1 and
// are not stored.
template <bool GATED>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(SkinnyParams p) {
  constexpr int TB = 4;  // 16-token blocks per workgroup
  __shared__ f32x4 red[3][TB][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c16 = lane & 15, g = lane >> 4;
  const int f0 = blockIdx.x * 16, t0 = blockIdx.y * 64, z = blockIdx.z;
  const int nblk = min(TB, (p.M - t0 + 15) / 16);
  const int K = p.K;
  const bf16_bits* wrow = p.W[z] + (size_t)(f0 + c16) * K + 8 * g;
  const bf16_bits* arow0[TB];
  const bf16_bits* arow1[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const size_t off = (size_t)min(t0 + tb * 16 + c16, p.M - 1) * K + 8 * g;
    arow0[tb] = p.A0 + off;
    arow1[tb] = GATED ? p.A1 + off : nullptr;
  }
  f32x4 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) acc[tb] = zero4();
  // U slabs of this wave per iteration, every load issued before the first
  // product so their latencies overlap.
  constexpr int U = 4;
  const int nk = K / 32;
  for (int ks0 = wave; ks0 < nk; ks0 += 4 * U) {
    u32x4 wv[U], av[U][TB], gv[U][GATED ? TB : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ks = ks0 + 4 * u;
      if (ks >= nk) break;  // wave-uniform
      wv[u] = ld16(wrow + ks * 32);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        if (tb < nblk) {
          av[u][tb] = ld16(arow0[tb] + ks * 32);
          if (GATED) gv[u][GATED ? tb : 0] = ld16(arow1[tb] + ks * 32);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ks0 + 4 * u >= nk) break;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        if (tb < nblk) {
          const u32x4 v = GATED ? gate8(av[u][tb], gv[u][GATED ? tb : 0]) : av[u][tb];
          acc[tb] = mfma(as_frag(wv[u]), as_frag(v), acc[tb]);
        }
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) red[wave - 1][tb][lane] = acc[tb];
  }
  __syncthreads();
  if (wave == 0) {
    // D layout: lane holds token c16 of the block, features 4g .. 4g+3.
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int tok = t0 + tb * 16 + c16;
      if (tb >= nblk || tok >= p.M) continue;
      const f32x4 r = acc[tb] + red[0][tb][lane] + red[1][tb][lane] + red[2][tb][lane];
      const size_t o = (size_t)tok * p.ldo + (size_t)z * p.F + f0 + 4 * g;
      if (p.out_bf16)
        *reinterpret_cast<u32x2*>(static_cast<bf16_bits*>(p.out) + o) = u32x2{pack2(r[0], r[1]), pack2(r[2], r[3])};
      else
        *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + o) = r;
    }
  }
}

// Sum over the N threads of a workgroup (N = 32: the lower half of one
// wave, whose exchanges stay inside it; 64, 128 or 256: N / 64 waves, added
// in wave order); every thread gets it.
template <int N>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = (N < 64 ? N : 64) / 2; off > 0; off >>= 1) v += shfl_xor(v, off);
  if (N <= 64) return v;
  __syncthreads();  // earlier readers of red are done
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < N / 64; ++w) t += red[w];
  return t;
}

// One workgroup of N threads per (b, h); thread n owns feature n of the head.
// The same steps as the projection epilogue of the full-sequence kernel:
// a = rx * (x W^T) with rx = rsqrt(mean(x^2) + eps) (fast_triton_attn.py:
// 29-32), per-head RMSNorm of q and k (:102-106), rotary (:132-141) at row
// pos[b], q times qscale, v plain, sigmoid(g) (:123). k and v go straight to
// cache row pos[b] (clamped to [0, Tc - 1]), where the attention reads them.
template <int N>
__global__ __launch_bounds__(N) void decode_proj_epilogue_kernel(DecodeProjParams p) {
  __shared__ float red[N / 64 > 1 ? N / 64 : 1];
  const int bh = blockIdx.x, b = bh / p.H, h = bh - b * p.H, n = threadIdx.x;
  const int HN = p.H * N;
  float ss = 0.f;
  for (int c = n; c < p.C; c += N) {
    const float v = bf2f(p.x[(size_t)b * p.C + c]);
    ss = __builtin_fmaf(v, v, ss);
  }
  const float rx = rsqrtf(block_sum<N>(ss, red) / (float)p.C + p.eps);
  const float* a = p.a + (size_t)b * 4 * HN + h * N + n;
  const float aq = a[0] * rx, ak = a[HN] * rx, av = a[2 * HN] * rx, ag = a[3 * HN] * rx;
  const float rq = rsqrtf(block_sum<N>(aq * aq, red) * p.inv_n + p.eps);
  const float rk = rsqrtf(block_sum<N>(ak * ak, red) * p.inv_n + p.eps);
  const float qh = aq * rq, kh = ak * rk;
  const int row = min(max(p.pos[b], 0), p.t_max - 1);
  const float f1 = p.f1[(size_t)row * N + n], f2 = p.f2[(size_t)row * N + n];
  const float qsw = shfl_xor(qh, 1), ksw = shfl_xor(kh, 1);
  p.q[(size_t)bh * N + n] = f2bf((qh * f1 + qsw * f2) * p.qscale);
  const size_t c = ((size_t)bh * p.Tc + min(max(p.pos[b], 0), p.Tc - 1)) * N + n;
  p.k_cache[c] = f2bf(kh * f1 + ksw * f2);
  p.v_cache[c] = f2bf(av);
  p.sig[(size_t)b * HN + h * N + n] = f2bf(1.0f / (1.0f + __expf(-ag)));
}

}  // namespace

hipError_t launch_skinny_gemm(const SkinnyParams& p, hipStream_t s) {
  if (p.F % 16 != 0 || p.K % 32 != 0 || p.nw < 1 || p.nw > 4 || p.M < 1) return hipErrorInvalidValue;
  const dim3 grid(p.F / 16, (p.M + 63) / 64, p.nw);
  if (p.A1 != nullptr)
    hipLaunchKernelGGL(skinny_gemm_kernel<true>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(skinny_gemm_kernel<false>, grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_decode_proj_epilogue(const DecodeProjParams& p, int N, hipStream_t s) {
  if (N == 32)
    hipLaunchKernelGGL(decode_proj_epilogue_kernel<32>, dim3(p.B * p.H), dim3(32), 0, s, p);
  else if (N == 64)
    hipLaunchKernelGGL(decode_proj_epilogue_kernel<64>, dim3(p.B * p.H), dim3(64), 0, s, p);
  else if (N == 128)
    hipLaunchKernelGGL(decode_proj_epilogue_kernel<128>, dim3(p.B * p.H), dim3(128), 0, s, p);
  else if (N == 256)
    hipLaunchKernelGGL(decode_proj_epilogue_kernel<256>, dim3(p.B * p.H), dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

void decode_splits(int B, int H, int Tc, int* S, int* chunk) {
  const int bh = B * H;
  int s = (kTargetWaves + bh - 1) / bh;
  const int max_s = (Tc + 63) / 64;  // at least 64 keys per split
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  s = (s + kDecodeWaves - 1) / kDecodeWaves * kDecodeWaves;
  int ch = (Tc + s - 1) / s;
  ch = (ch + 63) / 64 * 64;
  *S = s;
  *chunk = ch;
}

hipError_t launch_attn_decode(const DecodeParams& p, int N, hipStream_t s) {
  if (p.S % kDecodeWaves != 0 || p.chunk % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid(p.B * p.H, p.S / kDecodeWaves);
  if (N == 32)
    hipLaunchKernelGGL(attn_decode_kernel<32>, grid, dim3(64 * kDecodeWaves), 0, s, p);
  else if (N == 64)
    hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(64 * kDecodeWaves), 0, s, p);
  else if (N == 128)
    hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(64 * kDecodeWaves), 0, s, p);
  else if (N == 256)
    hipLaunchKernelGGL(attn_decode_kernel<256>, grid, dim3(64 * kDecodeWaves), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_attn_decode_combine(const DecodeParams& p, int N, hipStream_t s) {
  if (N == 32)
    hipLaunchKernelGGL(attn_decode_combine_kernel<32>, dim3(p.B * p.H), dim3(256), 0, s, p);
  else if (N == 64)
    hipLaunchKernelGGL(attn_decode_combine_kernel<64>, dim3(p.B * p.H), dim3(256), 0, s, p);
  else if (N == 128)
    hipLaunchKernelGGL(attn_decode_combine_kernel<128>, dim3(p.B * p.H), dim3(256), 0, s, p);
  else if (N == 256)
    hipLaunchKernelGGL(attn_decode_combine_kernel<256>, dim3(p.B * p.H), dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mea
