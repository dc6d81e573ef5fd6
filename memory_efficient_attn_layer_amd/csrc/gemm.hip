// GEMM-shaped kernels of the block, each with its elementwise neighbours
// fused into operand fetch (prologue) or into the tile epilogue:
//
//   gate_oproj  y = (O * sig) Wo^T                 gate_repack_kernel
//               (fast_triton_attn.py:146-176) + F.linear (:460)
//   dz_gate_bwd dZ = dy Wo, dO = dZ*sig, da_g, delta   (:577-584, :601) and the
//               row sums rowsum(dO*O) the attention backward needs
//   dx          dx = rmsnorm_bwd([da_q|da_k|da_v|da_g] Wcat)   (:655-669)
//   dw          dW_p = da_p^T xh, dWo = dy^T (O*sig)           (:579, :642-652)
//               as token-split fp32 partials plus a deterministic reduction.
//
// Projection-gradient rows arrive pre-scaled by rx = 1/rms(x), so
//   dW_p = (rx da_p)^T x   and   dx = acc - x * rx^2 * (acc . x) / C
// with acc = sum_p (rx da_p) W_p; neither xh nor dxh is ever stored.
#include "gemm_core.cuh"
#include "kernels.h"

namespace mea {

// ---------------------------------------------------------------------------
// y = (O * sig) Wo^T
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gate_oproj_kernel(OprojParams p) {
  constexpr int BM = 128, BN = 256, SP = BN + 8;
  constexpr int SM_MAIN = NtSmem<BM, BN>::elems, SM_STG = BM * SP;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SM_MAIN > SM_STG ? SM_MAIN : SM_STG];
  const int M = p.M, C = p.C, HN = p.HN;
  const int nct = C / BN, ntm = (M + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, ntm * nct);
  const int m0 = (L / nct) * BM, n0 = (L % nct) * BN;
  const int tid = threadIdx.x, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;

  auto load_a = [&](int row, int k0, int kc, int) -> u32x4 {
    const int m = m0 + row;
    if (m >= M) return u32x4{0u, 0u, 0u, 0u};
    const size_t off = (size_t)m * HN + k0 + kc * 8;
    float o[8], s[8];
    unpack8(ld16(p.o + off), o);
    unpack8(ld16(p.sig + off), s);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= s[i];
    return pack8(o);
  };
  auto load_b = [&](int row, int k0, int kc, int) -> u32x4 {
    return ld16(p.wo + (size_t)(n0 + row) * HN + k0 + kc * 8);
  };
  f32x4 acc[4][8];
  mainloop_nt<BM, BN, 2, 2>(HN, smem, load_a, load_b, acc);

  stage_acc_bf16<4, 8, SP>(smem, wm * 64, wn * 128, acc, [](int, int, float v) { return v; });
  __syncthreads();
#pragma unroll 4
  for (int it = 0; it < BM * (BN / 8) / 256; ++it) {
    const int id = tid + 256 * it, row = id / (BN / 8), cc = id % (BN / 8);
    const int m = m0 + row;
    if (m < M) st16(p.y + (size_t)m * C + n0 + cc * 8, *reinterpret_cast<const u32x4*>(smem + row * SP + cc * 8));
  }
}

hipError_t launch_gate_oproj(const OprojParams& p, hipStream_t s) {
  const int G = ((p.M + 127) / 128) * (p.C / 256);
  hipLaunchKernelGGL(gate_oproj_kernel, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dZ = dy Wo with the gate backward in the epilogue.
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void dz_gate_bwd_kernel(DzParams p) {
  constexpr int BM = 128, BN = 256, FP = 128 + 4;
  constexpr int SM_MAIN = NtSmem<BM, BN>::elems * 2, SM_STG = 4 * 32 * FP * 4;  // bytes
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM_MAIN > SM_STG ? SM_MAIN : SM_STG];
  const int M = p.M, C = p.C, H = p.H, T = p.T, HN = H * N;
  const int nct = (HN + BN - 1) / BN, ntm = (M + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, ntm * nct);
  const int m0 = (L / nct) * BM, n0 = (L % nct) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int c16 = lane & 15, g = lane >> 4;

  auto load_a = [&](int row, int k0, int kc, int) -> u32x4 {
    const int m = m0 + row;
    return m < M ? ld16(p.dy + (size_t)m * C + k0 + kc * 8) : u32x4{0u, 0u, 0u, 0u};
  };
  auto load_b = [&](int row, int k0, int kc, int) -> u32x4 {
    const int j = n0 + row;
    return j < HN ? ld16(p.woT + (size_t)j * C + k0 + kc * 8) : u32x4{0u, 0u, 0u, 0u};
  };
  f32x4 acc[4][8];
  mainloop_nt<BM, BN, 2, 2>(C, reinterpret_cast<bf16_bits*>(smem), load_a, load_b, acc);

  float* stg = reinterpret_cast<float*>(smem) + wave * 32 * FP;
  constexpr int CPH = N / 8;  // 16-byte chunks per head row
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) stg[(mb * 16 + 4 * g + r) * FP + nb * 16 + c16] = acc[2 * hf + mb][nb][r];
    __syncthreads();
#pragma unroll 1
    for (int pass = 0; pass < 8; ++pass) {
      const int row = pass * 4 + (lane >> 4), cc = lane & 15;
      const int m = m0 + wm * 64 + hf * 32 + row;
      const int j = n0 + wn * 128 + cc * 8;
      const bool valid = m < M && j < HN;
      const int mc = m < M ? m : M - 1, jc = j < HN ? j : 0;
      float dz[8], sg[8], ov[8];
      {
        const f32x4 a = *reinterpret_cast<const f32x4*>(stg + row * FP + cc * 8);
        const f32x4 c = *reinterpret_cast<const f32x4*>(stg + row * FP + cc * 8 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { dz[i] = a[i]; dz[4 + i] = c[i]; }
      }
      const size_t off = (size_t)mc * HN + jc;
      unpack8(ld16(p.sig + off), sg);
      unpack8(ld16(p.o + off), ov);
      const float rxv = p.rx[mc];
      float dov[8], dag[8], dl = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // delta uses the bf16-rounded dO the attention backward consumes, so
        // dP - delta cancels exactly where it should (a single key, T = 1).
        dov[i] = bf2f(f2bf(dz[i] * sg[i]));
        dag[i] = rxv * dz[i] * ov[i] * sg[i] * (1.0f - sg[i]);
        dl += dov[i] * ov[i];
      }
      dl += xor1(dl);
      dl += xor2(dl);
      dl += shfl_xor(dl, 4);
      if (CPH == 16) dl += shfl_xor(dl, 8);
      if (valid) {
        const int hh = jc / N, n = jc % N;
        const int b = mc / T, t = mc - b * T;
        const size_t hrow = ((size_t)b * H + hh) * T + t;
        st16(p.dO + hrow * N + n, pack8(dov));
        st16(p.dag + off, pack8(dag));
        if (n == 0) p.delta[hrow] = dl;
      }
    }
    __syncthreads();
  }
}

hipError_t launch_dz_gate_bwd(const DzParams& p, hipStream_t s) {
  const int HN = p.H * p.N;
  const int G = ((p.M + 127) / 128) * ((HN + 255) / 256);
  if (p.N == 64)
    hipLaunchKernelGGL(dz_gate_bwd_kernel<64>, dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(dz_gate_bwd_kernel<128>, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dx = rmsnorm_bwd([da_q|da_k|da_v|da_g] Wcat); one workgroup owns full rows.
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(256) void dx_kernel(DxParams p) {
  constexpr int BM = 32768 / C, BN = C;
  constexpr int MB = BM / 16, NB = C / 64;
  constexpr int XP = C + 8;
  constexpr int SM_MAIN = NtSmem<BM, BN>::elems, SM_X = BM * XP;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SM_MAIN > SM_X ? SM_MAIN : SM_X];
  __shared__ float dotp[4][BM];
  const int M = p.M, HN = p.HN, K4 = 4 * HN;
  const int ntm = (M + BM - 1) / BM;
  const int m0 = xcd_remap(blockIdx.x, ntm) * BM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;

  auto load_a = [&](int row, int k0, int kc, int) -> u32x4 {
    const int m = m0 + row;
    if (m >= M) return u32x4{0u, 0u, 0u, 0u};
    const int pj = k0 / HN, col = k0 - pj * HN + kc * 8;
    const bf16_bits* src = pj == 0 ? p.daq : pj == 1 ? p.dak : pj == 2 ? p.dav : p.dag;
    return ld16(src + (size_t)m * HN + col);
  };
  auto load_b = [&](int row, int k0, int kc, int) -> u32x4 {
    return ld16(p.wcatT + (size_t)row * K4 + k0 + kc * 8);
  };
  f32x4 acc[MB][NB];
  mainloop_nt<BM, BN, 1, 4>(K4, smem, load_a, load_b, acc);

  // x tile -> LDS.
  for (int id = tid; id < BM * (C / 8); id += 256) {
    const int row = id / (C / 8), cc = id % (C / 8);
    const int m = m0 + row;
    const u32x4 v = m < M ? ld16(p.x + (size_t)m * C + cc * 8) : u32x4{0u, 0u, 0u, 0u};
    st16(smem + row * XP + cc * 8, v);
  }
  __syncthreads();
  const int col0 = wave * (C / 4);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mb * 16 + 4 * g + r;
      float s = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s += acc[mb][nb][r] * bf2f(smem[row * XP + col0 + nb * 16 + c16]);
      s = sum16(s);
      if (c16 == 0) dotp[wave][row] = s;
    }
  __syncthreads();
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mb * 16 + 4 * g + r;
      const int m = m0 + row;
      const float rxv = m < M ? p.rx[m] : 0.f;
      const float dot = dotp[0][row] + dotp[1][row] + dotp[2][row] + dotp[3][row];
      const float cf = rxv * rxv * dot / (float)C;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        bf16_bits& xr = smem[row * XP + col0 + nb * 16 + c16];
        xr = f2bf(acc[mb][nb][r] - bf2f(xr) * cf);
      }
    }
  __syncthreads();
  for (int id = tid; id < BM * (C / 8); id += 256) {
    const int row = id / (C / 8), cc = id % (C / 8);
    const int m = m0 + row;
    if (m < M) st16(p.dx + (size_t)m * C + cc * 8, *reinterpret_cast<const u32x4*>(smem + row * XP + cc * 8));
  }
}

hipError_t launch_dx(const DxParams& p, hipStream_t s) {
  switch (p.C) {
    case 256:
      hipLaunchKernelGGL(dx_kernel<256>, dim3((p.M + 127) / 128), dim3(256), 0, s, p);
      break;
    case 512:
      hipLaunchKernelGGL(dx_kernel<512>, dim3((p.M + 63) / 64), dim3(256), 0, s, p);
      break;
    case 1024:
      hipLaunchKernelGGL(dx_kernel<1024>, dim3((p.M + 31) / 32), dim3(256), 0, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weight gradients: D(i, j) = sum_m A(m, i) B(m, j) over a token slice.
// Both operands are token-major, so each 32-token slab is written into LDS
// transposed (pairs of tokens packed into 32-bit words) and then read as
// ordinary k-contiguous MFMA fragments.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dw_partial_kernel(DwParams p) {
  constexpr int BT = 128, P = kLdsPitch;  // tile 128 x 128, 32 tokens per step
  __shared__ __attribute__((aligned(16))) bf16_bits At[BT * P];
  __shared__ __attribute__((aligned(16))) bf16_bits Bt[BT * P];
  const int M = p.M, C = p.C, HN = p.HN, K4 = 4 * HN;
  const int ti0 = K4 / BT, tj0 = C / BT;                  // dWcat tiles
  const int tj1 = (HN + BT - 1) / BT;                     // dWo tiles
  const int tile = blockIdx.x, z = blockIdx.y;
  const bool prob1 = tile >= ti0 * tj0;
  const int lt = prob1 ? tile - ti0 * tj0 : tile;
  const int ntj = prob1 ? tj1 : tj0;
  const int i0 = (lt / ntj) * BT, j0 = (lt % ntj) * BT;
  const int I = prob1 ? C : K4, J = prob1 ? HN : C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int c16 = lane & 15, g = lane >> 4;

  const int chunk = ((M + (int)gridDim.y - 1) / (int)gridDim.y + 31) / 32 * 32;
  const int mbeg = z * chunk, mend = min(M, mbeg + chunk);

  // One row pair x 8 columns per thread per operand.
  const int rp = tid >> 4, cc = tid & 15;
  auto ld_a = [&](int m) -> u32x4 {
    const int i = i0 + cc * 8;
    if (m >= mend || i >= I) return u32x4{0u, 0u, 0u, 0u};
    if (prob1) return ld16(p.dy + (size_t)m * C + i);
    const int pj = i / HN, col = i - pj * HN;
    const bf16_bits* src = pj == 0 ? p.daq : pj == 1 ? p.dak : pj == 2 ? p.dav : p.dag;
    return ld16(src + (size_t)m * HN + col);
  };
  auto ld_b = [&](int m) -> u32x4 {
    const int j = j0 + cc * 8;
    if (m >= mend || j >= J) return u32x4{0u, 0u, 0u, 0u};
    if (!prob1) return ld16(p.x + (size_t)m * C + j);
    float o[8], s[8];
    unpack8(ld16(p.o + (size_t)m * HN + j), o);
    unpack8(ld16(p.sig + (size_t)m * HN + j), s);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= s[e];
    return pack8(o);
  };
  auto put_t = [&](bf16_bits* dstT, const u32x4& r0, const u32x4& r1) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(dstT + (cc * 8) * P + 2 * rp);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dst[(2 * e) * P / 2] = (r0[e] & 0xffffu) | (r1[e] << 16);
      dst[(2 * e + 1) * P / 2] = (r0[e] >> 16) | (r1[e] & 0xffff0000u);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[a][c] = zero4();

  u32x4 a0, a1, b0, b1;
  auto fetch = [&](int m) {
    a0 = ld_a(m + 2 * rp);
    a1 = ld_a(m + 2 * rp + 1);
    b0 = ld_b(m + 2 * rp);
    b1 = ld_b(m + 2 * rp + 1);
  };
  if (mbeg < mend) fetch(mbeg);
  for (int m = mbeg; m < mend; m += 32) {
    put_t(At, a0, a1);
    put_t(Bt, b0, b1);
    __syncthreads();
    if (m + 32 < mend) fetch(m + 32);
    bf16x8 af[4], bfr[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) af[a] = as_frag(*reinterpret_cast<const u32x4*>(At + (wm * 64 + a * 16 + c16) * P + 8 * g));
#pragma unroll
    for (int c = 0; c < 4; ++c) bfr[c] = as_frag(*reinterpret_cast<const u32x4*>(Bt + (wn * 64 + c * 16 + c16) * P + 8 * g));
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[a][c] = mfma(af[a], bfr[c], acc[a][c]);
    __syncthreads();
  }

  const size_t per_split = (size_t)K4 * C + (size_t)C * HN;
  float* out = p.part + (size_t)z * per_split + (prob1 ? (size_t)K4 * C : 0);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j = j0 + wn * 64 + c * 16 + c16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + wm * 64 + a * 16 + 4 * g + r;
        if (i < I && j < J) out[(size_t)i * J + j] = acc[a][c][r];
      }
    }
}

hipError_t launch_dw_partial(const DwParams& p, hipStream_t s) {
  const int K4 = 4 * p.HN;
  const int tiles = (K4 / 128) * (p.C / 128) + (p.C / 128) * ((p.HN + 127) / 128);
  hipLaunchKernelGGL(dw_partial_kernel, dim3(tiles, p.splits), dim3(256), 0, s, p);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void dw_reduce_kernel(DwReduceParams p) {
  const int C = p.C, HN = p.HN;
  const size_t n_cat = (size_t)4 * HN * C, total = n_cat + (size_t)C * HN;
  const size_t e = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= total) return;
  f32x4 s = zero4();
  for (int z = 0; z < p.splits; ++z) s += *reinterpret_cast<const f32x4*>(p.part + (size_t)z * total + e);
  const u32x2 w = {pack2(s[0], s[1]), pack2(s[2], s[3])};
  bf16_bits* dst;
  if (e < n_cat) {
    const size_t per = (size_t)HN * C;
    const int pj = (int)(e / per);
    bf16_bits* base = pj == 0 ? p.dwq : pj == 1 ? p.dwk : pj == 2 ? p.dwv : p.dwg;
    dst = base + (e - (size_t)pj * per);
  } else {
    dst = p.dwo + (e - n_cat);
  }
  *reinterpret_cast<u32x2*>(dst) = w;
}

hipError_t launch_dw_reduce(const DwReduceParams& p, hipStream_t s) {
  const size_t total = (size_t)4 * p.HN * p.C + (size_t)p.C * p.HN;
  const int G = (int)((total / 4 + 255) / 256);
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(G), dim3(256), 0, s, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Small helpers.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void transpose_kernel(const bf16_bits* in, int rows, int cols, int ld_in,
                                                        bf16_bits* out, int ld_out, int col_off) {
  __shared__ bf16_bits tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int rr = r0 + r, cc = c0 + tx;
    tile[r][tx] = (rr < rows && cc < cols) ? in[(size_t)rr * ld_in + cc] : (bf16_bits)0;
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int cc = c0 + c, rr = r0 + tx;
    if (cc < cols && rr < rows) out[(size_t)cc * ld_out + col_off + rr] = tile[tx][c];
  }
}

hipError_t launch_transpose(const bf16_bits* in, int rows, int cols, int ld_in, bf16_bits* out, int ld_out,
                            int col_off, hipStream_t s) {
  hipLaunchKernelGGL(transpose_kernel, dim3((cols + 63) / 64, (rows + 63) / 64), dim3(256), 0, s, in, rows, cols,
                     ld_in, out, ld_out, col_off);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0.f;
}

hipError_t launch_zero_f32(float* p, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t G = (n + 255) / 256;
  if (G > 4096) G = 4096;
  hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)G), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

}  // namespace mea
