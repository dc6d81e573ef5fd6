// Tiled bf16 MFMA main loop shared by the GEMM-shaped kernels.
// Loader signature: u32x4 load(row, k0, kc, i) returns the 8 elements
// (row, k0 + 8*kc .. +7); i is the thread's chunk slot (a compile-time
// constant after unrolling, row = (threadIdx.x >> 2) + 64 * i).
//
// A workgroup of 256 threads (4 waves) computes a BM x BN tile of
// D = A * B^T where both operands are read "k-contiguous": A(row, k) and
// B(col, k) come in 8-element (16-byte) chunks from caller-supplied loader
// functors, so a loader can fuse elementwise work (the output gate, a row
// scale, a concatenation of several weight matrices) into the operand fetch.
//
// Pipeline: the next k-slab is fetched into registers while the current slab
// is multiplied out of LDS (one LDS buffer, register double buffering).
// LDS rows are padded by 8 elements so the 16-byte fragment reads of 16
// consecutive rows fall on distinct bank groups.
#pragma once

#include "common.cuh"

namespace mea {

constexpr int kBK = 32;          // k-slab per step (one MFMA depth)
constexpr int kLdsPitch = kBK + 8;

template <int BM, int BN>
struct NtSmem {
  static constexpr int elems = (BM + BN) * kLdsPitch;
};

// acc[MB][NB] with MB = BM/WM/16, NB = BN/WN/16; waves laid out WM x WN.
template <int BM, int BN, int WM, int WN, class LA, class LB>
__device__ __forceinline__ void mainloop_nt(int K, bf16_bits* smem, LA load_a, LB load_b,
                                            f32x4 (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int MB = BM / WM / 16, NB = BN / WN / 16;
  constexpr int ACHUNKS = BM * 4, BCHUNKS = BN * 4;
  constexpr int ACH = (ACHUNKS + 255) / 256, BCH = (BCHUNKS + 255) / 256;
  static_assert(WM * WN == 4, "4 waves");
  bf16_bits* As = smem;
  bf16_bits* Bs = smem + BM * kLdsPitch;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;
  const int wm = wave / WN, wn = wave % WN;

#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = zero4();

  u32x4 ra[ACH], rb[BCH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int id = tid + 256 * i;
      if (ACHUNKS % 256 == 0 || id < ACHUNKS) ra[i] = load_a(id >> 2, k0, id & 3, i);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int id = tid + 256 * i;
      if (BCHUNKS % 256 == 0 || id < BCHUNKS) rb[i] = load_b(id >> 2, k0, id & 3, i);
    }
  };

  fetch(0);
  for (int k0 = 0; k0 < K; k0 += kBK) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int id = tid + 256 * i;
      if (ACHUNKS % 256 == 0 || id < ACHUNKS) st16(As + (id >> 2) * kLdsPitch + (id & 3) * 8, ra[i]);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int id = tid + 256 * i;
      if (BCHUNKS % 256 == 0 || id < BCHUNKS) st16(Bs + (id >> 2) * kLdsPitch + (id & 3) * 8, rb[i]);
    }
    __syncthreads();
    if (k0 + kBK < K) fetch(k0 + kBK);
    bf16x8 af[MB], bfr[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      af[mb] = as_frag(*reinterpret_cast<const u32x4*>(As + (wm * MB * 16 + mb * 16 + c16) * kLdsPitch + 8 * g));
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      bfr[nb] = as_frag(*reinterpret_cast<const u32x4*>(Bs + (wn * NB * 16 + nb * 16 + c16) * kLdsPitch + 8 * g));
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma(af[mb], bfr[nb], acc[mb][nb]);
    __syncthreads();
  }
}

// Writes a wave's accumulator tile (after an elementwise map f(row, col, v))
// as bf16 into an LDS staging tile of pitch SP elements.
// Rows/cols are tile-local. Caller synchronises.
template <int MB, int NB, int SP, class F>
__device__ __forceinline__ void stage_acc_bf16(bf16_bits* stg, int row0, int col0,
                                               const f32x4 (&acc)[MB][NB], F f) {
  const int lane = threadIdx.x & 63, c16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + mb * 16 + 4 * g + r, col = col0 + nb * 16 + c16;
        stg[row * SP + col] = f2bf(f(row, col, acc[mb][nb][r]));
      }
}

}  // namespace mea
