// Token-block GEMM main loop for the memory-bound GEMMs of the block whose
// output has at most 1024 features per token (output projection, dZ).
//
// D(f, t) = sum_k A(f, k) B(t, k): A is an (NF, K) weight matrix with
// element (f, k) at f * a_row + (k / 32) * a_slab + k % 32 (row-major:
// a_row = K, a_slab = 32; k-slab-major: a_row = 32, a_slab = 32 * rows;
// (K / 32) * a_slab < 2^31),
// B a row-major (M, K) activation matrix. Computed transposed like the other
// token-major GEMMs: one workgroup covers all NF features of BT tokens, so
// every activation row is read from HBM exactly once, and WF x WT waves own
// 128 features x 64 tokens each (in the accumulator a lane holds one token
// and 4 consecutive features). K streams in slabs of 32 through two LDS
// stages laid out as slab.cuh describes. Both operands are fetched into
// registers RS slabs ahead of the slab being written to LDS, with ordinary
// loads, so the compiler's own wait tracking retires exactly the slab it
// writes; with GATED the B row is the elementwise product of two
// matrices, B = B0 * B1, formed while the slab is written to LDS.
#pragma once

#include <type_traits>

#include "slab.cuh"

namespace mea {

template <int NF>
struct TokShape {
  static_assert(NF % 128 == 0 && NF <= 1024, "features per token");
  static constexpr int WF = NF / 128;                    // waves along features
  static constexpr int WT = 8 % WF == 0 ? 8 / WF : 1;    // waves along tokens
  static constexpr int NW = WF * WT, NT = 64 * NW;       // waves, threads
  static constexpr int BT = 64 * WT;                     // tokens per workgroup
  static constexpr int BK = 32, FB = 8, TB = 4;          // slab width, 16-blocks per wave
  static constexpr int A_CH = NF * BK / 8, B_CH = BT * BK / 8;  // 16-byte chunks per slab
  static constexpr int NA = (A_CH + NT - 1) / NT, NB = (B_CH + NT - 1) / NT;
  static constexpr int STAGE = (NF + BT) * BK;           // elements per LDS stage
  static constexpr int RS = NF <= 512 ? 2 : 1;           // register slabs in flight
  static constexpr int SMEM = 2 * STAGE;
};

__device__ __forceinline__ u32x4 gate8(const u32x4& a, const u32x4& b) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack2(lo_bf(a[i]) * lo_bf(b[i]), hi_bf(a[i]) * hi_bf(b[i]));
  return r;
}

// Accumulates this wave's 128 x 64 block of D over the whole K into acc
// (zeroed here). Rows of A past na - 1 read row na - 1 and rows of B past
// M - 1 read row M - 1 (their results are not to be stored). K % 32 == 0.
template <int NF, bool GATED>
__device__ __forceinline__ void tok_mainloop(int K, bf16_bits* smem, const bf16_bits* A, int a_row, int a_slab, int na,
                                             const bf16_bits* B0, const bf16_bits* B1, int ldb, int m0, int M,
                                             f32x4 (&acc)[8][4]) {
  using S = TokShape<NF>;
  constexpr int BK = S::BK;
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = tid >> 6, wf = wave % S::WF, wt = wave / S::WF;

  struct Regs {
    u32x4 a[S::NA], b0[S::NB], b1[GATED ? S::NB : 1];
  };
  Regs R[S::RS];
  // Chunk id -> (row, 16-byte chunk of the 64-byte row segment).
  auto load = [&](Regs& r, int k0) {
#pragma unroll
    for (int i = 0; i < S::NA; ++i) {
      const int id = tid + S::NT * i;
      if (S::A_CH % S::NT == 0 || id < S::A_CH)
        r.a[i] = ld16(A + (size_t)min(id >> 2, na - 1) * a_row + (uint32_t)((k0 / BK) * a_slab) + (id & 3) * 8);
    }
#pragma unroll
    for (int i = 0; i < S::NB; ++i) {
      const int id = tid + S::NT * i;
      if (S::B_CH % S::NT == 0 || id < S::B_CH) {
        const size_t off = (size_t)min(m0 + (id >> 2), M - 1) * ldb + k0 + (id & 3) * 8;
        r.b0[i] = ld16(B0 + off);
        if (GATED) r.b1[i] = ld16(B1 + off);
      }
    }
  };
  auto store = [&](const Regs& r, int st) {
    bf16_bits* As = smem + st * S::STAGE;
    bf16_bits* Bs = As + NF * BK;
#pragma unroll
    for (int i = 0; i < S::NA; ++i) {
      const int id = tid + S::NT * i, row = id >> 2;
      if (S::A_CH % S::NT == 0 || id < S::A_CH)
        *reinterpret_cast<u32x4*>(As + row * BK + (((id & 3) ^ slab_swz<BK>(row)) << 3)) = r.a[i];
    }
#pragma unroll
    for (int i = 0; i < S::NB; ++i) {
      const int id = tid + S::NT * i, row = id >> 2;
      if (S::B_CH % S::NT == 0 || id < S::B_CH)
        *reinterpret_cast<u32x4*>(Bs + row * BK + (((id & 3) ^ slab_swz<BK>(row)) << 3)) =
            GATED ? gate8(r.b0[i], r.b1[i]) : r.b0[i];
    }
  };
  auto multiply = [&](int st) {
    const bf16_bits* As = smem + st * S::STAGE;
    const bf16_bits* Bs = As + NF * BK;
    bf16x8 af[S::FB], bfr[S::TB];
#pragma unroll
    for (int fb = 0; fb < S::FB; ++fb) af[fb] = as_frag(slab_read<BK>(As, wf * 128 + fb * 16 + c16, g));
#pragma unroll
    for (int tb = 0; tb < S::TB; ++tb) bfr[tb] = as_frag(slab_read<BK>(Bs, wt * 64 + tb * 16 + c16, g));
#pragma unroll
    for (int fb = 0; fb < S::FB; ++fb)
#pragma unroll
      for (int tb = 0; tb < S::TB; ++tb) acc[fb][tb] = mfma(af[fb], bfr[tb], acc[fb][tb]);
    reads_then_products<S::FB + S::TB, S::FB * S::TB>();
  };

#pragma unroll
  for (int fb = 0; fb < S::FB; ++fb)
#pragma unroll
    for (int tb = 0; tb < S::TB; ++tb) acc[fb][tb] = zero4();

  // Slab s is held in register set s % RS and multiplied from LDS stage s % 2.
  const int nk = K / BK;
  load(R[0], 0);
  if (S::RS == 2 && nk > 1) load(R[S::RS - 1], BK);
  store(R[0], 0);
  if (nk > S::RS) load(R[0], S::RS * BK);
  __syncthreads();
  // One slab: multiply slab ks, write slab ks + 1 to the other stage (its
  // last reader, slab ks - 1, is behind the previous barrier) and refill the
  // freed register set with slab ks + 1 + RS.
  auto slab = [&](int ks, auto par) {
    constexpr int P = decltype(par)::value;
    multiply(P);
    if (ks + 1 < nk) store(R[(1 - P) % S::RS], 1 - P);
    if (ks + 1 + S::RS < nk) load(R[(1 - P) % S::RS], (ks + 1 + S::RS) * BK);
    __syncthreads();
  };
  for (int ks = 0; ks < nk; ks += 2) {
    slab(ks, std::integral_constant<int, 0>{});
    if (ks + 1 < nk) slab(ks + 1, std::integral_constant<int, 1>{});
  }
}

}  // namespace mea
