// LDS k-slabs for the GEMM-shaped kernels (gfx950).
//
// A slab holds R operand rows x KS bf16 of the reduction dimension k, KS = 64
// (8 chunks of 16 bytes per row) or 32 (4 chunks). Chunk c of row r sits at
// chunk slot c ^ slab_swz<KS>(r). The MFMA operand read has lane 16g + i
// fetch chunk g of row r0 + i. For 32-element rows the slot of row r is
// (r >> 1) & 3: measured on gfx950 (ds_read_b128 in this pattern, rocprofv3
// SQ_LDS_BANK_CONFLICT), it is conflict-free and reads 223 B/clk per CU,
// where (r >> 2) & 3, r & 3 or no swizzle conflict on half the cycles
// (132 B/clk). 64-element rows use (r >> 1) & 7.
//
// Slabs are filled straight from global memory with global_load_lds_dwordx4:
// one wave instruction writes 1 KB of LDS (64 / CH rows), lane L filling slot
// L % CH of row L / CH; the swizzle is applied by choosing which global chunk
// each lane fetches, so every CH lanes still read one contiguous row segment.
#pragma once

#include "common.cuh"

namespace mea {

constexpr int kSlabK = 64;  // k elements per row of a 64-wide slab

template <int KS>
__device__ __forceinline__ int slab_swz(int row) {
  static_assert(KS == 64 || KS == 32, "slab width");
  return KS == 64 ? ((row >> 1) & 7) : ((row >> 1) & 3);
}

// Issues the loads of an R-row slab into LDS byte address lds, shared by the
// NW waves of the workgroup. One load instruction covers RPI = 64 / CH rows;
// rows come in groups of G = NW * RPI (one round of instructions, the last
// round possibly partial): group u starts at the wave-uniform address base(u)
// (element k0 of its first row) and its row i (0 <= i < G) is read from row
// row_of(u, i) >= 0 of that base, rows being stride elements apart. Callers
// clamp rows past the end of their matrix inside row_of.
template <int R, int NW, int KS, class Base, class RowOf>
__device__ __forceinline__ void slab_issue(uint32_t lds, int wave, int stride, Base base, RowOf row_of) {
  constexpr int CH = KS / 8, RPI = 64 / CH, NI = R / RPI;
  static_assert(R % RPI == 0, "slab rows");
  const int lane = threadIdx.x & 63;
  const int i = wave * RPI + lane / CH;
#pragma unroll
  for (int u = 0; u < (NI + NW - 1) / NW; ++u) {
    const int ins = u * NW + wave;
    if (NI % NW != 0 && ins >= NI) break;  // wave-uniform: partial last round
    const int row = ins * RPI + lane / CH;
    const int chunk = (lane % CH) ^ slab_swz<KS>(row);
    const uint32_t voff = (uint32_t)(row_of(u, i) * stride + chunk * 8) * 2u;
    g2lds16_s(base(u), voff, lds + (uint32_t)ins * 1024u);
  }
}

// The per-lane half of slab_issue, for callers that fetch many slabs with
// the same rows: byte offset of this lane's 16-byte chunk for each of its
// load instructions (row_of and the swizzle do not depend on k). Slabs are
// then issued with slab_issue_planned, which only adds a per-slab base.
template <int R, int NW, int KS>
struct SlabPlan {
  static constexpr int CH = KS / 8, RPI = 64 / CH, NI = R / RPI, NU = (NI + NW - 1) / NW;
  uint32_t voff[NU];
};
template <int R, int NW, int KS, class RowOf>
__device__ __forceinline__ void slab_plan(SlabPlan<R, NW, KS>& pl, int wave, int stride, RowOf row_of) {
  using P = SlabPlan<R, NW, KS>;
  static_assert(R % P::RPI == 0, "slab rows");
  const int lane = threadIdx.x & 63;
  const int i = wave * P::RPI + lane / P::CH;
#pragma unroll
  for (int u = 0; u < P::NU; ++u) {
    const int ins = u * NW + wave;
    const int row = ins * P::RPI + lane / P::CH;
    const int chunk = (lane % P::CH) ^ slab_swz<KS>(row);
    pl.voff[u] = (uint32_t)(row_of(u, i) * stride + chunk * 8) * 2u;
  }
}
template <int R, int NW, int KS, class Base>
__device__ __forceinline__ void slab_issue_planned(uint32_t lds, int wave, const SlabPlan<R, NW, KS>& pl, Base base) {
  using P = SlabPlan<R, NW, KS>;
#pragma unroll
  for (int u = 0; u < P::NU; ++u) {
    const int ins = u * NW + wave;
    if (P::NI % NW != 0 && ins >= P::NI) break;  // wave-uniform: partial last round
    g2lds16_s(base(u), pl.voff[u], lds + (uint32_t)ins * 1024u);
  }
}

// 16-byte read of chunk `chunk` of slab row `row`.
template <int KS>
__device__ __forceinline__ u32x4 slab_read(const bf16_bits* lds, int row, int chunk) {
  return *reinterpret_cast<const u32x4*>(lds + row * KS + ((chunk ^ slab_swz<KS>(row)) << 3));
}

// Scheduling of one slab step of an MFMA main loop: the wave's NREAD LDS
// fragment reads first, then its NMFMA products (placed after them in the
// same basic block). Left to itself the scheduler keeps one or two fragments
// in registers and waits for each read in turn, one LDS round trip per group
// of four products; issued together the reads return while the first
// products run, and the waits count down (lgkmcnt(n-1), ..., 0).
template <int NREAD, int NMFMA>
__device__ __forceinline__ void reads_then_products() {
  __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);  // DS reads
  __builtin_amdgcn_sched_group_barrier(0x008, NMFMA, 0);  // MFMA
}

// Sum of squares of 8 bf16 values (exact fp32 products, fp32 accumulation).
__device__ __forceinline__ float sumsq8(const u32x4& v, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = lo_bf(v[i]), hi = hi_bf(v[i]);
    acc = __builtin_fmaf(lo, lo, acc);
    acc = __builtin_fmaf(hi, hi, acc);
  }
  return acc;
}

}  // namespace mea
