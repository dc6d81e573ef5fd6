// LDS k-slabs for the GEMM-shaped kernels (gfx950).
//
// A slab holds R operand rows x 64 bf16 of the reduction dimension k
// (128 bytes = 8 chunks of 16 bytes per row). Chunk c of row r sits at chunk
// slot c ^ ((r >> 1) & 7): two rows fill one 256-byte LDS bank line, so the
// 16 rows that one 16-lane group reads at one chunk index land in 16 distinct
// 16-byte bank groups.
//
// Slabs are filled straight from global memory with global_load_lds_dwordx4:
// one wave instruction writes 1 KB (8 rows) of LDS, lane L filling slot L & 7
// of row L >> 3; the swizzle is applied by choosing which global chunk each
// lane fetches, so every 8 lanes still read one contiguous 128-byte row
// segment.
#pragma once

#include "common.cuh"

namespace mea {

constexpr int kSlabK = 64;  // k elements per slab row

__device__ __forceinline__ int slab_swz(int row) { return (row >> 1) & 7; }

// Issues the loads of an R-row slab into LDS byte address lds, shared by the
// NW waves of the workgroup (R a multiple of 8 NW). Rows come in groups of
// 8 NW: group u starts at the wave-uniform address base(u) (element k0 of its
// first row) and its row i (0 <= i < 8 NW) is read from row row_of(u, i) >= 0
// of that base, rows being stride elements apart. Callers clamp rows past the
// end of their matrix inside row_of.
template <int R, int NW, class Base, class RowOf>
__device__ __forceinline__ void slab_issue(uint32_t lds, int wave, int stride, Base base, RowOf row_of) {
  static_assert(R % (8 * NW) == 0, "slab rows");
  const int lane = threadIdx.x & 63;
  const int i = wave * 8 + (lane >> 3);
#pragma unroll
  for (int u = 0; u < R / (8 * NW); ++u) {
    const int row = u * 8 * NW + i;
    const int chunk = (lane & 7) ^ slab_swz(row);
    const uint32_t voff = (uint32_t)(row_of(u, i) * stride + chunk * 8) * 2u;
    g2lds16_s(base(u), voff, lds + (uint32_t)(u * NW + wave) * 1024u);
  }
}

// 16-byte read of chunk `chunk` (0..7) of slab row `row`.
__device__ __forceinline__ u32x4 slab_read(const bf16_bits* lds, int row, int chunk) {
  return *reinterpret_cast<const u32x4*>(lds + row * kSlabK + ((chunk ^ slab_swz(row)) << 3));
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
