// Input RMSNorm + q/k/v/g projection + per-head q/k RMSNorm + rotary +
// sigmoid, as one MFMA GEMM with a fused prologue and epilogue.
//
// Replaces rms_norm_kernel (fast_triton_attn.py:12-34) and
// fused_qkvg_norm_rope_kernel (:36-144), and their backward-recompute
// variants (:181-332) when rx/rq/rk are requested.
//
// The product is computed transposed, D^T = W x^T: the A operand is a slice
// of the stacked weights of one head h (features; [Wq_h; Wv_h; Wk_h; Wg_h]
// for N = 64, [Wq_h; Wk_h] and [Wv_h; Wg_h] tiles for N = 128; for N = 32
// the same four of a head pair, [Wq; Wv; Wk; Wg] rows 64h .. 64h + 63), the B
// operand a tile of x rows (tokens). In the 16x16 accumulator layout a
// lane then holds one token and 4 consecutive features, so the head RMSNorm
// is an in-lane sum plus two lane exchanges, both members of every rotary
// pair (n, n^1) sit in one lane, and results leave as 8-byte stores.
//
// Tile: 256 features x 128 tokens. k-slabs of 32 stream through a 3-stage
// LDS ring filled by direct global->LDS loads, two slabs ahead, continuously
// across the tiles a workgroup walks (one barrier per slab). The block entry
// points pass k-slab-major copies of the weights (a slab of a tile's rows is
// one contiguous block, 1 KB per load instruction; from the row-major
// matrices each instruction gathers 16 rows of 64 bytes): 0.714 -> 0.680 ms
// per launch at B64 T4096 C512 H8 N64. Four waves of
// 128 features x 64 tokens (32 accumulators of 16x16): for N = 64 a wave owns
// one rotary projection (q or k) and one plain one (v or g) of its tokens, so
// the epilogue work is the same in every wave. Two workgroups share a CU, so
// one's epilogue can overlap the other's products.
//
// The input RMSNorm is never materialised: diag(1/rms(x)) commutes with the
// GEMM, so the row scale multiplies the fp32 accumulator. The row sums of
// squares come from the matrix cores: the diagonal of the 16x16 Gram matrix
// X X^T of each 16-token block, one extra MFMA per block and k-step on the x
// fragments already in registers (the two waves sharing a token half split
// the blocks).
#include <type_traits>

#include "kernels.h"
#include "slab.cuh"

namespace mea {

// Tile coordinates of logical tile L (head-minor order, so the tiles of one
// token tile are consecutive and share their x rows in L2).
struct ProjTile {
  int m0, h, f0;
};

constexpr int kProjBT = 128;  // tokens per tile
constexpr int kProjBF = 256;  // stacked-weight rows per tile
constexpr int kProjBK = 32;   // k per slab
constexpr int kProjStages = 3;

// N = 32: a tile holds the four projections of a head pair, h is the pair
// (heads 2h and 2h + 1; H is even).
template <int N>
__device__ __forceinline__ ProjTile proj_tile(int L, int H) {
  if constexpr (N == 32) {
    const int np = H / 2, tt = L / np;
    return ProjTile{tt * kProjBT, L - tt * np, 0};
  } else {
    constexpr int NFT = 4 * N / kProjBF;
    const int tt = L / (H * NFT), rem = L - tt * (H * NFT);
    return ProjTile{tt * kProjBT, rem / NFT, (rem % NFT) * kProjBF};
  }
}
// Tiles of one 128-token tile: 4 * H * N stacked-weight rows in tiles of 256.
__host__ __device__ __forceinline__ int proj_tiles_per_token_tile(int H, int N) { return H * 4 * N / kProjBF; }

// Persistent: workgroups walk tiles; workgroup w runs on XCD w % 8 and takes
// tiles from a contiguous range owned by that XCD, so the workgroups of one
// XCD work on neighbouring tiles at the same time.
// POS: every token reads its rotary row from p.tpos (packed sequences); a
// separate instantiation, so the (B, T) kernel keeps its code.
// PK: the epilogue reads the packed bf16 tables p.tabp (one 16-byte load per
// 4 features for both tables) instead of the fp32 f1 / f2 rows (two).
template <int N, bool POS, bool PK>
__global__ __launch_bounds__(256, 2) void qkvg_proj_kernel(ProjParams p) {
  constexpr int BT = kProjBT, BF = kProjBF, BK = kProjBK, NS = kProjStages;
  constexpr int STAGE = (BF + BT) * BK;
  constexpr int WF = 2, WT = 2;        // waves along features x tokens
  constexpr int FB = 8;                // 16-feature blocks per wave (128 features)
  constexpr int TB = BT / WT / 16;     // 16-token blocks per wave (4)
  constexpr int GB = TB / WF;          // Gram blocks per wave
  // N = 256 (HALF): a tile is one projection of one head and each wave holds
  // half of it (128 of its 256 features); the head RMSNorm and the row norms
  // then add the two waves' halves through LDS.
  constexpr bool HALF = N == 256;
  constexpr int NW128 = N < 128 ? N : 128;  // features of one projection in one wave
  constexpr int NPW = 128 / NW128;     // projections per wave
  constexpr int GF = NW128 / 16;       // feature blocks per projection in one wave
  constexpr int NSEG = BF / N;         // projections per stacked-weight slab
  constexpr int LOADS = (BF + BT) * BK / 8 / 64 / 4;  // load instructions per wave per slab
  __shared__ __attribute__((aligned(16))) bf16_bits smem[NS * STAGE];
  __shared__ float ssq_s[BT];
  __shared__ float xch[2][HALF ? 2 : 1][HALF ? BT : 1];  // [ss | norm][wf][token] (HALF)

  // Locals, not captures of the argument block: a lambda holding &p would
  // force the block into scratch memory.
  const bf16_bits* __restrict__ xg = p.x;
  const bf16_bits *wq = p.wq, *wk = p.wk, *wv = p.wv, *wg = p.wg;
  const int w_row = p.w_row;
  const int64_t w_slab = p.w_slab;
  const int M = p.M, C = p.C, H = p.H, T = p.T, HN = H * N;
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave % WF, wt = wave / WF;

  // This workgroup's tiles: start + j0 + i * nj for i < ntl.
  const int ntiles = ((M + BT - 1) / BT) * proj_tiles_per_token_tile(H, N);
  const int G = gridDim.x, xcd = blockIdx.x & 7, j0 = blockIdx.x >> 3;
  const int nj = (G - xcd + 7) >> 3;
  const int q8 = ntiles >> 3, r8 = ntiles & 7;
  const int start = xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8;
  const int cnt = xcd < r8 ? q8 + 1 : q8;
  const int ntl = j0 < cnt ? (cnt - j0 + nj - 1) / nj : 0;
  const int nk = C / BK;
  const int nslab = ntl * nk;  // slabs this workgroup streams, over all its tiles

  const uint32_t lds0 = lds_addr(smem);
  // Fetch cursor: slabs are issued in stream order, tile after tile. The
  // per-tile part of every load address (row-group bases, uniform; lane
  // offsets with the x rows clamped to the last token) is set when the
  // cursor enters a tile, so issuing a slab only adds its k offset.
  SlabPlan<BF, 4, BK> wplan;
  slab_plan(wplan, wave, p.w_row, [](int, int i) { return i; });
  SlabPlan<BT, 4, BK> xplan;
  constexpr int NUW = SlabPlan<BF, 4, BK>::NU, NUX = SlabPlan<BT, 4, BK>::NU;
  const bf16_bits* wbase[NUW];
  const bf16_bits* xbase[NUX];
  // iss_rot: the tile's head staggers its k order (slab kk = (ks + h) mod nk
  // is issued at step ks), so the 8 head tiles of a token tile that run
  // together on an XCD request each x slab at different times: the first
  // request fetches it into L2, the others hit (requested together, most
  // of them went past L2). The outputs are stored non-temporally so that
  // they do not evict the x slabs and weights from L2.
  int iss_ti = 0, iss_ks = 0, iss_st = 0, iss_rot = 0;
  auto plan_tile = [&](int ti) {
    const ProjTile tl = proj_tile<N>(start + j0 + ti * nj, H);
    iss_rot = tl.h % nk;
    if constexpr (N == 32) {
      // [q; v; k; g] of the head pair: rows 64h .. 64h + 63 of each matrix,
      // one 64-row load group each, so each wave's 128 features hold the
      // pair's rows of one rotary and one plain projection.
      const bf16_bits* wsel[4] = {wq, wv, wk, wg};
#pragma unroll
      for (int u = 0; u < NUW; ++u) wbase[u] = wsel[u] + (size_t)(tl.h * 64) * w_row;
    } else {
    const bf16_bits* wseg[NSEG];
    if (NSEG == 4) {
      // [q; v; k; g]: each wave's 128 features hold one rotary projection.
      wseg[0] = wq;
      wseg[NSEG > 1 ? 1 : 0] = wv;
      wseg[NSEG > 2 ? 2 : 0] = wk;
      wseg[NSEG > 3 ? 3 : 0] = wg;
    } else if (NSEG == 1) {
      // One projection per tile: q, k, v, g for f0 = 0, N, 2N, 3N.
      wseg[0] = tl.f0 == 0 ? wq : tl.f0 == N ? wk : tl.f0 == 2 * N ? wv : wg;
    } else {
      wseg[0] = tl.f0 == 0 ? wq : wv;
      wseg[NSEG > 1 ? 1 : 0] = tl.f0 == 0 ? wk : wg;
    }
    // Stacked-weight rows: each 64-row load group lies inside one projection.
#pragma unroll
    for (int u = 0; u < NUW; ++u) {
      const int seg = (64 * u) / N;  // compile-time after unrolling
      wbase[u] = wseg[seg] + (size_t)(tl.h * N + 64 * u - seg * N) * w_row;
    }
    }
#pragma unroll
    for (int u = 0; u < NUX; ++u) xbase[u] = xg + (size_t)min(tl.m0 + 64 * u, M - 1) * C;
    slab_plan(xplan, wave, C,
              [&](int u, int i) { return min(tl.m0 + 64 * u + i, M - 1) - min(tl.m0 + 64 * u, M - 1); });
  };
  auto issue_next = [&]() {
    const uint32_t lds = lds0 + (uint32_t)(iss_st * STAGE) * 2u;
    const int kk = iss_ks + iss_rot >= nk ? iss_ks + iss_rot - nk : iss_ks + iss_rot;
    const int k0 = kk * BK;
    slab_issue_planned<BF, 4, BK>(lds, wave, wplan, [&](int u) { return wbase[u] + kk * w_slab; });
    slab_issue_planned<BT, 4, BK>(lds + BF * BK * 2, wave, xplan, [&](int u) { return xbase[u] + k0; });
    iss_st = iss_st == NS - 1 ? 0 : iss_st + 1;
    if (++iss_ks == nk) {
      iss_ks = 0;
      if (++iss_ti < ntl) plan_tile(iss_ti);
    }
  };
  if (ntl > 0) plan_tile(0);

  f32x4 acc[FB][TB];
  f32x4 gram[GB];  // Gram blocks of token blocks GB*wf .. GB*wf+GB-1

  if (nslab > 0) issue_next();
  if (nslab > 1) issue_next();
  int cmp_st = 0;  // stage of the slab being multiplied
  // Largest squared row norm of the wave's rotary projection over all its
  // tiles (wave wf holds q for wf = 0, k for wf = 1, in every rotary tile;
  // with N = 256 every wave sees whole q and k rows: nmax for q, nmax_k for k),
  // published once after the last tile.
  float nmax = 0.f, nmax_k = 0.f;
  for (int ti = 0; ti < ntl; ++ti) {
    const ProjTile tl = proj_tile<N>(start + j0 + ti * nj, H);
#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = zero4();
#pragma unroll
    for (int i = 0; i < GB; ++i) gram[i] = zero4();

    for (int ks = 0; ks < nk; ++ks) {
      const int q = ti * nk + ks;
      // Slab q has landed once at most the next slab's loads are pending.
      if (q + 1 < nslab)
        __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);  // vmcnt(LOADS)
      else
        wait_vmcnt0();
      __syncthreads();
      if (q + 2 < nslab) issue_next();
      const bf16_bits* As = smem + cmp_st * STAGE;
      cmp_st = cmp_st == NS - 1 ? 0 : cmp_st + 1;
      const bf16_bits* Bs = As + BF * BK;
      bf16x8 af[FB], bfr[TB];
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) af[fb] = as_frag(slab_read<BK>(As, wf * 128 + fb * 16 + c16, g));
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) bfr[tb] = as_frag(slab_read<BK>(Bs, wt * (TB * 16) + tb * 16 + c16, g));
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
      reads_then_products<FB + TB, FB * TB + GB>();
    }

    // Rotary table rows of the wave's tokens are fetched ahead of their use
    // and before the stores that precede it: a load waits for every memory
    // operation issued before it (vmcnt counts stores too), so a table row
    // fetched after a block's stores would wait for their acknowledgement.
    const int m0 = tl.m0, h = tl.h;
    const int b0 = m0 / T, t0 = m0 - b0 * T;
    const bool tile_whole = m0 + BT <= M && t0 + BT <= T;
    const bool has_rot = N <= 64 || (N == 128 ? tl.f0 == 0 : tl.f0 < 2 * N);  // the wave holds q or k
    const int col = HALF ? wf * 128 : 0;  // first head column of the wave's features
    auto tab_row = [&](int tb) {
      const int m = m0 + wt * (TB * 16) + tb * 16 + c16;
      if (POS) return min(max(p.tpos[min(m, M - 1)], 0), p.t_max - 1);
      return tile_whole ? t0 + (m - m0) : (m < M ? m - (m / T) * T : 0);
    };
    // N = 64: one slot of table rows, filled for block 0 at the start of the
    // epilogue and refilled, feature block by feature block, for block tb + 1
    // as block tb consumes it. N = 128 (twice the rows) reads each feature
    // block's rows just before use.
    constexpr bool PREF = N == 64;
    constexpr bool SLOT32 = PREF && !PK, SLOTW = PREF && PK;
    f32x4 tab1[SLOT32 ? GF : 1], tab2[SLOT32 ? GF : 1];
    u32x4 tabw[SLOTW ? GF : 1];
    // Features col + 16j + 4g .. +3 of block tb's token: fp32 row of f, or
    // the packed word (row t, features n..n+3) = 16-byte word t * N/4 + n/4.
    auto tab_at = [&](const float* f, int tb, int j) {
      return *reinterpret_cast<const f32x4*>(f + (size_t)tab_row(tb) * N + col + 16 * j + 4 * g);
    };
    auto tabw_at = [&](int tb, int j) {
      return *reinterpret_cast<const u32x4*>(p.tabp + 2 * ((size_t)tab_row(tb) * N + col + 16 * j + 4 * g));
    };
    auto load_tab_j = [&](int tb, int j) {
      if (SLOTW) {
        tabw[SLOTW ? j : 0] = tabw_at(tb, j);
      } else if (SLOT32) {
        tab1[SLOT32 ? j : 0] = tab_at(p.f1, tb, j);
        tab2[SLOT32 ? j : 0] = tab_at(p.f2, tb, j);
      }
    };
    // (f1, f2) of those features, from the slot (N = 64) or from memory.
    auto tab_vals = [&](int tb, int j, f32x4& a1, f32x4& a2) {
      if (PK) {
        const u32x4 w = SLOTW ? tabw[SLOTW ? j : 0] : tabw_at(tb, j);
        a1 = f32x4{lo_bf(w[0]), hi_bf(w[0]), lo_bf(w[1]), hi_bf(w[1])};
        a2 = f32x4{lo_bf(w[2]), hi_bf(w[2]), lo_bf(w[3]), hi_bf(w[3])};
      } else {
        a1 = SLOT32 ? tab1[SLOT32 ? j : 0] : tab_at(p.f1, tb, j);
        a2 = SLOT32 ? tab2[SLOT32 ? j : 0] : tab_at(p.f2, tb, j);
      }
    };

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
    // multiple of 128) needs no per-row division or bounds checks.
    const float inv_c = 1.0f / (float)C, inv_n = p.inv_n, eps = p.eps;
    // Everything below is instantiated twice: for a whole tile (one sequence,
    // inside M: no per-row division or bounds test) and for the rest.
    auto epilogue = [&](auto whole_tag) {
    constexpr bool whole = decltype(whole_tag)::value;
    int trow[TB], brow[TB];
    bool ok[TB];
    float rx[TB];
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
      rx[tb] = rsqrtf(ssq_s[tlr] * inv_c + eps);
      if (p.rx != nullptr && h == 0 && tl.f0 == 0 && wf == 0 && g == 0 && ok[tb]) p.rx[m] = rx[tb];
    }

    if (PREF && has_rot) {
#pragma unroll
      for (int j = 0; j < GF; ++j) load_tab_j(0, j);
    }

    // Output staging: the stage of the tile's last slab is free until the
    // next tile's third slab is issued (after that tile's first barrier).
    // Each wave owns a 16-token x (NPW * N) block of it, rows of N + 8
    // elements, filled with 8-byte writes from the accumulator layout and
    // drained as 16-byte row chunks, so every store covers whole rows.
    constexpr int SP = NW128 + 8;
    bf16_bits* stg = smem + ((ti * nk + nk - 1) % NS) * STAGE + wave * (NPW * 16 * SP);
    // Projection (0 q, 1 k, 2 v, 3 g) of the wave's gi-th N-feature block,
    // wave-uniform. For N = 64 the stacked rows are [q; v; k; g], so every
    // wave owns one rotary projection and one plain one and the epilogue work
    // is the same in all four waves; for N = 128 a tile is (q, k) or (v, g).
    // N = 32: blocks 0, 1 are the rotary projection of heads 2h, 2h + 1 and
    // blocks 2, 3 the plain one.
    auto proj_of = [&](int gi) {
      return N == 32   ? (gi < 2 ? wf : 2 + wf)
             : N == 64 ? (gi == 0 ? wf : 2 + wf)
             : N == 128 ? (tl.f0 == 0 ? 0 : 2) + wf
                        : tl.f0 / N;
    };
    // Head of the wave's gi-th N-feature block.
    auto head_of = [&](int gi) { return N == 32 ? 2 * h + (gi & 1) : h; };
    constexpr int CPR = NW128 / 8;           // 16-byte chunks per staged row
    // Drains the staged block of projection gi for token block tb into
    // dstp + b * bstride + t * tstride.
    // The lane index the store addresses derive from, opaque to the compiler
    // inside each tile: hoisted out of the tile loop, those lane-constant
    // 64-bit offsets would stay live across the main loop and spill.
    int lane_d = lane;
    asm volatile("" : "+v"(lane_d));
    auto drain = [&](int gi, int tb, bf16_bits* dstp, size_t bstride, size_t tstride) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
      bf16_bits* tile0 = dstp + (size_t)b0 * bstride + (size_t)t0 * tstride;  // whole tiles
#pragma unroll
      for (int it = 0; it < 16 * CPR / 64; ++it) {
        const int id = lane_d + 64 * it, row = id / CPR, ch = id % CPR;
        const int tl_row = wt * (TB * 16) + tb * 16 + row;
        const u32x4 val = *reinterpret_cast<const u32x4*>(stg + (gi * 16 + row) * SP + ch * 8);
        if (whole) {
          st16_nt(tile0 + (uint32_t)(tl_row * (int)tstride + ch * 8), val);
        } else if (m0 + tl_row < M) {
          const int m = m0 + tl_row, bb = m / T, tt = m - bb * T;
          st16_nt(dstp + (size_t)bb * bstride + (size_t)tt * tstride + ch * 8, val);
        }
      }
    };
    // Head RMSNorm over N (fast_triton_attn.py:102-106) of a = rx * acc:
    // 1/rms(a) = rsqrt(rx^2 mean(acc^2) + eps), one scale rx / rms(a) per
    // row. The rotary (:132-141) then acts on the fp32 normalised values:
    // out[n] = qh[n] f1[t,n] + qh[n^1] f2[t,n]; q rows are stored times
    // qscale. The largest squared row norm is recorded for the attention's
    // logit bound. `next` >= 0 names the block whose table rows refill the
    // slot.
    auto rot_block = [&](int tb, int gi, int next) {
      // Fenced, so the refill loads stay behind the reads of the slot.
      __builtin_amdgcn_sched_barrier(0);
      const int pj = proj_of(gi);
      const int t = ok[tb] ? trow[tb] : 0;
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < GF; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) ss += acc[gi * GF + j][tb][r] * acc[gi * GF + j][tb][r];
      ss += shfl_xor(ss, 16);
      ss += shfl_xor(ss, 32);
      const int tlr = wt * (TB * 16) + tb * 16 + c16;
      if (HALF) {
        // Add the other wave's half of the row (every wave of the workgroup
        // runs the same blocks, so the barrier is uniform).
        if (g == 0) xch[0][HALF ? wf : 0][HALF ? tlr : 0] = ss;
        __syncthreads();
        ss += xch[0][HALF ? wf ^ 1 : 0][HALF ? tlr : 0];
      }
      const float rr = rsqrtf(rx[tb] * rx[tb] * ss * inv_n + eps);
      const float sc = rx[tb] * rr * (pj == 0 ? p.qscale : 1.0f);  // folded into the table rows
      if (ok[tb] && g == 0 && (!HALF || wf == 0)) {
        float* rstat = pj == 0 ? p.rq : p.rk;
        if (rstat != nullptr) rstat[((size_t)brow[tb] * H + head_of(gi)) * T + t] = rr;
      }
      float nrm = 0.f;
#pragma unroll
      for (int j = 0; j < GF; ++j) {
        const int n = 16 * j + 4 * g;
        f32x4 a1, a2;
        tab_vals(tb, j, a1, a2);
        a1 *= sc;
        a2 *= sc;
        if (next >= 0) load_tab_j(next, j);
        const f32x4& a = acc[gi * GF + j][tb];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[r] = a[r] * a1[r] + a[r ^ 1] * a2[r];
          nrm += o[r] * o[r];
        }
        *reinterpret_cast<u32x2*>(stg + (gi * 16 + c16) * SP + n) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
      nrm += shfl_xor(nrm, 16);
      nrm += shfl_xor(nrm, 32);
      if (HALF) {
        if (g == 0) xch[1][HALF ? wf : 0][HALF ? tlr : 0] = nrm;
        __syncthreads();
        nrm += xch[1][HALF ? wf ^ 1 : 0][HALF ? tlr : 0];
        if (pj == 0)
          nmax = fmaxf(nmax, nrm);
        else
          nmax_k = fmaxf(nmax_k, nrm);
      } else {
        nmax = fmaxf(nmax, nrm);
      }
    };
    // v = rx acc; g = sigmoid(rx acc) = 1 / (1 + exp2(-log2(e) rx acc)).
    auto plain_block = [&](int tb, int gi) {
      __builtin_amdgcn_sched_barrier(0);
      const int pj = proj_of(gi);
      const float kx = pj == 2 ? rx[tb] : -kLog2e * rx[tb];
#pragma unroll
      for (int j = 0; j < GF; ++j) {
        const f32x4& a = acc[gi * GF + j][tb];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = pj == 2 ? a[r] * kx : __builtin_amdgcn_rcpf(1.0f + fast_exp2(a[r] * kx));
        *reinterpret_cast<u32x2*>(stg + (gi * 16 + c16) * SP + 16 * j + 4 * g) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
    };
    auto drain_pj = [&](int gi, int tb) {
      const int pj = proj_of(gi), hg = head_of(gi);
      if (pj < 2)
        drain(gi, tb, (pj == 0 ? p.q : p.k) + (size_t)hg * T * N + col, (size_t)H * T * N, (size_t)N);
      else if (pj == 2)
        drain(gi, tb, p.v + (size_t)hg * T * N + col, (size_t)H * T * N, (size_t)N);
      else
        drain(gi, tb, p.sig + (size_t)hg * N + col, (size_t)T * HN, (size_t)HN);
    };
    if (N == 64) {
      // Plain (v or g) and rotary (q or k) blocks interleaved as P0 P1 R0 P2
      // R1 P3 R2 R3: block 0's table rows arrive during P0 and P1, and each
      // rotary block refills the slot with the next block's rows, which then
      // have a plain block's time to land (the table loads are latency-bound;
      // all plain blocks first and the rotary ones after ran 1.7% slower).
      plain_block(0, 1);
      drain_pj(1, 0);
      plain_block(1, 1);
      drain_pj(1, 1);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        rot_block(tb, 0, tb + 1 < TB ? tb + 1 : -1);
        drain_pj(0, tb);
        if (tb + 2 < TB) {
          plain_block(tb + 2, 1);
          drain_pj(1, tb + 2);
        }
      }
    } else if (N == 32) {
      // Per token block: the two heads' rotary blocks, then their plain ones.
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          if (gi < 2)
            rot_block(tb, gi, -1);
          else
            plain_block(tb, gi);
          drain_pj(gi, tb);
        }
      }
    } else {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        if (has_rot)
          rot_block(tb, 0, -1);
        else
          plain_block(tb, 0);
        drain_pj(0, tb);
      }
    }
    };
    if (tile_whole)
      epilogue(std::true_type{});
    else
      epilogue(std::false_type{});
  }
  if (p.qk_norm2 != nullptr && ntl > 0) {
    auto publish = [&](float v, int slot) {
      v = fmaxf(v, xor1(v));
      v = fmaxf(v, xor2(v));
      v = fmaxf(v, shfl_xor(v, 4));
      v = fmaxf(v, shfl_xor(v, 8));
      // Non-negative floats order like their bit patterns.
      if (lane == 0) atomicMax(reinterpret_cast<unsigned int*>(p.qk_norm2) + slot, __float_as_uint(v));
    };
    if (HALF) {
      publish(nmax, 0);
      publish(nmax_k, 1);
    } else {
      publish(nmax, wf);
    }
  }
}

// Workgroups per device for the persistent kernels: one per CU.
int persistent_grid(int tiles, int per_cu) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return tiles < per_cu * cus[dev] ? tiles : per_cu * cus[dev];
}

template <int N>
static void launch_proj_n(const ProjParams& p, int G, hipStream_t s) {
  const bool pos = p.tpos != nullptr, pk = p.tabp != nullptr;
  if (!pos && !pk)
    hipLaunchKernelGGL((qkvg_proj_kernel<N, false, false>), dim3(G), dim3(256), 0, s, p);
  else if (!pos)
    hipLaunchKernelGGL((qkvg_proj_kernel<N, false, true>), dim3(G), dim3(256), 0, s, p);
  else if (!pk)
    hipLaunchKernelGGL((qkvg_proj_kernel<N, true, false>), dim3(G), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((qkvg_proj_kernel<N, true, true>), dim3(G), dim3(256), 0, s, p);
}

hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s) {
  if (N == 32 && p.H % 2 != 0) return hipErrorInvalidValue;  // tiles hold head pairs
  const int G = persistent_grid(((p.M + kProjBT - 1) / kProjBT) * proj_tiles_per_token_tile(p.H, N), 2);
  if (N == 32)
    launch_proj_n<32>(p, G, s);
  else if (N == 64)
    launch_proj_n<64>(p, G, s);
  else if (N == 128)
    launch_proj_n<128>(p, G, s);
  else if (N == 256)
    launch_proj_n<256>(p, G, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

namespace {

// One thread per 4-feature group i = t * N/4 + n/4 of rows 0 .. rows-1:
// (f1[4i .. 4i+3], f2[4i .. 4i+3]) rounded to bf16 into word i.
__global__ __launch_bounds__(256) void rotary_pack_kernel(const f32x4* f1, const f32x4* f2, int groups, u32x4* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= groups) return;
  const f32x4 a = f1[i], b = f2[i];
  out[i] = u32x4{pack2(a[0], a[1]), pack2(a[2], a[3]), pack2(b[0], b[1]), pack2(b[2], b[3])};
}

}  // namespace

hipError_t launch_rotary_pack(const float* f1, const float* f2, int rows, int N, bf16_bits* tabp, hipStream_t s) {
  const int groups = rows * (N / 4);
  hipLaunchKernelGGL(rotary_pack_kernel, dim3((groups + 255) / 256), dim3(256), 0, s,
                     reinterpret_cast<const f32x4*>(f1), reinterpret_cast<const f32x4*>(f2), groups,
                     reinterpret_cast<u32x4*>(tabp));
  return hipGetLastError();
}

namespace {

// One thread per token: the sequence holding token m by binary search over
// the nseq + 1 offsets cu (cu[0] = 0, increasing).
__global__ __launch_bounds__(256) void token_positions_kernel(const int* cu, int nseq, int M, int* tpos) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (m >= M) return;
  int lo = 0, hi = nseq;  // cu[lo] <= m < cu[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= m)
      lo = mid;
    else
      hi = mid;
  }
  tpos[m] = m - cu[lo];
}

}  // namespace

hipError_t launch_token_positions(const int* cu, int nseq, int M, int* tpos, hipStream_t s) {
  hipLaunchKernelGGL(token_positions_kernel, dim3((M + 255) / 256), dim3(256), 0, s, cu, nseq, M, tpos);
  return hipGetLastError();
}

}  // namespace mea
