// Causal flash attention forward on gfx950 MFMA.
//
// Replaces the aten._scaled_dot_product_flash_attention call of the
// reference (fast_triton_attn.py:425-444): softmax(q k^T * scale) v with
// scale = 1/sqrt(N) (:426), causal, no dropout, returning the output and the
// natural-log row normaliser (lse).
//
// One workgroup = one (batch, head) and BQ = 4*QW queries; wave w owns QW =
// 32 consecutive queries (for N = 64, 128 registers: four workgroups per
// CU; 64 queries per wave, two per SIMD with a software-pipelined tile,
// ran 10% slower). Keys stream through LDS in tiles of 64 (N = 128: 32, so
// that three workgroups fit the LDS; at 168 registers that ran 7% faster
// than two workgroups with 64-key tiles), loaded straight from global memory
// into a swizzled row-major layout (global_load_lds, double-buffered, one
// barrier per tile). Each tile is consumed in 32-key steps with
// v_mfma_f32_32x32x16_bf16:
//   S^T = K Q^T     A = K rows from LDS, B = Q^T held in registers;
//                   the query index sits on the lane, so every softmax
//                   statistic is a per-lane value (plus one exchange with
//                   lane ^ 32, which holds the other 16 keys of the step);
//   O^T += V^T P^T  A = V^T read from the row-major V tile with the
//                   transposing ds_read_b64_tr_b16, B = P^T straight from
//                   the S^T accumulator registers (keys in the order the
//                   accumulator holds them, matched by the V^T rows read).
//
// Two softmax forms:
//  - fixed offset: q and k come out of a per-head RMSNorm, so every logit is
//    bounded by |q| |k|. When the caller passes the row-norm bounds, q is
//    stored in log2 units (sl2e == 1) and the bound is at most kFixedBound,
//    P = exp2(q.k) needs no running maximum at all: P lies in
//    [2^-60, 2^60], far inside the fp32/bf16 range, and O = sum P v / sum P
//    is the same quotient the running-maximum form computes. Per score that
//    leaves one exp2, one add and half a convert.
//  - online: the running maximum is only raised when a new score exceeds it
//    by more than 2^8 (in exp2 units), so the costly rescale of the output
//    accumulator is skipped on almost every step.
// The output is written straight into the (B, T, H*N) layout the output
// projection reads (the reference's gate_repack layout, :171-176).
#include <type_traits>

#include "common.cuh"
#include "kernels.h"

namespace mea {

// VARLEN: packed sequences (p.cu); a workgroup's (b, h, query block) becomes
// (sequence, h, query block) and every row index is taken relative to the
// sequence's first token.
template <int N, bool VARLEN>
__global__ __launch_bounds__(256, N <= 64 ? 4 : N == 128 ? 3 : 1) void attn_fwd_kernel(AttnFwdParams p) {
  constexpr int QW = 32;  // queries per wave
  constexpr int QB = QW / 32;            // 32-query MFMA blocks per wave
  constexpr int BQ = 4 * QW;             // queries per workgroup
  constexpr int BKV = N == 128 ? 32 : 64;  // keys per LDS tile
  constexpr int CH = N / 8;              // 16-byte chunks per row
  constexpr int KS = N / 16;             // MFMA k-steps over the head dim
  constexpr int DB = N / 32;             // 32-wide output column blocks
  constexpr int TILE = BKV * N;          // elements of one K or V tile
  constexpr int LOADS = TILE / 8 / 256;  // 16-byte loads per thread per tile
  constexpr float TAU = 8.f;
  constexpr int OP = N + 8;              // output staging pitch
  constexpr int SMEM = 4 * TILE > 4 * QW * OP ? 4 * TILE : 4 * QW * OP;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SMEM];  // [stage][K | V], then output staging

  // Each XCD walks whole heads (heaviest query block of a head first), so
  // the K/V tiles of a head are fetched once into that XCD's L2.
  int T, bh, qi, b, hd;
  size_t head_row0, tok_row0;  // first row of the (b, h) sequence in (B*H, T) / (B*T) order
  if constexpr (!VARLEN) {
    T = p.T;
    const int nqb = (T + BQ - 1) / BQ;
    const int lid = attn_item(blockIdx.x, p.B * p.H * nqb, nqb, N <= 64 ? 3 : 1);
    bh = lid / nqb;
    qi = nqb - 1 - lid % nqb;
    b = bh / p.H;
    hd = bh % p.H;
    head_row0 = (size_t)bh * T;
    tok_row0 = (size_t)b * T;
  } else {
    const int nqb = (p.max_len + BQ - 1) / BQ;
    const int lid = attn_item(blockIdx.x, p.nseq * p.H * nqb, nqb, N <= 64 ? 3 : 1);
    bh = lid / nqb;  // sequence-major (s, h)
    qi = nqb - 1 - lid % nqb;
    b = bh / p.H;
    hd = bh % p.H;
    // Offsets clamped to [0, total]: a malformed list cannot index outside.
    const int start = min(max(p.cu[b], 0), p.T);
    T = min(max(p.cu[b + 1], start), p.T) - start;
    head_row0 = (size_t)hd * p.T + start;
    tok_row0 = (size_t)start;
    if (qi * BQ >= T) return;  // past this sequence's end: uniform, before any barrier
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, h = lane >> 5;
  const int q0w = qi * BQ + wave * QW;
  const int kv_end = min(T, qi * BQ + BQ);
  const size_t head_off = head_row0 * N;
  const bf16_bits* kg = p.k + head_off;
  const bf16_bits* vg = p.v + head_off;

  bool fixed = false;
  if (p.qk_norm2 != nullptr && p.sl2e == 1.0f) {
    const float bound = sqrtf(p.qk_norm2[0] * p.qk_norm2[1]) * 1.01f;
    fixed = bound <= kFixedBound;
  }

  // Q^T fragments (B operand): lane holds query q0w + 32qb + c, d = 16ks + 8h.
  bf16x8 qf[QB][KS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int t = min(q0w + 32 * qb + c, T - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[qb][ks] = as_frag(ld16(p.q + head_off + (size_t)t * N + 16 * ks + 8 * h));
  }

  // Tile loads: lane L of load u fills 16-byte slot L of row block u*4+wave;
  // its row and swizzled chunk are fixed, so a whole tile is fetched from a
  // wave-uniform base (row j0) plus a lane-constant byte offset. Only a tile
  // that runs past the sequence end takes per-lane clamped addresses.
  uint32_t ld_row[LOADS], ld_off[LOADS];
#pragma unroll
  for (int u = 0; u < LOADS; ++u) {
    const int slot = (u * 4 + wave) * 64 + lane;
    const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
    ld_row[u] = row;
    ld_off[u] = (uint32_t)(row * N + cc * 8) * 2u;
  }
  const uint32_t smem_b = lds_addr(smem);
  auto issue_tile = [&](int j0, int stage) {
    const uint32_t kt = smem_b + (uint32_t)(stage * 2 * TILE) * 2u;
    if (j0 + BKV <= T) {
      const bf16_bits* kb = kg + (size_t)j0 * N;
      const bf16_bits* vb = vg + (size_t)j0 * N;
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        g2lds16_s(kb, ld_off[u], kt + (uint32_t)(u * 4 + wave) * 1024u);
        g2lds16_s(vb, ld_off[u], kt + (uint32_t)(TILE * 2) + (uint32_t)(u * 4 + wave) * 1024u);
      }
    } else {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int row = min(j0 + (int)ld_row[u], T - 1);
        const uint32_t off = ld_off[u] + (uint32_t)((row - j0 - (int)ld_row[u]) * N) * 2u;
        g2lds16_s(kg + (size_t)j0 * N, off, kt + (uint32_t)(u * 4 + wave) * 1024u);
        g2lds16_s(vg + (size_t)j0 * N, off, kt + (uint32_t)(TILE * 2) + (uint32_t)(u * 4 + wave) * 1024u);
      }
    }
  };

  float m_i[QB], l_i[QB];
  f32x16 o[QB][DB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = fixed ? 0.f : -INFINITY;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[qb][db] = zero16();
  }

  // Lane-constant parts of the fragment addresses (elements). The swizzle of
  // a row depends on row & 15 only, so the step (32 rows) and k-step (16
  // rows) parts of an address are plain offsets.
  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * h + (i16 >> 2);             // + 16*kstep + 8*x (+ 32*st)
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);  // + 32*db
  int koff[KS], voff[2][DB];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = swz_off<CH>(c, 16 * ks + 8 * h);
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int db = 0; db < DB; ++db) voff[x][db] = swz_off<CH>(tr_row + 8 * x, 32 * db + tr_col);

  // Row sums of P on the matrix core: a 16x16x32 MFMA with B = the P^T
  // fragment of one 16-key MFMA step sees, in lane 16g + n, query n + 16(g&1)
  // and the keys of half g >> 1. With A row m selecting the groups with
  // g & 1 == m, D row 0 (1) of column n is the sum of P over those 16 keys for
  // query n (n + 16): lanes 0..15, registers 0 and 1.
  const uint32_t selw = (i16 == (g16 & 1)) ? 0x3F803F80u : 0u;
  const bf16x8 sel = as_frag(u32x4{selw, selw, selw, selw});
  f32x4 lsum[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) lsum[qb] = zero4();

  // One 32-key step of every query block of this wave. FIXED: exp2 of the
  // raw logit; otherwise the online form. MASK: the step touches the causal
  // diagonal or the end of the sequence.
  auto step = [&](const bf16_bits* ks_t, const bf16_bits* vs_t, int st, int kb0, auto fixed_tag, auto mask_tag) {
    constexpr bool FIXED = decltype(fixed_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
    bf16x8 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[ks] = as_frag(*reinterpret_cast<const u32x4*>(ks_t + st * 32 * N + koff[ks]));
    // N <= 64: the V^T fragments of the step are read with the K fragments,
    // before the S products, and the scheduling fence keeps them there (N =
    // 64: 128 registers, still four workgroups per CU): read next to the PV
    // products that use them, each read's LDS round trip stalled the wave
    // (the kernel ran 1.9% slower). N = 128 and 256 have no registers to
    // spare and read them at the products.
    constexpr bool VEARLY = N <= 64;
    auto vread = [&](int kst, int db) {
      const bf16_bits* vr = vs_t + (st * 32 + 16 * kst) * N;
      return frag_from2(lds_read_tr4(vr + voff[0][db]), lds_read_tr4(vr + voff[1][db]));
    };
    bf16x8 vfr[VEARLY ? 2 : 1][VEARLY ? DB : 1];
    if constexpr (VEARLY) {
#pragma unroll
      for (int kst = 0; kst < 2; ++kst)
#pragma unroll
        for (int db = 0; db < DB; ++db) vfr[kst][db] = vread(kst, db);
      __builtin_amdgcn_sched_barrier(0);
    }
    bf16x8 pf[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qb0 = q0w + 32 * qb;
      if (MASK && kb0 > qb0 + 31) {
        // The whole step is in this query block's future: contributes nothing.
        pf[qb][0] = pf[qb][1] = as_frag(u32x4{0u, 0u, 0u, 0u});
        continue;
      }
      f32x16 s = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s = mfma32(kf[ks], qf[qb][ks], s);
      if (MASK) {
        const int qq = qb0 + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb0 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key > qq || key >= T) s[i] = -INFINITY;
        }
      }
      float ls = 0.f;
      if (FIXED) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = fast_exp2(s[i]);
      } else {
        float mx = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float ms = mx * p.sl2e;
        const bool up = ms > m_i[qb] + TAU;
        if (__any(up)) {
          const float mn = up ? ms : m_i[qb];
          const float alpha = fast_exp2(m_i[qb] - mn);
          l_i[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[qb][db] *= alpha;
          m_i[qb] = mn;
        }
        const float nm = -m_i[qb];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = fast_exp2(__builtin_fmaf(s[i], p.sl2e, nm));
          s[i] = e;
          ls += e;
        }
      }
      if (!FIXED) l_i[qb] += ls;
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack2(s[8 * kst + 2 * e], s[8 * kst + 2 * e + 1]);
        pf[qb][kst] = as_frag(w);
        if (FIXED) lsum[qb] = mfma(sel, pf[qb][kst], lsum[qb]);
      }
    }
    // O^T += V^T P^T, two 16-key MFMA steps.
#pragma unroll
    for (int kst = 0; kst < 2; ++kst) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x8 vf = VEARLY ? vfr[VEARLY ? kst : 0][VEARLY ? db : 0] : vread(kst, db);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (MASK && kb0 > q0w + 32 * qb + 31) continue;
          o[qb][db] = mfma32(vf, pf[qb][kst], o[qb][db]);
        }
      }
    }
  };

  // Tiles wholly below a wave's first query (and inside the sequence) need
  // no mask for that wave and run in a branch-free loop; the rest of the
  // diagonal region and a ragged sequence end follow in a second loop. The
  // split point is per wave: every wave still passes one barrier per tile,
  // so the two loops together keep the waves in step.
  auto main_loop = [&](auto fixed_tag) {
    const int nkv = (kv_end + BKV - 1) / BKV;
    const int nfull = min(nkv, min(q0w + 1, T) / BKV);
    issue_tile(0, 0);
    wait_vmcnt0();  // also retires the Q fragment loads
    __syncthreads();
    int j = 0;
    for (; j < nfull; ++j) {
      if (j + 1 < nkv) issue_tile((j + 1) * BKV, (j + 1) & 1);
      const bf16_bits* ks_t = smem + (j & 1) * 2 * TILE;
      const bf16_bits* vs_t = ks_t + TILE;
#pragma unroll
      for (int st = 0; st < BKV / 32; ++st) step(ks_t, vs_t, st, j * BKV + 32 * st, fixed_tag, std::false_type{});
      wait_vmcnt0();
      __syncthreads();
    }
    for (; j < nkv; ++j) {
      if (j + 1 < nkv) issue_tile((j + 1) * BKV, (j + 1) & 1);
      const bf16_bits* ks_t = smem + (j & 1) * 2 * TILE;
      const bf16_bits* vs_t = ks_t + TILE;
#pragma unroll
      for (int st = 0; st < BKV / 32; ++st) {
        const int kb0 = j * BKV + st * 32;
        if (kb0 <= q0w + QW - 1) step(ks_t, vs_t, st, kb0, fixed_tag, std::true_type{});
      }
      wait_vmcnt0();
      __syncthreads();
    }
  };
  if (fixed) {
    main_loop(std::true_type{});
    // Row sums from the MFMA accumulators (lanes 0..15), spread so that both
    // halves h of each query column see the whole sum in l_i.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float v0 = __shfl(lsum[qb][0], c & 15, 64), v1 = __shfl(lsum[qb][1], c & 15, 64);
      l_i[qb] = h == 0 ? (c < 16 ? v0 : v1) : 0.f;
    }
  } else {
    main_loop(std::false_type{});
  }

  // Normalise, write lse and stage O^T (lane = query) as rows for 16-byte stores.
  bf16_bits* stg = smem + wave * QW * OP;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l = l_i[qb] + __shfl_xor(l_i[qb], 32, 64);
    const float inv = 1.0f / l;
    const int qq = q0w + 32 * qb + c;
    if (p.lse != nullptr && h == 0 && qq < T) p.lse[head_row0 + qq] = (m_i[qb] + __log2f(l)) * kLn2;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x16& a = o[qb][db];
        const u32x2 w = {pack2(a[4 * r4] * inv, a[4 * r4 + 1] * inv), pack2(a[4 * r4 + 2] * inv, a[4 * r4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(stg + (32 * qb + c) * OP + 32 * db + 8 * r4 + 4 * h) = w;
      }
  }
  __syncthreads();
  const size_t HN = (size_t)p.H * N;
#pragma unroll
  for (int it = 0; it < QW * CH / 64; ++it) {
    const int id = lane + 64 * it, row = id / CH, dc = id % CH;
    const int t = q0w + row;
    if (t < T) {
      const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * OP + dc * 8);
      st16(p.o + (tok_row0 + t) * HN + (size_t)hd * N + dc * 8, val);
    }
  }
}

hipError_t launch_attn_fwd(const AttnFwdParams& p, int N, hipStream_t s) {
  const int BQ = 128;
  const bool var = p.cu != nullptr;
  const int G = var ? p.nseq * p.H * ((p.max_len + BQ - 1) / BQ) : p.B * p.H * ((p.T + BQ - 1) / BQ);
  if (N == 32 && !var)
    hipLaunchKernelGGL((attn_fwd_kernel<32, false>), dim3(G), dim3(256), 0, s, p);
  else if (N == 32)
    hipLaunchKernelGGL((attn_fwd_kernel<32, true>), dim3(G), dim3(256), 0, s, p);
  else if (N == 64 && !var)
    hipLaunchKernelGGL((attn_fwd_kernel<64, false>), dim3(G), dim3(256), 0, s, p);
  else if (N == 64)
    hipLaunchKernelGGL((attn_fwd_kernel<64, true>), dim3(G), dim3(256), 0, s, p);
  else if (N == 128 && !var)
    hipLaunchKernelGGL((attn_fwd_kernel<128, false>), dim3(G), dim3(256), 0, s, p);
  else if (N == 128)
    hipLaunchKernelGGL((attn_fwd_kernel<128, true>), dim3(G), dim3(256), 0, s, p);
  else if (N == 256 && !var)
    hipLaunchKernelGGL((attn_fwd_kernel<256, false>), dim3(G), dim3(256), 0, s, p);
  else if (N == 256)
    hipLaunchKernelGGL((attn_fwd_kernel<256, true>), dim3(G), dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mea
