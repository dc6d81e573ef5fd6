// Causal flash attention backward on gfx950 MFMA, fused with the backward of
// the per-head q/k RMSNorm and rotary and with the input-RMSNorm row scale.
//
// Replaces aten._scaled_dot_product_flash_attention_backward
// (fast_triton_attn.py:586-596) and the q/k gradient chain after it
// (:603-634). The chain is computed exactly for any rotary table with
// invertible 2x2 pair blocks, instead of the reference's rotated-space
// shortcut, which is exact only for orthonormal tables:
//   q = R qh with R the per-pair block [[f1[2i], f2[2i]], [f2[2i+1], f1[2i+1]]]
//   dqh = R^T dq
//   da_q = rq * (dqh - qh * (dqh . qh) / N)
// qh is recovered from the stored rotated q by inverting R per pair, so the
// recompute pass does not have to keep the pre-rotation values.
// Table gradients (fast_triton_attn.py:622-639), when asked for:
//   dF1[t, n] = sum over batch and heads of dq[n] qh[n] + dk[n] kh[n],
//   dF2[t, n] likewise with qh[n^1], kh[n^1]
// come from table_grad_kernel after both kernels: it rebuilds dq and dk from
// the stored da_q, da_k, q, k and the per-row dot products (dqh . qh) the
// kernels leave, and sums over batch and heads in a fixed order.
//
// Two kernels (deterministic, no atomics on dQ):
//   dq kernel   : one workgroup per (b, h, 4 waves of queries), streams key
//                 tiles. S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T -
//                 delta), dQ^T += K^T dS^T.
//   dkdv kernel : one workgroup per (b, h, 4 waves of keys), streams query
//                 tiles. S = Q K^T, dP = dO V^T, dV^T += dO^T P,
//                 dK^T += Q^T dS.
// Operands that reduce over a sequence index (K^T, Q^T, dO^T) are read from
// row-major LDS tiles with the transposing ds_read_b64_tr_b16.
#include <type_traits>

#include "common.cuh"
#include "kernels.h"

namespace mea {

// Row-wise tail for one wave: 32 staged rows of fp32 gradient (pitch FP)
// for sequence positions t0 .. t0+31 of head (b, h).
//   rotary != 0 : head RMSNorm + rotary backward of q or k (xrot = q or k
//                 as stored, xrot * xscale the rotated rows themselves).
//   rotary == 0 : plain copy (v).
// Output row t goes to out[(head_row0 + t)*N ...] (head-major, like q, k, v),
// scaled by rx[tok_row0 + t]. out may be xrot itself: every lane writes only
// the 16 bytes it has read, after reading them, and rows past T are not
// written.
// dot_out (rotary rows, or null): row t's dot product dqh . qh goes to
// dot_out[head_row0 + t] (the table gradients rebuild dq from it).
template <int N>
__device__ __forceinline__ void head_row_bwd(const float* stg, int FP, int t0, const AttnBwdParams& p, int T,
                                             size_t tok_row0, size_t head_row0, bool rotary,
                                             const bf16_bits* xrot, float xscale, const float* rstat,
                                             bf16_bits* out, float* dot_out) {
  constexpr int CPR = N / 8, RPP = 64 / CPR;
  // Passes, and passes whose global operands are fetched together (N = 64:
  // all four, one memory round trip per call).
  constexpr int NP = 32 / RPP, PB = N == 64 ? NP : 2;
  static_assert(NP % PB == 0, "pass batches");
  const int lane = threadIdx.x & 63;
#pragma unroll 1
  for (int p0 = 0; p0 < NP; p0 += PB) {
    // Every global operand of the batch's rows is requested first: one
    // memory round trip per batch instead of one per pass.
    u32x4 xw[PB];
    f32x4 f1w[PB][2], f2w[PB][2];
    float rxw[PB], rrw[PB];
#pragma unroll
    for (int k = 0; k < PB; ++k) {
      const int row = (p0 + k) * RPP + lane / CPR, dc = lane % CPR;
      const int t = t0 + row, tc = t < T ? t : T - 1;
      rxw[k] = p.rx[tok_row0 + tc];
      if (rotary) {
        xw[k] = ld16(xrot + (head_row0 + tc) * N + dc * 8);
        const float* f1r = p.f1 + (size_t)tc * N + dc * 8;
        const float* f2r = p.f2 + (size_t)tc * N + dc * 8;
        f1w[k][0] = *reinterpret_cast<const f32x4*>(f1r);
        f1w[k][1] = *reinterpret_cast<const f32x4*>(f1r + 4);
        f2w[k][0] = *reinterpret_cast<const f32x4*>(f2r);
        f2w[k][1] = *reinterpret_cast<const f32x4*>(f2r + 4);
        rrw[k] = rstat[head_row0 + tc];
      }
    }
#pragma unroll
    for (int k = 0; k < PB; ++k) {
      const int row = (p0 + k) * RPP + lane / CPR, dc = lane % CPR;
      const int t = t0 + row;
      const bool valid = t < T;
      float dv[8];
      {
        const f32x4 a = *reinterpret_cast<const f32x4*>(stg + row * FP + dc * 8);
        const f32x4 c = *reinterpret_cast<const f32x4*>(stg + row * FP + dc * 8 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { dv[i] = a[i]; dv[4 + i] = c[i]; }
      }
      const float rxv = rxw[k];
      float res[8];
      if (rotary) {
        float xv[8], a1[8], a2[8];
        unpack8(xw[k], xv);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] *= xscale;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a1[e] = f1w[k][0][e];
          a1[4 + e] = f1w[k][1][e];
          a2[e] = f2w[k][0][e];
          a2[4 + e] = f2w[k][1][e];
        }
        float xh[8], dh[8], dot = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const float det = a1[i] * a1[i + 1] - a2[i] * a2[i + 1];
          // v_rcp_f32 (1 ulp): the IEEE division cost 0.8% of dQ. A zero pair
          // block (the padding columns of a narrow head given zero tables)
          // maps its rows to zero, where the forward put them, not to
          // 0 * inf = NaN.
          const float inv = det != 0.f ? __builtin_amdgcn_rcpf(det) : 0.f;
          xh[i] = (a1[i + 1] * xv[i] - a2[i] * xv[i + 1]) * inv;
          xh[i + 1] = (a1[i] * xv[i + 1] - a2[i + 1] * xv[i]) * inv;
          dh[i] = a1[i] * dv[i] + a2[i + 1] * dv[i + 1];
          dh[i + 1] = a1[i + 1] * dv[i + 1] + a2[i] * dv[i];
          dot += dh[i] * xh[i] + dh[i + 1] * xh[i + 1];
        }
        // Reduce the dot product over the CPR lanes of this row.
        dot += xor1(dot);
        dot += xor2(dot);
        if (CPR >= 8) dot += shfl_xor(dot, 4);
        if (CPR >= 16) dot += shfl_xor(dot, 8);
        if (CPR == 32) dot += shfl_xor(dot, 16);
        const float rr = rrw[k];
        const float sc = rxv * rr, cf = dot * p.inv_n;
#pragma unroll
        for (int i = 0; i < 8; ++i) res[i] = sc * (dh[i] - xh[i] * cf);
        // Every lane of the row holds the same sum (a butterfly of commutative
        // adds), so all of them store it: no lane test, no extra register.
        if (dot_out != nullptr && valid) dot_out[head_row0 + t] = dot;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) res[i] = rxv * dv[i];
      }
      if (valid) st16(out + (head_row0 + t) * N + dc * 8, pack8(res));
    }
  }
}

// ---------------------------------------------------------------------------
// dQ
//
// One workgroup = one (batch, head) and BQ = 4*QW queries; wave w owns QW =
// 32 consecutive queries whose q and dO rows stay in registers as the B
// operands of
//   S^T = K Q^T   and   dP^T = V dO^T      (A = K, V rows from LDS)
// on v_mfma_f32_32x32x16_bf16. The query index sits on the lane, and the
// accumulators start from the lane's row statistics (stored q is in log2
// units): -lse*log2e for S^T and -delta for dP^T, four copies of each per
// query in a wave-private LDS area, read straight into the accumulator
// registers (four 16-byte reads per product). They come out as log2 P and
// dP - delta, and dS^T = P^T (dP^T - delta) is one exp2 and one multiply per
// score, already the B operand (k = key) of
//   dQ^T += K^T dS^T
// whose A operand K^T is read from the row-major K tile with the transposing
// ds_read_b64_tr_b16. Key tiles of 64 stream through LDS (global_load_lds,
// double-buffered, one barrier per tile); tiles wholly below a wave's first
// query run in a branch-free loop, the rest of the diagonal region after it.
// For N = 64 three workgroups share a CU (163 registers): 64 queries per wave
// (two blocks sharing every K/V fragment) held two per SIMD ran 4.4% slower.
// (The statistics were earlier added by one more MFMA k-block per product,
// their exact bf16 terms against (1, 1, 1) selectors; the LDS start values
// save those MFMAs: dQ -0.9%, dK/dV -3%.)
// ---------------------------------------------------------------------------
template <int N, bool VARLEN>
__global__ __launch_bounds__(256, N <= 64 ? 3 : N == 256 ? 1 : 2) void attn_bwd_dq_kernel(AttnBwdParams p) {
  constexpr int QW = 32;                 // queries per wave
  constexpr int QB = QW / 32;            // 32-query MFMA blocks per wave
  constexpr int BQ = 4 * QW;             // queries per workgroup
  constexpr int BKV = 64;                // keys per LDS tile
  constexpr int CH = N / 8, KS = N / 16, DB = N / 32;
  constexpr int TILE = BKV * N;
  constexpr int LOADS = TILE / 8 / 256;
  constexpr int FP = N + 4;  // fp32 staging pitch
  constexpr int SM_LOOP = 4 * TILE * 2;  // bytes: [stage][K | V]
  constexpr int SM_STAT = 4 * QB * 2 * 4 * 32 * 16;  // bytes: [wave][qb][lse | delta][copy][query] x 4
  constexpr int SM_OUT = 4 * QW * FP * 4;
  constexpr int SMEM = SM_LOOP + SM_STAT > SM_OUT ? SM_LOOP + SM_STAT : SM_OUT;
  __shared__ __attribute__((aligned(16))) unsigned char smem_raw[SMEM];
  bf16_bits* smem = reinterpret_cast<bf16_bits*>(smem_raw);

  // Each XCD walks whole heads (heaviest query block first), so the K/V
  // tiles of a head are fetched once into that XCD's L2. VARLEN: packed
  // sequences (p.cu), rows relative to the sequence's first token.
  int T, qi, b, h_first;
  size_t hrow_base, hrow_step, tok_row0;  // head hd's rows start at hrow_base + hd * hrow_step
  const int nh = p.H;                     // heads per grid row
  if constexpr (!VARLEN) {
    T = p.T;
    const int nqb = (T + BQ - 1) / BQ;
    const int lid = attn_item(blockIdx.x, p.B * nh * nqb, nqb, N <= 64 ? 3 : 1);
    const int bh = lid / nqb;
    qi = nqb - 1 - lid % nqb;
    b = bh / nh;
    h_first = bh % nh;
    hrow_base = (size_t)b * p.H * T;
    hrow_step = (size_t)T;
    tok_row0 = (size_t)b * T;
  } else {
    const int nqb = (p.max_len + BQ - 1) / BQ;
    const int lid = attn_item(blockIdx.x, p.nseq * nh * nqb, nqb, N <= 64 ? 3 : 1);
    const int bh = lid / nqb;
    qi = nqb - 1 - lid % nqb;
    b = bh / nh;
    h_first = bh % nh;
    // Offsets clamped to [0, total]: a malformed list cannot index outside.
    const int start = min(max(p.cu[b], 0), p.T);
    T = min(max(p.cu[b + 1], start), p.T) - start;
    hrow_base = (size_t)start;
    hrow_step = (size_t)p.T;
    tok_row0 = (size_t)start;
    if (qi * BQ >= T) return;  // past this sequence's end: uniform, before any barrier
  }
  {
    const int hd = h_first;
    const size_t head_row0 = hrow_base + (size_t)hd * hrow_step;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h = lane >> 5;
    const int q0w = qi * BQ + wave * QW;
    const int kv_end = min(T, qi * BQ + BQ);
    const size_t head_off = head_row0 * N;
    const bf16_bits* kg = p.k + head_off;
    const bf16_bits* vg = p.v + head_off;

    // q^T and dO^T fragments (B operands), and the start values of the S^T
    // and dP^T accumulators of the lane's query q0w + 32qb + c: -lse*log2e
    // (written by the lanes with h == 0) and -delta (h == 1), each as four
    // copies of a 16-byte row [qb][lse | delta][copy][query], in a
    // wave-private LDS area the loop does not touch. Four distinct copies keep
    // the four reads that fill an accumulator from being merged into one read
    // and twelve register moves.
    bf16x8 qf[QB][KS], df[QB][KS];
    f32x4* statq = reinterpret_cast<f32x4*>(smem_raw + SM_LOOP) + wave * QB * 256;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int t = min(q0w + 32 * qb + c, T - 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const size_t off = head_off + (size_t)t * N + 16 * ks + 8 * h;
        qf[qb][ks] = as_frag(ld16(p.q + off));
        df[qb][ks] = as_frag(ld16(p.dO + off));
      }
      // One load per lane (a selected pointer, not two loads under a branch).
      const float sl = (h == 0 ? p.lse : p.delta)[head_row0 + t];
      const float sv = h == 0 ? -sl * kLog2e : -sl;
#pragma unroll
      for (int j = 0; j < 4; ++j) statq[qb * 256 + h * 128 + j * 32 + c] = f32x4{sv, sv, sv, sv};
    }

    // Tile loads: lane L of load u fills 16-byte slot L of row block u*4+wave;
    // its row and swizzled chunk are fixed, so a whole tile is fetched from a
    // wave-uniform base (row j0) plus a lane-constant byte offset, and only a
    // tile that runs past the sequence end takes per-lane clamped addresses.
    uint32_t ld_off[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int slot = (u * 4 + wave) * 64 + lane;
      const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
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
          const int slot = (u * 4 + wave) * 64 + lane;
          const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
          const size_t off = (size_t)min(j0 + row, T - 1) * N + cc * 8;
          g2lds16(kg + off, kt + (uint32_t)(u * 4 + wave) * 1024u);
          g2lds16(vg + off, kt + (uint32_t)(TILE * 2) + (uint32_t)(u * 4 + wave) * 1024u);
        }
      }
    };

    f32x16 dq[QB][DB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int db = 0; db < DB; ++db) dq[qb][db] = zero16();

    // Lane-constant parts of the fragment addresses (elements): a row's
    // swizzle depends on row & 15 only, so the step and k-step parts of an
    // address are plain offsets.
    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * h + (i16 >> 2);
    const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);
    int koff[KS], toff[2][DB];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = swz_off<CH>(c, 16 * ks + 8 * h);
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int db = 0; db < DB; ++db) toff[x][db] = swz_off<CH>(tr_row + 8 * x, 32 * db + tr_col);

    // One 32-key step of every query block of this wave. MASK: the step
    // touches the causal diagonal or the end of the sequence.
    auto step = [&](const bf16_bits* ks_t, const bf16_bits* vs_t, int st, int kb0, auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      bf16x8 kf[KS], vf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[ks] = as_frag(*reinterpret_cast<const u32x4*>(ks_t + st * 32 * N + koff[ks]));
        vf[ks] = as_frag(*reinterpret_cast<const u32x4*>(vs_t + st * 32 * N + koff[ks]));
      }
      bf16x8 sf[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int qb0 = q0w + 32 * qb;
        if (MASK && kb0 > qb0 + 31) {
          sf[qb][0] = sf[qb][1] = as_frag(u32x4{0u, 0u, 0u, 0u});
          continue;
        }
        f32x16 s, dp;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 a = statq[qb * 256 + j * 32 + c], b = statq[qb * 256 + 128 + j * 32 + c];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[4 * j + e] = a[e];
            dp[4 * j + e] = b[e];
          }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = mfma32(kf[ks], qf[qb][ks], s);
          dp = mfma32(vf[ks], df[qb][ks], dp);
        }
        const int qq = qb0 + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float pv = fast_exp2(s[i]);
          if (MASK) {
            const int key = kb0 + 8 * (i >> 2) + 4 * h + (i & 3);
            pv = (key > qq || key >= T) ? 0.f : pv;
          }
          s[i] = pv * dp[i];
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = pack2(s[8 * kst + 2 * e], s[8 * kst + 2 * e + 1]);
          sf[qb][kst] = as_frag(w);
        }
        // Keeps the next query block's S and dP accumulators from going live
        // before this block's are consumed (they do not fit in registers
        // together with the resident q, dO and dQ fragments).
        if (QB > 1) __builtin_amdgcn_sched_barrier(0);
      }
      // dQ^T += K^T dS^T, two 16-key MFMA steps.
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16_bits* kr = ks_t + (st * 32 + 16 * kst) * N;
          const bf16x8 kt = frag_from2(lds_read_tr4(kr + toff[0][db]), lds_read_tr4(kr + toff[1][db]));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            if (MASK && kb0 > q0w + 32 * qb + 31) continue;
            dq[qb][db] = mfma32(kt, sf[qb][kst], dq[qb][db]);
          }
        }
      }
    };

    const int nkv = (kv_end + BKV - 1) / BKV;
    // Branch-free loop over the tiles wholly below this wave's first query and
    // inside the sequence; the split point is per wave (one barrier per tile
    // in either loop keeps the waves in step).
    const int nfull = min(nkv, min(q0w + 1, T) / BKV);
    issue_tile(0, 0);
    wait_vmcnt0();  // also retires the q/dO fragment loads
    __syncthreads();
    int j = 0;
    for (; j < nfull; ++j) {
      if (j + 1 < nkv) issue_tile((j + 1) * BKV, (j + 1) & 1);
      const bf16_bits* ks_t = smem + (j & 1) * 2 * TILE;
      step(ks_t, ks_t + TILE, 0, j * BKV, std::false_type{});
      step(ks_t, ks_t + TILE, 1, j * BKV + 32, std::false_type{});
      wait_vmcnt0();
      __syncthreads();
    }
    for (; j < nkv; ++j) {
      if (j + 1 < nkv) issue_tile((j + 1) * BKV, (j + 1) & 1);
      const bf16_bits* ks_t = smem + (j & 1) * 2 * TILE;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int kb0 = j * BKV + st * 32;
        if (kb0 <= q0w + QW - 1) step(ks_t, ks_t + TILE, st, kb0, std::true_type{});
      }
      wait_vmcnt0();
      __syncthreads();
    }

    // Stage dQ (times the softmax scale) as fp32 rows, then the q chain.
    float* stg = reinterpret_cast<float*>(smem_raw) + wave * QW * FP;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x16& a = dq[qb][db];
          const f32x4 v = {a[4 * r4], a[4 * r4 + 1], a[4 * r4 + 2], a[4 * r4 + 3]};
          *reinterpret_cast<f32x4*>(stg + (32 * qb + c) * FP + 32 * db + 8 * r4 + 4 * h) = v * p.scale;
        }
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
      head_row_bwd<N>(stg + 32 * qb * FP, FP, q0w + 32 * qb, p, T, tok_row0, head_row0, true, p.q,
                      1.0f / p.qscale, p.rq, p.daq, p.dotq);
  }
}

// ---------------------------------------------------------------------------
// dK, dV
//
// One workgroup = one (batch, head) and BKV = 4*KW keys; wave w owns KW = 32
// consecutive keys whose K rows stay in registers and whose V rows sit in a
// per-wave LDS block laid out as the lane's fragments, as the B operands of
//   S  = Q K^T   and   dP = dO V^T        (A = Q, dO rows from LDS)
// on v_mfma_f32_32x32x16_bf16, whose accumulators start from the query
// statistics (stored q is in log2 units): -lse*log2e and -delta of each
// query tile sit in LDS as fp32 rows, and a lane's 16 accumulator elements
// (queries 8j + 4h + 0..3, j = 0..3) are four 16-byte reads of each row. The
// accumulators come out as log2 P and dP - delta. The key index sits on the
// lane, so P and dS = P (dP - delta) are already the B operands (k = query) of
//   dV^T += dO^T P   and   dK^T += Q^T dS
// whose A operands dO^T, Q^T are read from the same row-major LDS tiles with
// the transposing ds_read_b64_tr_b16. Query tiles (64 queries for N = 64,
// 32 for N >= 128) stream through LDS (global_load_lds, double-buffered, one
// barrier per tile), from the last tile down to the one holding the block's
// first key (causal). For N = 64 three workgroups share a CU (168 registers,
// 50 KB of LDS each): the same work at two per CU, with V^T in registers and
// two 32-query steps interleaved for instruction-level parallelism, ran 7.4%
// slower. For N = 128 two workgroups share a CU (252 registers, 66 KB of LDS
// each); with 64-query tiles (97 KB of LDS) only one fitted, one wave per
// SIMD, and the kernel ran 36% longer. N = 256 (and N = 128 with table
// gradients, whose extra state would spill at 256 registers) runs one wave
// per SIMD.
// ---------------------------------------------------------------------------
template <int N, bool VARLEN>
__global__ __launch_bounds__(256, N <= 64 ? 3 : N == 128 ? 2 : 1) void attn_bwd_dkdv_kernel(AttnBwdParams p) {
  constexpr int KW = 32;                 // keys per wave
  constexpr int KB = KW / 32;            // 32-key MFMA blocks per wave
  static_assert(KB == 1, "one 32-key block per wave");
  constexpr int BKV = 4 * KW;            // keys per workgroup
  constexpr int BQ = N >= 128 ? 32 : 64;  // queries per LDS tile (N >= 128: 32, so that Q, dO and V^T of two
                                         // workgroups fit LDS at N = 128, and of one at N = 256)
  constexpr int CH = N / 8, KS = N / 16, DB = N / 32;
  constexpr int TILE = BQ * N;
  constexpr int LOADS = TILE / 8 / 256;
  constexpr int FP = N + 4;  // fp32 staging pitch
  constexpr int SM_LOOP = 2 * 2 * TILE * 2 + 2 * 2 * BQ * 4;  // bytes
  constexpr int SM_V = 4 * KS * 64 * 16;  // bytes: each wave's V^T fragments, [wave][ks][lane]
  constexpr int SM_OUT = 4 * 32 * FP * 4;
  constexpr int SMEM = SM_LOOP + SM_V > SM_OUT ? SM_LOOP + SM_V : SM_OUT;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  bf16_bits* tiles = reinterpret_cast<bf16_bits*>(smem);           // [stage][Q | dO]
  // [stage][-lse*log2e | -delta][query]: the accumulator start values of the
  // tile's queries.
  float* statf = reinterpret_cast<float*>(smem + 2 * 2 * TILE * 2);
  u32x4* vown = reinterpret_cast<u32x4*>(smem + SM_LOOP);

  // Each XCD walks whole heads, the key block that sees the most queries
  // first, so the Q/dO tiles of a head are shared in one L2. VARLEN: packed
  // sequences (p.cu), rows relative to the sequence's first token.
  int T, ki, b, h_first;
  size_t hrow_base, hrow_step, tok_row0;  // head hd's rows start at hrow_base + hd * hrow_step
  const int nh = p.H;                     // heads per grid row
  if constexpr (!VARLEN) {
    T = p.T;
    const int nkb = (T + BKV - 1) / BKV;
    const int lid = attn_item(blockIdx.x, p.B * nh * nkb, nkb, N <= 64 ? 3 : 1);
    const int bh = lid / nkb;
    ki = lid % nkb;
    b = bh / nh;
    h_first = bh % nh;
    hrow_base = (size_t)b * p.H * T;
    hrow_step = (size_t)T;
    tok_row0 = (size_t)b * T;
  } else {
    const int nkb = (p.max_len + BKV - 1) / BKV;
    const int lid = attn_item(blockIdx.x, p.nseq * nh * nkb, nkb, N <= 64 ? 3 : 1);
    const int bh = lid / nkb;
    ki = lid % nkb;
    b = bh / nh;
    h_first = bh % nh;
    // Offsets clamped to [0, total]: a malformed list cannot index outside.
    const int start = min(max(p.cu[b], 0), p.T);
    T = min(max(p.cu[b + 1], start), p.T) - start;
    hrow_base = (size_t)start;
    hrow_step = (size_t)p.T;
    tok_row0 = (size_t)start;
    if (ki * BKV >= T) return;  // past this sequence's end: uniform, before any barrier
  }
  {
    const int hd = h_first;
    const size_t head_row0 = hrow_base + (size_t)hd * hrow_step;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, h = lane >> 5;
    const int k0 = ki * BKV, kw0 = k0 + wave * KW;
    const size_t head_off = head_row0 * N;
    const bf16_bits* qg = p.q + head_off;
    const bf16_bits* dg = p.dO + head_off;

    // K^T, V^T fragments (B operands): lane holds key kw0 + 32kb + c, d = 16ks + 8h.
    bf16x8 kf[KB][KS];
    u32x4* vw = vown + (size_t)wave * KS * 64;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const size_t row = head_off + (size_t)min(kw0 + 32 * kb + c, T - 1) * N;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[kb][ks] = as_frag(ld16(p.k + row + 16 * ks + 8 * h));
        vw[ks * 64 + lane] = ld16(p.v + row + 16 * ks + 8 * h);
      }
    }

    float st_l = 0.f, st_d = 0.f;
    // Tile loads as in the dQ kernel: a whole tile from a uniform base plus a
    // lane-constant byte offset, a tile past the sequence end clamped per
    // lane. The LDS destination comes from a uniform wave index: held in a
    // vector register instead, it spilled from the main loop.
    uint32_t ld_off[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int slot = (u * 4 + wave) * 64 + lane;
      const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
      ld_off[u] = (uint32_t)(row * N + cc * 8) * 2u;
    }
    const uint32_t tiles_b = lds_addr(tiles);
    auto issue_tile = [&](int q0, int stage) {
      const uint32_t qt = tiles_b + (uint32_t)(stage * 2 * TILE) * 2u;
      const int wu = __builtin_amdgcn_readfirstlane(wave);
      if (q0 + BQ <= T) {
        const bf16_bits* qb = qg + (size_t)q0 * N;
        const bf16_bits* db = dg + (size_t)q0 * N;
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
          g2lds16_s(qb, ld_off[u], qt + (uint32_t)(u * 4 + wu) * 1024u);
          g2lds16_s(db, ld_off[u], qt + (uint32_t)(TILE * 2) + (uint32_t)(u * 4 + wu) * 1024u);
        }
      } else {
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
          const int slot = (u * 4 + wave) * 64 + lane;
          const int row = slot / CH, cc = (slot % CH) ^ chunk_swz<CH>(row);
          const size_t off = (size_t)min(q0 + row, T - 1) * N + cc * 8;
          g2lds16(qg + off, qt + (uint32_t)(u * 4 + wu) * 1024u);
          g2lds16(dg + off, qt + (uint32_t)(TILE * 2) + (uint32_t)(u * 4 + wu) * 1024u);
        }
      }
      if (tid < BQ) {
        const size_t t = head_row0 + min(q0 + tid, T - 1);
        st_l = p.lse[t];
        st_d = p.delta[t];
      }
    };
    // Called after wait_vmcnt0(): st_l / st_d are consumed only once every load
    // of the tile has landed, so no wait is placed inside the prefetch.
    auto publish_stats = [&](int stage) {
      if (tid < BQ) {
        statf[stage * 2 * BQ + tid] = -st_l * kLog2e;
        statf[stage * 2 * BQ + BQ + tid] = -st_d;
      }
    };

    f32x16 dv[KB][DB], dk[KB][DB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int db = 0; db < DB; ++db) dv[kb][db] = dk[kb][db] = zero16();

    // Lane-constant parts of the fragment addresses (elements); a row's swizzle
    // depends on row & 15 only.
    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * h + (i16 >> 2);
    const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);
    // (Recomputed per use rather than held: registers are what bound the
    // workgroups per CU.)
    auto kofs = [&](int ks) { return swz_off<CH>(c, 16 * ks + 8 * h); };
    auto tofs = [&](int x, int db) { return swz_off<CH>(tr_row + 8 * x, 32 * db + tr_col); };

    // Query tiles are walked from the last one down: every workgroup of a
    // head then reads the same tile at about the same time (walking up from
    // each block's own diagonal, they read as many different tiles at once as
    // there are key blocks), which cut this kernel's HBM reads from 2.74 to
    // 2.27 GB per launch at B64 T4096 C512 H8 N64.
    const int nq = (T - k0 + BQ - 1) / BQ;
    issue_tile(k0 + (nq - 1) * BQ, 0);
    wait_vmcnt0();
    publish_stats(0);
    __syncthreads();
    // One query tile. MASKED: the tile may touch the causal diagonal or the
    // sequence end (per-step tests and masks); the tiles between hold only
    // full steps for every wave and run without any test.
    auto tile = [&](int it, auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const int q0 = k0 + (nq - 1 - it) * BQ;
      if (it + 1 < nq) issue_tile(q0 - BQ, (it + 1) & 1);
      const bf16_bits* qt = tiles + (it & 1) * 2 * TILE;
      const bf16_bits* dt = qt + TILE;
      const float* stf = statf + (it & 1) * 2 * BQ;
      // One 32-query step in three parts: S and dP (MFMA), P and dS (exp2,
      // multiply, convert; DIAG steps also mask key > query and query >= T),
      // then the dV and dK updates (MFMA).
      struct Sub {
        f32x16 s, dp;
        bf16x8 pb[2], sb[2];
      };
      auto sdp = [&](int sub, Sub& u) {
        // Start values: element 4j + e holds query qs0 + 8j + 4h + e.
        const float* sl = stf + 32 * sub + 4 * h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(sl + 8 * j);
          const f32x4 b = *reinterpret_cast<const f32x4*>(sl + BQ + 8 * j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            u.s[4 * j + e] = a[e];
            u.dp[4 * j + e] = b[e];
          }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 qa = as_frag(*reinterpret_cast<const u32x4*>(qt + 32 * sub * N + kofs(ks)));
          const bf16x8 da = as_frag(*reinterpret_cast<const u32x4*>(dt + 32 * sub * N + kofs(ks)));
          u.s = mfma32(qa, kf[0][ks], u.s);
          u.dp = mfma32(da, as_frag(vw[ks * 64 + lane]), u.dp);
        }
      };
      auto soft = [&](int sub, Sub& u, auto diag_tag) {
        constexpr bool DIAG = decltype(diag_tag)::value;
        const int qs0 = q0 + 32 * sub, key = kw0 + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float pv = fast_exp2(u.s[i]);
          if (DIAG) {
            const int q = qs0 + 8 * (i >> 2) + 4 * h + (i & 3);
            pv = (key > q || q >= T) ? 0.f : pv;
          }
          u.s[i] = pv;
          u.dp[i] = pv * u.dp[i];
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
          u32x4 w, v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[e] = pack2(u.s[8 * kst + 2 * e], u.s[8 * kst + 2 * e + 1]);
            v[e] = pack2(u.dp[8 * kst + 2 * e], u.dp[8 * kst + 2 * e + 1]);
          }
          u.pb[kst] = as_frag(w);
          u.sb[kst] = as_frag(v);
        }
      };
      auto kv = [&](int sub, const Sub& u) {
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int rb = (32 * sub + 16 * kst) * N;
            const int o0 = rb + tofs(0, db), o1 = rb + tofs(1, db);
            const bf16x8 dT = frag_from2(lds_read_tr4(dt + o0), lds_read_tr4(dt + o1));
            const bf16x8 qT = frag_from2(lds_read_tr4(qt + o0), lds_read_tr4(qt + o1));
            dv[0][db] = mfma32(dT, u.pb[kst], dv[0][db]);
            dk[0][db] = mfma32(qT, u.sb[kst], dk[0][db]);
          }
        }
      };
#pragma unroll
      for (int sub = 0; sub < BQ / 32; ++sub) {
        const int qs0 = q0 + 32 * sub;
        if (MASKED && (qs0 + 31 < kw0 || qs0 >= T)) continue;  // wave-uniform: nothing to add
        Sub u;
        sdp(sub, u);
        if (MASKED && (qs0 < kw0 + KW - 1 || qs0 + 31 >= T))
          soft(sub, u, std::true_type{});
        else
          soft(sub, u, std::false_type{});
        kv(sub, u);
        // Keeps the next step's S and dP from being scheduled into this one
        // (their registers would not fit beside this step's).
        if (!MASKED) __builtin_amdgcn_sched_barrier(0);
      }
      wait_vmcnt0();
      if (it + 1 < nq) publish_stats((it + 1) & 1);
      __syncthreads();
    };
    // Tiles it < nfull lie wholly above the block's keys (q0 >= k0 + BKV);
    // the first one (the highest queries) may run past the sequence end.
    const int nfull = nq - BKV / BQ;
    int it = 0;
    if (nfull > 0 && (T - k0) % BQ != 0) tile(it++, std::true_type{});
    for (; it < nfull; ++it) tile(it, std::false_type{});
    for (; it < nq; ++it) tile(it, std::true_type{});

    // Epilogue per 32-key block: stage dV (then dK * scale) as fp32 rows and run
    // the row-wise tails (rx scale; k RMSNorm + rotary backward for dK).
    float* stg = reinterpret_cast<float*>(smem) + wave * 32 * FP;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 v = {dv[kb][db][4 * r4], dv[kb][db][4 * r4 + 1], dv[kb][db][4 * r4 + 2], dv[kb][db][4 * r4 + 3]};
          *reinterpret_cast<f32x4*>(stg + c * FP + 32 * db + 8 * r4 + 4 * h) = v;
        }
      __syncthreads();
      head_row_bwd<N>(stg, FP, kw0 + 32 * kb, p, T, tok_row0, head_row0, false, nullptr, 1.0f, nullptr, p.dav,
                      nullptr);
      __syncthreads();
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 v = {dk[kb][db][4 * r4], dk[kb][db][4 * r4 + 1], dk[kb][db][4 * r4 + 2], dk[kb][db][4 * r4 + 3]};
          *reinterpret_cast<f32x4*>(stg + c * FP + 32 * db + 8 * r4 + 4 * h) = v * (p.scale / p.qscale);
        }
      __syncthreads();
      head_row_bwd<N>(stg, FP, kw0 + 32 * kb, p, T, tok_row0, head_row0, true, p.k, 1.0f, p.rk, p.dak, p.dotk);
      __syncthreads();
    }
  }
}

template <int N, bool VAR>
struct DqKernel {
  static void launch(const AttnBwdParams& p, int G, hipStream_t s) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<N, VAR>), dim3(G), dim3(256), 0, s, p);
  }
};
template <int N, bool VAR>
struct DkdvKernel {
  static void launch(const AttnBwdParams& p, int G, hipStream_t s) {
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<N, VAR>), dim3(G), dim3(256), 0, s, p);
  }
};

template <template <int, bool> class K>
static hipError_t launch_bwd_variant(const AttnBwdParams& p, int N, int blocks_per_seq, hipStream_t s) {
  if (p.sl2e != 1.0f) return hipErrorInvalidValue;  // stored q must be in log2 units
  const bool var = p.cu != nullptr;
  // Grid: (sequence, head, block).
  const int G = (var ? p.nseq : p.B) * p.H * blocks_per_seq;
  if (G <= 0) return hipSuccess;
  if (N != 32 && N != 64 && N != 128 && N != 256) return hipErrorInvalidValue;
  const int v = (N == 128 ? 2 : N == 256 ? 4 : N == 32 ? 6 : 0) | (var ? 1 : 0);
  switch (v) {
    case 6: K<32, false>::launch(p, G, s); break;
    case 7: K<32, true>::launch(p, G, s); break;
    case 0: K<64, false>::launch(p, G, s); break;
    case 1: K<64, true>::launch(p, G, s); break;
    case 2: K<128, false>::launch(p, G, s); break;
    case 3: K<128, true>::launch(p, G, s); break;
    case 4: K<256, false>::launch(p, G, s); break;
    default: K<256, true>::launch(p, G, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_attn_bwd_dq(const AttnBwdParams& p, int N, hipStream_t s) {
  const int BQ = 128, len = p.cu != nullptr ? p.max_len : p.T;
  return launch_bwd_variant<DqKernel>(p, N, (len + BQ - 1) / BQ, s);
}

hipError_t launch_attn_bwd_dkdv(const AttnBwdParams& p, int N, hipStream_t s) {
  const int BKV = 128, len = p.cu != nullptr ? p.max_len : p.T;
  return launch_bwd_variant<DkdvKernel>(p, N, (len + BKV - 1) / BKV, s);
}

// ---------------------------------------------------------------------------
// Table gradients (fast_triton_attn.py:622-639):
//   dF1[t, n] = sum_{b, h} dq[n] qh[n] + dk[n] kh[n]
//   dF2[t, n] = sum_{b, h} dq[n] qh[n^1] + dk[n] kh[n^1]
// with dq, dk the gradients of the rotated q, k rows and qh, kh the rows
// before the rotary. Neither dq nor qh is stored: per row, with R the rotary
// pair blocks of position t, r = rx * rq and s = dqh . qh (left by the dQ
// kernel in p.dotq),
//   qh  = R^-1 q                       (q as stored, over qscale)
//   dqh = da_q / r + qh * s / N        (the head RMSNorm backward, inverted)
//   dq  = R^-T dqh
// and likewise for k (p.dotk, da_k). da_q and da_k are the bf16 gradients the
// weight and input gradients use, so dF sees the same rounding they do.
// One workgroup covers PT positions: its threads take (slice, position,
// 8-column chunk), each slice walks every SL-th (sequence, head) pair, and
// the slices' sums meet in LDS in a fixed order (deterministic). Packed
// sequences: position t of sequence s is token cu[s] + t, skipped where
// the sequence is shorter.
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void table_grad_kernel(TableGradParams p) {
  constexpr int CPR = N / 8, PT = 4, SL = 256 / (CPR * PT);
  __shared__ __attribute__((aligned(16))) float red[SL][PT][2 * N];
  const int tid = threadIdx.x;
  const int dc = tid % CPR, pp = (tid / CPR) % PT, sl = tid / (CPR * PT);
  const int t = blockIdx.x * PT + pp;
  const bool live = t < p.rows;
  const int tc = live ? t : p.rows - 1;
  float a1[8], a2[8], inv[4];
  {
    const float* f1r = p.f1 + (size_t)tc * N + dc * 8;
    const float* f2r = p.f2 + (size_t)tc * N + dc * 8;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const f32x4 u = *reinterpret_cast<const f32x4*>(f1r + 4 * hf);
      const f32x4 w = *reinterpret_cast<const f32x4*>(f2r + 4 * hf);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a1[4 * hf + e] = u[e];
        a2[4 * hf + e] = w[e];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const float det = a1[i] * a1[i + 1] - a2[i] * a2[i + 1];
      inv[i / 2] = det != 0.f ? __builtin_amdgcn_rcpf(det) : 0.f;  // zero pair block: zero rows
    }
  }
  float u[8], w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) u[e] = w[e] = 0.f;

  // One row's contribution: x as stored (times xscale), its da, r = rx * rr
  // and the dot product s.
  auto add_row = [&](const u32x4& xw, const u32x4& daw, float xscale, float r_inv, float sdot) {
    float xv[8], da[8], xh[8], dh[8];
    unpack8(xw, xv);
    unpack8(daw, da);
    const float cf = sdot * p.inv_n;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const float x0 = xv[i] * xscale, x1 = xv[i + 1] * xscale;
      xh[i] = (a1[i + 1] * x0 - a2[i] * x1) * inv[i / 2];
      xh[i + 1] = (a1[i] * x1 - a2[i + 1] * x0) * inv[i / 2];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) dh[i] = da[i] * r_inv + xh[i] * cf;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const float d0 = (a1[i + 1] * dh[i] - a2[i + 1] * dh[i + 1]) * inv[i / 2];
      const float d1 = (a1[i] * dh[i + 1] - a2[i] * dh[i]) * inv[i / 2];
      u[i] += d0 * xh[i];
      u[i + 1] += d1 * xh[i + 1];
      w[i] += d0 * xh[i + 1];
      w[i + 1] += d1 * xh[i];
    }
  };

  const bool var = p.cu != nullptr;
  const int nbh = (var ? p.nseq : p.B) * p.H;
  if (live) {
#pragma unroll 2
    for (int i = sl; i < nbh; i += SL) {
      const int b = i / p.H, h = i - b * p.H;
      size_t row, tok;
      if (!var) {
        row = ((size_t)b * p.H + h) * p.T + t;
        tok = (size_t)b * p.T + t;
      } else {
        // Offsets clamped to [0, total], as in the attention kernels.
        const int start = min(max(p.cu[b], 0), p.T);
        const int len = min(max(p.cu[b + 1], start), p.T) - start;
        if (t >= len) continue;
        row = (size_t)h * p.T + start + t;
        tok = (size_t)start + t;
      }
      const u32x4 qw = ld16(p.q + row * N + dc * 8), daqw = ld16(p.daq + row * N + dc * 8);
      const u32x4 kw = ld16(p.k + row * N + dc * 8), dakw = ld16(p.dak + row * N + dc * 8);
      const float rxv = p.rx[tok];
      const float rq = p.rq[row], rk = p.rk[row], sq = p.dotq[row], sk = p.dotk[row];
      add_row(qw, daqw, 1.0f / p.qscale, __builtin_amdgcn_rcpf(rxv * rq), sq);
      add_row(kw, dakw, 1.0f, __builtin_amdgcn_rcpf(rxv * rk), sk);
    }
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    *reinterpret_cast<f32x4*>(&red[sl][pp][dc * 8 + 4 * hf]) = f32x4{u[4 * hf], u[4 * hf + 1], u[4 * hf + 2], u[4 * hf + 3]};
    *reinterpret_cast<f32x4*>(&red[sl][pp][N + dc * 8 + 4 * hf]) =
        f32x4{w[4 * hf], w[4 * hf + 1], w[4 * hf + 2], w[4 * hf + 3]};
  }
  __syncthreads();
  if (sl == 0 && live) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x4 s1 = *reinterpret_cast<const f32x4*>(&red[0][pp][dc * 8 + 4 * hf]);
      f32x4 s2 = *reinterpret_cast<const f32x4*>(&red[0][pp][N + dc * 8 + 4 * hf]);
#pragma unroll
      for (int k = 1; k < SL; ++k) {
        s1 += *reinterpret_cast<const f32x4*>(&red[k][pp][dc * 8 + 4 * hf]);
        s2 += *reinterpret_cast<const f32x4*>(&red[k][pp][N + dc * 8 + 4 * hf]);
      }
      *reinterpret_cast<f32x4*>(p.df1 + (size_t)t * N + dc * 8 + 4 * hf) = s1;
      *reinterpret_cast<f32x4*>(p.df2 + (size_t)t * N + dc * 8 + 4 * hf) = s2;
    }
  }
}

hipError_t launch_table_grad(const TableGradParams& p, int N, hipStream_t s) {
  constexpr int PT = 4;
  if (p.rows <= 0) return hipSuccess;
  const dim3 grid((p.rows + PT - 1) / PT);
  if (N == 32)
    hipLaunchKernelGGL(table_grad_kernel<32>, grid, dim3(256), 0, s, p);
  else if (N == 64)
    hipLaunchKernelGGL(table_grad_kernel<64>, grid, dim3(256), 0, s, p);
  else if (N == 128)
    hipLaunchKernelGGL(table_grad_kernel<128>, grid, dim3(256), 0, s, p);
  else if (N == 256)
    hipLaunchKernelGGL(table_grad_kernel<256>, grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mea
