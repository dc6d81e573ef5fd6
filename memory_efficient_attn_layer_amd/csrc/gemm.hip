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
#include "kernels.h"
#include "slab.cuh"
#include "tokgemm.cuh"

namespace mea {

// ---------------------------------------------------------------------------
// y = (O * sig) Wo^T, on the token-block main loop: A = Wo rows (output
// features, k = HN), B = O * sig rows, gated while the slab is written to
// LDS. A workgroup covers the NF output features from group * NF of BT
// tokens (the last group may reach past C); y rows leave through an LDS
// staging block as whole-row segments.
// ---------------------------------------------------------------------------
template <int NF>
__global__ __launch_bounds__(TokShape<NF>::NT, 1) void gate_oproj_kernel(OprojParams p) {
  using S = TokShape<NF>;
  constexpr int SP = 128 + 8;  // staging pitch (elements)
  static_assert(S::NW * 16 * SP <= S::SMEM, "staging fits the slab stages");
  __shared__ __attribute__((aligned(16))) bf16_bits smem[S::SMEM];
  const int M = p.M, C = p.C, HN = p.HN;
  // Workgroup (token block, feature group); the groups of one token block
  // are consecutive on one XCD, so its O and sig rows come from HBM once.
  const int ngrp = (C + NF - 1) / NF, lid = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (lid / ngrp) * S::BT, f0 = (lid % ngrp) * NF;
  f32x4 acc[8][4];
  tok_mainloop<NF, true>(HN, smem, p.wo + (size_t)f0 * HN, HN, 32, min(NF, C - f0), p.o, p.sig, HN, m0, M, acc);

  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = tid >> 6, wf = wave % S::WF, wt = wave / S::WF;
  bf16_bits* stg = smem + wave * 16 * SP;  // the main loop ended on a barrier
#pragma unroll
  for (int tb = 0; tb < S::TB; ++tb) {
#pragma unroll
    for (int fb = 0; fb < S::FB; ++fb) {
      const f32x4& a = acc[fb][tb];
      *reinterpret_cast<u32x2*>(stg + c16 * SP + 16 * fb + 4 * g) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
#pragma unroll
    for (int it = 0; it < 16 * 16 / 64; ++it) {
      const int id = lane + 64 * it, row = id >> 4, ch = id & 15;
      const int m = m0 + wt * 64 + tb * 16 + row;
      const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * SP + ch * 8);
      if (m < M && f0 + wf * 128 + ch * 8 < C) st16(p.y + (size_t)m * C + f0 + wf * 128 + ch * 8, val);
    }
  }
}

template <int NF>
static void launch_oproj_nf(const OprojParams& p, hipStream_t s) {
  const dim3 grid(((p.M + TokShape<NF>::BT - 1) / TokShape<NF>::BT) * ((p.C + NF - 1) / NF));
  hipLaunchKernelGGL(gate_oproj_kernel<NF>, grid, dim3(TokShape<NF>::NT), 0, s, p);
}

hipError_t launch_gate_oproj(const OprojParams& p, hipStream_t s) {
  if (p.C < 32 || p.C % 32 != 0 || p.HN % 32 != 0) return hipErrorInvalidValue;
  // Feature groups of 512 (or 256): a group of 1024 would shrink the token
  // block to 64 and re-read all of Wo from L2 for every 64 tokens. A width
  // that is no multiple of 256 ends in a partial group (its Wo rows past
  // C - 1 read row C - 1, its stores stop at C).
  if (p.C == 768)
    launch_oproj_nf<768>(p, s);
  else if (p.C % 512 == 0)
    launch_oproj_nf<512>(p, s);
  else
    launch_oproj_nf<256>(p, s);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dZ = dy Wo with the gate backward in the epilogue, on the token-block main
// loop: A = Wo^T rows (HN features, k = C), B = dy rows. A workgroup
// covers features group * NF .. + NF - 1 (clamped to HN; groups hold whole
// heads since NF is a multiple of N) of BT tokens. Each wave stages its fp32
// dZ block per 16 tokens and walks it as rows: lane (row, 8-feature chunk)
// loads sig and O, writes dO into the head-major (B, H, T, N) layout, da_g,
// z = O * sig over sig, and delta = rowsum(dO * O) per (token, head), summed
// over the N / 8 lanes of the head (N = 256: over the two waves of the head).
// ---------------------------------------------------------------------------
template <int NF>
__global__ __launch_bounds__(TokShape<NF>::NT, 1) void dz_gate_bwd_kernel(DzParams p) {
  using S = TokShape<NF>;
  constexpr int FP = 128 + 4;  // fp32 staging pitch
  constexpr int SM_BYTES = S::SMEM * 2 > S::NW * 16 * FP * 4 ? S::SMEM * 2 : S::NW * 16 * FP * 4;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM_BYTES];
  __shared__ float dpart[S::WF][S::BT];  // N = 256: each wave's half of delta
  const int M = p.M, C = p.C, H = p.H, T = p.T, N = p.N, HN = H * N;
  // Workgroup (token block, feature group), the groups of a token block
  // consecutive on one XCD (its dy rows come from HBM once).
  const int ngrp = (HN + NF - 1) / NF, lid = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (lid / ngrp) * S::BT, f0 = (lid % ngrp) * NF;
  f32x4 acc[8][4];
  // Wo^T is k-slab-major (C / 32, HN, 32): a slab of the group's rows is one
  // contiguous block (from row-major rows the loads ran 5.7% longer).
  tok_mainloop<NF, false>(C, reinterpret_cast<bf16_bits*>(smem), p.woT + (size_t)f0 * 32, 32, 32 * HN, HN - f0,
                          p.dy, nullptr,
                          C, m0, M, acc);

  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = tid >> 6, wf = wave % S::WF, wt = wave / S::WF;
  float* stg = reinterpret_cast<float*>(smem) + wave * 16 * FP;  // the main loop ended on a barrier
#pragma unroll
  for (int tb = 0; tb < S::TB; ++tb) {
    // The block's sigmoid(a_g), O and rx rows are requested before its
    // staging, so one memory round trip serves all four row groups (a load
    // issued after this block's stores would also wait for them).
    u32x4 sgw[4], ovw[4];
    float rxw[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = it * 4 + (lane >> 4), cc = lane & 15;
      const int m = m0 + wt * 64 + tb * 16 + row;
      const int j = f0 + wf * 128 + cc * 8;
      const int mc = m < M ? m : M - 1, jc = j < HN ? j : 0;
      const size_t off = (size_t)mc * HN + jc;
      sgw[it] = ld16(p.sig + off);
      ovw[it] = ld16(p.o + off);
      rxw[it] = p.rx[mc];
    }
#pragma unroll
    for (int fb = 0; fb < S::FB; ++fb)
      *reinterpret_cast<f32x4*>(stg + c16 * FP + 16 * fb + 4 * g) = acc[fb][tb];
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = it * 4 + (lane >> 4), cc = lane & 15;
      const int m = m0 + wt * 64 + tb * 16 + row;
      const int j = f0 + wf * 128 + cc * 8;
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
      unpack8(sgw[it], sg);
      unpack8(ovw[it], ov);
      const float rxv = rxw[it];
      float dov[8], dag[8], zv[8], dl = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // delta uses the bf16-rounded dO the attention backward consumes, so
        // dP - delta cancels exactly where it should (a single key, T = 1).
        dov[i] = bf2f(f2bf(dz[i] * sg[i]));
        dag[i] = rxv * dz[i] * ov[i] * sg[i] * (1.0f - sg[i]);
        zv[i] = ov[i] * sg[i];
        dl += dov[i] * ov[i];
      }
      dl += xor1(dl);
      dl += xor2(dl);
      if (N >= 64) dl += shfl_xor(dl, 4);  // N is uniform
      if (N >= 128) dl += shfl_xor(dl, 8);
      if (N == 256) {
        // A 256-wide head spans waves wf and wf ^ 1 (heads align to the
        // 256-feature groups): add the other wave's half. N is uniform, and
        // every (block, row) has its own slot.
        const int tl = wt * 64 + tb * 16 + row;
        if (cc == 0) dpart[wf][tl] = dl;
        __syncthreads();
        dl += dpart[wf ^ 1][tl];
      }
      if (valid) {
        const int hh = jc / N, n = jc - hh * N;
        const int b = mc / T, t = mc - b * T;
        const size_t hrow = ((size_t)b * H + hh) * T + t;
        st16(p.dO + hrow * N + n, pack8(dov));
        st16(p.dag + (size_t)mc * p.ld_dag + jc, pack8(dag));
        st16(p.sig + off, pack8(zv));  // sigmoid(a_g) is dead from here on
        if (n == 0) p.delta[hrow] = dl;
      }
    }
  }
}

template <int NF>
static void launch_dz_nf(const DzParams& p, int HN, hipStream_t s) {
  const dim3 grid(((p.M + TokShape<NF>::BT - 1) / TokShape<NF>::BT) * ((HN + NF - 1) / NF));
  hipLaunchKernelGGL(dz_gate_bwd_kernel<NF>, grid, dim3(TokShape<NF>::NT), 0, s, p);
}

hipError_t launch_dz_gate_bwd(const DzParams& p, hipStream_t s) {
  const int HN = p.H * p.N;
  if (p.C % 32 != 0 || (p.N != 32 && p.N != 64 && p.N != 128 && p.N != 256)) return hipErrorInvalidValue;
  // Feature groups of 512 where HN allows (see launch_gate_oproj).
  if (HN == 768)
    launch_dz_nf<768>(p, HN, s);
  else if (HN % 512 == 0)
    launch_dz_nf<512>(p, HN, s);
  else
    launch_dz_nf<256>(p, HN, s);
  return hipGetLastError();
}

// Part `part` of da as a pointer, without branches or an indexed read (a
// pointer picked by index from the parameters is read from a private copy).
__device__ __forceinline__ const bf16_bits* da_part(const DaParts& dp, int part) {
  auto m = [&](const bf16_bits* ptr, int i) { return (uint64_t)(uintptr_t)ptr & (0ull - (uint64_t)(part == i)); };
  return reinterpret_cast<const bf16_bits*>((uintptr_t)(m(dp.q, 0) | m(dp.k, 1) | m(dp.v, 2) | m(dp.g, 3)));
}

// ---------------------------------------------------------------------------
// dx = rmsnorm_bwd([da_q|da_k|da_v|da_g] Wcat), one workgroup owns full rows.
//
// Computed transposed, D^T = Wcat^T da^T: A = Wcat^T rows (C features, k =
// 4HN, stored k-slab-major by wcat_pack_kernel so that a slab is one
// contiguous block), B = da rows (tokens). A 32-wide k-slab of da lies in one
// head of one part (N >= 64): each slab has one base address, and a lane's
// row offset from it, the same in every slab, is precomputed for the
// head-major parts (q, k, v) and for the token-major da_g. A workgroup
// covers all C features of BT tokens with WF x WT waves of 128 features x 64
// tokens; k-slabs of 32 stream through a 3-stage LDS ring filled by direct
// global->LDS loads. In
// the accumulator layout a lane holds one token and 4 consecutive features,
// so the RMSNorm backward dot (acc . x) is an in-lane sum, two lane
// exchanges and a cross-wave sum through LDS; dx rows leave through an LDS
// staging block as whole-row stores.
//
// CP is the padded width the workgroup layout is built for; the model width
// C = p.C is a multiple of 32 with CP - 256 < C <= CP. Weight rows past C - 1
// read row C - 1, x columns past the row are clamped into it, accumulators of
// features past C are zeroed before the dot, and their stores are skipped.
//
// GROUPS = 2 (CP = 512, 768 < C <= 1024): the 512-feature layout over 128
// tokens walks the features in two groups, so each weight slab is re-read
// per 128 tokens rather than per 64 (the 1024-wide layout holds 64 tokens).
// The dot (acc . x) is summed over both groups in LDS. Group 0 leaves its
// uncorrected acc as bf16 in p.scratch (M x 512; the reference's dx_hat is a
// bf16 matmul output too, fast_triton_attn.py:655-660), group 1 writes its
// result, then every thread re-reads the scratch chunks it stored, applies
// the correction and writes those dx chunks (a thread's own store is visible
// to its own later load once vmcnt has drained). da_g may live in dx: each
// workgroup writes only its own rows, after both groups have read them.
// ---------------------------------------------------------------------------
template <int CP, int GROUPS = 1>
__global__ __launch_bounds__(64 * ((CP / 128) * (8 % (CP / 128) == 0 ? 8 / (CP / 128) : 1)), 1) void dx_kernel(DxParams p) {
  static_assert(GROUPS == 1 || CP == 512, "feature groups use the 512-wide layout");
  constexpr int WF = CP / 128;                          // waves along features
  constexpr int WT = 8 % WF == 0 ? 8 / WF : 1;          // waves along tokens
  constexpr int NW = WF * WT;
  constexpr int BT = 64 * WT;                           // tokens per workgroup
  constexpr int BK = 32, NS = CP * 2 <= 1024 ? 3 : 2;   // slab width, ring depth
  constexpr int STAGE = (CP + BT) * BK;
  constexpr int FB = 8, TB = 4;                         // 16-blocks per wave
  // Load instructions every wave issues per slab at least (waves whose
  // share is larger wait for more of their own loads, which is still right).
  constexpr int LOADS = (CP / 16) / NW + (BT / 16) / NW;
  constexpr int XW = 64 * 128;                          // x block of one wave (elements)
  constexpr int SMEM = NS * STAGE > NW * XW ? NS * STAGE : NW * XW;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[SMEM];
  __shared__ float dotp[WF][BT];
  __shared__ float dsum[GROUPS > 1 ? BT : 1];  // dot summed over the groups

  const int M = p.M, C = p.C, K4 = 4 * p.HN;
  const int m0 = xcd_remap(blockIdx.x, (M + BT - 1) / BT) * BT;
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave % WF, wt = wave / WF;
  const bf16_bits* wt_g = p.wcatT;  // (4HN / 32, C, 32): k-slab-major
  const DaParts& dp = p.da;
  const int N = dp.N, T = dp.T;

  // Token rows of the da slabs: group u of load instructions starts at token
  // mf(u); hm(m) is token m's row in a head-major array, in units of N from
  // head 0 of batch 0.
  using Plan = SlabPlan<BT, NW, BK>;
  auto mf = [&](int u) { return min(m0 + u * NW * 16, M - 1); };
  auto hm = [&](int m) { return (m / T) * (dp.H - 1) * T + m; };
  Plan plan_t, plan_h;
  slab_plan(plan_t, wave, dp.ld_g, [&](int u, int i) { return min(m0 + u * NW * 16 + i, M - 1) - mf(u); });
  slab_plan(plan_h, wave, N, [&](int u, int i) { return hm(min(m0 + u * NW * 16 + i, M - 1)) - hm(mf(u)); });
  int hmf[Plan::NU];
#pragma unroll
  for (int u = 0; u < Plan::NU; ++u) hmf[u] = __builtin_amdgcn_readfirstlane(hm(mf(u)));
  if (GROUPS > 1 && tid < BT) dsum[GROUPS > 1 ? tid : 0] = 0.f;
  const uint32_t lds0 = lds_addr(smem);
  const float inv_c = 1.0f / (float)C;

#pragma unroll 1
  for (int grp = 0; grp < GROUPS; ++grp) {
  const int f0 = grp * CP;  // first feature of the group
  const bool last = grp == GROUPS - 1;
  // Slabs are issued in order ks = 0, 1, 2, ...; (part, hh, n0) locate the
  // next one: part of da, head, first column within the head.
  int part = 0, hh = 0, n0 = 0;
  auto issue = [&](int ks, int st) {
    const uint32_t lds = lds0 + (uint32_t)(st * STAGE) * 2u;
    // The weight slab is one contiguous C x 32 block: 1 KB per load
    // instruction (rows past C - 1 read row C - 1; a clamped base keeps every
    // row offset non-negative).
    const bf16_bits* wslab = wt_g + (size_t)ks * C * BK;
    slab_issue<CP, NW, BK>(
        lds, wave, BK, [&](int u) { return wslab + (size_t)min(f0 + u * NW * 16, C - 1) * BK; },
        [&](int u, int i) { return min(f0 + u * NW * 16 + i, C - 1) - min(f0 + u * NW * 16, C - 1); });
    {
      const bool tokm = part == 3;
      const bf16_bits* src = da_part(dp, part);
      constexpr int NU = Plan::NU, NI = Plan::NI;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int ins = u * NW + wave;
        if (NI % NW != 0 && ins >= NI) break;  // wave-uniform: partial last round
        const size_t off = tokm ? (size_t)mf(u) * dp.ld_g + (hh * N + n0) : ((size_t)hh * T + hmf[u]) * N + n0;
        g2lds16_s(src + off, tokm ? plan_t.voff[u] : plan_h.voff[u],
                  lds + (uint32_t)(CP * BK * 2) + (uint32_t)ins * 1024u);
      }
    }
    n0 += BK;
    if (n0 == N) {
      n0 = 0;
      if (++hh == dp.H) {
        hh = 0;
        ++part;
      }
    }
  };

  f32x4 acc[FB][TB];
#pragma unroll
  for (int fb = 0; fb < FB; ++fb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = zero4();

  // Ring of NS stages, NS - 1 slabs in flight ahead of the one multiplied.
  const int nk = K4 / BK;
  for (int s0 = 0; s0 < NS - 1 && s0 < nk; ++s0) issue(s0, s0);
  for (int ks = 0; ks < nk; ++ks) {
    if (NS == 3 && ks + 1 < nk)
      __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);  // vmcnt(LOADS): only slab ks + 1 may be pending
    else
      wait_vmcnt0();
    __syncthreads();
    if (ks + NS - 1 < nk) issue(ks + NS - 1, (ks + NS - 1) % NS);
    const bf16_bits* As = smem + (ks % NS) * STAGE;
    const bf16_bits* Bs = As + CP * BK;
    bf16x8 af[FB], bfr[TB];
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) af[fb] = as_frag(slab_read<BK>(As, wf * 128 + fb * 16 + c16, g));
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) bfr[tb] = as_frag(slab_read<BK>(Bs, wt * 64 + tb * 16 + c16, g));
#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = mfma(af[fb], bfr[tb], acc[fb][tb]);
    reads_then_products<FB + TB, FB * TB>();
  }

  // Epilogue. The x block of each wave (its 64 tokens x 128 features, 16 KB)
  // comes through LDS once the ring is free: 16 direct global->LDS loads of
  // four whole 256-byte row segments each, chunk c of row r at 16-byte slot
  // c ^ (r & 15), so the accumulator-layout reads below (lane: one token,
  // 4 features) are conflict-free. Each wave reads only its own block.
  __syncthreads();  // every wave is past its last slab read
  // With GROUPS > 1 the lane index is opaque to the compiler inside each
  // group, so the epilogue's lane-constant offsets are recomputed per group
  // rather than hoisted out of the group loop and held across it.
  int lane_e = lane;
  if (GROUPS > 1) asm volatile("" : "+v"(lane_e));
  const int c16e = lane_e & 15, ge = lane_e >> 4;
  bf16_bits* xs = smem + wave * XW;
  int mrow[TB];
  float rxr[TB];
  if (f0 + wf * 128 + 128 > C) {
    // Features 16 fb + 4 g .. + 3 past C: their accumulators (products with
    // the clamped weight row) must not enter the dot (wave-uniform branch).
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) {
      const bool out = f0 + wf * 128 + 16 * fb + 4 * ge >= C;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = out ? zero4() : acc[fb][tb];
    }
  }
  {
    const int r0 = min(m0 + wt * 64, M - 1);
    const bf16_bits* xb = p.x + (size_t)r0 * C;
    const uint32_t lds = lds_addr(xs);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 4 * j + (lane_e >> 4), ch = (lane_e & 15) ^ (r & 15);
      const int col = min(f0 + wf * 128 + ch * 8, C - 8);  // columns past the row: clamped, never used
      const uint32_t voff = (uint32_t)((min(m0 + wt * 64 + r, M - 1) - r0) * C + col) * 2u;
      g2lds16_s(xb, voff, lds + (uint32_t)j * 1024u);
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      mrow[tb] = min(m0 + wt * 64 + tb * 16 + c16e, M - 1);
      rxr[tb] = p.rx[mrow[tb]];
    }
  }
  // Features 16 fb + 4 g .. + 3 of token row r of the wave's block.
  auto xs_at = [&](int r, int fb) {
    return reinterpret_cast<u32x2*>(xs + r * 128 + (((2 * fb + (ge >> 1)) ^ (r & 15)) << 3) + 4 * (ge & 1));
  };
  wait_vmcnt0();  // this wave's x block has landed

  // acc . x over this wave's 128 features, per token, then across the WF
  // waves that share the tokens.
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    float d = 0.f;
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) {
      const u32x2 xw = *xs_at(tb * 16 + c16e, fb);
      d += acc[fb][tb][0] * lo_bf(xw[0]) + acc[fb][tb][1] * hi_bf(xw[0]) + acc[fb][tb][2] * lo_bf(xw[1]) +
           acc[fb][tb][3] * hi_bf(xw[1]);
    }
    d += shfl_xor(d, 16);
    d += shfl_xor(d, 32);
    if (ge == 0) dotp[wf][wt * 64 + tb * 16 + c16e] = d;
  }
  __syncthreads();
  if (GROUPS > 1) {
    if (tid < BT) {
      float t = dsum[GROUPS > 1 ? tid : 0];
#pragma unroll
      for (int i = 0; i < WF; ++i) t += dotp[i][tid];
      dsum[GROUPS > 1 ? tid : 0] = t;
    }
    __syncthreads();
  }

  // dx = acc - x rx^2 (acc . x) / C, written over the x values it consumes
  // (each lane overwrites exactly the 8 bytes it read), then stored per 16
  // tokens as whole 256-byte row segments. An earlier group stores acc.
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    float dot = 0.f;
    if (GROUPS > 1) {
      dot = dsum[GROUPS > 1 ? wt * 64 + tb * 16 + c16e : 0];
    } else {
#pragma unroll
      for (int i = 0; i < WF; ++i) dot += dotp[i][wt * 64 + tb * 16 + c16e];
    }
    const float cf = last ? rxr[tb] * rxr[tb] * dot * inv_c : 0.f;
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) {
      u32x2* xp = xs_at(tb * 16 + c16e, fb);
      const u32x2 xw = *xp;
      const f32x4& a = acc[fb][tb];
      const float o0 = a[0] - lo_bf(xw[0]) * cf, o1 = a[1] - hi_bf(xw[0]) * cf;
      const float o2 = a[2] - lo_bf(xw[1]) * cf, o3 = a[3] - hi_bf(xw[1]) * cf;
      *xp = u32x2{pack2(o0, o1), pack2(o2, o3)};
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes are done
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = tb * 16 + it * 4 + (lane_e >> 4), ch = lane_e & 15;
      const int m = m0 + wt * 64 + r;
      const u32x4 val = *reinterpret_cast<const u32x4*>(xs + r * 128 + ((ch ^ (r & 15)) << 3));
      if (!last) {
        if (m < M) st16(p.scratch + (size_t)m * CP + wf * 128 + ch * 8, val);
      } else if (m < M && f0 + wf * 128 + ch * 8 < C)
        st16(p.dx + (size_t)m * C + f0 + wf * 128 + ch * 8, val);
    }
  }
  if (GROUPS > 1) __syncthreads();  // the x blocks are the next group's slab ring
  }  // groups

  if constexpr (GROUPS > 1) {
    // Group 0's features (all below 512 < C): reload the acc chunks this
    // thread stored, correct them, write dx.
    wait_vmcnt0();
    int lane_c = lane;
    asm volatile("" : "+v"(lane_c));
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = tb * 16 + it * 4 + (lane_c >> 4), ch = lane_c & 15;
        const int m = m0 + wt * 64 + r;
        if (m >= M) continue;
        const int col = wf * 128 + ch * 8;
        const float rxv = p.rx[m];
        const float cf = rxv * rxv * dsum[wt * 64 + r] * inv_c;
        float a[8], xv[8], o[8];
        unpack8(ld16(p.scratch + (size_t)m * CP + col), a);
        unpack8(ld16(p.x + (size_t)m * C + col), xv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = a[e] - xv[e] * cf;
        st16(p.dx + (size_t)m * C + col, pack8(o));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dx for C > 1024 (a multiple of 32): the workgroup layout of dx_kernel<1024>
// (8 waves of 128 features x 64 tokens) walks the output features in groups
// of 1024. The RMSNorm-backward dot (acc . x) needs the whole row, so it is
// summed over the groups in LDS; every group but the last leaves its
// uncorrected acc (bf16) in dx, the last group writes its result directly,
// and then every thread re-reads exactly the 16-byte chunks it wrote for the
// earlier groups, applies the correction and writes them back (a thread's
// own store is visible to its own later load once vmcnt has drained; no
// other workgroup touches these rows, and da_g does not live in dx here).
// Weight rows past C are clamped on load. Only the last group can reach past
// C: there features from C on read no x, add nothing to the dot and store
// nothing (a wave's slice wholly past C skips its loads and stores).
// ---------------------------------------------------------------------------
constexpr int kDxGroup = 1024;

__global__ __launch_bounds__(512, 1) void dx_wide_kernel(DxParams p) {
  constexpr int CG = kDxGroup, WF = 8, NW = 8, BT = 64, BK = 32, NS = 2;
  constexpr int STAGE = (CG + BT) * BK;
  constexpr int FB = 8, TB = 4;
  constexpr int SP = 128 + 8;  // staging pitch (elements)
  __shared__ __attribute__((aligned(16))) bf16_bits smem[NS * STAGE];
  __shared__ float dotp[WF][BT];
  __shared__ float dsum[BT];

  const int M = p.M, C = p.C, K4 = 4 * p.HN;
  const int m0 = xcd_remap(blockIdx.x, (M + BT - 1) / BT) * BT;
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave;  // one token block of 64: waves run along features only
  const bf16_bits* wt_g = p.wcatT;  // (4HN / 32, C, 32): k-slab-major
  const DaParts& dp = p.da;
  const int N = dp.N, T = dp.T;
  const int ngroups = (C + CG - 1) / CG;
  if (tid < BT) dsum[tid] = 0.f;

  using Plan = SlabPlan<BT, NW, BK>;
  auto mf = [&](int u) { return min(m0 + u * NW * 16, M - 1); };
  auto hm = [&](int m) { return (m / T) * (dp.H - 1) * T + m; };
  Plan plan_t, plan_h;
  slab_plan(plan_t, wave, dp.ld_g, [&](int u, int i) { return min(m0 + u * NW * 16 + i, M - 1) - mf(u); });
  slab_plan(plan_h, wave, N, [&](int u, int i) { return hm(min(m0 + u * NW * 16 + i, M - 1)) - hm(mf(u)); });
  int hmf[Plan::NU];
#pragma unroll
  for (int u = 0; u < Plan::NU; ++u) hmf[u] = __builtin_amdgcn_readfirstlane(hm(mf(u)));
  const uint32_t lds0 = lds_addr(smem);
  const bf16_bits* xg = p.x;
  const float inv_c = 1.0f / (float)C;
  int mrow[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) mrow[tb] = min(m0 + tb * 16 + c16, M - 1);

  for (int grp = 0; grp < ngroups; ++grp) {
    const int f0 = grp * CG;
    const bool wave_live = f0 + wf * 128 < C;  // wave-uniform
    const bool last = grp == ngroups - 1;
    int part = 0, hh = 0, n0 = 0;
    auto issue = [&](int ks, int st) {
      const uint32_t lds = lds0 + (uint32_t)(st * STAGE) * 2u;
      // Weight rows f0 .. f0 + CG - 1 of slab ks, clamped to C - 1 (a clamped
      // base keeps every row offset non-negative).
      const bf16_bits* wslab = wt_g + (size_t)ks * C * BK;
      slab_issue<CG, NW, BK>(
          lds, wave, BK, [&](int u) { return wslab + (size_t)min(f0 + u * NW * 16, C - 1) * BK; },
          [&](int u, int i) { return min(f0 + u * NW * 16 + i, C - 1) - min(f0 + u * NW * 16, C - 1); });
      {
        const bool tokm = part == 3;
        const bf16_bits* src = da_part(dp, part);
        constexpr int NU = Plan::NU, NI = Plan::NI;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const int ins = u * NW + wave;
          if (NI % NW != 0 && ins >= NI) break;  // wave-uniform: partial last round
          const size_t off = tokm ? (size_t)mf(u) * dp.ld_g + (hh * N + n0) : ((size_t)hh * T + hmf[u]) * N + n0;
          g2lds16_s(src + off, tokm ? plan_t.voff[u] : plan_h.voff[u],
                    lds + (uint32_t)(CG * BK * 2) + (uint32_t)ins * 1024u);
        }
      }
      n0 += BK;
      if (n0 == N) {
        n0 = 0;
        if (++hh == dp.H) {
          hh = 0;
          ++part;
        }
      }
    };

    f32x4 acc[FB][TB];
#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = zero4();

    const int nk = K4 / BK;
    issue(0, 0);
    for (int ks = 0; ks < nk; ++ks) {
      wait_vmcnt0();
      __syncthreads();
      if (ks + 1 < nk) issue(ks + 1, (ks + 1) % NS);
      const bf16_bits* As = smem + (ks % NS) * STAGE;
      const bf16_bits* Bs = As + CG * BK;
      bf16x8 af[FB], bfr[TB];
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) af[fb] = as_frag(slab_read<BK>(As, wf * 128 + fb * 16 + c16, g));
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) bfr[tb] = as_frag(slab_read<BK>(Bs, tb * 16 + c16, g));
#pragma unroll
      for (int fb = 0; fb < FB; ++fb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[fb][tb] = mfma(af[fb], bfr[tb], acc[fb][tb]);
    }

    // acc . x over this wave's 128 features, summed over the waves and the
    // groups in dsum.
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      float d = 0.f;
      if (wave_live) {
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) {
          const int f = f0 + wf * 128 + 16 * fb + 4 * g;
          if (f >= C) continue;
          const u32x2 xv = *reinterpret_cast<const u32x2*>(xg + (size_t)mrow[tb] * C + f);
          d += acc[fb][tb][0] * lo_bf(xv[0]) + acc[fb][tb][1] * hi_bf(xv[0]) + acc[fb][tb][2] * lo_bf(xv[1]) +
               acc[fb][tb][3] * hi_bf(xv[1]);
        }
      }
      d += shfl_xor(d, 16);
      d += shfl_xor(d, 32);
      if (g == 0) dotp[wf][tb * 16 + c16] = d;
    }
    __syncthreads();  // also: every wave is past its last slab read
    if (tid < BT) {
      float t = dsum[tid];
#pragma unroll
      for (int i = 0; i < WF; ++i) t += dotp[i][tid];
      dsum[tid] = t;
    }
    __syncthreads();

    // The last group writes dx = acc - x rx^2 (acc . x) / C; the others write
    // acc. Staged per 16-token block and stored as whole 256-byte segments.
    bf16_bits* stg = smem + wave * 16 * SP;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int tl = tb * 16 + c16;
      const float rxv = p.rx[mrow[tb]];
      const float cf = last ? rxv * rxv * dsum[tl] * inv_c : 0.f;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        u32x2 xv = {0u, 0u};
        const int f = f0 + wf * 128 + 16 * fb + 4 * g;
        if (last && f < C) xv = *reinterpret_cast<const u32x2*>(xg + (size_t)mrow[tb] * C + f);
        const f32x4& a = acc[fb][tb];
        const float o0 = a[0] - lo_bf(xv[0]) * cf, o1 = a[1] - hi_bf(xv[0]) * cf;
        const float o2 = a[2] - lo_bf(xv[1]) * cf, o3 = a[3] - hi_bf(xv[1]) * cf;
        *reinterpret_cast<u32x2*>(stg + c16 * SP + 16 * fb + 4 * g) = u32x2{pack2(o0, o1), pack2(o2, o3)};
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
#pragma unroll
      for (int it = 0; it < 16 * 16 / 64; ++it) {
        const int id = lane + 64 * it, row = id >> 4, ch = id & 15;
        const int m = m0 + tb * 16 + row;
        const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * SP + ch * 8);
        if (m < M && f0 + wf * 128 + ch * 8 < C) st16(p.dx + (size_t)m * C + f0 + wf * 128 + ch * 8, val);
      }
    }
    __syncthreads();  // the staging area is the next group's slab ring
  }

  // Correct the earlier groups: each thread reloads the chunks it stored.
  wait_vmcnt0();
  for (int grp = 0; grp + 1 < ngroups; ++grp) {
    const int f0 = grp * CG;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int it = 0; it < 16 * 16 / 64; ++it) {
        const int id = lane + 64 * it, row = id >> 4, ch = id & 15;
        const int m = m0 + tb * 16 + row;
        if (m >= M || f0 + wf * 128 >= C) continue;
        const size_t off = (size_t)m * C + f0 + wf * 128 + ch * 8;
        const float rxv = p.rx[m];
        const float cf = rxv * rxv * dsum[tb * 16 + row] * inv_c;
        float a[8], xv[8], o[8];
        unpack8(ld16(p.dx + off), a);
        unpack8(ld16(xg + off), xv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = a[e] - xv[e] * cf;
        st16(p.dx + off, pack8(o));
      }
    }
  }
}

hipError_t launch_dx(const DxParams& p, hipStream_t s) {
  // Model widths are multiples of 32; a width runs on the smallest padded
  // layout that holds it, widths past 1024 on the feature-group kernel.
  if (p.C < 32 || p.C % 32 != 0) return hipErrorInvalidValue;
  if (p.C <= 256)
    hipLaunchKernelGGL(dx_kernel<256>, dim3((p.M + 255) / 256), dim3(512), 0, s, p);
  else if (p.C <= 512)
    hipLaunchKernelGGL(dx_kernel<512>, dim3((p.M + 127) / 128), dim3(512), 0, s, p);
  else if (p.C <= 768)
    hipLaunchKernelGGL(dx_kernel<768>, dim3((p.M + 63) / 64), dim3(384), 0, s, p);
  else if (p.C <= 1024 && p.scratch != nullptr)
    hipLaunchKernelGGL((dx_kernel<512, 2>), dim3((p.M + 127) / 128), dim3(512), 0, s, p);
  else if (p.C <= 1024)
    hipLaunchKernelGGL(dx_kernel<1024>, dim3((p.M + 63) / 64), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL(dx_wide_kernel, dim3((p.M + 63) / 64), dim3(512), 0, s, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weight gradients D(i, j) = sum_m A(m, i) B(m, j) over a token range:
//   problem 0: A = da (M, 4HN), B = x (M, C)   -> dWcat (4HN, C)
//   problem 1: A = dy (M, C),   B = z (M, HN)  -> dWo   (C, HN)
// Operands run along tokens (da's head-major parts are read per head as
// (B, T) rows of N, see DaParts). Slabs of 32 tokens x 256 features land in
// LDS row-major (direct global->LDS loads, 3 stages); the MFMA operands,
// which run along tokens, are read with the transposing ds_read_b64_tr_b16.
// Tile 256 x 256, eight waves of 64 (i) x 128 (j). The token range is split
// so that all tiles x splits fill the CUs once; fp32 partials are summed by
// dw_reduce in a fixed order.
// ---------------------------------------------------------------------------
namespace {

constexpr int kDwBK = 32;     // tokens per slab
constexpr int kDwTile = 256;  // output tile edge
constexpr int kDwSlab = kDwBK * kDwTile;  // elements per operand slab

// Chunk c (16 bytes) of slab row r sits at slot c ^ dw_swz(r). The eight
// rows that one half-wave reads in a transposing read (rows 0-3 and 8-11 of
// an 8-row group pair) then cover eight distinct 32-byte bank segments.
__device__ __forceinline__ int dw_swz(int r) { return ((r & 3) | ((r >> 1) & 4)) << 1; }

// Loads one 32 x 256 slab: rows m0 .. m0+31 (clamped to M-1), columns
// c0 .. c0+255 (clamped to ncol-8) of a row-major (M, ld) matrix.
__device__ __forceinline__ void dw_issue(uint32_t lds, int wave, const bf16_bits* src, int ld, int m0, int M,
                                         int c0, int ncol) {
  const int lane = threadIdx.x & 63;
  const int mb = min(m0, M - 1);
  const bf16_bits* base = src + (size_t)mb * ld + c0;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ins = u * 8 + wave;         // 16 instructions of 2 rows each
    const int row = 2 * ins + (lane >> 5);
    const int chunk = (lane & 31) ^ dw_swz(row);
    const int r = min(m0 + row, M - 1) - mb;
    const int col = min(8 * chunk, ncol - c0 - 8);
    g2lds16_s(base, (uint32_t)(r * ld + col) * 2u, lds + (uint32_t)ins * 1024u);
  }
}

// The A slabs of problem 0 read da, whose parts have two layouts (da_q,
// da_k, da_v head-major, da_g token-major). A lane's column is the same in
// every slab and its token row advances by kDwBK per slab, so each lane
// keeps a cursor: the column's address in row 0 and the row's batch. In a
// head-major part token m = b*T + t sits at row b*H*T + t = m + b*(H-1)*T
// (in units of N from the column's head in batch 0).
struct DaCursor {
  const bf16_bits* col;  // part + the lane's column offset
  int rstride;           // elements per row: N, or ld_g for da_g
  int bstep;             // (H-1)*T, or 0 for da_g
  int m, b, nb;          // token row, its batch, first token of batch b+1
  int last;              // row of token M-1
};

__device__ __forceinline__ void da_cursor_init(DaCursor& c, const DaParts& dp, int HN, int feature, int m, int M) {
  const int part = feature / HN, f = feature - part * HN;
  if (part == 3) {
    c.col = dp.g + f;
    c.rstride = dp.ld_g;
    c.bstep = 0;
  } else {
    const bf16_bits* src = part == 0 ? dp.q : part == 1 ? dp.k : dp.v;
    const int hh = f / dp.N;
    c.col = src + (size_t)hh * dp.T * dp.N + (f - hh * dp.N);
    c.rstride = dp.N;
    c.bstep = (dp.H - 1) * dp.T;
  }
  c.m = m;
  c.b = m / dp.T;
  c.nb = (c.b + 1) * dp.T;
  c.last = (M - 1) + ((M - 1) / dp.T) * c.bstep;
}

// Address of the cursor's current row (rows past M - 1 read row M - 1),
// then one slab further.
__device__ __forceinline__ const bf16_bits* da_cursor_next(DaCursor& c, int T, int M) {
  while (c.m >= c.nb) {
    ++c.b;
    c.nb += T;
  }
  const int row = c.m < M ? c.m + c.b * c.bstep : c.last;
  c.m += kDwBK;
  return c.col + (size_t)row * c.rstride;
}

// MFMA operand of feature block f (16 features) from a slab: lane (g, c16)
// gets feature 16 f + c16 of tokens 8g .. 8g+7.
__device__ __forceinline__ bf16x8 dw_frag(const bf16_bits* slab, int f, int lane) {
  const int c16 = lane & 15, g = lane >> 4;
  const int r0 = 8 * g + (c16 >> 2);
  const int col = 16 * f + 4 * (c16 & 3);
  const int ch = col >> 3, within = col & 7;
  const bf16_bits* p0 = slab + r0 * kDwTile + ((ch ^ dw_swz(r0)) << 3) + within;
  const bf16_bits* p1 = slab + (r0 + 4) * kDwTile + ((ch ^ dw_swz(r0 + 4)) << 3) + within;
  return frag_from2(lds_read_tr4(p0), lds_read_tr4(p1));
}

}  // namespace

template <bool FAST>
__global__ __launch_bounds__(512, 1) void dw_partial_kernel(DwParams p) {
  constexpr int STAGES = 3;
  __shared__ __attribute__((aligned(16))) bf16_bits smem[STAGES * 2 * kDwSlab];
  const int M = p.M, C = p.C, HN = p.HN, K4 = 4 * HN;
  const int nc = (C + kDwTile - 1) / kDwTile;              // tiles along C (the last may be partial)
  const int t0 = (K4 / kDwTile) * nc;                       // problem-0 tiles
  const int t1 = nc * ((HN + kDwTile - 1) / kDwTile);
  const int ntile = t0 + t1;
  // Consecutive logical ids (same token split, neighbouring tiles) share an
  // XCD, so the operand rows of a split are fetched into one L2.
  const int L = xcd_remap(blockIdx.x, ntile * p.splits);
  const int z = L / ntile, tile = L - z * ntile;
  const bool prob1 = tile >= t0;
  const int lt = prob1 ? tile - t0 : tile;
  const int ntj = prob1 ? (HN + kDwTile - 1) / kDwTile : nc;
  const int i0 = (lt / ntj) * kDwTile, j0 = (lt % ntj) * kDwTile;
  const int I = prob1 ? C : K4, J = prob1 ? HN : C;
  const bf16_bits* bsrc = prob1 ? p.z : p.x;
  const int ldb = prob1 ? HN : C;

  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave & 3, wj = wave >> 2;

  const int chunk = ((M + p.splits - 1) / p.splits + kDwBK - 1) / kDwBK * kDwBK;
  const int mbeg = z * chunk, mend = min(M, mbeg + chunk);
  const int ns = mbeg < mend ? (mend - mbeg + kDwBK - 1) / kDwBK : 0;

  // A slabs (this lane: rows 2 * ins + lane / 32, ins = 8u + wave; column
  // chunk as in dw_issue). Slabs are issued in order s = 0, 1, 2, ...
  //  FAST (T a multiple of kDwBK, HN and C of kDwTile; then every token chunk is a
  //  multiple of kDwBK): no slab crosses a sequence or runs past M and the
  //  tile's columns lie in one part, so slab s reads from the uniform base
  //  asrc + arow * ald, arow being the row of its first token (head-major
  //  parts: b*H*T + t; token-major sources: m), at a per-lane offset that is
  //  the same in every slab. Each issue advances arow (and stt, the first
  //  token's position in its sequence, to step arow over the other heads).
  //  Otherwise problem 0 follows every lane's row with a cursor.
  const DaParts& dp = p.da;
  const bf16_bits* asrc = nullptr;
  int ald = 0, bstep = 0, arow = 0, stt = 0;
  uint32_t avoff[2] = {0u, 0u};
  DaCursor cur[2];
  if (FAST) {
    const int apart = prob1 ? 4 : i0 / HN;
    const bool hmaj = apart < 3;
    asrc = prob1 ? p.dy : da_part(dp, apart);
    ald = prob1 ? C : hmaj ? dp.N : dp.ld_g;
    bstep = hmaj ? (dp.H - 1) * dp.T : 0;
    const int sb = mbeg / dp.T;
    stt = mbeg - sb * dp.T;
    arow = hmaj ? sb * dp.H * dp.T + stt : mbeg;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 2 * (u * 8 + wave) + (lane >> 5);
      const int f = i0 - (prob1 ? 0 : apart * HN) + 8 * ((lane & 31) ^ dw_swz(row));
      const int hh = f / dp.N;
      avoff[u] = (uint32_t)(hmaj ? (hh * dp.T + row) * dp.N + f - hh * dp.N : row * ald + f) * 2u;
    }
  } else if (!prob1) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 2 * (u * 8 + wave) + (lane >> 5);
      const int col = min(8 * ((lane & 31) ^ dw_swz(row)), I - i0 - 8);
      da_cursor_init(cur[u], dp, HN, i0 + col, mbeg + row, M);
    }
  }

  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int s) {
    const int st = s % STAGES;
    const uint32_t lds = lds0 + (uint32_t)(st * 2 * kDwSlab) * 2u;
    const int m0 = mbeg + s * kDwBK;
    if (FAST) {
      const bf16_bits* base = asrc + (size_t)arow * ald;
#pragma unroll
      for (int u = 0; u < 2; ++u) g2lds16_s(base, avoff[u], lds + (uint32_t)(u * 8 + wave) * 1024u);
      arow += kDwBK;
      stt += kDwBK;
      if (stt == dp.T) {
        stt = 0;
        arow += bstep;
      }
    } else if (prob1) {
      dw_issue(lds, wave, p.dy, C, m0, M, i0, I);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) g2lds16(da_cursor_next(cur[u], dp.T, M), lds + (uint32_t)(u * 8 + wave) * 1024u);
    }
    dw_issue(lds + kDwSlab * 2, wave, bsrc, ldb, m0, M, j0, J);
  };

  f32x4 acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = zero4();

  if (ns > 0) issue(0);
  if (ns > 1) issue(1);
  for (int s = 0; s < ns; ++s) {
    // Slab s has landed once at most the next slab's 4 loads are pending.
    if (s + 1 < ns)
      __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
    else
      wait_vmcnt0();
    __syncthreads();
    bf16_bits* As = smem + (s % STAGES) * 2 * kDwSlab;
    const int valid = mend - (mbeg + s * kDwBK);
    if (valid < kDwBK) {
      // Last slab of the matrix: token rows past the end contribute zero.
      for (int e = tid; e < (kDwBK - valid) * kDwTile; e += 512) As[valid * kDwTile + e] = 0;
      __syncthreads();
    }
    if (s + 2 < ns) issue(s + 2);
    bf16x8 af[4], bfr[8];
#pragma unroll
    for (int a = 0; a < 4; ++a) af[a] = dw_frag(As, wi * 4 + a, lane);
#pragma unroll
    for (int b = 0; b < 8; ++b) bfr[b] = dw_frag(As + kDwSlab, wj * 8 + b, lane);
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[a][b] = mfma(af[a], bfr[b], acc[a][b]);
  }

  const size_t per_split = (size_t)K4 * C + (size_t)C * HN;
  float* out = p.part + (size_t)z * per_split + (prob1 ? (size_t)K4 * C : 0);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int j = j0 + wj * 128 + b * 16 + c16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + wi * 64 + a * 16 + 4 * g + r;
        if (i < I && j < J) out[(size_t)i * J + j] = acc[a][b][r];
      }
    }
}

// Output tiles of both problems (tiles along C rounded up).
static int dw_tiles(int C, int HN) {
  const int nc = (C + kDwTile - 1) / kDwTile;
  return (4 * HN / kDwTile) * nc + nc * ((HN + kDwTile - 1) / kDwTile);
}

int dw_splits(int M, int C, int HN) {
  const int tiles = dw_tiles(C, HN);
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus = n;
  }
  int s = cus / tiles;
  const int max_s = (M + kDwBK - 1) / kDwBK;
  if (s > max_s) s = max_s;
  return s < 1 ? 1 : s;
}

hipError_t launch_dw_partial(const DwParams& p, hipStream_t s) {
  if (p.C % 32 != 0 || (4 * p.HN) % kDwTile != 0) return hipErrorInvalidValue;
  const int tiles = dw_tiles(p.C, p.HN);
  // The fast path reads dy's columns unclamped: whole tiles along C only.
  if (p.da.T % kDwBK == 0 && p.HN % kDwTile == 0 && p.C % kDwTile == 0)
    hipLaunchKernelGGL(dw_partial_kernel<true>, dim3(tiles * p.splits), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL(dw_partial_kernel<false>, dim3(tiles * p.splits), dim3(512), 0, s, p);
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
// SLABS: out is k-slab-major instead, element (c, r) of the transpose at
// (r / 32) * cols * 32 + c * 32 + r % 32 (ld_out and col_off unused).
template <bool SLABS>
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
    if (cc < cols && rr < rows) {
      if (SLABS)
        out[(size_t)(rr >> 5) * cols * 32 + (size_t)cc * 32 + (rr & 31)] = tile[tx][c];
      else
        out[(size_t)cc * ld_out + col_off + rr] = tile[tx][c];
    }
  }
}

hipError_t launch_transpose(const bf16_bits* in, int rows, int cols, int ld_in, bf16_bits* out, int ld_out,
                            int col_off, hipStream_t s) {
  hipLaunchKernelGGL(transpose_kernel<false>, dim3((cols + 63) / 64, (rows + 63) / 64), dim3(256), 0, s, in, rows,
                     cols, ld_in, out, ld_out, col_off);
  return hipGetLastError();
}

hipError_t launch_transpose_slabs(const bf16_bits* in, int rows, int cols, int ld_in, bf16_bits* out, hipStream_t s) {
  if (rows % 32 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(transpose_kernel<true>, dim3((cols + 63) / 64, (rows + 63) / 64), dim3(256), 0, s, in, rows,
                     cols, ld_in, out, 0, 0);
  return hipGetLastError();
}

// Wcat^T in k-slab-major order (the dx A operand): element (f, k) at
// (k / 32) * C * 32 + f * 32 + k % 32, k indexing the stacked rows of
// [Wq; Wk; Wv; Wg] (part blockIdx.z, rows z * HN ..). A 64 x 64 tile of one
// part goes through LDS; each thread writes 16-byte chunks (8 consecutive k
// of one feature), so every 32-k slab of the tile leaves as 64 contiguous
// 64-byte rows.
__global__ __launch_bounds__(256) void wcat_pack_kernel(WcatPackParams p) {
  __shared__ bf16_bits tile[64][64 + 2];  // [k][f]
  const int z = blockIdx.z, HN = p.HN, C = p.C;
  const bf16_bits* in = z == 0 ? p.wq : z == 1 ? p.wk : z == 2 ? p.wv : p.wg;  // (HN, C)
  const int k0 = blockIdx.y * 64, f0 = blockIdx.x * 64, tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int i = tid + 256 * it, r = i >> 3, c = (i & 7) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (k0 + r < HN && f0 + c < C) v = ld16(in + (size_t)(k0 + r) * C + f0 + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[r][c + 2 * e] = (bf16_bits)(v[e] & 0xFFFFu);
      tile[r][c + 2 * e + 1] = (bf16_bits)(v[e] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    // i = (slab half s, feature f, chunk ch): consecutive threads write consecutive 16-byte chunks.
    const int i = tid + 256 * it, s = i >> 8, f = (i >> 2) & 63, ch = i & 3;
    const int kl = s * 32 + ch * 8;
    if (k0 + kl >= HN || f0 + f >= C) continue;
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = (uint32_t)tile[kl + 2 * e][f] | ((uint32_t)tile[kl + 2 * e + 1][f] << 16);
    const int k = z * HN + k0 + kl;  // HN and k0 are multiples of 32
    st16(p.out + (size_t)(k >> 5) * C * 32 + (size_t)(f0 + f) * 32 + (k & 31), v);
  }
}

hipError_t launch_wcat_pack(const WcatPackParams& p, hipStream_t s) {
  if (p.HN % 32 != 0 || p.C % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(wcat_pack_kernel, dim3((p.C + 63) / 64, (p.HN + 63) / 64, 4), dim3(256), 0, s, p);
  return hipGetLastError();
}

namespace {

// One thread per 16-byte chunk of the packed output: matrix blockIdx.z,
// k-slab kk, row r, chunk c8 (8 elements) <- row r, columns 32 kk + 8 c8.
__global__ __launch_bounds__(256) void wslab_pack_kernel(WcatPackParams p) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // chunk index within one matrix
  const int nch = p.HN * (p.C / 8);
  if (i >= nch) return;
  const int c8 = i & 3, r = (i >> 2) % p.HN, kk = (i >> 2) / p.HN;
  const bf16_bits* w = blockIdx.z == 0 ? p.wq : blockIdx.z == 1 ? p.wk : blockIdx.z == 2 ? p.wv : p.wg;
  const u32x4 v = ld16(w + (size_t)r * p.C + kk * 32 + c8 * 8);
  *reinterpret_cast<u32x4*>(p.out + (size_t)blockIdx.z * p.HN * p.C + (size_t)i * 8) = v;
}

}  // namespace

hipError_t launch_wslab_pack(const WcatPackParams& p, hipStream_t s) {
  if (p.C % 32 != 0) return hipErrorInvalidValue;
  const int nch = p.HN * (p.C / 8);
  hipLaunchKernelGGL(wslab_pack_kernel, dim3((nch + 255) / 256, 1, 4), dim3(256), 0, s, p);
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
