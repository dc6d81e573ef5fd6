// Parameter blocks and host-side launchers of the block's kernels.
// Every launcher enqueues on `stream` and returns hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mea {

typedef uint16_t bf16_bits;

// Input RMSNorm + q/k/v/g projection + q/k head RMSNorm + rotary + sigmoid.
struct ProjParams {
  const bf16_bits* x;                       // (M, C)
  // (H*N, C) weights: element (row, k) at row * w_row + (k / 32) * w_slab +
  // k % 32. Row-major: w_row = C, w_slab = 32; the k-slab-major copy of
  // launch_wslab_pack: w_row = 32, w_slab = 32 * H*N.
  const bf16_bits *wq, *wk, *wv, *wg;
  int w_row;
  int64_t w_slab;
  const float *f1, *f2;                     // (T_max, N)
  // Packed bf16 copy of the tables (t_max rows of N / 4 16-byte words, word
  // n / 4 of row t = f1[t, n..n+3], f2[t, n..n+3]), or null: the epilogue
  // then reads f1 / f2. Used when every table value is a bf16 number.
  const bf16_bits* tabp;
  bf16_bits *q, *k, *v;                     // (B, H, T, N)
  bf16_bits* sig;                           // (M, H*N)
  float* rx;                                // (M) or null
  float *rq, *rk;                           // (B, H, T) or null
  // Largest squared norms of the stored q and k rows (2 floats, zeroed
  // beforehand, raised with atomic max) or null.
  float* qk_norm2;
  // Rotary row of every token (M), or null (row = t of the (B, T) layout):
  // packed sequences give each token its position inside its sequence.
  const int* tpos;
  int t_max;                                // rows of f1 / f2 or tabp (tpos is clamped to it)
  int M, T, C, H;
  float eps;
  float qscale;                             // the stored q rows are q * qscale
  float inv_n;                              // 1 / head dimensions in use (head RMSNorm mean)
};
hipError_t launch_qkvg_proj(const ProjParams& p, int N, hipStream_t s);

// tabp (ProjParams) from rows 0 .. rows-1 of f1 and f2: values rounded to
// bf16, so exact for tables whose values are bf16 numbers.
hipError_t launch_rotary_pack(const float* f1, const float* f2, int rows, int N, bf16_bits* tabp, hipStream_t s);

// tpos[m] = m - cu[s] for cu[s] <= m < cu[s+1] (packed sequences).
hipError_t launch_token_positions(const int* cu, int nseq, int M, int* tpos, hipStream_t s);

// Causal flash attention forward.
struct AttnFwdParams {
  const bf16_bits *q, *k, *v;               // (B, H, T, N)
  bf16_bits* o;                             // (B, T, H*N)
  float* lse;                               // (B, H, T) natural log, or null
  // Squared-norm bounds of the q and k rows (see ProjParams) or null. When
  // given and sl2e * |q| |k| <= kFixedBound, the softmax runs without a max.
  const float* qk_norm2;
  int B, H, T;
  float sl2e;                               // multiplies q.k into log2 units
  // Packed sequences (or null): sequence s holds tokens cu[s] .. cu[s+1]-1 of
  // a (1, H, T, N) / (T, H*N) layout with T the total; nseq sequences of at
  // most max_len tokens. Attention stays inside each sequence.
  const int* cu;
  int nseq, max_len;
};
constexpr float kFixedBound = 60.0f;
hipError_t launch_attn_fwd(const AttnFwdParams& p, int N, hipStream_t s);

// Causal flash attention backward fused with the q/k RMSNorm + rotary
// backward and the input-RMSNorm row scale of the projection gradients.
struct AttnBwdParams {
  const bf16_bits *q, *k, *v, *dO;          // (B, H, T, N)
  const float *lse, *delta;                 // (B, H, T)
  const float *f1, *f2;                     // (T_max, N)
  const float* rx;                          // (M)
  const float *rq, *rk;                     // (B, H, T)
  // Gradients of the q, k, v projection outputs, (B, H, T, N), rows scaled
  // by rx. dak / dav may be k / v themselves: the dK/dV kernel reads only
  // its own key rows of k and v, each before writing them.
  bf16_bits *daq, *dak, *dav;
  // Per-row dot products dqh . qh and dkh . kh of the head RMSNorm backward,
  // (B, H, T) fp32, written when non-null (table gradients; then dak must
  // not be k, which table_grad_kernel reads afterwards).
  float *dotq, *dotk;
  int B, H, T;
  float scale;                              // softmax scale 1/sqrt(N)
  float sl2e;                               // must be 1: stored q . k is in log2 units
  float qscale;                             // stored q = q * qscale
  float inv_n;                              // 1 / head dimensions in use (head RMSNorm mean)
  const int* cu;                            // packed sequences, as in AttnFwdParams (or null)
  int nseq, max_len;
};
hipError_t launch_attn_bwd_dq(const AttnBwdParams& p, int N, hipStream_t s);
hipError_t launch_attn_bwd_dkdv(const AttnBwdParams& p, int N, hipStream_t s);
// dF1 / dF2 (rows, N) fp32 from the stored q, k, their gradients da_q,
// da_k and the per-row dot products of the attention backward, summed over
// batch (or packed sequences) and heads in a fixed order.
struct TableGradParams {
  const bf16_bits *q, *daq, *k, *dak;       // (B, H, T, N) head-major; q as stored (times qscale)
  const float *dotq, *dotk, *rq, *rk;       // (B, H, T)
  const float* rx;                          // (M)
  const float *f1, *f2;                     // (rows, N) fp32 tables
  float *df1, *df2;                         // (rows, N) out
  float qscale, inv_n;
  int B, H, T, rows;
  const int* cu;                            // packed sequences (B = 1, T = total tokens) or null
  int nseq;
};
hipError_t launch_table_grad(const TableGradParams& p, int N, hipStream_t s);

// y = (o * sig) Wo^T.
struct OprojParams {
  const bf16_bits *o, *sig;                 // (M, HN)
  const bf16_bits* wo;                      // (C, HN)
  bf16_bits* y;                             // (M, C)
  int M, C, HN;
};
hipError_t launch_gate_oproj(const OprojParams& p, hipStream_t s);

// dZ = dy Wo, then the gate backward:
//   dO = dZ * sig            -> (B, H, T, N)
//   da_g = rx * dZ * O * sig * (1 - sig)   -> (M, HN), row stride ld_dag
//   delta = rowsum_N(dO * O) -> (B, H, T)
//   z = O * sig              -> (M, HN), written over sig (the output
//                               projection's input, for dWo)
struct DzParams {
  const bf16_bits* dy;                      // (M, C)
  const bf16_bits* woT;                     // Wo^T k-slab-major: (C / 32, HN, 32)
  const bf16_bits* o;                       // (M, HN)
  bf16_bits* sig;                           // (M, HN): sigmoid(a_g) in, z out
  const float* rx;                          // (M)
  bf16_bits* dO;                            // (B, H, T, N)
  bf16_bits* dag;                           // (M, HN), row stride ld_dag
  float* delta;                             // (B, H, T)
  int M, T, C, H, N, ld_dag;
};
hipError_t launch_dz_gate_bwd(const DzParams& p, hipStream_t s);

// The gradient of the four projection outputs, da = [da_q | da_k | da_v |
// da_g] (M, 4*HN), rows pre-scaled by rx, as the dx and dW GEMMs read it:
// da_q, da_k, da_v head-major (B, H, T, N) like q, k, v; da_g token-major
// (M, HN) with row stride ld_g.
struct DaParts {
  const bf16_bits *q, *k, *v, *g;
  int ld_g, B, T, H, N;
};

// acc = da Wcat, then the input RMSNorm backward:
// dx = acc - x * rx^2 * (acc . x) / C.
struct DxParams {
  DaParts da;
  const bf16_bits* wcatT;                   // Wcat^T k-slab-major: (4*HN / 32, C, 32)
  const bf16_bits* x;                       // (M, C)
  const float* rx;                          // (M)
  bf16_bits* dx;                            // (M, C)
  // (M, 512) bf16 for 768 < C <= 1024 (feature groups of 512), or null: the
  // 1024-wide layout over 64 tokens runs instead.
  bf16_bits* scratch;
  int M, C, HN;
};
hipError_t launch_dx(const DxParams& p, hipStream_t s);

// Weight gradients, split over tokens into fp32 partial sums:
//   dWcat = da^T x        (4*HN, C)   da = [da_q | da_k | da_v | da_g]
//   dWo   = dy^T z        (C, HN)     z = O * sig
struct DwParams {
  DaParts da;
  const bf16_bits* x;                       // (M, C)
  const bf16_bits* dy;                      // (M, C)
  const bf16_bits* z;                       // (M, HN)
  float* part;                              // (splits, 4*HN*C + C*HN)
  int M, C, HN, splits;
};
// Token splits of the weight-gradient reduction for a shape (one workgroup
// per CU over all output tiles); the workspace holds that many partials.
int dw_splits(int M, int C, int HN);
hipError_t launch_dw_partial(const DwParams& p, hipStream_t s);
// Sums the partials and writes the five bf16 weight gradients.
struct DwReduceParams {
  const float* part;
  bf16_bits *dwq, *dwk, *dwv, *dwg, *dwo;
  int C, HN, splits;
};
hipError_t launch_dw_reduce(const DwReduceParams& p, hipStream_t s);

// out(cols, rows) = in(rows, cols)^T for a bf16 matrix with leading
// dimension ld_in; writes into out with leading dimension ld_out starting at
// column col_off.
hipError_t launch_transpose(const bf16_bits* in, int rows, int cols, int ld_in, bf16_bits* out,
                            int ld_out, int col_off, hipStream_t s);
// The same transpose stored k-slab-major: element (c, r) of out at
// (r / 32) * cols * 32 + c * 32 + r % 32 (rows a multiple of 32).
hipError_t launch_transpose_slabs(const bf16_bits* in, int rows, int cols, int ld_in, bf16_bits* out, hipStream_t s);

// Wcat^T for dx in k-slab-major order: element (f, k) at
// (k / 32) * C * 32 + f * 32 + k % 32, k over the stacked rows of
// [Wq; Wk; Wv; Wg] (each (HN, C)).
struct WcatPackParams {
  const bf16_bits *wq, *wk, *wv, *wg;
  bf16_bits* out;
  int HN, C;
};
hipError_t launch_wcat_pack(const WcatPackParams& p, hipStream_t s);

// Each of Wq, Wk, Wv, Wg (HN, C) into k-slab-major (C / 32, HN, 32) at
// out + i * HN * C (i = 0 q, 1 k, 2 v, 3 g): a 32-wide k-slab of any run of
// rows is one contiguous block, so the projection's weight-slab loads read
// 1 KB of contiguous memory per instruction.
hipError_t launch_wslab_pack(const WcatPackParams& p, hipStream_t s);

// Fills n floats with zero (a kernel, so it is safe inside captured graphs).
hipError_t launch_zero_f32(float* p, size_t n, hipStream_t s);

// KV-cache decode step: one new token per sequence at position pos[b]
// attends to cache rows 0 .. pos[b] (its own k / v included).
struct DecodeParams {
  const bf16_bits* q;                       // (B, H, N) stored q (log2 units)
  bf16_bits *k_cache, *v_cache;             // (B, H, Tc, N), the new token's rows already written
  const int* pos;                           // (B); clamped to [0, Tc - 1]
  float* part;                              // (B*H, S, N + 4): o[N], m, l per split
  bf16_bits* o;                             // (B, H*N) attention output
  int B, H, Tc;
  int S;                                    // key splits per (b, h), a multiple of 4
  int chunk;                                // keys per split, a multiple of 64
};
// Splits and keys per split for a cache of Tc rows (host side).
void decode_splits(int B, int H, int Tc, int* S, int* chunk);

// Few-token products of the decode step: out[t][f] = sum_k A[t][k] W[f][k]
// for t < M (M small), with A = A0 * A1 elementwise when A1 is given; up to
// four weight matrices (W[z], F rows each) side by side in one launch, their
// outputs at column z * F of out. fp32 or bf16 output.
struct SkinnyParams {
  const bf16_bits *A0, *A1;                 // (M, K), row stride K; A1 may be null
  const bf16_bits* W[4];                    // (F, K) each
  void* out;                                // (M, ldo)
  int M, K, F, nw, ldo;
  int out_bf16;
};
hipError_t launch_skinny_gemm(const SkinnyParams& p, hipStream_t s);

// Epilogue of the decode projection for the new token of every sequence:
// from a = [a_q | a_k | a_v | a_g] (B, 4HN) fp32 (products with the raw x)
// and x, the input RMSNorm scale, per-head RMSNorm of q and k, rotary at
// row pos[b] (clamped to t_max - 1), q times qscale, v, sigmoid(g).
struct DecodeProjParams {
  const float* a;                           // (B, 4HN)
  const bf16_bits* x;                       // (B, C)
  const float *f1, *f2;                     // (t_max, N)
  const int* pos;                           // (B)
  bf16_bits* q;                             // (B, H, N)
  bf16_bits *k_cache, *v_cache;             // (B, H, Tc, N): k, v go to row pos[b] (clamped to [0, Tc - 1])
  bf16_bits* sig;                           // (B, HN)
  int B, C, H, t_max, Tc;
  float eps, qscale;
  float inv_n;  // 1 / head dimensions in use (head RMSNorm mean)
};
hipError_t launch_decode_proj_epilogue(const DecodeProjParams& p, int N, hipStream_t s);
hipError_t launch_attn_decode(const DecodeParams& p, int N, hipStream_t s);
hipError_t launch_attn_decode_combine(const DecodeParams& p, int N, hipStream_t s);

}  // namespace mea
