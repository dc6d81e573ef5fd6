/*
 * mea.h - C ABI of the MI355X (gfx950) memory-efficient attention block.
 *
 * The block is the one computed by `fused_attn` in the reference
 * (fast_triton_attn.py:681-697) and by the eager path it replaces
 * (README.md:42-64):
 *
 *   xh = rmsnorm(x)                              per token over C
 *   a_p = xh W_p^T             p in {q,k,v,g}    W_p is (H*N, C)
 *   q = rope(rmsnorm_N(a_q)), k = rope(rmsnorm_N(a_k)), v = a_v, s = sigmoid(a_g)
 *   O = softmax_causal(q k^T / sqrt(N)) v        per (batch, head)
 *   y = (O * s) W_o^T                            W_o is (C, H*N)
 *
 * rope pairs adjacent lanes n and n^1: out[n] = t[n]*f1[t,n] + t[n^1]*f2[t,n]
 * (fast_triton_attn.py:132-141).
 *
 * Conventions shared by every entry point:
 *   - All device pointers are borrowed; the library never allocates device
 *     memory. Outputs and the workspace are allocated by the caller
 *     (mea_decode_static takes no workspace: it uses a static buffer of the
 *     library instead).
 *   - Activations and weights are bf16 (the only dtype the reference runs
 *     with, fast_triton_attn.py:32,103,123). Rotary tables, lse and the
 *     per-row statistics are fp32.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*) and is
 *     asynchronous; nothing synchronises the host.
 *   - A return of 0 means success. Negative values are argument errors found
 *     on the host before anything is launched; MEA_ERR_LAUNCH reports a HIP
 *     launch error. mea_strerror() names every code.
 *   - Tensors are dense row-major in the shapes documented per argument.
 *     Pointers must be 16-byte aligned.
 *
 * Supported shapes: N in {32, 64, 128, 256}, with H even for N = 32 (the
 * projection tiles hold head pairs); heads of 16 dimensions are carried
 * zero-padded to N = 32 or 64 (see N_active), and an odd number of 16- or
 * 32-wide heads with one zero head more (zero weight rows and Wo columns)
 * or as N = 64;
 * C a multiple of 32, 32 <= C <= 16384, with H * N * C < 2^29; H >= 1;
 * B, T >= 1; T <= T_max; and
 * for the backward H * (T + 256) * N < 2^30 (one batch's head-major gradient
 * rows are addressed with 32-bit byte offsets).
 */
#ifndef MEA_H
#define MEA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Shape of one block invocation. */
typedef struct mea_desc {
  int64_t B;      /* batch */
  int64_t T;      /* sequence length */
  int64_t C;      /* model width (x is B x T x C) */
  int64_t H;      /* heads */
  int64_t N;      /* head width */
  int64_t T_max;  /* rows of the rotary tables, >= T */
  float eps;      /* RMSNorm epsilon; the reference default is 1e-6 (fast_triton_attn.py:681) */
  int64_t N_active; /* head dimensions in use: 0 (all N), 16 with N = 32, or 16
                       or 32 with N = 64.
                       No counterpart in the reference: a head of N_active < N
                       dimensions is carried zero-padded to N (the last
                       N - N_active rows of every head in Wq, Wk, Wv, Wg and
                       columns in Wo are zero; the last N - N_active columns of
                       the rotary tables hold identity pairs, f1 = 1 and
                       f2 = 0, as the Python wrapper pads them; zero columns
                       are accepted too and give the same results, the
                       backward mapping a zero 2x2 pair block to zero rows);
                       the head RMSNorm then averages over N_active dimensions
                       and the attention scale is 1/sqrt(N_active). */
  int64_t tables_bf16; /* nonzero: every value in rows 0..T-1 of f1 and f2 is a
                          bf16 number (the caller's tables were bf16, the only
                          table dtype the reference runs with,
                          fast_triton_attn.py:110-111). mea_fwd, mea_bwd, their
                          varlen forms and mea_prefill then pack those rows
                          into a bf16 copy in the workspace (T * N * 4 more
                          bytes) that the projection epilogue reads, one
                          16-byte load per 4 features of both tables; results
                          are bitwise the same as with 0. Other values would be
                          rounded to bf16 by the copy. The stage entry points
                          and mea_decode read the fp32 tables either way. */
} mea_desc;

enum {
  MEA_OK = 0,
  MEA_ERR_NULL = -1,        /* a required pointer is NULL */
  MEA_ERR_SHAPE = -2,       /* B, T, H or T_max out of range */
  MEA_ERR_HEAD_DIM = -3,    /* N not supported */
  MEA_ERR_MODEL_DIM = -4,   /* C not supported */
  MEA_ERR_WORKSPACE = -5,   /* workspace smaller than mea_workspace_bytes() */
  MEA_ERR_ALIGN = -6,       /* a pointer is not 16-byte aligned */
  MEA_ERR_EPS = -7,         /* eps not finite and positive */
  MEA_ERR_LAUNCH = -8,      /* HIP reported an error at launch */
  MEA_ERR_ALIAS = -9,       /* dx overlaps another argument of mea_bwd */
  MEA_ERR_SCRATCH = -10,    /* shape needs more than MEA_STATIC_SCRATCH_BYTES */
  MEA_ERR_DEVICE = -11      /* no current device, or the stream is another device's */
};

/* Size of the static scratch buffer of mea_decode_static (per GPU). */
#define MEA_STATIC_SCRATCH_BYTES (16u << 20)

/* Which pass a workspace size is asked for: the forward, the backward, or a
 * backward that also writes the table gradients df1 / df2 (it needs
 * B * T * H * (2 * N + 8) more bytes: the gradient of the k projection beside
 * k, which the table gradients read after the attention backward, and one
 * fp32 dot product per (b, h, t) row of q and of k). */
enum { MEA_PASS_FWD = 0, MEA_PASS_BWD = 1, MEA_PASS_BWD_TABLES = 2 };

/*
 * Workspace bytes needed by mea_fwd (pass 0), mea_bwd (pass 1) or mea_bwd
 * with table gradients (pass 2).
 * Returns 0 when the descriptor is invalid.
 * Replaces the torch.empty transients of FusedAttentionFunction.forward
 * (fast_triton_attn.py:381,391-394,447) and .backward (:505-506,518-524,560).
 */
size_t mea_workspace_bytes(const mea_desc* d, int pass);

/*
 * Forward of the block. Replaces FusedAttentionFunction.forward
 * (fast_triton_attn.py:375-479): rms_norm_kernel (:12-34),
 * fused_qkvg_norm_rope_kernel (:36-144), aten flash attention (:438),
 * gate_repack_kernel (:146-176) and F.linear (:460).
 *
 *   x        (B, T, C) bf16
 *   wq..wg   (H*N, C)  bf16        nn.Linear.weight of q/k/v/g_proj
 *   wo       (C, H*N)  bf16        nn.Linear.weight of o_proj
 *   f1, f2   (T_max, N) fp32       rotary tables (rows 0..T-1 are read)
 *   y        (B, T, C) bf16        output
 *   o_save   (B, T, H*N) bf16      attention output, saved for mea_bwd (:465)
 *   lse_save (B, H, T) fp32        natural-log softmax normaliser (:465)
 *            o_save and lse_save may be NULL together (inference).
 */
int mea_fwd(const mea_desc* d, const void* x, const void* wq, const void* wk,
            const void* wv, const void* wg, const void* wo, const float* f1,
            const float* f2, void* y, void* o_save, float* lse_save, void* ws,
            size_t ws_bytes, void* stream);

/*
 * Backward of the block. Replaces FusedAttentionFunction.backward
 * (fast_triton_attn.py:481-675), with the exact q/k RMSNorm and rotary
 * backward (valid for any rotary table whose 2x2 pair blocks are invertible,
 * which every RoPE/YaRN table with a positive temperature is).
 *
 *   dy                  (B, T, C) bf16     gradient of y
 *   x, wq..wo, f1, f2   as in mea_fwd
 *   o_save, lse_save    as written by mea_fwd
 *   dx                  (B, T, C) bf16     out
 *   dwq, dwk, dwv, dwg  (H*N, C) bf16      out
 *   dwo                 (C, H*N) bf16      out
 *   df1, df2            (T_max, N) fp32    out, rows 0..T-1 written; both may
 *                                          be NULL to skip the table gradient.
 *                                          Given, they need the workspace of
 *                                          MEA_PASS_BWD_TABLES; the sum over
 *                                          batch and heads runs in a fixed
 *                                          order (deterministic)
 *
 * dx also holds the gradient of the gate projection's output (rows of H*N
 * values at stride C) until the last kernel overwrites it with the result,
 * when H*N <= C <= 1024, and partial results of the last kernel's feature
 * groups when C > 1024; it must not overlap any other argument
 * (MEA_ERR_ALIAS).
 */
int mea_bwd(const mea_desc* d, const void* dy, const void* x, const void* wq,
            const void* wk, const void* wv, const void* wg, const void* wo,
            const float* f1, const float* f2, const void* o_save,
            const float* lse_save, void* dx, void* dwq, void* dwk, void* dwv,
            void* dwg, void* dwo, float* df1, float* df2, void* ws,
            size_t ws_bytes, void* stream);

/*
 * Packed variable-length sequences (the cum_seq slots of the reference's
 * aten flash call, fast_triton_attn.py:431-432, which it leaves unused):
 * mea_fwd / mea_bwd over nseq sequences stored back to back, attention
 * causal inside each sequence and rotary rows counted from each sequence's
 * first token.
 *
 *   d->B                 1; d->T = total tokens = cu_seqlens[nseq]
 *   cu_seqlens           (nseq + 1) int32, device: 0 = cu[0] <= cu[1] <= ...
 *   max_len              >= every cu[s+1] - cu[s]; d->T_max >= max_len
 *   x, y, dy, dx         (T, C) bf16;  o_save (T, H*N);  lse_save (H, T)
 *   df1, df2             rows 0 .. max_len-1 written
 *   workspace            mea_workspace_bytes(d, pass) with d->T_max raised to
 *                        d->T if smaller (the sizes depend on B, T, C, H, N)
 * Everything else as in mea_fwd / mea_bwd.
 */
int mea_fwd_varlen(const mea_desc* d, const int32_t* cu_seqlens, int32_t nseq,
                   int32_t max_len, const void* x, const void* wq,
                   const void* wk, const void* wv, const void* wg,
                   const void* wo, const float* f1, const float* f2, void* y,
                   void* o_save, float* lse_save, void* ws, size_t ws_bytes,
                   void* stream);
int mea_bwd_varlen(const mea_desc* d, const int32_t* cu_seqlens, int32_t nseq,
                   int32_t max_len, const void* dy, const void* x,
                   const void* wq, const void* wk, const void* wv,
                   const void* wg, const void* wo, const float* f1,
                   const float* f2, const void* o_save, const float* lse_save,
                   void* dx, void* dwq, void* dwk, void* dwv, void* dwg,
                   void* dwo, float* df1, float* df2, void* ws,
                   size_t ws_bytes, void* stream);

/*
 * Prefill of a KV cache: the inference forward of a whole prompt (mea_fwd
 * with o_save = lse_save = NULL, same workspace) that also copies the
 * prompt's k and v rows, exactly as the attention consumed them, into rows
 * 0..T-1 of the caller's caches. No counterpart in the reference, which
 * trains only; it is the prompt half of the decode step below.
 *
 *   x .. f2, y           as in mea_fwd (d->T = prompt length)
 *   k_cache, v_cache     (B, H, cache_T, N) bf16; k rows are RMS-normalised
 *                        and rotated, v rows plain; T <= cache_T <= T_max
 */
int mea_prefill(const mea_desc* d, const void* x, const void* wq,
                const void* wk, const void* wv, const void* wg,
                const void* wo, const float* f1, const float* f2, void* y,
                void* k_cache, void* v_cache, int64_t cache_T, void* ws,
                size_t ws_bytes, void* stream);

/*
 * Workspace bytes needed by mea_decode (d->T = cache capacity). Returns 0
 * when the descriptor is invalid.
 */
size_t mea_decode_workspace_bytes(const mea_desc* d);

/*
 * KV-cache decode step: one new token per sequence. No counterpart in the
 * reference (training only); the block math is that of mea_fwd for the last
 * row of a causal sequence. The new token of sequence b sits at position
 * pos[b]: it reads rotary row pos[b], its k and v are written to cache row
 * pos[b], and it attends to cache rows 0..pos[b] (its own included).
 *
 *   d->T              cache capacity Tc (<= d->T_max)
 *   x                 (B, C) bf16            the new tokens
 *   wq .. wo, f1, f2  as in mea_fwd
 *   pos               (B) int32, device      0 <= pos[b] < Tc; values outside
 *                                            are clamped to that range
 *   k_cache, v_cache  (B, H, Tc, N) bf16     rows 0..pos[b]-1 hold the
 *                                            earlier tokens (mea_prefill or
 *                                            earlier steps); row pos[b] is
 *                                            written
 *   y                 (B, C) bf16            out
 */
int mea_decode(const mea_desc* d, const void* x, const void* wq,
               const void* wk, const void* wv, const void* wg, const void* wo,
               const float* f1, const float* f2, const int32_t* pos,
               void* k_cache, void* v_cache, void* y, void* ws,
               size_t ws_bytes, void* stream);

/*
 * mea_decode without a workspace argument: the step's scratch (the new
 * tokens' projections, q/k/v/gate rows and the split-attention partials,
 * mea_decode_workspace_bytes(d) bytes) lives in a static device buffer of
 * MEA_STATIC_SCRATCH_BYTES inside the library, so a call allocates nothing
 * and needs no caller-provided scratch. No counterpart in the reference; it
 * is for callers that cannot allocate device memory: serving loops with a
 * fixed memory budget, code under graph capture, harnesses that forbid
 * allocation. Shapes whose scratch exceeds the buffer return
 * MEA_ERR_SCRATCH (16 MiB covers, e.g., B * H * N * C up to ~10^9 with
 * 4H*N*B*4 bytes of projections; mea_decode_workspace_bytes tells).
 *
 * Runs on the calling thread's current device, which must be the stream's
 * (else MEA_ERR_DEVICE); the buffer's address on each device is looked up
 * on the first call there. Every call on one GPU shares that GPU's buffer:
 * calls that may overlap in time on one GPU (different streams, or threads
 * without ordering) race and must be serialised by the caller. Arguments
 * and results otherwise exactly as mea_decode.
 */
int mea_decode_static(const mea_desc* d, const void* x, const void* wq,
                      const void* wk, const void* wv, const void* wg,
                      const void* wo, const float* f1, const float* f2,
                      const int32_t* pos, void* k_cache, void* v_cache,
                      void* y, void* stream);

/*
 * Stage: input RMSNorm + q/k/v/g projection + per-head q/k RMSNorm + rotary +
 * sigmoid. Replaces rms_norm_kernel(_recompute) and
 * fused_qkvg_norm_rope_kernel(_recompute) (fast_triton_attn.py:12-144,
 * 181-332).
 *
 *   q, k, v  (B, H, T, N) bf16   rotated q/k, plain v
 *   sig      (B, T, H*N) bf16    sigmoid(a_g)
 *   rx       (B, T) fp32         1/rms of x rows          (may be NULL)
 *   rq, rk   (B, H, T) fp32      1/rms of a_q, a_k rows   (may be NULL)
 */
int mea_qkvg_proj(const mea_desc* d, const void* x, const void* wq,
                  const void* wk, const void* wv, const void* wg,
                  const float* f1, const float* f2, void* q, void* k, void* v,
                  void* sig, float* rx, float* rq, float* rk, void* stream);

/*
 * Stage: causal flash attention forward with scale 1/sqrt(N). Replaces
 * aten._scaled_dot_product_flash_attention (fast_triton_attn.py:425-444).
 *
 *   q, k, v  (B, H, T, N) bf16
 *   o        (B, T, H*N) bf16     out
 *   lse      (B, H, T) fp32       out (may be NULL)
 */
int mea_attn_fwd(const mea_desc* d, const void* q, const void* k,
                 const void* v, void* o, float* lse, void* stream);

/*
 * Stage: output gate and projection, y = (o * sig) W_o^T. Replaces
 * gate_repack_kernel (fast_triton_attn.py:146-176) and F.linear (:460).
 *
 *   o, sig   (B, T, H*N) bf16
 *   wo       (C, H*N) bf16
 *   y        (B, T, C) bf16       out
 */
int mea_gate_oproj(const mea_desc* d, const void* o, const void* sig,
                   const void* wo, void* y, void* stream);

/*
 * Stage: the first half of mea_bwd, stopping before the weight and input
 * gradients. Runs the recompute (fast_triton_attn.py:500-570), the o_proj
 * and gate backward (:577-584, :601), the aten flash backward (:586-596)
 * and the exact q/k RMSNorm + rotary backward (in place of :603-620), and
 * returns what the reference holds at :641 as the inputs of its dW / dx
 * GEMMs, plus the attention-backward operands:
 *
 *   daq, dak, dav   (B, H, T, N) bf16   rx * dL/da_q, rx * dL/da_k, rx * dL/da_v
 *   dag             (B, T, H*N) bf16    rx * dL/da_g
 *   dO              (B, H, T, N) bf16   dL/dO (the attention output's gradient)
 *   delta           (B, H, T) fp32      rowsum(dO * O)
 *   df1, df2        as in mea_bwd (may be NULL together)
 *
 * rx = 1/rms(x) per token; a_p = rmsnorm(x) W_p^T. All other arguments and
 * the workspace as in mea_bwd. Used to check the backward per row.
 */
int mea_bwd_stage_grads(const mea_desc* d, const void* dy, const void* x,
                        const void* wq, const void* wk, const void* wv,
                        const void* wg, const void* wo, const float* f1,
                        const float* f2, const void* o_save,
                        const float* lse_save, void* daq, void* dak, void* dav,
                        void* dag, void* dO, float* delta, float* df1,
                        float* df2, void* ws, size_t ws_bytes, void* stream);

/* Text for a status code returned by any entry point. */
const char* mea_strerror(int code);

/*
 * Kernel timing diagnostics (no counterpart in the reference; used by the
 * benchmark). While enabled, every kernel the library launches is bracketed
 * by a pair of HIP events recorded on the stream it is launched on.
 *   mea_profile_enable(1)  clears previous records and starts recording;
 *   mea_profile_enable(0)  stops recording (records are kept);
 *   mea_profile_read(k, &count, &total_ms) waits for the recorded events of
 *     kernel k and returns its launch count and summed duration;
 *   mea_profile_kernel_name(k) names kernel k, NULL past the last one;
 *   mea_profile_select(k) limits recording to kernel k (its launches alone
 *     are bracketed; each event pair adds about 8 us of queue time, so a
 *     caller timing a whole step can keep the other launches bare), k = -1
 *     (the initial state) records every kernel. MEA_ERR_NULL for any other k.
 * Recording is process-wide and serialised by a mutex.
 */
int mea_profile_enable(int on);
int mea_profile_read(int kernel, int* count, double* total_ms);
const char* mea_profile_kernel_name(int kernel);
int mea_profile_select(int kernel);

/* Library version string. */
const char* mea_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MEA_H */
