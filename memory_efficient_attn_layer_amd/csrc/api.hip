// C ABI of the attention block: argument validation, workspace layout and
// the launch sequence of each pass. Declarations and contracts: include/mea.h.
#include <math.h>
#include <stdint.h>

#include <mutex>
#include <utility>
#include <vector>

#include "../../include/mea.h"
#include "kernels.h"

namespace {

using mea::bf16_bits;

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Byte offsets of every transient inside the workspace.
struct Layout {
  size_t q, k, v, sig, tpos, o, qkn;         // forward (tpos: packed sequences only)
  size_t rot;                                // packed bf16 tables (tables_bf16 only)
  size_t wpk;                                // k-slab-major copies of Wq, Wk, Wv, Wg
  size_t dO, daq, dag;                       // backward (da_k, da_v overwrite k, v)
  size_t rx, rq, rk, delta, woT, wcatT, part;
  size_t dak, dotq, dotk;                    // table gradients (MEA_PASS_BWD_TABLES): da_k beside k, row dots
  size_t total;
};

Layout make_layout(const mea_desc& d, int pass) {
  const size_t M = (size_t)(d.B * d.T), HN = (size_t)(d.H * d.N), C = (size_t)d.C;
  const size_t act = align_up(M * HN * 2), stat = align_up(M * (size_t)d.H * 4);
  Layout L = {};
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes); return o; };
  L.q = take(act);
  L.k = take(act);
  L.v = take(act);
  L.sig = take(act);
  L.tpos = take(M * 4);
  // Rows 0 .. T-1 (packed sequences: max_len <= T) of both tables, 8 bytes
  // per (row, feature).
  if (d.tables_bf16 != 0) L.rot = take((size_t)d.T * (size_t)d.N * 4);
  L.wpk = take(4 * HN * C * 2);
  if (pass == MEA_PASS_FWD) {
    L.o = take(act);
    L.qkn = take(2 * sizeof(float));
  } else {
    L.dO = take(act);
    L.daq = take(act);
    // da_g lives in the caller's dx buffer when its rows fit (HN <= C) and
    // dx is written once, at the end (C <= 1024; wider rows take dx as
    // scratch for their feature groups).
    L.dag = HN <= C && C <= 1024 ? 0 : take(act);
    L.rx = take(M * 4);
    L.rq = take(stat);
    L.rk = take(stat);
    L.delta = take(stat);
    L.woT = take(HN * C * 2);
    L.wcatT = take(C * 4 * HN * 2);
    L.part = take((size_t)mea::dw_splits((int)M, (int)C, (int)HN) * (4 * HN * C + C * HN) * 4);
    if (pass == MEA_PASS_BWD_TABLES) {
      // The table gradients read k after the dK/dV kernel: da_k gets its own
      // rows, and the kernels leave one dot product per (b, h, t) row.
      L.dak = take(act);
      L.dotq = take(stat);
      L.dotk = take(stat);
    }
  }
  L.total = off;
  return L;
}

// Widest model: the kernels walk C in 32-wide k-slabs and 1024-wide feature
// groups, so any multiple of 32 works; the cap keeps every 32-bit slab and
// row offset far from overflow.
constexpr int64_t kMaxC = 16384;

int validate(const mea_desc* d, int pass) {
  if (d == nullptr) return MEA_ERR_NULL;
  if (d->B < 1 || d->T < 1 || d->H < 1 || d->T_max < d->T) return MEA_ERR_SHAPE;
  if (d->N != 32 && d->N != 64 && d->N != 128 && d->N != 256) return MEA_ERR_HEAD_DIM;
  // 32-wide heads: the projection tiles hold head pairs.
  if (d->N == 32 && d->H % 2 != 0) return MEA_ERR_HEAD_DIM;
  if (d->N_active != 0 && d->N_active != d->N && !(d->N == 32 && d->N_active == 16) &&
      !(d->N == 64 && (d->N_active == 16 || d->N_active == 32)))
    return MEA_ERR_HEAD_DIM;
  if (d->C < 32 || d->C % 32 != 0) return MEA_ERR_MODEL_DIM;
  const bool bwd = pass == MEA_PASS_BWD || pass == MEA_PASS_BWD_TABLES;
  if (d->C > kMaxC) return MEA_ERR_MODEL_DIM;
  if (!(d->eps > 0.f) || !isfinite(d->eps)) return MEA_ERR_EPS;
  // All row and element indices used by the kernels fit in 31 bits.
  const int64_t M = d->B * d->T, HN = d->H * d->N;
  if (M >= (INT64_C(1) << 31) || HN >= 65536 || d->B * d->H * d->T >= (INT64_C(1) << 31) ||
      d->T_max * d->N >= (INT64_C(1) << 31))
    return MEA_ERR_SHAPE;
  // Element indices into the four stacked weight matrices (4 * H*N * C) are
  // 32-bit.
  if (HN * d->C >= (INT64_C(1) << 29)) return MEA_ERR_MODEL_DIM;
  // The backward GEMMs address a head-major gradient with 32-bit byte
  // offsets spanning up to one head of one batch plus a few hundred rows.
  if (bwd && d->H * (d->T + 256) * d->N >= (INT64_C(1) << 30)) return MEA_ERR_SHAPE;
  return MEA_OK;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Packed sequences: sequence s holds tokens cu[s] .. cu[s+1]-1 of a B = 1,
// T = total batch; no sequence is longer than max_len.
struct Varlen {
  const int* cu;
  int nseq, max_len;
};

// validate() for a pass; with packed sequences the rotary tables need only
// max_len rows (T is the total token count), B must be 1 and cu a 4-byte
// aligned device array of nseq + 1 offsets.
int validate_pass(const mea_desc* d, int pass, const Varlen* var) {
  if (var == nullptr) return validate(d, pass);
  if (d == nullptr) return MEA_ERR_NULL;
  mea_desc dd = *d;
  dd.T_max = d->T_max > d->T ? d->T_max : d->T;
  const int rc = validate(&dd, pass);
  if (rc != MEA_OK) return rc;
  if (d->B != 1 || var->nseq < 1 || var->max_len < 1 || var->max_len > d->T || d->T_max < var->max_len)
    return MEA_ERR_SHAPE;
  if (var->cu == nullptr) return MEA_ERR_NULL;
  if (((uintptr_t)var->cu & 3u) != 0) return MEA_ERR_ALIGN;
  return MEA_OK;
}

// Whether byte ranges [a, a + na) and [b, b + nb) overlap (null b: no).
bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  if (b == nullptr) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + nb && y < x + na;
}

int check_ptrs(std::initializer_list<const void*> ps) {
  for (const void* p : ps) {
    if (p == nullptr) return MEA_ERR_NULL;
    if (!aligned16(p)) return MEA_ERR_ALIGN;
  }
  return MEA_OK;
}

#define MEA_TRY(expr)                                  \
  do {                                                 \
    if ((expr) != hipSuccess) return MEA_ERR_LAUNCH;   \
  } while (0)

template <class T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<unsigned char*>(ws) + off);
}

// ---- kernel timing diagnostics -------------------------------------------
enum KernelId {
  K_QKVG_PROJ, K_ATTN_FWD, K_GATE_OPROJ, K_TRANSPOSE, K_ZERO, K_DZ_GATE_BWD,
  K_ATTN_BWD_DQ, K_ATTN_BWD_DKDV, K_DW_PARTIAL, K_DW_REDUCE, K_DX,
  K_ATTN_DECODE, K_DECODE_COMBINE, K_SKINNY_GEMM, K_DECODE_PROJ, K_TABLE_GRAD, K_ROTARY_PACK, K_WEIGHT_PACK, K_COUNT
};
const char* const kKernelNames[K_COUNT] = {
    "qkvg_proj", "attn_fwd", "gate_oproj", "transpose", "zero_f32", "dz_gate_bwd",
    "attn_bwd_dq", "attn_bwd_dkdv", "dw_partial", "dw_reduce", "dx",
    "attn_decode", "attn_decode_combine", "skinny_gemm", "decode_proj", "table_grad", "rotary_pack", "weight_pack"};

struct ProfRec {
  int kernel;
  hipEvent_t a, b;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
int g_prof_only = -1;  // record only this kernel (-1: all)
std::vector<ProfRec> g_prof;
std::vector<hipEvent_t> g_pool;

hipEvent_t pool_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Runs `launch` (which returns a hipError_t); when profiling is on, brackets
// it with events on stream s.
template <class F>
hipError_t timed(int kernel, hipStream_t s, F launch) {
  std::unique_lock<std::mutex> lk(g_prof_mu);
  if (!g_prof_on || (g_prof_only >= 0 && kernel != g_prof_only)) {
    lk.unlock();
    return launch();
  }
  hipEvent_t a = pool_event(), b = pool_event();
  if (a == nullptr || b == nullptr) return hipErrorOutOfMemory;
  (void)hipEventRecord(a, s);
  const hipError_t e = launch();
  (void)hipEventRecord(b, s);
  g_prof.push_back({kernel, a, b});
  return e;
}

}  // namespace

extern "C" {

size_t mea_workspace_bytes(const mea_desc* d, int pass) {
  if (pass != MEA_PASS_FWD && pass != MEA_PASS_BWD && pass != MEA_PASS_BWD_TABLES) return 0;
  if (validate(d, pass) != MEA_OK) return 0;
  return make_layout(*d, pass).total;
}

}  // extern "C"

namespace {

// log2(e)/sqrt(N): the block stores q in these units, so the attention's
// logits come out of the MFMA ready for exp2.
float q_log2_scale(int64_t N) { return (float)(1.4426950408889634 / sqrt((double)N)); }
// Head dimensions in use (the rest of each head is zero padding).
int64_t n_active(const mea_desc* d) { return d->N_active != 0 ? d->N_active : d->N; }

// Launch sequence pieces; the public entry points validate before calling.
// Packed tables (tabp, tab_rows rows; see pack_tables) or null: f1 / f2.
// wpk: the k-slab-major weight copies (see pack_weights) or null: the
// row-major weights wq .. wg.
int proj_launch(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
                const float* f1, const float* f2, void* q, void* k, void* v, void* sig, float* rx, float* rq,
                float* rk, float qscale, float* qk_norm2, const int* tpos, const bf16_bits* tabp, int tab_rows,
                const bf16_bits* wpk, void* stream) {
  mea::ProjParams p;
  p.x = static_cast<const bf16_bits*>(x);
  const size_t wsz = (size_t)(d->H * d->N) * (size_t)d->C;
  p.wq = wpk != nullptr ? wpk : static_cast<const bf16_bits*>(wq);
  p.wk = wpk != nullptr ? wpk + wsz : static_cast<const bf16_bits*>(wk);
  p.wv = wpk != nullptr ? wpk + 2 * wsz : static_cast<const bf16_bits*>(wv);
  p.wg = wpk != nullptr ? wpk + 3 * wsz : static_cast<const bf16_bits*>(wg);
  p.w_row = wpk != nullptr ? 32 : (int)d->C;
  p.w_slab = wpk != nullptr ? 32 * d->H * d->N : 32;
  p.f1 = f1;
  p.f2 = f2;
  p.tabp = tabp;
  p.q = static_cast<bf16_bits*>(q);
  p.k = static_cast<bf16_bits*>(k);
  p.v = static_cast<bf16_bits*>(v);
  p.sig = static_cast<bf16_bits*>(sig);
  p.rx = rx;
  p.rq = rq;
  p.rk = rk;
  p.qk_norm2 = qk_norm2;
  p.qscale = qscale;
  p.tpos = tpos;
  p.t_max = tabp != nullptr ? tab_rows : (int)d->T_max;
  p.M = (int)(d->B * d->T);
  p.T = (int)d->T;
  p.C = (int)d->C;
  p.H = (int)d->H;
  p.eps = d->eps;
  p.inv_n = 1.0f / (float)n_active(d);
  hipStream_t s = static_cast<hipStream_t>(stream);
  MEA_TRY(timed(K_QKVG_PROJ, s, [&] { return mea::launch_qkvg_proj(p, (int)d->N, s); }));
  return MEA_OK;
}

int proj_impl(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
              const float* f1, const float* f2, void* q, void* k, void* v, void* sig, float* rx, float* rq,
              float* rk, float qscale, float* qk_norm2, void* stream) {
  int rc = validate(d, MEA_PASS_FWD);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({x, wq, wk, wv, wg, f1, f2, q, k, v, sig});
  if (rc != MEA_OK) return rc;
  return proj_launch(d, x, wq, wk, wv, wg, f1, f2, q, k, v, sig, rx, rq, rk, qscale, qk_norm2, nullptr, nullptr, 0,
                     nullptr, stream);
}

}  // namespace

extern "C" {

int mea_qkvg_proj(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv,
                  const void* wg, const float* f1, const float* f2, void* q, void* k, void* v, void* sig,
                  float* rx, float* rq, float* rk, void* stream) {
  return proj_impl(d, x, wq, wk, wv, wg, f1, f2, q, k, v, sig, rx, rq, rk, 1.0f, nullptr, stream);
}

}  // extern "C"

namespace {

int attn_fwd_launch(const mea_desc* d, const void* q, const void* k, const void* v, void* o, float* lse, float sl2e,
                    const float* qk_norm2, const Varlen* var, void* stream) {
  mea::AttnFwdParams p;
  p.q = static_cast<const bf16_bits*>(q);
  p.k = static_cast<const bf16_bits*>(k);
  p.v = static_cast<const bf16_bits*>(v);
  p.o = static_cast<bf16_bits*>(o);
  p.lse = lse;
  p.B = (int)d->B;
  p.H = (int)d->H;
  p.T = (int)d->T;
  p.sl2e = sl2e;
  p.qk_norm2 = qk_norm2;
  p.cu = var != nullptr ? var->cu : nullptr;
  p.nseq = var != nullptr ? var->nseq : 0;
  p.max_len = var != nullptr ? var->max_len : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  MEA_TRY(timed(K_ATTN_FWD, s, [&] { return mea::launch_attn_fwd(p, (int)d->N, s); }));
  return MEA_OK;
}

int attn_fwd_impl(const mea_desc* d, const void* q, const void* k, const void* v, void* o, float* lse, float sl2e,
                  const float* qk_norm2, void* stream) {
  int rc = validate(d, MEA_PASS_FWD);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({q, k, v, o});
  if (rc != MEA_OK) return rc;
  return attn_fwd_launch(d, q, k, v, o, lse, sl2e, qk_norm2, nullptr, stream);
}

int gate_oproj_launch(const mea_desc* d, const void* o, const void* sig, const void* wo, void* y, void* stream) {
  mea::OprojParams p;
  p.o = static_cast<const bf16_bits*>(o);
  p.sig = static_cast<const bf16_bits*>(sig);
  p.wo = static_cast<const bf16_bits*>(wo);
  p.y = static_cast<bf16_bits*>(y);
  p.M = (int)(d->B * d->T);
  p.C = (int)d->C;
  p.HN = (int)(d->H * d->N);
  hipStream_t s = static_cast<hipStream_t>(stream);
  MEA_TRY(timed(K_GATE_OPROJ, s, [&] { return mea::launch_gate_oproj(p, s); }));
  return MEA_OK;
}

}  // namespace

extern "C" {

int mea_attn_fwd(const mea_desc* d, const void* q, const void* k, const void* v, void* o, float* lse,
                 void* stream) {
  return attn_fwd_impl(d, q, k, v, o, lse, q_log2_scale(n_active(d)), nullptr, stream);
}

int mea_gate_oproj(const mea_desc* d, const void* o, const void* sig, const void* wo, void* y, void* stream) {
  int rc = validate(d, MEA_PASS_FWD);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({o, sig, wo, y});
  if (rc != MEA_OK) return rc;
  return gate_oproj_launch(d, o, sig, wo, y, stream);
}

}  // extern "C"

namespace {

// With d->tables_bf16: packs the table rows the projection reads (0 .. T-1;
// packed sequences 0 .. max_len-1) into the workspace and returns the copy in
// *tabp and its row count in *rows; otherwise *tabp = null.
hipError_t pack_tables(const mea_desc* d, const Varlen* var, const float* f1, const float* f2, void* ws,
                       const Layout& L, hipStream_t s, const bf16_bits** tabp, int* rows) {
  *tabp = nullptr;
  *rows = 0;
  if (d->tables_bf16 == 0) return hipSuccess;
  bf16_bits* out = at<bf16_bits>(ws, L.rot);
  const int n = var != nullptr ? var->max_len : (int)d->T;
  const hipError_t e = timed(K_ROTARY_PACK, s, [&] { return mea::launch_rotary_pack(f1, f2, n, (int)d->N, out, s); });
  *tabp = out;
  *rows = n;
  return e;
}

// Wq, Wk, Wv, Wg into k-slab-major copies in the workspace (2 * 4HN * C
// bytes) for the projection's weight-slab loads; returns the copy.
hipError_t pack_weights(const mea_desc* d, const void* wq, const void* wk, const void* wv, const void* wg, void* ws,
                        const Layout& L, hipStream_t s, const bf16_bits** wpk) {
  bf16_bits* out = at<bf16_bits>(ws, L.wpk);
  mea::WcatPackParams wp{static_cast<const bf16_bits*>(wq), static_cast<const bf16_bits*>(wk),
                         static_cast<const bf16_bits*>(wv), static_cast<const bf16_bits*>(wg), out,
                         (int)(d->H * d->N), (int)d->C};
  *wpk = out;
  return timed(K_WEIGHT_PACK, s, [&] { return mea::launch_wslab_pack(wp, s); });
}

int fwd_impl(const mea_desc* d, const Varlen* var, const void* x, const void* wq, const void* wk, const void* wv,
             const void* wg, const void* wo, const float* f1, const float* f2, void* y, void* o_save,
             float* lse_save, void* ws, size_t ws_bytes, void* stream) {
  int rc = validate_pass(d, MEA_PASS_FWD, var);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({x, wq, wk, wv, wg, wo, f1, f2, y, ws});
  if (rc != MEA_OK) return rc;
  if ((o_save == nullptr) != (lse_save == nullptr)) return MEA_ERR_NULL;
  if (o_save != nullptr && !aligned16(o_save)) return MEA_ERR_ALIGN;
  const Layout L = make_layout(*d, MEA_PASS_FWD);
  if (ws_bytes < L.total) return MEA_ERR_WORKSPACE;
  void* q = at<void>(ws, L.q);
  void* k = at<void>(ws, L.k);
  void* v = at<void>(ws, L.v);
  void* sig = at<void>(ws, L.sig);
  void* o = o_save != nullptr ? o_save : at<void>(ws, L.o);
  // q is stored in log2 units; the projection records the largest q and k
  // row norms so the attention can take its fixed-offset softmax.
  float* qkn = at<float>(ws, L.qkn);
  MEA_TRY(timed(K_ZERO, static_cast<hipStream_t>(stream),
                [&] { return mea::launch_zero_f32(qkn, 2, static_cast<hipStream_t>(stream)); }));
  const float qs = q_log2_scale(n_active(d));
  int* tpos = nullptr;
  if (var != nullptr) {
    tpos = at<int>(ws, L.tpos);
    MEA_TRY(mea::launch_token_positions(var->cu, var->nseq, (int)d->T, tpos, static_cast<hipStream_t>(stream)));
  }
  const bf16_bits* tabp;
  int tab_rows;
  MEA_TRY(pack_tables(d, var, f1, f2, ws, L, static_cast<hipStream_t>(stream), &tabp, &tab_rows));
  const bf16_bits* wpk;
  MEA_TRY(pack_weights(d, wq, wk, wv, wg, ws, L, static_cast<hipStream_t>(stream), &wpk));
  rc = proj_launch(d, x, wq, wk, wv, wg, f1, f2, q, k, v, sig, nullptr, nullptr, nullptr, qs, qkn, tpos, tabp,
                   tab_rows, wpk, stream);
  if (rc != MEA_OK) return rc;
  rc = attn_fwd_launch(d, q, k, v, o, lse_save, 1.0f, qkn, var, stream);
  if (rc != MEA_OK) return rc;
  return gate_oproj_launch(d, o, sig, wo, y, stream);
}

// Buffers of one backward pass inside the workspace (and dx).
struct BwdBufs {
  bf16_bits *q, *k, *v, *sig, *dO, *daq, *dak, *dag, *woT, *wcatT;
  float *rx, *rq, *rk, *delta, *part;
  float *dotq, *dotk;  // table gradients only, else null
  int ld_dag;
};

// tables: the backward also writes df1 / df2 (MEA_PASS_BWD_TABLES layout).
BwdBufs bwd_bufs(const mea_desc* d, void* ws, void* dag_ext, int ld_dag_ext, bool tables) {
  const Layout L = make_layout(*d, tables ? MEA_PASS_BWD_TABLES : MEA_PASS_BWD);
  BwdBufs b;
  b.q = at<bf16_bits>(ws, L.q);
  b.k = at<bf16_bits>(ws, L.k);
  b.v = at<bf16_bits>(ws, L.v);
  b.sig = at<bf16_bits>(ws, L.sig);
  b.dO = at<bf16_bits>(ws, L.dO);
  b.daq = at<bf16_bits>(ws, L.daq);
  b.dag = dag_ext != nullptr ? static_cast<bf16_bits*>(dag_ext) : at<bf16_bits>(ws, L.dag);
  b.ld_dag = dag_ext != nullptr ? ld_dag_ext : (int)(d->H * d->N);
  b.woT = at<bf16_bits>(ws, L.woT);
  b.wcatT = at<bf16_bits>(ws, L.wcatT);
  b.rx = at<float>(ws, L.rx);
  b.rq = at<float>(ws, L.rq);
  b.rk = at<float>(ws, L.rk);
  b.delta = at<float>(ws, L.delta);
  b.part = at<float>(ws, L.part);
  // da_k overwrites k (its last reader is the dK/dV kernel itself) unless
  // the table gradients still need k.
  b.dak = tables ? at<bf16_bits>(ws, L.dak) : b.k;
  b.dotq = tables ? at<float>(ws, L.dotq) : nullptr;
  b.dotk = tables ? at<float>(ws, L.dotk) : nullptr;
  return b;
}

// First half of the backward: weight transposes, the recompute of q, k, v,
// sigmoid(g) and the RMS statistics, dZ with the gate backward, and the
// attention backward with the exact q/k chain, and the table gradients when
// df1 is set. Leaves the projection-output gradients (rows scaled by rx) in
// bf.daq, bf.dak, bf.v (da_v) and bf.dag, and dO / delta in their buffers.
int bwd_front(const mea_desc* d, const Varlen* var, const void* dy, const void* x, const void* wq, const void* wk,
              const void* wv, const void* wg, const void* wo, const float* f1, const float* f2, const void* o_save,
              const float* lse_save, float* df1, float* df2, const BwdBufs& bf, void* ws, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = (int)(d->B * d->T), T = (int)d->T, H = (int)d->H, N = (int)d->N, C = (int)d->C;
  const int HN = H * N;
  const Layout L = make_layout(*d, df1 != nullptr ? MEA_PASS_BWD_TABLES : MEA_PASS_BWD);

  // Weight transposes (k-contiguous B operands for dZ and dx).
  MEA_TRY(timed(K_TRANSPOSE, s, [&] { return mea::launch_transpose_slabs(static_cast<const bf16_bits*>(wo), C, HN, HN, bf.woT, s); }));
  {
    mea::WcatPackParams wp{static_cast<const bf16_bits*>(wq), static_cast<const bf16_bits*>(wk),
                           static_cast<const bf16_bits*>(wv), static_cast<const bf16_bits*>(wg), bf.wcatT, HN, C};
    MEA_TRY(timed(K_TRANSPOSE, s, [&] { return mea::launch_wcat_pack(wp, s); }));
  }
  // Recompute q, k, v, sigmoid(g) and the three RMS statistics.
  const float qs = q_log2_scale(n_active(d));
  int* tpos = nullptr;
  if (var != nullptr) {
    tpos = at<int>(ws, L.tpos);
    MEA_TRY(mea::launch_token_positions(var->cu, var->nseq, T, tpos, s));
  }
  const bf16_bits* tabp;
  int tab_rows;
  MEA_TRY(pack_tables(d, var, f1, f2, ws, L, s, &tabp, &tab_rows));
  const bf16_bits* wpk;
  MEA_TRY(pack_weights(d, wq, wk, wv, wg, ws, L, s, &wpk));
  int rc = proj_launch(d, x, wq, wk, wv, wg, f1, f2, bf.q, bf.k, bf.v, bf.sig, bf.rx, bf.rq, bf.rk, qs, nullptr, tpos,
                       tabp, tab_rows, wpk, stream);
  if (rc != MEA_OK) return rc;

  mea::DzParams dz;
  dz.dy = static_cast<const bf16_bits*>(dy);
  dz.woT = bf.woT;
  dz.o = static_cast<const bf16_bits*>(o_save);
  dz.sig = bf.sig;
  dz.rx = bf.rx;
  dz.dO = bf.dO;
  dz.dag = bf.dag;
  dz.delta = bf.delta;
  dz.M = M;
  dz.T = T;
  dz.C = C;
  dz.H = H;
  dz.N = N;
  dz.ld_dag = bf.ld_dag;
  MEA_TRY(timed(K_DZ_GATE_BWD, s, [&] { return mea::launch_dz_gate_bwd(dz, s); }));

  mea::AttnBwdParams ab;
  ab.q = bf.q;
  ab.k = bf.k;
  ab.v = bf.v;
  ab.dO = bf.dO;
  ab.lse = lse_save;
  ab.delta = bf.delta;
  ab.f1 = f1;
  ab.f2 = f2;
  ab.rx = bf.rx;
  ab.rq = bf.rq;
  ab.rk = bf.rk;
  ab.daq = bf.daq;
  ab.dak = bf.dak;
  ab.dav = bf.v;
  ab.dotq = bf.dotq;
  ab.dotk = bf.dotk;
  ab.B = (int)d->B;
  ab.H = H;
  ab.T = T;
  ab.scale = (float)(1.0 / sqrt((double)n_active(d)));
  ab.sl2e = 1.0f;  // q was stored in log2 units by the recompute above
  ab.qscale = qs;
  ab.inv_n = 1.0f / (float)n_active(d);
  ab.cu = var != nullptr ? var->cu : nullptr;
  ab.nseq = var != nullptr ? var->nseq : 0;
  ab.max_len = var != nullptr ? var->max_len : 0;
  MEA_TRY(timed(K_ATTN_BWD_DQ, s, [&] { return mea::launch_attn_bwd_dq(ab, N, s); }));
  MEA_TRY(timed(K_ATTN_BWD_DKDV, s, [&] { return mea::launch_attn_bwd_dkdv(ab, N, s); }));
  if (df1 != nullptr) {
    mea::TableGradParams tg;
    tg.q = bf.q;
    tg.daq = bf.daq;
    tg.k = bf.k;
    tg.dak = bf.dak;
    tg.dotq = bf.dotq;
    tg.dotk = bf.dotk;
    tg.rq = bf.rq;
    tg.rk = bf.rk;
    tg.rx = bf.rx;
    tg.f1 = f1;
    tg.f2 = f2;
    tg.df1 = df1;
    tg.df2 = df2;
    tg.qscale = qs;
    tg.inv_n = ab.inv_n;
    tg.B = (int)d->B;
    tg.H = H;
    tg.T = T;
    // Table rows the block touches: positions 0 .. T-1 (packed: max_len - 1).
    tg.rows = var != nullptr ? var->max_len : T;
    tg.cu = ab.cu;
    tg.nseq = ab.nseq;
    MEA_TRY(timed(K_TABLE_GRAD, s, [&] { return mea::launch_table_grad(tg, N, s); }));
  }
  return MEA_OK;
}

// Pointer checks shared by the backward entry points.
int bwd_check(const mea_desc* d, const Varlen* var, std::initializer_list<const void*> ps, float* df1, float* df2) {
  int rc = validate_pass(d, MEA_PASS_BWD, var);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs(ps);
  if (rc != MEA_OK) return rc;
  if ((df1 == nullptr) != (df2 == nullptr)) return MEA_ERR_NULL;
  if (df1 != nullptr && (!aligned16(df1) || !aligned16(df2))) return MEA_ERR_ALIGN;
  return MEA_OK;
}

int bwd_impl(const mea_desc* d, const Varlen* var, const void* dy, const void* x, const void* wq, const void* wk,
             const void* wv, const void* wg, const void* wo, const float* f1, const float* f2, const void* o_save,
             const float* lse_save, void* dx, void* dwq, void* dwk, void* dwv, void* dwg, void* dwo, float* df1,
             float* df2, void* ws, size_t ws_bytes, void* stream) {
  int rc = bwd_check(d, var, {dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, dx, dwq, dwk, dwv, dwg, dwo, ws},
                     df1, df2);
  if (rc != MEA_OK) return rc;
  {
    // dx is written before the end (it holds da_g while HN <= C): it may
    // overlap nothing else.
    const size_t M = (size_t)(d->B * d->T), HN = (size_t)(d->H * d->N), C = (size_t)d->C;
    const size_t act_c = M * C * 2, wbytes = HN * C * 2, tbytes = (size_t)d->T_max * (size_t)d->N * 4;
    const std::pair<const void*, size_t> others[] = {
        {dy, act_c},  {x, act_c},   {wq, wbytes},  {wk, wbytes},  {wv, wbytes},  {wg, wbytes},
        {wo, wbytes}, {f1, tbytes}, {f2, tbytes},  {o_save, M * HN * 2},       {lse_save, M * (size_t)d->H * 4},
        {dwq, wbytes}, {dwk, wbytes}, {dwv, wbytes}, {dwg, wbytes}, {dwo, wbytes}, {df1, tbytes},
        {df2, tbytes}, {ws, ws_bytes}};
    for (const auto& o : others)
      if (overlaps(dx, act_c, o.first, o.second)) return MEA_ERR_ALIAS;
  }
  const Layout L = make_layout(*d, df1 != nullptr ? MEA_PASS_BWD_TABLES : MEA_PASS_BWD);
  if (ws_bytes < L.total) return MEA_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = (int)(d->B * d->T), T = (int)d->T, H = (int)d->H, N = (int)d->N, C = (int)d->C;
  const int HN = H * N;

  // Gradients of the projection outputs: da_q, and da_k / da_v written over
  // k / v by the dK/dV kernel (the last reader of k and v), head-major;
  // da_g token-major, in the rows of dx when they are wide enough (each dx
  // workgroup reads the da_g rows it later overwrites, and nothing else
  // reads them after the weight gradients).
  const bool dag_in_dx = HN <= C && C <= 1024;
  const BwdBufs bf = bwd_bufs(d, ws, dag_in_dx ? dx : nullptr, C, df1 != nullptr);
  rc = bwd_front(d, var, dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, df1, df2, bf, ws, stream);
  if (rc != MEA_OK) return rc;
  const mea::DaParts da = {bf.daq, bf.dak, bf.v, bf.dag, bf.ld_dag, (int)d->B, T, H, N};

  mea::DwParams dw;
  dw.da = da;
  dw.x = static_cast<const bf16_bits*>(x);
  dw.dy = static_cast<const bf16_bits*>(dy);
  dw.z = bf.sig;  // the dZ kernel replaced sigmoid(a_g) by z = O * sigmoid(a_g)
  dw.part = bf.part;
  dw.M = M;
  dw.C = C;
  dw.HN = HN;
  dw.splits = mea::dw_splits(M, C, HN);
  MEA_TRY(timed(K_DW_PARTIAL, s, [&] { return mea::launch_dw_partial(dw, s); }));
  mea::DwReduceParams dr;
  dr.part = bf.part;
  dr.dwq = static_cast<bf16_bits*>(dwq);
  dr.dwk = static_cast<bf16_bits*>(dwk);
  dr.dwv = static_cast<bf16_bits*>(dwv);
  dr.dwg = static_cast<bf16_bits*>(dwg);
  dr.dwo = static_cast<bf16_bits*>(dwo);
  dr.C = C;
  dr.HN = HN;
  dr.splits = dw.splits;
  MEA_TRY(timed(K_DW_REDUCE, s, [&] { return mea::launch_dw_reduce(dr, s); }));

  mea::DxParams dxp;
  dxp.da = da;
  dxp.wcatT = bf.wcatT;
  dxp.x = static_cast<const bf16_bits*>(x);
  dxp.rx = bf.rx;
  dxp.dx = static_cast<bf16_bits*>(dx);
  // 768 < C <= 1024: feature groups of 512 over 128 tokens, group 0's
  // uncorrected rows parked in the recomputed q buffer (dead after the
  // attention backward; M x HN >= M x 512 elements).
  dxp.scratch = C > 768 && C <= 1024 && HN >= 512 ? bf.q : nullptr;
  dxp.M = M;
  dxp.C = C;
  dxp.HN = HN;
  MEA_TRY(timed(K_DX, s, [&] { return mea::launch_dx(dxp, s); }));
  return MEA_OK;
}

}  // namespace

extern "C" {

int mea_fwd(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
            const void* wo, const float* f1, const float* f2, void* y, void* o_save, float* lse_save, void* ws,
            size_t ws_bytes, void* stream) {
  return fwd_impl(d, nullptr, x, wq, wk, wv, wg, wo, f1, f2, y, o_save, lse_save, ws, ws_bytes, stream);
}

int mea_bwd(const mea_desc* d, const void* dy, const void* x, const void* wq, const void* wk, const void* wv,
            const void* wg, const void* wo, const float* f1, const float* f2, const void* o_save,
            const float* lse_save, void* dx, void* dwq, void* dwk, void* dwv, void* dwg, void* dwo, float* df1,
            float* df2, void* ws, size_t ws_bytes, void* stream) {
  return bwd_impl(d, nullptr, dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, dx, dwq, dwk, dwv, dwg, dwo, df1,
                  df2, ws, ws_bytes, stream);
}

int mea_fwd_varlen(const mea_desc* d, const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, const void* x,
                   const void* wq, const void* wk, const void* wv, const void* wg, const void* wo, const float* f1,
                   const float* f2, void* y, void* o_save, float* lse_save, void* ws, size_t ws_bytes,
                   void* stream) {
  const Varlen var{cu_seqlens, nseq, max_len};
  return fwd_impl(d, &var, x, wq, wk, wv, wg, wo, f1, f2, y, o_save, lse_save, ws, ws_bytes, stream);
}

int mea_bwd_varlen(const mea_desc* d, const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, const void* dy,
                   const void* x, const void* wq, const void* wk, const void* wv, const void* wg, const void* wo,
                   const float* f1, const float* f2, const void* o_save, const float* lse_save, void* dx, void* dwq,
                   void* dwk, void* dwv, void* dwg, void* dwo, float* df1, float* df2, void* ws, size_t ws_bytes,
                   void* stream) {
  const Varlen var{cu_seqlens, nseq, max_len};
  return bwd_impl(d, &var, dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, dx, dwq, dwk, dwv, dwg, dwo, df1,
                  df2, ws, ws_bytes, stream);
}

int mea_bwd_stage_grads(const mea_desc* d, const void* dy, const void* x, const void* wq, const void* wk,
                        const void* wv, const void* wg, const void* wo, const float* f1, const float* f2,
                        const void* o_save, const float* lse_save, void* daq, void* dak, void* dav, void* dag,
                        void* dO, float* delta, float* df1, float* df2, void* ws, size_t ws_bytes, void* stream) {
  int rc = bwd_check(d, nullptr, {dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, daq, dak, dav, dag, dO, delta, ws},
                     df1, df2);
  if (rc != MEA_OK) return rc;
  const Layout L = make_layout(*d, df1 != nullptr ? MEA_PASS_BWD_TABLES : MEA_PASS_BWD);
  if (ws_bytes < L.total) return MEA_ERR_WORKSPACE;
  const int HN = (int)(d->H * d->N);
  // da_g goes straight to the caller's buffer (token-major rows of H*N).
  const BwdBufs bf = bwd_bufs(d, ws, dag, HN, df1 != nullptr);
  rc = bwd_front(d, nullptr, dy, x, wq, wk, wv, wg, wo, f1, f2, o_save, lse_save, df1, df2, bf, ws, stream);
  if (rc != MEA_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t act = (size_t)(d->B * d->T) * (size_t)HN * 2, stat = (size_t)(d->B * d->H * d->T) * 4;
  MEA_TRY(hipMemcpyAsync(daq, bf.daq, act, hipMemcpyDeviceToDevice, s));
  MEA_TRY(hipMemcpyAsync(dak, bf.dak, act, hipMemcpyDeviceToDevice, s));
  MEA_TRY(hipMemcpyAsync(dav, bf.v, act, hipMemcpyDeviceToDevice, s));
  MEA_TRY(hipMemcpyAsync(dO, bf.dO, act, hipMemcpyDeviceToDevice, s));
  MEA_TRY(hipMemcpyAsync(delta, bf.delta, stat, hipMemcpyDeviceToDevice, s));
  return MEA_OK;
}

int mea_prefill(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
                const void* wo, const float* f1, const float* f2, void* y, void* k_cache, void* v_cache,
                int64_t cache_T, void* ws, size_t ws_bytes, void* stream) {
  int rc = validate(d, MEA_PASS_FWD);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({k_cache, v_cache});
  if (rc != MEA_OK) return rc;
  if (cache_T < d->T || cache_T > d->T_max) return MEA_ERR_SHAPE;
  rc = mea_fwd(d, x, wq, wk, wv, wg, wo, f1, f2, y, nullptr, nullptr, ws, ws_bytes, stream);
  if (rc != MEA_OK) return rc;
  // The prompt's k / v rows (as the attention consumed them) into rows
  // 0 .. T-1 of every (b, h) block of the caches.
  const Layout L = make_layout(*d, MEA_PASS_FWD);
  const size_t row = (size_t)(d->T * d->N * 2), pitch = (size_t)(cache_T * d->N * 2);
  const size_t rows = (size_t)(d->B * d->H);
  hipStream_t s = static_cast<hipStream_t>(stream);
  MEA_TRY(hipMemcpy2DAsync(k_cache, pitch, at<void>(ws, L.k), row, row, rows, hipMemcpyDeviceToDevice, s));
  MEA_TRY(hipMemcpy2DAsync(v_cache, pitch, at<void>(ws, L.v), row, row, rows, hipMemcpyDeviceToDevice, s));
  return MEA_OK;
}

}  // extern "C"

namespace {

// Decode workspace: the raw products [a_q|a_k|a_v|a_g] (B x 4HN fp32), the
// new token's q, sigmoid(g) and attention output (B x H*N bf16 each; its k
// and v go straight to the caches) and the split partials.
struct DecLayout {
  size_t a, q, sig, o, part, total;
  int S, chunk;
};

DecLayout make_dec_layout(const mea_desc& d) {
  DecLayout L = {};
  mea::decode_splits((int)d.B, (int)d.H, (int)d.T, &L.S, &L.chunk);
  const size_t row = (size_t)(d.B * d.H * d.N) * 2;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes); return o; };
  L.a = take(row * 2 * 4);
  L.q = take(row);
  L.sig = take(row);
  L.o = take(row);
  L.part = take((size_t)(d.B * d.H) * L.S * (size_t)(d.N + 4) * 4);
  L.total = off;
  return L;
}

}  // namespace

extern "C" {

size_t mea_decode_workspace_bytes(const mea_desc* d) {
  if (validate(d, MEA_PASS_FWD) != MEA_OK) return 0;
  return make_dec_layout(*d).total;
}

}  // extern "C"

namespace {

// Argument checks of the decode step (everything but the scratch memory).
int decode_check(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
                 const void* wo, const float* f1, const float* f2, const int32_t* pos, void* k_cache, void* v_cache,
                 void* y) {
  int rc = validate(d, MEA_PASS_FWD);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({x, wq, wk, wv, wg, wo, f1, f2, k_cache, v_cache, y});
  if (rc != MEA_OK) return rc;
  if (pos == nullptr) return MEA_ERR_NULL;
  if (((uintptr_t)pos & 3u) != 0) return MEA_ERR_ALIGN;
  return MEA_OK;
}

// The decode step's launches; ws holds make_dec_layout(*d).total bytes.
int decode_launch(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
                  const void* wo, const float* f1, const float* f2, const int32_t* pos, void* k_cache, void* v_cache,
                  void* y, void* ws, void* stream) {
  const DecLayout L = make_dec_layout(*d);
  const int N = (int)d->N, B = (int)d->B, C = (int)d->C, HN = (int)(d->H * d->N);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* a = at<float>(ws, L.a);
  bf16_bits* q = at<bf16_bits>(ws, L.q);
  bf16_bits* sig = at<bf16_bits>(ws, L.sig);
  bf16_bits* o = at<bf16_bits>(ws, L.o);
  // Projections of the B new tokens (a few rows: every weight row is read
  // once over a wide grid), then their epilogue at rotary rows pos[b].
  mea::SkinnyParams sp;
  sp.A0 = static_cast<const bf16_bits*>(x);
  sp.A1 = nullptr;
  sp.W[0] = static_cast<const bf16_bits*>(wq);
  sp.W[1] = static_cast<const bf16_bits*>(wk);
  sp.W[2] = static_cast<const bf16_bits*>(wv);
  sp.W[3] = static_cast<const bf16_bits*>(wg);
  sp.out = a;
  sp.M = B;
  sp.K = C;
  sp.F = HN;
  sp.nw = 4;
  sp.ldo = 4 * HN;
  sp.out_bf16 = 0;
  MEA_TRY(timed(K_SKINNY_GEMM, s, [&] { return mea::launch_skinny_gemm(sp, s); }));
  mea::DecodeProjParams pp;
  pp.a = a;
  pp.x = static_cast<const bf16_bits*>(x);
  pp.f1 = f1;
  pp.f2 = f2;
  pp.pos = pos;
  pp.q = q;
  pp.k_cache = static_cast<bf16_bits*>(k_cache);
  pp.v_cache = static_cast<bf16_bits*>(v_cache);
  pp.sig = sig;
  pp.Tc = (int)d->T;
  pp.B = B;
  pp.C = C;
  pp.H = (int)d->H;
  pp.t_max = (int)d->T_max;
  pp.eps = d->eps;
  pp.qscale = q_log2_scale(n_active(d));
  pp.inv_n = 1.0f / (float)n_active(d);
  MEA_TRY(timed(K_DECODE_PROJ, s, [&] { return mea::launch_decode_proj_epilogue(pp, N, s); }));
  mea::DecodeParams dp;
  dp.q = q;
  dp.k_cache = static_cast<bf16_bits*>(k_cache);
  dp.v_cache = static_cast<bf16_bits*>(v_cache);
  dp.pos = pos;
  dp.part = at<float>(ws, L.part);
  dp.o = o;
  dp.B = (int)d->B;
  dp.H = (int)d->H;
  dp.Tc = (int)d->T;
  dp.S = L.S;
  dp.chunk = L.chunk;
  MEA_TRY(timed(K_ATTN_DECODE, s, [&] { return mea::launch_attn_decode(dp, N, s); }));
  MEA_TRY(timed(K_DECODE_COMBINE, s, [&] { return mea::launch_attn_decode_combine(dp, N, s); }));
  // y = (O * sigmoid(g)) W_o^T for the B tokens.
  mea::SkinnyParams op;
  op.A0 = o;
  op.A1 = sig;
  op.W[0] = static_cast<const bf16_bits*>(wo);
  op.W[1] = op.W[2] = op.W[3] = nullptr;
  op.out = y;
  op.M = B;
  op.K = HN;
  op.F = C;
  op.nw = 1;
  op.ldo = C;
  op.out_bf16 = 1;
  MEA_TRY(timed(K_SKINNY_GEMM, s, [&] { return mea::launch_skinny_gemm(op, s); }));
  return MEA_OK;
}

// Scratch of mea_decode_static: a file-scope device array, one copy per GPU
// (each GPU the library runs on holds it until the process ends). In host
// code `scratch` is only a handle: its device address on the current GPU
// comes from hipGetSymbolAddress, looked up once per device and kept in
// g_scratch_addr, and only that address is handed to kernels.
__device__ __attribute__((aligned(256))) unsigned char scratch[MEA_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of `scratch` on the current device (the stream's device).
int static_scratch(void* stream, void** addr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MEA_ERR_DEVICE;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || sdev != dev)
      return MEA_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return MEA_ERR_DEVICE;
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return MEA_OK;
}

}  // namespace

extern "C" {

int mea_decode(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv, const void* wg,
               const void* wo, const float* f1, const float* f2, const int32_t* pos, void* k_cache, void* v_cache,
               void* y, void* ws, size_t ws_bytes, void* stream) {
  int rc = decode_check(d, x, wq, wk, wv, wg, wo, f1, f2, pos, k_cache, v_cache, y);
  if (rc != MEA_OK) return rc;
  rc = check_ptrs({ws});
  if (rc != MEA_OK) return rc;
  if (ws_bytes < make_dec_layout(*d).total) return MEA_ERR_WORKSPACE;
  return decode_launch(d, x, wq, wk, wv, wg, wo, f1, f2, pos, k_cache, v_cache, y, ws, stream);
}

int mea_decode_static(const mea_desc* d, const void* x, const void* wq, const void* wk, const void* wv,
                      const void* wg, const void* wo, const float* f1, const float* f2, const int32_t* pos,
                      void* k_cache, void* v_cache, void* y, void* stream) {
  int rc = decode_check(d, x, wq, wk, wv, wg, wo, f1, f2, pos, k_cache, v_cache, y);
  if (rc != MEA_OK) return rc;
  // Every scratch byte the step reads is written by the step first, so the
  // previous call's contents need no clearing.
  if (make_dec_layout(*d).total > (size_t)MEA_STATIC_SCRATCH_BYTES) return MEA_ERR_SCRATCH;
  void* ws = nullptr;
  rc = static_scratch(stream, &ws);
  if (rc != MEA_OK) return rc;
  return decode_launch(d, x, wq, wk, wv, wg, wo, f1, f2, pos, k_cache, v_cache, y, ws, stream);
}

const char* mea_strerror(int code) {
  switch (code) {
    case MEA_OK: return "ok";
    case MEA_ERR_NULL: return "a required pointer is NULL (or only one of a pair was given)";
    case MEA_ERR_SHAPE: return "B, T, H must be >= 1, T <= T_max, and indices must fit 31 bits";
    case MEA_ERR_HEAD_DIM: return "head width N must be 32 (with H even), 64, 128 or 256, N_active 0, N or 16 (N = 32, 64) or 32 (N = 64)";
    case MEA_ERR_MODEL_DIM: return "model width C must be a multiple of 32 in [32, 16384] with H*N*C < 2^29";
    case MEA_ERR_WORKSPACE: return "workspace smaller than mea_workspace_bytes()";
    case MEA_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case MEA_ERR_EPS: return "eps must be finite and positive";
    case MEA_ERR_LAUNCH: return "HIP kernel launch failed";
    case MEA_ERR_ALIAS: return "dx overlaps another argument of the backward";
    case MEA_ERR_SCRATCH: return "the decode step needs more scratch than mea_decode_static's static buffer";
    case MEA_ERR_DEVICE: return "no current device, or the stream belongs to another device";
    default: return "unknown status";
  }
}

const char* mea_version(void) { return "mea 0.1.0 gfx950"; }

int mea_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (on && !g_prof_on) {
    for (const ProfRec& r : g_prof) {
      (void)hipEventSynchronize(r.b);
      g_pool.push_back(r.a);
      g_pool.push_back(r.b);
    }
    g_prof.clear();
  }
  g_prof_on = on != 0;
  return MEA_OK;
}

int mea_profile_read(int kernel, int* count, double* total_ms) {
  if (kernel < 0 || kernel >= K_COUNT || count == nullptr || total_ms == nullptr) return MEA_ERR_NULL;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  int n = 0;
  double ms = 0.0;
  for (const ProfRec& r : g_prof) {
    if (r.kernel != kernel) continue;
    if (hipEventSynchronize(r.b) != hipSuccess) return MEA_ERR_LAUNCH;
    float t = 0.f;
    if (hipEventElapsedTime(&t, r.a, r.b) != hipSuccess) return MEA_ERR_LAUNCH;
    ms += t;
    ++n;
  }
  *count = n;
  *total_ms = ms;
  return MEA_OK;
}

const char* mea_profile_kernel_name(int kernel) {
  return kernel >= 0 && kernel < K_COUNT ? kKernelNames[kernel] : nullptr;
}

int mea_profile_select(int kernel) {
  if (kernel < -1 || kernel >= K_COUNT) return MEA_ERR_NULL;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_only = kernel;
  return MEA_OK;
}

}  // extern "C"
