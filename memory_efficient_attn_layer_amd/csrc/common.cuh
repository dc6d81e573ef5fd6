// Device helpers shared by the gfx950 kernels of the attention block.
//
// MFMA convention used throughout (v_mfma_f32_16x16x32_bf16, one wave of 64
// lanes, lane = 16*g + c with g in 0..3 and c in 0..15):
//   A operand (16 rows x 32 k):  lane holds row c, k = 8g .. 8g+7
//   B operand (32 k x 16 cols):  lane holds col c, k = 8g .. 8g+7
//   D (16 x 16 fp32):            lane holds col c, rows 4g .. 4g+3
// Only the D layout matters for correctness of a plain product: the k order
// inside A and B is the same function of (g, element), so any consistent
// permutation of k between the two operands gives the same sum. The attention
// kernels rely on that to feed an accumulator straight back as an operand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mea {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_bits;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Zero accumulators as splat constants, so a first MFMA can take the inline
// constant 0 as its accumulator input instead of zeroed registers.
__device__ __forceinline__ f32x4 zero4() { return (f32x4)(0.0f); }

// v_mfma_f32_32x32x16_bf16, lane = 32*h + c (h in 0..1, c in 0..31):
//   A operand (32 rows x 16 k): lane holds row c, k = 8h .. 8h+7
//   B operand (16 k x 32 cols): lane holds col c, k = 8h .. 8h+7
//   D (32 x 32 fp32, 16 regs):  reg i of lane holds row 8*(i/4) + 4h + i%4, col c
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 zero16() { return (f32x16)(0.0f); }

// LDS pointer types for the gfx950 LDS-only instructions.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

// ds_read_b64_tr_b16: within each group of 16 lanes, lane 4a+b receives
// element b of the 4-element rows addressed by lanes a, 4+a, 8+a, 12+a (in
// that order). With lane i of the group addressing row r0 + (i >> 2),
// column c0 + 4*(i & 3) of a row-major bf16 matrix, lane j gets column
// c0 + j of rows r0 .. r0+3: a k-major MFMA operand read from a tile whose
// rows run along k.
__device__ __forceinline__ u32x2 lds_read_tr4(const bf16_bits* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// global_load_lds_dwordx4: lane L copies 16 bytes from its own global
// address to lds_wave_base + 16*L (lds_wave_base must be wave-uniform).
// Completion is tracked by vmcnt only: the caller waits with wait_vmcnt0()
// before the barrier that publishes the tile. Issued as inline asm so the
// compiler does not guard every later LDS read (it cannot tell the tile
// being filled from the one being read) with a wait for all of these loads.
// The kernels that use it set m0 nowhere else.
__device__ __forceinline__ void g2lds16(const void* gsrc, bf16_bits* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)((lds_void*)lds_wave_base));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gsrc), "s"(lds) : "memory");
}
// The same, into the LDS byte address lds (wave-uniform).
__device__ __forceinline__ void g2lds16(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gsrc),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a 32-bit
// per-lane byte offset (saddr form), into the LDS byte address lds (also
// wave-uniform). Saves the per-lane 64-bit address arithmetic.
__device__ __forceinline__ void g2lds16_s(const void* sbase, uint32_t voff, uint32_t lds) {
  // The base and the LDS address must sit in SGPRs; readfirstlane states
  // that they are uniform where the compiler cannot prove it (free where it
  // can).
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"((const void*)(uintptr_t)u),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)((lds_void*)p); }

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left open), as a builtin so the
// compiler's own wait tracking also sees every earlier vector load retired.
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// bf16 bit patterns <-> fp32.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(bf16_bits h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16 bits, round to nearest even (hardware conversion on gfx950).
__device__ __forceinline__ bf16_bits f2bf(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(bf16_bits, b);
}
// Two fp32 -> packed bf16 pair with one v_cvt_pk_bf16_f32 (round to nearest
// even).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo_bf(v[i]);
    f[2 * i + 1] = hi_bf(v[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack2(f[2 * i], f[2 * i + 1]);
  return v;
}

__device__ __forceinline__ bf16x8 as_frag(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }
// Concatenation of two 64-bit halves into one MFMA operand; written as a
// shuffle so the two halves can be loaded straight into adjacent registers.
__device__ __forceinline__ bf16x8 frag_from2(const u32x2& a, const u32x2& b) {
  const u32x4 v = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  return __builtin_bit_cast(bf16x8, v);
}

// 16-byte global load / store.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
// Non-temporal (streaming) 16-byte store: for outputs not read again soon.
__device__ __forceinline__ void st16_nt(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Cross-lane helpers. xor 1 / xor 2 use DPP quad permutes; wider distances go
// through ds_bpermute (no memory traffic).
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
}
// Sum over the 16 lanes that share g (lane = 16g + c).
__device__ __forceinline__ float sum16(float v) {
  v += xor1(v);
  v += xor2(v);
  v += shfl_xor(v, 4);
  v += shfl_xor(v, 8);
  return v;
}
// Sum / max over the 4 lane groups g that share c.
__device__ __forceinline__ float sum_g(float v) {
  v += shfl_xor(v, 16);
  v += shfl_xor(v, 32);
  return v;
}
__device__ __forceinline__ float max_g(float v) {
  v = fmaxf(v, shfl_xor(v, 16));
  v = fmaxf(v, shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf(float a) { return 1.0f / (1.0f + __expf(-a)); }
// sigmoid with the hardware exp2 and reciprocal (about 2 ulp in fp32; the
// result is rounded to bf16).
__device__ __forceinline__ float fast_sigmoid(float a) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-a * kLog2e));
}

// Row-major bf16 tiles in LDS are stored as 16-byte chunks; chunk c of row r
// sits at chunk slot c ^ swz(r). Two access patterns must be conflict-free:
//  - 16-byte row reads: 16 lanes read one chunk of 16 consecutive rows. For
//    rows of 8 chunks (128 B) two rows share a 256-byte bank line, so the 8
//    rows of each parity need distinct swizzles: p = (r >> 1) & 7 does that.
//    For rows of 16 chunks any permutation of r & 15 does.
//  - transposing 8-byte reads (ds_read_b64_tr_b16): 64 lanes read 4 aligned
//    chunks of 8 consecutive rows. The swizzle's bit 2 (8-chunk rows, over row
//    pairs) or bits 2-3 (16-chunk rows, over rows) must then take each value
//    equally often, so the 4-chunk groups of the rows spread over the whole
//    bank line instead of stacking on one quarter of it.
// p ^ ((p & 1) << 2) and r ^ ((r & 3) << 2) satisfy both. Rows of 32 chunks
// (256 bf16) take the 16-chunk swizzle: it permutes the low four bits of the
// slot, so 16 consecutive rows still fill 16 distinct bank groups. Rows of 4
// chunks (32 bf16, 64 B): four rows share a bank line, so the four rows of
// each residue r & 3 among 16 consecutive rows need distinct swizzles:
// (r >> 2) & 3. A transposing read then covers 8 whole rows, two full bank
// lines, whatever the swizzle.
// Every swizzle depends on row & 15 only.
template <int CH>
__device__ __forceinline__ int chunk_swz(int row) {
  static_assert(CH == 4 || CH == 8 || CH == 16 || CH == 32, "rows of 32, 64, 128 or 256 bf16");
  if (CH == 4) return (row >> 2) & 3;
  if (CH == 8) {
    const int p = (row >> 1) & 7;
    return p ^ ((p & 1) << 2);
  }
  const int r = row & 15;
  return r ^ ((r & 3) << 2);
}
// Element offset of (row, col) in a swizzled tile with CH chunks per row.
template <int CH>
__device__ __forceinline__ int swz_off(int row, int col) {
  return row * (CH * 8) + (((col >> 3) ^ chunk_swz<CH>(row)) << 3) + (col & 7);
}

// Block-id remapping so that consecutive logical tiles run on the same XCD.
// The hardware hands workgroup L to XCD L % 8; logical tile ids
// [start(x), start(x)+count(x)) are made to run on XCD x, which keeps
// neighbouring tiles (that share operand rows) inside one L2.
__host__ __device__ __forceinline__ int xcd_remap(int L, int G) {
  const int x = L & 7, i = L >> 3;
  const int q = G >> 3, r = G & 7;
  const int start = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  return start + i;
}

// Work-item order of the attention kernels. Logical item l = head * nb + k,
// where block k = 0 of a head is its heaviest (the most key or query tiles)
// and k = nb - 1 its lightest. Each XCD runs a contiguous range of items
// (xcd_remap) in order, so it walks whole heads and the K/V (or Q/dO) tiles
// of the heads it is working on stay in its L2. Walked head by head to the
// end, the last head's heaviest blocks would start last and run alone (a
// list schedule over 96 workgroup slots per XCD ends 4.8% after its mean
// load at B64 T4096 in the backward, 6.8% in the forward). So the last
// tail_heads heads' worth of each XCD's range (at most a quarter of it, so
// that long sequences keep their head-by-head L2 reuse) is taken
// heaviest-first across those heads: the heaviest block of every one of its
// heads first, then the next heaviest of each, and so on. Any range of
// tail * nb consecutive items holds each block index exactly tail times, so
// the tail is a permutation of itself whatever head it starts in. Four heads:
// a wider tail balances the end better in a model, but its heads no longer
// share L2 (B64 T4096 H8 N64 HBM reads per launch, forward / dQ / dK-dV:
// 0 heads 0.83 / 2.29 / 2.26 GB, 4 heads 0.87 / 2.35 / 2.33 GB, 8 heads
// 1.32 / 2.76 / 2.78 GB, 16 heads 2.66 / 4.01 / 4.10 GB) and 4 ran the
// fastest step (8.25 ms against 8.29, 8.32 and 8.35 ms for 8, 16 and 0).
constexpr int kTailHeads = 4;
// Before the tail, the order is dealt out so that the workgroups sharing a
// CU run blocks of different weight. In plain order, an XCD's first
// kCusPerXcd * slots workgroups (which fill its CUs, slots = workgroups per
// CU) would put the same block index of consecutive heads on the slots of a
// CU: blocks of the same length, which start, wait for their first tiles,
// run their epilogues and finish in step, leaving the matrix cores to fewer
// waves each time. So within every run of kCusPerXcd * slots items, the
// items of slot j = r / kCusPerXcd (r the position in the run) are rotated
// by j * ceil(kCusPerXcd / slots): a permutation of the run, whose slots
// start blocks a third of a head apart. Measured on B64 T4096 H8 N64 (same
// box, rotation against plain order, three runs on three boxes): dK/dV
// -2.3 to -3.4%, dQ -1.4 to -2.6%, forward -0.9 to -1.5% (three slots in
// all three kernels; four in the forward, its occupancy, gained 0.2%); the
// step -0.5 to -1.3%. With 128-wide heads (two slots) dK/dV ran 1.1% slower
// and T = 32768 was unchanged, so only N <= 64 uses it (slots = 1: plain).
// Packed sequences take the same order over their (sequence, head, block)
// items, blocks past a sequence's end exiting at once (64 sequences of 1024
// to 4096 tokens, against plain per-XCD ranges: dK/dV -4.2%, dQ -2.2%,
// forward -2.7%, the step -1.7%).
constexpr int kCusPerXcd = 32;
// (Host and device: tests/work_order.cpp checks on the CPU that it is a
// permutation of 0 .. G - 1.)
__host__ __device__ __forceinline__ int attn_item(int L, int G, int nb, int slots, int tail_heads = kTailHeads) {
  const int x = L & 7, i = L >> 3;
  const int q = G >> 3, rm = G & 7;
  const int n = q + (x < rm ? 1 : 0);
  const int s = x < rm ? x * (q + 1) : rm * (q + 1) + (x - rm) * q;
  const int h4 = n / nb / 4 > 1 ? n / nb / 4 : 1;
  const int th = n < nb ? 0 : (tail_heads < h4 ? tail_heads : h4);  // heads in the tail (th * nb <= n)
  const int R = th * nb;
  if (i < n - R) {
    const int run = kCusPerXcd * slots, blk = i / run, r = i - blk * run;
    if (slots == 1 || (blk + 1) * run > n - R) return s + i;  // the last partial run: as is
    const int slot = r / kCusPerXcd, c = r - slot * kCusPerXcd;
    const int rot = slot * ((kCusPerXcd + slots - 1) / slots);
    return s + blk * run + slot * kCusPerXcd + (c + rot) % kCusPerXcd;
  }
  const int j = i - (n - R);
  const int k = j / th, c = j - k * th;     // block k (heaviness rank), its c-th head in the tail
  const int base = s + n - R;
  const int first = base + (k - base % nb + nb) % nb;  // first item of block k at or after base
  return first + c * nb;
}

}  // namespace mea
