// Shared device helpers for the gfx950 attention kernels.
//
// MFMA conventions used throughout (CDNA3/CDNA4 32x32 family, wave64):
//   C[32x32] fp32 accumulator: lane l, register r holds
//       column n = l % 32, row m = 8*(r/4) + 4*(l/32) + (r%4).
//   v_mfma_f32_32x32x16_bf16: lane l supplies A[m = l%32][k = 8*(l/32) .. +7]
//       and B[k = 8*(l/32) .. +7][n = l%32] (8 bf16 each).
//   v_mfma_f32_32x32x2_f32:   lane l supplies A[m = l%32][k = l/32] and
//       B[k = l/32][n = l%32] (one float each).
// A contraction may visit its k indices in any order as long as A and B
// agree; the kernels use that freedom to feed accumulator registers straight
// back in as B operands (acc_row below gives the rows a lane holds), paired
// with transposing LDS reads of the other operand that visit the same rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mf {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTile = 128;  // block-map tile edge (queries and keys)
constexpr int kD = 64;      // head dimension served by the kernels
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// Row (within a 32-row accumulator block) held by register r of lane l.
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b,
                                               const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32x32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// v_permlane32_swap with both operands = x leaves, in every lane l, the pair
// {x[l], x[l ^ 32]} across its two results (which one lands where does not
// matter for a symmetric combine).
__device__ __forceinline__ float halves_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float halves_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x rounded to bf16 (nearest even) and widened back to fp32.  The conversion
// is inline asm so that no floating-point rewrite can drop it: written as
// (float)(bf16)x, the compiler has fused a product rounded this way into a
// following add (one FMA, the rounding gone).
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, 0" : "=v"(r) : "v"(x));
  return __builtin_bit_cast(float, r << 16);
}

// x and y rounded to bf16 (nearest even) by one conversion, packed (x in the
// low half); inline asm for the same reason as round_bf16.
__device__ __forceinline__ uint32_t round_bf16_pair(float x, float y) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
  return r;
}
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __builtin_bit_cast(float, u & 0xffff0000u); }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j receives
// element e (0..3) = halfword (j & 3) of the 8 bytes addressed by lane
// (j >> 2) + 4e.  If lane i of the group addresses row base + (i >> 2),
// column c0 + 4 (i & 3) of a row-major 16-bit tile, lane j receives rows
// base .. base+3 of column c0 + j: a 4-deep k-slice of a transposed operand.
typedef __fp16 f16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) f16x4_raw* lds_ptr;
  const f16x4_raw r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_ptr)(p));
  return __builtin_bit_cast(u32x2, r);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// 8 consecutive floats -> bf16x8 (round to nearest even).
__device__ __forceinline__ bf16x8 pack8(const f32x16& v, int base) {
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (bf16)v[base + i];
  return o;
}

// Four accumulator values times `mul` as bf16 (round to nearest even), or
// zeros where `keep` is false.  The select acts on the two packed words, not
// on each value, so the conversions pair up (one v_cvt_pk_bf16_f32 per two
// values and no repacking): a select per value before the cast makes the
// compiler convert one value at a time and merge the halves afterwards.
__device__ __forceinline__ bf16x4 scaled_bf16x4(const f32x16& v, int base, float mul, bool keep) {
  bf16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (bf16)(v[base + i] * mul);
  u32x2 w = __builtin_bit_cast(u32x2, o);
  w[0] = keep ? w[0] : 0u;
  w[1] = keep ? w[1] : 0u;
  return __builtin_bit_cast(bf16x4, w);
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const void* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ u32x4 ld_u32x4(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ void st_u32x4(void* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// The lane id, computed afresh by instructions the compiler cannot merge
// with an earlier copy: code after a long loop uses it instead of keeping
// lane-derived values alive (or spilled to scratch) across the loop.
__device__ __forceinline__ int fresh_lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// A wave-uniform integer forced into a scalar register.  Index arithmetic
// on blockIdx with runtime divisors is lowered through VALU; without this the
// dependent loads become vector loads and the work loops become divergent.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Division of integers in [0, 2^31) by a divisor d >= 1 fixed at launch, by
// the round-up method of Granlund and Montgomery ("Division by invariant
// integers using multiplication", 1994): with shr = ceil(log2 d) and
// m = 2^32 + mul = floor(2^(32 + shr) / d) + 1, x / d = floor(x m / 2^(32 + shr)).
// m d exceeds 2^(32 + shr) by e in (0, d], so x m / 2^(32 + shr) exceeds x / d
// by x e / (d 2^(32 + shr)) < 1 / d for x < 2^32, which never carries the
// quotient past the next integer.  umulhi(x, mul) < x keeps the 32-bit sum
// below 2^32 for x < 2^31.  The grid-index decompositions use it in place of
// the compiler's generic division (about 30 dependent scalar instructions).
struct FastDiv {
  uint32_t d, mul, shr;
};

inline FastDiv make_fastdiv(int d) {
  FastDiv f;
  f.d = (uint32_t)d;
  f.shr = 0;
  while ((1ull << f.shr) < f.d) ++f.shr;
  f.mul = (uint32_t)(((1ull << 32) * ((1ull << f.shr) - f.d)) / f.d + 1);
  return f;
}

__device__ __forceinline__ int fast_div(int x, const FastDiv& f) {
  return (int)((__umulhi((uint32_t)x, f.mul) + (uint32_t)x) >> f.shr);
}

// Read of a wave-uniform index from memory that is immutable for the whole
// kernel (the plan's work lists): the constant address space lets the
// compiler use a scalar load, which does not queue behind the vector loads
// in flight.
__device__ __forceinline__ int ld_const(const int* p, int i) {
  return ((const __attribute__((address_space(4))) int*)(p))[__builtin_amdgcn_readfirstlane(i)];
}

// Eight consecutive entries p[i .. i+7] of such an array in one scalar load
// (i wave-uniform; only dword alignment is required of p + i).  The caller
// guarantees that the 32 bytes lie inside the allocation.
typedef int i32x8u __attribute__((ext_vector_type(8), aligned(4)));
__device__ __forceinline__ i32x8u ld_const8(const int* p, int i) {
  return *((const __attribute__((address_space(4))) i32x8u*)(p + __builtin_amdgcn_readfirstlane(i)));
}

// Wait for every outstanding memory operation.  Used once, after the
// per-wave operands that stay in registers for the whole kernel are loaded:
// the compiler's wait insertion cannot see across the work loop's back edge
// that those loads completed, and would otherwise wait for all in-flight
// prefetches at the top of every step.
__device__ __forceinline__ void drain_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Mask element: nonzero means active.
__device__ __forceinline__ int mask_at(const void* mask, int mask_u8, long idx) {
  return mask_u8 ? (int)reinterpret_cast<const uint8_t*>(mask)[idx]
                 : reinterpret_cast<const int32_t*>(mask)[idx];
}

// Plan section offsets (bytes), shared by host and device code.
struct PlanLayout {
  size_t qid, kid, tmap, qcnt, qlist, kcnt, klist, qorder, korder, runs, total;
  int nq, nk, tq_pad, tk_pad;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Per-tile run record written by the block-map builder.
struct Run {
  int id, start, stop;  // absolute token positions [start, stop)
};
constexpr int kMaxRuns = kTile;  // a 128-token tile has at most 128 runs

__host__ __device__ inline PlanLayout plan_layout(int batch, int q_len, int kv_len) {
  PlanLayout p;
  p.nq = (q_len + kTile - 1) / kTile;
  p.nk = (kv_len + kTile - 1) / kTile;
  p.tq_pad = p.nq * kTile;
  p.tk_pad = p.nk * kTile;
  size_t off = 0;
  p.qid = off;   off = align256(off + sizeof(int) * (size_t)batch * p.tq_pad);
  p.kid = off;   off = align256(off + sizeof(int) * (size_t)batch * p.tk_pad);
  p.tmap = off;  off = align256(off + (size_t)batch * p.nq * p.nk);
  p.qcnt = off;  off = align256(off + sizeof(int) * (size_t)batch * p.nq);
  // work lists of 64-row stages: [B][nq][2 nk] key stages, [B][nk][2 nq] query stages.
  // The forward and dq read a query tile's list eight entries at a time and
  // may read up to 7 entries past its end: a section must follow qlist.
  p.qlist = off; off = align256(off + sizeof(int) * (size_t)batch * p.nq * 2 * p.nk);
  p.kcnt = off;  off = align256(off + sizeof(int) * (size_t)batch * p.nk);
  p.klist = off; off = align256(off + sizeof(int) * (size_t)batch * p.nk * 2 * p.nq);
  // launch orders: (row, tile) items by decreasing work-list length
  p.qorder = off; off = align256(off + sizeof(int) * (size_t)batch * p.nq);
  p.korder = off; off = align256(off + sizeof(int) * (size_t)batch * p.nk);
  // run records: q tiles then k tiles, each (count int + kMaxRuns Runs)
  p.runs = off;
  off = align256(off + (sizeof(int) + sizeof(Run) * kMaxRuns) * (size_t)batch * (p.nq + p.nk));
  p.total = off;
  return p;
}

}  // namespace mf
