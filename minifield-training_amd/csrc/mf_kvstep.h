// Staging of one 64-key step (K and V rows of one KV head, natural
// row-major layout) from HBM into LDS, shared by the bf16 forward and the
// bf16 dq kernel.  A workgroup of T threads moves 2 x 64 rows x 128 bytes
// per step as 1024 16-byte chunks (8 consecutive threads cover one 128-byte
// row, so every wavefront load is eight full lines); LDS rows are padded to
// 144 bytes so the 16-byte MFMA operand reads that follow are conflict-free.
#pragma once

#include "mf_common.h"

namespace mf {

constexpr int kKvStep = 64;       // keys per step
constexpr int kKvPitch = kD + 8;  // bf16 elements per LDS row

struct KvStepLds {
  bf16 k[2][kKvStep * kKvPitch];
  bf16 v[2][kKvStep * kKvPitch];
  int kid[2][kKvStep];
};

template <int T>
struct KvStepStage {
  static constexpr int kChunks = 1024 / T;
  u32x4 r[kChunks];
  int kid;
};

// Rows kb .. kb+63 of K and V (zero past S) and their canonical ids.
// `base` is the element offset of (row b, key 0, KV head, d 0); consecutive
// keys are `key_stride` elements apart.
template <int T>
__device__ __forceinline__ void kvstep_load(const void* k, const void* v, const int* kid_row,
                                            size_t base, size_t key_stride, int S, int kb,
                                            KvStepStage<T>& st) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < KvStepStage<T>::kChunks; ++i) {
    const int u = tid + T * i;
    const int row = (u & 511) >> 3, ch = u & 7;
    const bf16* src = reinterpret_cast<const bf16*>(u < 512 ? k : v);
    // rows past the sequence end re-read the last row: their keys carry id 0,
    // so every score against them is masked (P = 0) and the finite values
    // they bring into P V are multiplied by 0.  An unconditional load keeps
    // the staging registers free of a zero-fill that would have to wait for
    // the previous load of the same registers.
    const int key = min(kb + row, S - 1);
    st.r[i] = ld_u32x4(src + base + key * key_stride + ch * 8);
  }
  st.kid = kid_row[kb + (tid & (kKvStep - 1))];  // every thread loads: no branch
}

template <int T>
__device__ __forceinline__ void kvstep_store(const KvStepStage<T>& st, KvStepLds& lds, int buf) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < KvStepStage<T>::kChunks; ++i) {
    const int u = tid + T * i;
    const int row = (u & 511) >> 3, ch = u & 7;
    st_u32x4((u < 512 ? lds.k[buf] : lds.v[buf]) + row * kKvPitch + ch * 8, st.r[i]);
  }
  if (tid < kKvStep) lds.kid[buf][tid] = st.kid;
}

// Lane addressing of the transposing reads that build a [d][key] operand
// from a natural [key][d] LDS tile: add (block base + tr_row) rows and
// (32 * d block + tr_col) columns; the second read of a k-step is 8 rows on.
__device__ __forceinline__ int tr_row_of(int lane) { return ((lane & 15) >> 2) + 4 * (lane >> 5); }
__device__ __forceinline__ int tr_col_of(int lane) { return 16 * ((lane >> 4) & 1) + 4 * (lane & 3); }

// 8-deep k-slice (rows base + {0..3, 8..11} for lane half 0, {4..7, 12..15}
// for half 1, matching acc_row) of the transpose of a natural LDS tile.
__device__ __forceinline__ bf16x8 tr_operand(const bf16* tile, int pitch, int row, int col) {
  const bf16* p = tile + row * pitch + col;
  const u32x2 lo = lds_read_tr16(p);
  const u32x2 hi = lds_read_tr16(p + 8 * pitch);
  const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(bf16x8, w);
}

}  // namespace mf
