// LDS tiles filled by direct global->LDS DMA (gfx950 global_load_lds_dwordx4).
//
// A tile is 64 rows x 128 bytes (64 bf16 of one token and head).  Its 16-byte
// chunks are XOR-swizzled per row -- chunk c of row r lives at position
// c ^ swz(r) -- so that
//   * eight consecutive rows read at the same chunk (the 16-byte MFMA operand
//     reads, lanes r..r+7) hit eight different 16-byte bank groups, and
//   * four consecutive rows read as 32-byte pairs (the transposing reads of
//     ds_read_b64_tr_b16) hit four different 32-byte bank groups.
// A DMA instruction writes lane L's 16 bytes to LDS base + 16 L, so a wave
// moves 8 rows per instruction; the swizzle is applied on the source side by
// choosing which global chunk each lane fetches.
//
// Synchronisation is explicit: the staging loop waits on this wave's own DMAs
// with vmcnt(N) and then crosses a raw s_barrier.  __syncthreads() would add a
// release fence that waits for every DMA in flight, including the ones
// prefetching later stages.
#pragma once

#include "mf_common.h"

namespace mf {

constexpr int kRowBytes = 128;
constexpr int kTileBytes = 64 * kRowBytes;

typedef __attribute__((address_space(3))) void* lds_void_ptr;

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

__device__ __forceinline__ int chunk_off(int r, int c) { return r * kRowBytes + ((c ^ swz(r)) << 4); }

// Tile rows r0 .. r0+7 = global rows first + r0 .. first + r0 + 7 (global
// row 0 at g_base, rows row_stride bytes apart; rows past `last` re-read row
// `last`, so every access stays inside the tensor) into the LDS tile.
__device__ __forceinline__ void dma_rows8(const char* g_base, size_t row_stride, int first, int r0,
                                          int last, char* tile) {
  const int lane = __lane_id();
  const int r = r0 + (lane >> 3);
  const int c = (lane & 7) ^ swz(r);
  const char* src = g_base + (size_t)min(first + r, last) * row_stride + c * 16;
  __builtin_amdgcn_global_load_lds(src, (lds_void_ptr)(tile + r0 * kRowBytes), 16, 0, 0);
}

// `count` consecutive 4-byte words (count <= 64), lanes >= count idle:
// dst[i] = src[i].  Used for the per-row ids and softmax statistics.
__device__ __forceinline__ void dma_words(const void* src, void* dst, int count) {
  const int lane = __lane_id();
  if (lane < count)
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const int*>(src) + lane, (lds_void_ptr)dst, 4,
                                     0, 0);
}

// One 4-byte word per lane, all 64 lanes: lane L's word (read from its own
// address `src`) lands at dst + 4 L.  Unconditional, so it adds no
// divergent branch to the staging code.
__device__ __forceinline__ void dma_word64(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const int*>(src), (lds_void_ptr)dst, 4, 0, 0);
}

// 16-byte operand: chunk c of row r.
__device__ __forceinline__ bf16x8 tile_chunk(const char* tile, int r, int c) {
  return *reinterpret_cast<const bf16x8*>(tile + chunk_off(r, c));
}

// Transposed 8-deep k-slice for the calling lane: rows row+{0..3} and
// row+{8..11} (lane half 0; the caller adds 4 for half 1 through tr_row) of
// column col (a multiple of 4), read with ds_read_b64_tr_b16.
__device__ __forceinline__ bf16x8 tile_tr_operand(const char* tile, int row, int col) {
  const int c = col >> 3, within = (col & 7) * 2;
  const u32x2 lo = lds_read_tr16(tile + row * kRowBytes + ((c ^ swz(row)) << 4) + within);
  const int row2 = row + 8;
  const u32x2 hi = lds_read_tr16(tile + row2 * kRowBytes + ((c ^ swz(row2)) << 4) + within);
  const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(bf16x8, w);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate out of range");
  __builtin_amdgcn_s_waitcnt(0xF70 | N);
}

__device__ __forceinline__ void barrier() { __builtin_amdgcn_s_barrier(); }

// One stage of the key-side ring: K tile, V tile and the 64 canonical key ids.
constexpr int kStageBytes = 2 * kTileBytes + 256;  // K tile, V tile, 64 key ids

template <int W>
struct KvDma {
  static constexpr int kGroups = 8 / W;            // 8-row groups per tile per wave
  static constexpr int kIds = 64 / W;              // key ids per wave
  static constexpr int kPerStep = 2 * kGroups + 1; // DMA instructions per wave per step
};

// DMA of keys kb .. kb+63 (K rows, V rows, canonical ids) into one stage.
template <int W>
__device__ __forceinline__ void kv_dma(const char* kg, const char* vg, size_t row_stride, int S,
                                       const int* kid_row, int kb, int wave, char* stage) {
#pragma unroll
  for (int j = 0; j < KvDma<W>::kGroups; ++j) {
    const int r0 = 8 * (wave + W * j);
    dma_rows8(kg, row_stride, kb, r0, S - 1, stage);
    dma_rows8(vg, row_stride, kb, r0, S - 1, stage + kTileBytes);
  }
  constexpr int E = KvDma<W>::kIds;
  dma_words(kid_row + kb + E * wave, stage + 2 * kTileBytes + 4 * E * wave, E);
}

}  // namespace mf
