// LDS tiles filled by direct global->LDS DMA (gfx950 global_load_lds_dwordx4).
//
// A tile is 64 rows x 128 bytes (64 bf16 of one token and head).  Its 16-byte
// chunks are XOR-swizzled per row -- chunk c of row r lives at position
// c ^ swz(r), with swz a bijection of r & 7 -- so that
//   * eight consecutive rows read at the same chunk (the 16-byte MFMA operand
//     reads) hit eight different 16-byte bank groups, and
//   * four consecutive rows read as 32-byte pairs (the transposing reads of
//     ds_read_b64_tr_b16) hit four different 32-byte bank groups.
// gfx950's LDS has 64 banks and serves a 16-byte read 16 lanes per clock, so
// rows r and r + 8 of such a read share a bank group (a 2-way conflict).  A
// key that also depends on bit 3 of the row removes it, but its row-dependent
// addresses cost the forward kernel more registers than its budget of 128
// (spills), which costs far more than the conflict; with swz depending on
// r & 7 only, every lane's chunk offset is the same for rows 8 apart.
// A DMA instruction writes lane L's 16 bytes to LDS base + 16 L, so a wave
// moves 8 rows per instruction; the swizzle is applied on the source side by
// choosing which global chunk each lane fetches.  Sources are addressed as a
// wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane byte offset (the
// instruction's saddr form): one VGPR and 32-bit arithmetic per DMA instead
// of a 64-bit address.  The launchers keep every offset below 2^32.
//
// The DMAs, the vmcnt waits and the barriers are issued as inline asm with
// "memory" clobbers, and synchronisation is explicit: a staging loop waits on
// its own DMAs with vmcnt and then crosses s_barrier.  The compiler is not
// told about the DMAs on purpose.  Its wait insertion tracks which LDS object
// a DMA in flight writes only as far as its alias analysis reaches, and when
// that fails for a later LDS read (which happens for reads in conditionally
// executed blocks) it waits for every DMA in flight, including the ones that
// prefetch later stages, so the ring no longer overlaps copies with compute.
// The asm statements are also compiler memory barriers, so no LDS access is
// moved across a DMA issue, a wait or a barrier.
//
// The DMA asm writes M0 (the LDS destination).  No other instruction in the
// kernels that include this header uses M0, so nothing the compiler keeps in
// M0 is lost.
#pragma once

#include "mf_common.h"

namespace mf {

constexpr int kRowBytes = 128;
constexpr int kTileBytes = 64 * kRowBytes;

typedef __attribute__((address_space(3))) void* lds_void_ptr;

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

__device__ __forceinline__ int chunk_off(int r, int c) { return r * kRowBytes + ((c ^ swz(r)) << 4); }

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)p;  // low 32 bits of a generic LDS address
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is reserved; see the header comment
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// Tile rows r0 .. r0+7 = global rows first + r0 .. first + r0 + 7 (global
// row 0 at g_base, rows row_stride bytes apart; rows past `last` re-read row
// `last`, so every access stays inside the tensor) into the LDS tile.  g_base,
// the tile address and r0 must be wave-uniform; last * row_stride + 128 must
// stay below 2^32.
__device__ __forceinline__ void dma_rows8(const char* g_base, uint32_t row_stride, int first,
                                          int r0, int last, char* tile) {
  const int lane = __lane_id();
  const int r = r0 + (lane >> 3);
  const int c = (lane & 7) ^ swz(r);
  const uint32_t voff = (uint32_t)min(first + r, last) * row_stride + (uint32_t)(c * 16);
  dma16(g_base, voff, uniform((int)lds_offset(tile + r0 * kRowBytes)));
}

// One 4-byte word per lane, all 64 lanes: lane L's word at byte offset
// voff (per lane) from the wave-uniform base lands at dst + 4 L (dst
// wave-uniform).
__device__ __forceinline__ void dma_word64(const void* sbase, uint32_t voff, void* dst) {
  dma4(sbase, voff, uniform((int)lds_offset(dst)));
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
  const char* p = tile + chunk_off(row, c) + within;
  const u32x2 lo = lds_read_tr16(p);
  const u32x2 hi = lds_read_tr16(p + 8 * kRowBytes);  // swz(row + 8) == swz(row)
  const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(bf16x8, w);
}

constexpr int kKvStep = 64;  // rows per ring stage (keys, or queries in dk/dv)

// Lane addressing of the transposing reads that build a [d][row] operand
// from a natural [row][d] tile: add (block base + tr_row) rows and
// (32 * d block + tr_col) columns; the second read of a k-step is 8 rows on.
__device__ __forceinline__ int tr_row_of(int lane) { return ((lane & 15) >> 2) + 4 * (lane >> 5); }
__device__ __forceinline__ int tr_col_of(int lane) { return 16 * ((lane >> 4) & 1) + 4 * (lane & 3); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate out of range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// One stage of the key-side ring: K tile, V tile and the 64 canonical key ids.
constexpr int kStageBytes = 2 * kTileBytes + 256;  // K tile, V tile, 64 key ids

template <int W>
struct KvDma {
  static constexpr int kGroups = 8 / W;            // 8-row groups per tile per wave
};

// Per-lane source offsets of a wave's kv_dma rows, relative to the stage's
// first key row: group j covers tile rows r0 = 8 (wave + W j) .. r0 + 7, and
// the lane fetches chunk (lane & 7) ^ swz(r) of row r = r0 + lane / 8.
// Computed once per kernel; the stages that lie inside the tensor then issue
// their DMAs with scalar address arithmetic only.
template <int W>
struct KvLanes {
  uint32_t off[KvDma<W>::kGroups];
};

template <int W>
__device__ __forceinline__ KvLanes<W> kv_lanes(uint32_t row_stride, int wave) {
  KvLanes<W> l;
  const int lane = __lane_id();
#pragma unroll
  for (int j = 0; j < KvDma<W>::kGroups; ++j) {
    const int r = 8 * (wave + W * j) + (lane >> 3);
    l.off[j] = (uint32_t)r * row_stride + (uint32_t)(((lane & 7) ^ swz(r)) * 16);
  }
  return l;
}

// DMA of keys kb .. kb+63 (K rows, V rows, canonical ids) into one stage.
// kid_row must hold at least kb + 64 entries (the plan pads ids to whole tiles).
template <int W>
__device__ __forceinline__ void kv_dma(const char* kg, const char* vg, uint32_t row_stride, int S,
                                       const int* kid_row, int kb, int wave, char* stage) {
  if (wave == 0) dma_word64(kid_row + kb, 4u * __lane_id(), stage + 2 * kTileBytes);
#pragma unroll
  for (int j = 0; j < KvDma<W>::kGroups; ++j) {
    const int r0 = 8 * (wave + W * j);
    dma_rows8(kg, row_stride, kb, r0, S - 1, stage);
    dma_rows8(vg, row_stride, kb, r0, S - 1, stage + kTileBytes);
  }
}

// The same DMA with the lanes' source offsets precomputed (kv_lanes).
// A stage that reaches past key S - 1 re-reads row S - 1 for those rows.
template <int W>
__device__ __forceinline__ void kv_dma(const char* kg, const char* vg, uint32_t row_stride, int S,
                                       const int* kid_row, int kb, int wave, char* stage,
                                       const KvLanes<W>& lanes) {
  if (wave == 0) dma_word64(kid_row + kb, 4u * __lane_id(), stage + 2 * kTileBytes);
  if (kb + kKvStep <= S) {
    const uint32_t first = (uint32_t)kb * row_stride;
#pragma unroll
    for (int j = 0; j < KvDma<W>::kGroups; ++j) {
      const uint32_t dst = uniform((int)lds_offset(stage + 8 * (wave + W * j) * kRowBytes));
      dma16(kg + first, lanes.off[j], dst);
      dma16(vg + first, lanes.off[j], dst + kTileBytes);
    }
  } else {
#pragma unroll
    for (int j = 0; j < KvDma<W>::kGroups; ++j) {
      const int r0 = 8 * (wave + W * j);
      dma_rows8(kg, row_stride, kb, r0, S - 1, stage);
      dma_rows8(vg, row_stride, kb, r0, S - 1, stage + kTileBytes);
    }
  }
}

}  // namespace mf
