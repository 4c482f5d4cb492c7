// Block-mask builder: segment ids + masks -> canonical token ids, per-tile
// run lists, the EMPTY/PARTIAL/FULL tile map and compacted work lists.
//
// Semantics (reference: src/minifield_training/kernels/attention.py:94-107
// and kernels/bidirectional.py:21-31):
//   packed causal : active = mask > 0 && seg != 0; pair valid iff both active,
//                   same segment and key <= query.
//   packed bidir  : active = mask != 0 && seg != 0; pair valid iff both active
//                   and same segment.
//   key-mask bidir: every query of a row with at least one active key is a
//                   query of "segment" 1; key j is in segment 1 iff mask != 0.
// Canonical ids: the segment id of an active token, 0 for inactive tokens and
// for the tile padding past the sequence end.  Useful pairs are pairs of
// equal NONZERO ids (plus causality), which is exactly the reference grid
// with the self-fallback rows of inactive queries removed (their outputs are
// multiplied by 0 in the reference, attention.py:261).
//
// Tiles are classified from run-length encodings of the ids, so the cost is
// O(runs_q * runs_k) per tile pair instead of 128 * 128; it stays exact for
// arbitrary (non-contiguous, repeated) ids because every run is compared.
#include "mf_common.h"

namespace mf {

struct MapArgs {
  const int32_t* seg;
  const void* mask;
  int mask_u8;
  int mode;
  int batch, q_len, kv_len;
  PlanLayout lay;
  char* plan;
  int ids_ready;  // qid/kid already hold the canonical ids (key-mask mode, placements)
};

__device__ __forceinline__ int* plan_i32(char* plan, size_t off) {
  return reinterpret_cast<int*>(plan + off);
}

// Key-mask mode ids, one block per (position chunk, row): every query of a
// row with at least one active key gets id 1 (present = any(mask[b, :]),
// bidirectional.py:23), key j gets id 1 iff mask != 0.  The packed modes'
// ids are derived inside the run pass instead.
__global__ __launch_bounds__(256) void token_ids_kernel(MapArgs a) {
  const int b = blockIdx.y;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  int* qid = plan_i32(a.plan, a.lay.qid) + (size_t)b * a.lay.tq_pad;
  int* kid = plan_i32(a.plan, a.lay.kid) + (size_t)b * a.lay.tk_pad;
  int any = 0;
  for (int j = threadIdx.x; j < a.kv_len; j += blockDim.x)
    any |= mask_at(a.mask, a.mask_u8, (long)b * a.kv_len + j) != 0;
  any = __syncthreads_or(any);
  if (p < a.lay.tq_pad) qid[p] = (p < a.q_len && any) ? 1 : 0;
  if (p < a.lay.tk_pad)
    kid[p] = (p < a.kv_len && mask_at(a.mask, a.mask_u8, (long)b * a.kv_len + p) != 0) ? 1 : 0;
}

// Canonical id of token p of row b in the packed modes (q_len == kv_len).
__device__ __forceinline__ int packed_id(const MapArgs& a, int b, int p) {
  if (p >= a.q_len) return 0;
  const long idx = (long)b * a.q_len + p;
  const int m = mask_at(a.mask, a.mask_u8, idx);
  const int s = a.seg[idx];
  const bool active = (a.mode == 0 ? m > 0 : m != 0) && s != 0;
  return active ? s : 0;
}

// One wave per (tile, row): tiles [0, nq) are query tiles, [nq, nq+nk) key
// tiles.  Writes the ordered maximal runs of equal nonzero ids.  In the
// packed modes it also derives the tile's canonical ids from the segment ids
// and mask and stores them (query tiles into qid, key tiles into kid), so no
// separate id pass runs.
__global__ __launch_bounds__(64) void tile_runs_kernel(MapArgs a) {
  const int b = blockIdx.y;
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const bool is_q = t < a.lay.nq;
  const int tile = is_q ? t : t - a.lay.nq;
  int* ids = is_q ? plan_i32(a.plan, a.lay.qid) + (size_t)b * a.lay.tq_pad
                  : plan_i32(a.plan, a.lay.kid) + (size_t)b * a.lay.tk_pad;
  const size_t rec_bytes = sizeof(int) + sizeof(Run) * kMaxRuns;
  char* rec = a.plan + a.lay.runs +
              rec_bytes * ((size_t)b * (a.lay.nq + a.lay.nk) + (size_t)t);
  Run* runs = reinterpret_cast<Run*>(rec + sizeof(int));
  const int p0 = tile * kTile;
  int x[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int p = p0 + half * 64 + lane;
    if (a.ids_ready) {
      x[half] = ids[p];
    } else {
      x[half] = packed_id(a, b, p);
      ids[p] = x[half];
    }
  }
  int n_start = 0, n_stop = 0;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int i = half * 64 + lane;
    const int xv = x[half];
    // neighbours within the tile (the value each source lane offers is
    // chosen for the reader it serves): token i - 1 is lane - 1 of the same
    // half, or for half 1 lane 0 the last token of half 0 (lane 63, x[0]);
    // token i + 1 is lane + 1, or for half 0 lane 63 the first token of half
    // 1 (lane 0, x[1])
    const int up = __shfl(half == 0 ? x[0] : (lane == 63 ? x[0] : x[1]), lane == 0 ? 63 : lane - 1);
    const int dn = __shfl(half == 0 ? (lane == 0 ? x[1] : x[0]) : x[1], lane == 63 ? 0 : lane + 1);
    const int prev = i > 0 ? up : 0;
    const int next = i < kTile - 1 ? dn : 0;
    const bool st = xv != 0 && (i == 0 || prev != xv);
    const bool sp = xv != 0 && (i == kTile - 1 || next != xv);
    const uint64_t bs = __ballot(st);
    const uint64_t bp = __ballot(sp);
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (st) {
      const int k = n_start + __popcll(bs & below);
      runs[k].id = xv;
      runs[k].start = p0 + i;
    }
    if (sp) {
      const int k = n_stop + __popcll(bp & below);
      runs[k].stop = p0 + i + 1;
    }
    n_start += __popcll(bs);
    n_stop += __popcll(bp);
  }
  if (lane == 0) *reinterpret_cast<int*>(rec) = n_start;
}

// A tile's run record with its first kCachedRuns runs loaded into
// registers: the loads of the count and of those runs are independent, so
// they take one memory round trip, and the classification below runs from
// registers unless a record has more runs (then it reads the rest from
// memory).  Slots past the count are read but never used.
constexpr int kCachedRuns = 4;

struct RunList {
  int n;
  Run r[kCachedRuns];
  const Run* all;
};

__device__ __forceinline__ const char* run_record(const MapArgs& a, int b, int t) {
  const size_t rec_bytes = sizeof(int) + sizeof(Run) * kMaxRuns;
  return a.plan + a.lay.runs + rec_bytes * ((size_t)b * (a.lay.nq + a.lay.nk) + (size_t)t);
}

__device__ __forceinline__ RunList load_runs(const char* rec) {
  RunList l;
  l.n = *reinterpret_cast<const int*>(rec);
  l.all = reinterpret_cast<const Run*>(rec + sizeof(int));
#pragma unroll
  for (int i = 0; i < kCachedRuns; ++i) l.r[i] = l.all[i];  // records hold kMaxRuns slots
  return l;
}

// The runs of a list clipped to [lo, hi): how many there are, the id of the
// last one, and whether it covers the whole range.
struct Clip {
  int n, id;
  bool whole;
};

__device__ __forceinline__ Clip clip_runs(const RunList& l, int lo, int hi) {
  Clip c = {0, 0, false};
  auto take = [&](const Run u) {
    const int s = max(u.start, lo), e = min(u.stop, hi);
    if (s < e) {
      ++c.n;
      c.id = u.id;
      c.whole = s == lo && e == hi;
    }
  };
  if (l.n <= kCachedRuns) {
#pragma unroll
    for (int x = 0; x < kCachedRuns; ++x)
      if (x < l.n) take(l.r[x]);
  } else {
    for (int x = 0; x < l.n; ++x) take(l.all[x]);
  }
  return c;
}

// Class of the query rows [q_lo, q_hi) against the keys [k_lo, k_hi) of one
// row, from the query tile's and the key tile's run lists: 0 EMPTY, 1
// PARTIAL, 2 FULL.  The pair is non-empty iff some query run and key run,
// clipped to the ranges, share an id, with the key run starting at or before
// the query run's last token when causal; FULL iff both ranges are one run of
// the same id and, when causal, every key precedes every query.
__device__ __forceinline__ int range_class(bool causal, const RunList& rq, int q_lo, int q_hi,
                                           const RunList& rk, int k_lo, int k_hi) {
  if (causal && k_lo > q_hi - 1) return 0;
  auto meets = [&](const Run u, const Run w) {
    const int us = max(u.start, q_lo), ue = min(u.stop, q_hi);
    const int ws = max(w.start, k_lo), we = min(w.stop, k_hi);
    return us < ue && ws < we && u.id == w.id && (!causal || ws <= ue - 1);
  };
  bool any = false;
  if (rq.n <= kCachedRuns && rk.n <= kCachedRuns) {
#pragma unroll
    for (int x = 0; x < kCachedRuns; ++x)
#pragma unroll
      for (int y = 0; y < kCachedRuns; ++y)
        any |= x < rq.n && y < rk.n && meets(rq.r[x], rk.r[y]);
  } else {
    for (int x = 0; x < rq.n && !any; ++x)
      for (int y = 0; y < rk.n && !any; ++y) any = meets(rq.all[x], rk.all[y]);
  }
  if (!any) return 0;
  const Clip cq = clip_runs(rq, q_lo, q_hi), ck = clip_runs(rk, k_lo, k_hi);
  if (cq.n == 1 && ck.n == 1 && cq.whole && ck.whole && cq.id == ck.id &&
      (!causal || k_hi - 1 <= q_lo))
    return 2;
  return 1;
}

// One block per query-tile row (tile map row and work list of 64-key
// stages) or key-tile column (work list of 64-query stages): the row's or
// column's stage pairs are classified one per thread, and the non-empty ones
// are compacted in increasing stage order as `stage * 4 + class` (ballots
// within each wave, a prefix over the block's waves through LDS).  A tile's
// class in the tile map is that of its two stages together (EMPTY when both
// are, FULL when both are).  Column blocks classify their pairs again rather
// than waiting for the row blocks.  The block has one thread per stage of
// the longer side, up to kListMaxThreads, so that a row takes one round of
// classification wherever it fits (a round's latency is that of the run
// record loads, which no other block hides when the batch is small).
constexpr int kListMaxThreads = 1024;

static int list_threads(int nq, int nk) {
  const int stages = 2 * (nq > nk ? nq : nk);
  const int t = (stages + 63) / 64 * 64;
  return t < kListMaxThreads ? t : kListMaxThreads;
}

__global__ __launch_bounds__(kListMaxThreads) void tile_lists_kernel(MapArgs a) {
  __shared__ int wave_n[kListMaxThreads / 64];
  const int nwaves = blockDim.x >> 6;
  const int b = blockIdx.y;
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nq = a.lay.nq, nk = a.lay.nk;
  uint8_t* tmap = reinterpret_cast<uint8_t*>(a.plan + a.lay.tmap) + (size_t)b * nq * nk;
  const bool row = t < nq;
  const int fixed = row ? t : t - nq;
  const int len = 2 * (row ? nk : nq);  // stages of the other side
  int* list = row ? plan_i32(a.plan, a.lay.qlist) + ((size_t)b * nq + fixed) * 2 * nk
                  : plan_i32(a.plan, a.lay.klist) + ((size_t)b * nk + fixed) * 2 * nq;
  int* count = row ? plan_i32(a.plan, a.lay.qcnt) + (size_t)b * nq + fixed
                   : plan_i32(a.plan, a.lay.kcnt) + (size_t)b * nk + fixed;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const bool causal = a.mode == 0;
  // the row's (column's) own tile record, the same for every thread
  const RunList mine = load_runs(run_record(a, b, row ? fixed : nq + fixed));
  int n = 0;  // entries written by earlier rounds (same value in every thread)
  for (int base = 0; base < len; base += blockDim.x) {
    const int i = base + threadIdx.x;
    int cls = 0;
    if (i < len) {
      const int other = i >> 1, h = i & 1;
      const RunList theirs = load_runs(run_record(a, b, row ? nq + other : other));
      if (row) {
        const int q0 = fixed * kTile, k0 = other * kTile + h * (kTile / 2);
        cls = range_class(causal, mine, q0, q0 + kTile, theirs, k0, k0 + kTile / 2);
      } else {
        const int k0 = fixed * kTile, q0 = other * kTile + h * (kTile / 2);
        cls = range_class(causal, theirs, q0, q0 + kTile / 2, mine, k0, k0 + kTile);
      }
    }
    if (row) {
      // the tile class from the two stage classes (lanes 2j, 2j + 1)
      const int pair = __shfl_xor(cls, 1);
      if (i < len && (i & 1) == 0)
        tmap[(size_t)fixed * nk + (i >> 1)] =
            (uint8_t)((cls == 0 && pair == 0) ? 0 : (cls == 2 && pair == 2) ? 2 : 1);
    }
    const uint64_t bits = __ballot(cls != 0);
    if (lane == 0) wave_n[wave] = __popcll(bits);
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < nwaves; ++w) {
      before += w < wave ? wave_n[w] : 0;
      total += wave_n[w];
    }
    if (cls != 0) list[n + before + __popcll(bits & below)] = i * 4 + cls;
    n += total;
    __syncthreads();  // wave_n is rewritten by the next round
  }
  if (threadIdx.x == 0) *count = n;
}

// Launch orders for the attention grids: the (row, tile) items sorted by
// work-list length, longest first, so that the hardware's in-order dispatch
// approximates longest-processing-time scheduling and the long tiles do not
// end up in the last wave of workgroups.  Equal lengths keep index order
// (the sort is a stable counting sort), so the plan is deterministic.
// Block 0 orders the query tiles, block 1 the key tiles.  Lengths of
// kOrderBuckets - 1 and more share the first bucket.
constexpr int kOrderThreads = 128;
constexpr int kOrderBuckets = 64;

__device__ __forceinline__ int order_bucket(int len) {
  return kOrderBuckets - 1 - min(len, kOrderBuckets - 1);
}

__global__ __launch_bounds__(kOrderThreads) void order_kernel(MapArgs a) {
  // column t of hist belongs to thread t: counts, then scatter cursors.  Rows
  // are padded by one word, so the scan below (lane t walking half of a row)
  // spreads a wave's reads over the banks instead of one bank.
  __shared__ int hist[kOrderBuckets][kOrderThreads + 1];
  __shared__ int part[kOrderThreads];
  const bool qside = blockIdx.x == 0;
  const int n = a.batch * (qside ? a.lay.nq : a.lay.nk);
  const int* len = plan_i32(a.plan, qside ? a.lay.qcnt : a.lay.kcnt);
  int* order = plan_i32(a.plan, qside ? a.lay.qorder : a.lay.korder);
  const int t = threadIdx.x;
  const int per = (n + kOrderThreads - 1) / kOrderThreads;
  const int lo = min(n, t * per), hi = min(n, lo + per);
  for (int k = 0; k < kOrderBuckets; ++k) hist[k][t] = 0;
  for (int i = lo; i < hi; ++i) hist[order_bucket(len[i])][t] += 1;
  __syncthreads();
  // exclusive scan of hist in (bucket, thread) order; thread j owns the E
  // consecutive entries hist[j / 2][(j % 2) E + e], e < E, half of a bucket's
  // row
  static_assert(kOrderThreads == 2 * kOrderBuckets, "scan split");
  constexpr int E = kOrderThreads / 2;
  int* row = &hist[t >> 1][(t & 1) * E];
  int sum = 0;
  for (int e = 0; e < E; ++e) sum += row[e];
  part[t] = sum;
  __syncthreads();
  for (int step = 1; step < kOrderThreads; step <<= 1) {
    const int add = t >= step ? part[t - step] : 0;
    __syncthreads();
    part[t] += add;
    __syncthreads();
  }
  int base = part[t] - sum;
  for (int e = 0; e < E; ++e) {
    const int v = row[e];
    row[e] = base;
    base += v;
  }
  __syncthreads();
  for (int i = lo; i < hi; ++i) order[hist[order_bucket(len[i])][t]++] = i;
}

// Canonical ids straight from the packer's placements (row, start, length)
// -- batching/packing.py:74-102 gives the i-th placed sequence segment id
// i + 1 and positions arange(length) -- so no [B, T] id array has to be
// built on the host and copied in.  Two passes: clear, then one block per
// placement writes its tokens (placements do not overlap, as the packer
// guarantees; tokens outside [0, T) are dropped).
__global__ __launch_bounds__(256) void placement_clear_kernel(MapArgs a, int32_t* seg_out,
                                                              int32_t* pos_out) {
  const int b = blockIdx.y;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < a.lay.tq_pad) plan_i32(a.plan, a.lay.qid)[(size_t)b * a.lay.tq_pad + p] = 0;
  if (p < a.lay.tk_pad) plan_i32(a.plan, a.lay.kid)[(size_t)b * a.lay.tk_pad + p] = 0;
  if (p < a.q_len) {
    if (seg_out) seg_out[(size_t)b * a.q_len + p] = 0;
    if (pos_out) pos_out[(size_t)b * a.q_len + p] = 0;
  }
}

__global__ __launch_bounds__(256) void placement_ids_kernel(MapArgs a, const int32_t* placements,
                                                            int32_t* seg_out, int32_t* pos_out) {
  const int i = blockIdx.x;
  const int row = placements[3 * i], start = placements[3 * i + 1], len = placements[3 * i + 2];
  if (row < 0 || row >= a.batch) return;
  const int lo = max(start, 0), hi = min(start + len, a.q_len);
  for (int t = lo + threadIdx.x; t < hi; t += blockDim.x) {
    plan_i32(a.plan, a.lay.qid)[(size_t)row * a.lay.tq_pad + t] = i + 1;
    plan_i32(a.plan, a.lay.kid)[(size_t)row * a.lay.tk_pad + t] = i + 1;
    if (seg_out) seg_out[(size_t)row * a.q_len + t] = i + 1;
    if (pos_out) pos_out[(size_t)row * a.q_len + t] = t - start;
  }
}

static void launch_map_tail(const MapArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(tile_runs_kernel, dim3(a.lay.nq + a.lay.nk, a.batch), dim3(64), 0, stream, a);
  hipLaunchKernelGGL(tile_lists_kernel, dim3(a.lay.nq + a.lay.nk, a.batch),
                     dim3(list_threads(a.lay.nq, a.lay.nk)), 0, stream, a);
  hipLaunchKernelGGL(order_kernel, dim3(2), dim3(kOrderThreads), 0, stream, a);
}

hipError_t launch_block_map_placements(const int32_t* placements, int count, int mode, int batch,
                                       int length, void* plan, int32_t* seg_out, int32_t* pos_out,
                                       hipStream_t stream) {
  MapArgs a;
  a.seg = nullptr;
  a.mask = nullptr;
  a.mask_u8 = 0;
  a.mode = mode;
  a.batch = batch;
  a.q_len = length;
  a.kv_len = length;
  a.lay = plan_layout(batch, length, length);
  a.plan = reinterpret_cast<char*>(plan);
  a.ids_ready = 1;
  hipLaunchKernelGGL(placement_clear_kernel, dim3((a.lay.tq_pad + 255) / 256, batch), dim3(256), 0,
                     stream, a, seg_out, pos_out);
  if (count > 0)
    hipLaunchKernelGGL(placement_ids_kernel, dim3(count), dim3(256), 0, stream, a, placements,
                       seg_out, pos_out);
  launch_map_tail(a, stream);
  return hipGetLastError();
}

hipError_t launch_block_map(const int32_t* seg, const void* mask, int mask_u8, int mode,
                            int batch, int q_len, int kv_len, void* plan,
                            hipStream_t stream) {
  MapArgs a;
  a.seg = seg;
  a.mask = mask;
  a.mask_u8 = mask_u8;
  a.mode = mode;
  a.batch = batch;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.lay = plan_layout(batch, q_len, kv_len);
  a.plan = reinterpret_cast<char*>(plan);
  // packed modes: the run pass derives the ids itself; the key-mask mode
  // needs a row-wide "any key active" first
  a.ids_ready = mode == 2;
  if (a.ids_ready) {
    const int pad = a.lay.tq_pad > a.lay.tk_pad ? a.lay.tq_pad : a.lay.tk_pad;
    hipLaunchKernelGGL(token_ids_kernel, dim3((pad + 255) / 256, batch), dim3(256), 0, stream, a);
  }
  launch_map_tail(a, stream);
  return hipGetLastError();
}

}  // namespace mf
