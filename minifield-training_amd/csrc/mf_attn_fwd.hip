// Flash-style forward for segment-masked GQA attention on gfx950.
//
// Two kernels: the bf16 one (further below; the benchmarked path) and an
// fp32 one.  fp32 work unit: one workgroup = 4 waves = one 128-query
// tile of one row, for HPW (1 or 2) query heads that share a KV head.  Each
// wave owns 32 queries for all HPW heads, so every K / V^T fragment it reads
// from LDS feeds HPW MFMAs (the GQA sharing of K/V tiles).  The workgroup
// walks the compacted list of non-empty 128-key tiles of its query tile (from
// the block map) in 64-key steps, double-buffering K and V in LDS.
//
// Scores are formed transposed, S^T = K Q^T, so an accumulator column is one
// query: the row max and row sum are in-lane reductions plus one
// v_permlane32_swap, and the exponentiated block is already in the register
// layout of the B operand of O^T += V^T P^T.  PARTIAL tiles compare the
// canonical ids (and causality) per element; FULL tiles skip the compare.
// Online softmax in base 2 with the logit scale folded into one FMA.
#include "mf_common.h"
#include "mf_lds.h"

namespace mf {

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  const int* qid;
  const int* kid;
  const int* qcnt;
  const int* qlist;
  const int* qorder;
  int T, S, Hq, Hkv, G, hchunks;
  int nq, nk, tq_pad, tk_pad;
  int causal;
  float scale, scale_log2;
  FastDiv div_nh, div_hchunks, div_nq;  // Hkv * hchunks, hchunks, nq
  // query prologue fused into the bf16 kernel's query loads (ROPE instances)
  const void* q_gain;           // [64], tensor dtype
  const int32_t* positions;     // [B, T] or null (0 .. T-1 on every row)
  const uint32_t* rope_table;   // [B * T][32] (bf16 cos | bf16 sin << 16)
  float eps;
  float freq[kD / 2];
};

constexpr int kStepK = 64;          // keys per inner step
constexpr int kLdsRowF = kD + 1;    // fp32 LDS row pitch (65 floats)

struct FwdLdsF32 {
  float k[2][kStepK * kLdsRowF];  // K [key][d]
  float v[2][kStepK * kLdsRowF];  // V [key][d]
  int kid[2][kStepK];
};

// Global -> register staging of one 64-key step (K and V) for the workgroup.
struct FwdStageF32 {
  u32x4 r[8];
};

__device__ __forceinline__ void fwd_load_f32(const FwdArgs& a, int b, int kvh, int kb,
                                             FwdStageF32& st) {
  const int tid = threadIdx.x;
  const float* ks = reinterpret_cast<const float*>(a.k);
  const float* vs = reinterpret_cast<const float*>(a.v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i;
    const int key = kb + (u >> 4), ch = u & 15;
    const size_t off = (((size_t)b * a.S + key) * a.Hkv + kvh) * kD + ch * 4;
    st.r[i] = key < a.S ? ld_u32x4(ks + off) : u32x4{0, 0, 0, 0};
    st.r[4 + i] = key < a.S ? ld_u32x4(vs + off) : u32x4{0, 0, 0, 0};
  }
}

__device__ __forceinline__ void fwd_store_f32(const FwdArgs& a, int b, int kb,
                                              const FwdStageF32& st, FwdLdsF32& lds, int buf) {
  const int tid = threadIdx.x;
  if (tid < kStepK) lds.kid[buf][tid] = a.kid[(size_t)b * a.tk_pad + kb + tid];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i;
    const int key = u >> 4, ch = u & 15;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds.k[buf][key * kLdsRowF + ch * 4 + e] = __uint_as_float(st.r[i][e]);
      lds.v[buf][key * kLdsRowF + ch * 4 + e] = __uint_as_float(st.r[4 + i][e]);
    }
  }
}

template <int HPW>
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(FwdArgs a) {
  __shared__ FwdLdsF32 lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = lane >> 5;
  // 1-D grid: (query-tile item in launch order, kvh, head chunk), heads fastest
  const int nh = a.Hkv * a.hchunks;
  const int slot = uniform(fast_div(blockIdx.x, a.div_nh));
  const int hr = uniform(blockIdx.x - slot * nh);
  const int kvh = uniform(fast_div(hr, a.div_hchunks));
  const int hc = uniform(hr - kvh * a.hchunks);
  const int item = ld_const(a.qorder, slot);  // (row, query tile), longest first
  const int b = uniform(fast_div(item, a.div_nq));
  const int qt = uniform(item - b * a.nq);
  const int qpos = qt * kTile + wave * 32 + (lane & 31);
  const int myqid = a.qid[(size_t)b * a.tq_pad + qpos];
  const bool qvalid = qpos < a.T;
  int head[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) head[j] = kvh * a.G + hc * HPW + j;

  // ---- query fragments (B operand of S^T = K Q^T) -----------------------
  float qf[HPW][32];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const float* src = reinterpret_cast<const float*>(a.q) +
                       (((size_t)b * a.T + qpos) * a.Hq + head[j]) * kD + half;
#pragma unroll
    for (int st = 0; st < 32; ++st) qf[j][st] = qvalid ? src[2 * st] : 0.f;
  }

  f32x16 oacc[HPW][2];
  float m[HPW], l[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    oacc[j][0] = zero16();
    oacc[j][1] = zero16();
    m[j] = kNegInf;
    l[j] = 0.f;
  }

  const int count = ld_const(a.qcnt, b * a.nq + qt);
  const int* list = a.qlist + ((size_t)b * a.nq + qt) * 2 * a.nk;
  const int nsteps = count;  // one 64-key stage per list entry
  const float c = a.scale_log2;

  FwdStageF32 stage;
  if (nsteps > 0) {
    const int e0 = list[0];
    fwd_load_f32(a, b, kvh, (e0 >> 2) * kStepK, stage);
    fwd_store_f32(a, b, (e0 >> 2) * kStepK, stage, lds, 0);
  }
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const int entry = list[step];
    const int kb = (entry >> 2) * kStepK;
    const bool partial = (entry & 3) == 1;
    int next_kb = 0;
    if (step + 1 < nsteps) {
      next_kb = (list[step + 1] >> 2) * kStepK;
      fwd_load_f32(a, b, kvh, next_kb, stage);
    }

    // ---- S^T = K Q^T for two 32-key blocks --------------------------------
    f32x16 s[HPW][2];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int j = 0; j < HPW; ++j) s[j][kb2] = zero16();
      const float* krow = &lds.k[buf][(kb2 * 32 + (lane & 31)) * kLdsRowF + half];
#pragma unroll
      for (int st = 0; st < 32; ++st) {
        const float af = krow[2 * st];
#pragma unroll
        for (int j = 0; j < HPW; ++j) s[j][kb2] = mfma32x32x2(af, qf[j][st], s[j][kb2]);
      }
    }

    // ---- element mask on PARTIAL tiles ------------------------------------
    if (partial) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int kk0 = kb2 * 32 + 8 * g4 + 4 * half;
          const int4 kids = *reinterpret_cast<const int4*>(&lds.kid[buf][kk0]);
          const int kv[4] = {kids.x, kids.y, kids.z, kids.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool ok = kv[i] == myqid && (!a.causal || kb + kk0 + i <= qpos);
#pragma unroll
            for (int j = 0; j < HPW; ++j)
              s[j][kb2][g4 * 4 + i] = ok ? s[j][kb2][g4 * 4 + i] : kNegInf;
          }
        }
      }
    }

    // ---- online softmax (base 2) -------------------------------------------
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      float mx = kNegInf;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[j][kb2][r], s[j][kb2][r + 1]));
      mx = halves_max(mx);
      const float mnew = fmaxf(m[j], mx);
      const float msafe = mnew == kNegInf ? 0.f : mnew;
      const float alpha = fast_exp2((m[j] - msafe) * c);
      m[j] = mnew;
      l[j] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        oacc[j][0][r] *= alpha;
        oacc[j][1][r] *= alpha;
      }
      const float mc = msafe * c;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(fmaf(s[j][kb2][r], c, -mc));
          s[j][kb2][r] = p;
          l[j] += p;
        }
    }

    // ---- O^T += V^T P^T -------------------------------------------------------
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float vf = lds.v[buf][(kb2 * 32 + acc_row(r, lane)) * kLdsRowF + db * 32 + (lane & 31)];
#pragma unroll
          for (int j = 0; j < HPW; ++j) oacc[j][db] = mfma32x32x2(vf, s[j][kb2][r], oacc[j][db]);
        }

    if (step + 1 < nsteps) fwd_store_f32(a, b, next_kb, stage, lds, buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----------------------------------------------------------------
  const bool qactive = qvalid && myqid != 0;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const float lt = halves_sum(l[j]);
    const bool has = qactive && lt > 0.f;
    const float inv = has ? 1.f / lt : 0.f;
    if (qvalid) {
      if (half == 0)
        a.lse[((size_t)b * a.Hq + head[j]) * a.T + qpos] =
            has ? fmaf(m[j], a.scale, __logf(lt)) : kPosInf;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d0 = db * 32 + 8 * g4 + 4 * half;
          const size_t off = (((size_t)b * a.T + qpos) * a.Hq + head[j]) * kD + d0;
          f32x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = has ? oacc[j][db][g4 * 4 + i] * inv : 0.f;
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + off) = o;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 forward: one head per wave, 4*HPW waves per workgroup.
//
// Wave w serves head hc*HPW + w/4 of the KV group and queries
// [qt*128 + 32 (w%4), +32).  All waves of the workgroup share each 64-key
// step's K and V tiles (the GQA sharing).  The tiles are DMA'd from HBM into a
// two-slot LDS ring of 128-key slots, one slot ahead of use (no staging
// registers); K feeds the S^T = K Q^T MFMAs directly and V^T is read with
// transposing LDS reads.  Rescaling of the output accumulator is lazy: the
// running max used for the exponentials only moves when the true max exceeds
// it by more than 8 in log2 units, so P <= 2^8 and the final division by the
// row sum is unchanged.  Row sums are v_dot2 of the bf16 probabilities with
// (1, 1), a full-rate VALU op that halves the adds.
// ---------------------------------------------------------------------------
// The query half of the attention prologue on the query fragments a lane
// holds (dims 16 ks + 8 half .. +7 of one query row, ks = 0..3; the other
// half of the row is in lane ^ 32): RMS normalisation with the per-dimension
// gain, then the rotary embedding, with the arithmetic and the bf16 rounding
// points of qk_norm_rope_kernel step for step, so the fragments equal that
// kernel's output bit for bit.  Its sum of squares adds the fma-chain sums
// of the eight 8-dim chunks as ((c0 + c1) + (c2 + c3)) + ((c7 + c6) + (c5 +
// c4)) (its 8-lane DPP butterfly); here chunk 2 ks + half is this lane's and
// chunk 2 ks + (1 - half) comes from lane ^ 32.  The rotation partner of
// dims 16 ks + .. (ks < 2) is the same lane's fragment ks + 2.  cos and sin
// come from the token's row of the table rope_table_kernel fills.
__device__ __forceinline__ void rope_query(const FwdArgs& a, int b, int qpos, int half,
                                           bf16x8 (&qf)[4]) {
  const int t = min(qpos, a.T - 1);
  // angle pairs of this lane's dims: angles 8 half + i (fragments 0, 2) and
  // 16 + 8 half + i (fragments 1, 3), i < 8
  uint32_t cs[2][8];
  const uint32_t* row = a.rope_table + ((size_t)b * a.T + t) * (kD / 2) + 8 * half;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(row + 16 * j);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(row + 16 * j + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t l = lo[i], h = hi[i];  // through scalars (vector element reads)
      cs[j][i] = l;
      cs[j][4 + i] = h;
    }
  }
  bf16x8 w[4];  // gains of this lane's dims
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    w[ks] = ld_bf16x8(reinterpret_cast<const bf16*>(a.q_gain) + 16 * ks + 8 * half);
  // chunk sums: mine[ks] is chunk 2 ks + half, theirs[ks] chunk 2 ks + 1 - half
  float mine[4], theirs[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = (float)qf[ks][i];
      ss = fmaf(x, x, ss);
    }
    mine[ks] = ss;
    theirs[ks] = __shfl_xor(ss, 32);
  }
  float c[8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    c[2 * ks] = half ? theirs[ks] : mine[ks];
    c[2 * ks + 1] = half ? mine[ks] : theirs[ks];
  }
  const float total = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[7] + c[6]) + (c[5] + c[4]));
  const float inv = rsqrtf(total * (1.f / kD) + a.eps);
  // n = bf16(bf16(x * inv) * gain), kept as bf16 pairs
  uint32_t n[4][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const uint32_t y = round_bf16_pair((float)qf[ks][i] * inv, (float)qf[ks][i + 1] * inv);
      n[ks][i / 2] = round_bf16_pair(bf16_lo(y) * (float)w[ks][i], bf16_hi(y) * (float)w[ks][i + 1]);
    }
  auto nval = [&](int ks, int i) { return (i & 1) ? bf16_hi(n[ks][i / 2]) : bf16_lo(n[ks][i / 2]); };
  const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int j = ks & 1;  // angle block of fragment ks
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // rotate_half: dims < 32 take -n[d + 32], dims >= 32 take n[d - 32]
      const float r = ks < 2 ? -nval(ks + 2, i) : nval(ks - 2, i);
      const float cv = bf16_lo(cs[j][i]), sv = bf16_hi(cs[j][i]);
      const uint32_t pq = round_bf16_pair(nval(ks, i) * cv, r * sv);
      qf[ks][i] = (bf16)__builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pq), ones, 0.f,
                                                        false);
    }
  }
}

template <int HPW, bool ROPE>
__global__ __launch_bounds__(256 * HPW) __attribute__((amdgpu_waves_per_eu(2 * HPW)))
void attn_fwd_bf16_kernel(FwdArgs a) {
  constexpr int W = 4 * HPW;
  // two ring slots of 128 keys, each two 64-key stages
  __shared__ __attribute__((aligned(16))) char slotA[2 * kStageBytes], slotB[2 * kStageBytes];
  const int lane = threadIdx.x & 63;
  // scalar wave index: keeps the DMA destinations scalar expressions of the
  // stage arrays, so the compiler sees which stage each DMA writes
  const int wave = uniform(threadIdx.x >> 6);
  const int half = lane >> 5;
  // 1-D grid: (query-tile item in launch order, kvh, head chunk), heads fastest
  const int nh = a.Hkv * a.hchunks;
  const int slot = uniform(fast_div(blockIdx.x, a.div_nh));
  const int hr = uniform(blockIdx.x - slot * nh);
  const int kvh = uniform(fast_div(hr, a.div_hchunks));
  const int hc = uniform(hr - kvh * a.hchunks);
  const int item = ld_const(a.qorder, slot);  // (row, query tile), longest first
  const int b = uniform(fast_div(item, a.div_nq));
  const int qt = uniform(item - b * a.nq);
  const int head = kvh * a.G + hc * HPW + (wave >> 2);
  const int qpos = qt * kTile + (wave & 3) * 32 + (lane & 31);
  const int myqid = a.qid[(size_t)b * a.tq_pad + qpos];

  bf16x8 qf[4];
  {
    const bf16* src = reinterpret_cast<const bf16*>(a.q) +
                      (((size_t)b * a.T + min(qpos, a.T - 1)) * a.Hq + head) * kD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = ld_bf16x8(src + ks * 16);
  }
  if constexpr (ROPE) rope_query(a, b, qpos, half, qf);
  drain_memory();

  f32x16 oacc[2] = {zero16(), zero16()};
  // Exponentials are taken of x = s*c - shift (base 2).  shift is the running
  // max in log2 units once a valid key was seen (0 before); it only moves
  // when a new max exceeds it by more than `lag` (8 once set, -inf before).
  float shift = 0.f, lag = kNegInf;
  float l0 = 0.f, l1 = 0.f;  // row-sum partials
  const float c = a.scale_log2;

  const int count = ld_const(a.qcnt, b * a.nq + qt);
  const int* list = a.qlist + ((size_t)b * a.nq + qt) * 2 * a.nk;
  const int nsteps = count;  // one 64-key stage per list entry
  const int tr_row = tr_row_of(lane);
  const int tr_col = tr_col_of(lane);
  const int* kid_row = a.kid + (size_t)b * a.tk_pad;
  const uint32_t row_stride = (uint32_t)a.Hkv * kD * sizeof(bf16);
  const char* kg = reinterpret_cast<const char*>(a.k) + ((size_t)b * a.S * a.Hkv + kvh) * kD * sizeof(bf16);
  const char* vg = reinterpret_cast<const char*>(a.v) + ((size_t)b * a.S * a.Hkv + kvh) * kD * sizeof(bf16);

  const KvLanes<W> kv_lane = kv_lanes<W>(row_stride, wave);
  auto issue = [&](int entry, char* stage) {
    kv_dma<W>(kg, vg, row_stride, a.S, kid_row, (entry >> 2) * kStepK, wave, stage, kv_lane);
  };

  // Sub-block classification inside PARTIAL tiles.  A wave's 32 queries
  // against one 32-key block are skipped when no pair can be valid, run
  // without masks when every pair is valid, and masked otherwise (ids only,
  // causal only, or both).  When the wave's query ids are not all equal
  // every block of a PARTIAL tile is masked.
  const int q0 = qt * kTile + (wave & 3) * 32;
  const int u = uniform(myqid);
  const bool quni = __all(myqid == u);

  auto scores = [&](const char* kt, int kb2) {
    f32x16 s = zero16();
    const int krow = kb2 * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) s = mfma32x32x16(tile_chunk(kt, krow, 2 * ks + half), qf[ks], s);
    return s;
  };

  // masks of one block; returns the row max of its raw scores (both halves)
  auto mask_block = [&](f32x16& s, const int* kids_lds, int kb, int kb2, bool mask_ids, bool diag) {
    if (mask_ids) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int kk0 = kb2 * 32 + 8 * g4 + 4 * half;
        const int4 kids = *reinterpret_cast<const int4*>(&kids_lds[kk0]);
        const int kv[4] = {kids.x, kids.y, kids.z, kids.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) s[g4 * 4 + i] = kv[i] == myqid ? s[g4 * 4 + i] : kNegInf;
      }
    }
    if (diag) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        s[r] = kb + kb2 * 32 + acc_row(r, lane) <= qpos ? s[r] : kNegInf;
    }
    float mx = fmaxf(s[0], s[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) mx = fmaxf(fmaxf(mx, s[r]), s[r + 1]);
    return mx;
  };
  // probabilities 2^(s c - shift), row sums and O += P V of one block
  auto finish_pv = [&](f32x16& s, const char* vt, int kb2) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], c, -shift));
    const bf16x8 p0 = pack8(s, 0), p1 = pack8(s, 8);
    // row sum of the bf16 probabilities that P V uses: one v_dot2 with
    // (1, 1) per pair (copied through scalars: __builtin_bit_cast of a
    // vector element reads element 0 whatever the index, clang 22)
    {
      const u32x4 w0 = __builtin_bit_cast(u32x4, p0), w1 = __builtin_bit_cast(u32x4, p1);
      const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a0 = w0[j], a1 = w1[j];
        l0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a0), ones, l0, false);
        l1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a1), ones, l1, false);
      }
    }
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const bf16x8 v0 = tile_tr_operand(vt, kb2 * 32 + tr_row, db * 32 + tr_col);
      const bf16x8 v1 = tile_tr_operand(vt, kb2 * 32 + 16 + tr_row, db * 32 + tr_col);
      oacc[db] = mfma32x32x16(v0, p0, oacc[db]);
      oacc[db] = mfma32x32x16(v1, p1, oacc[db]);
    }
  };

  // One step = two 32-key blocks.  Both score blocks are issued before any
  // softmax work, so the second block's MFMAs run under the first block's
  // masks and max; both blocks share one shift decision; the first block's
  // P V then runs under the second block's exponentials.
  auto compute = [&](int step, int entry, const char* stage) {
    const int kb = (entry >> 2) * kStepK;
    const bool partial = (entry & 3) == 1;
    const char* kt = stage;
    const char* vt = stage + kTileBytes;
    const int* kids_lds = reinterpret_cast<const int*>(stage + 2 * kTileBytes);
    bool run[2] = {true, true}, mask_ids[2] = {false, false}, diag[2] = {false, false};
    if (partial) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        const int k0 = kb + kb2 * 32;
        const bool above = a.causal && k0 > q0 + 31;
        diag[kb2] = a.causal && k0 + 31 > q0;
        if (quni) {
          const uint64_t m = __ballot(kids_lds[kb2 * 32 + (lane & 31)] == u);
          run[kb2] = !above && u != 0 && m != 0;
          mask_ids[kb2] = m != ~0ull;
        } else {
          run[kb2] = !above;
          mask_ids[kb2] = true;
        }
      }
    }
    f32x16 s0, s1;
    if (run[0]) s0 = scores(kt, 0);
    if (run[1]) s1 = scores(kt, 1);
    // One shift decision for the step's two blocks, taken on the raw scores
    // before either block's probabilities exist: c > 0 and the rounding of
    // an FMA is monotone, so fma(max s, c, -shift) is exactly the max of the
    // shifted scores.  A growing lane moves its shift to the new max: d > 0
    // and finite, so alpha = 2^-d is finite (a lane with no valid key yet has
    // l = 0, O = 0).  At a tile's first step every lane has l = 0 and O = 0,
    // so the rescale is skipped there.
    float mx = kNegInf;
    if (run[0]) mx = mask_block(s0, kids_lds, kb, 0, mask_ids[0], diag[0]);
    if (run[1]) mx = fmaxf(mx, mask_block(s1, kids_lds, kb, 1, mask_ids[1], diag[1]));
    mx = fmaf(halves_max(mx), c, -shift);
    const bool grow = mx > lag;
    if (__any(grow)) {
      const float d = grow ? mx : 0.f;
      shift += d;
      lag = grow ? 8.f : lag;
      if (step > 0) {
        const float alpha = fast_exp2(-d);
        l0 *= alpha;
        l1 *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          oacc[0][r] *= alpha;
          oacc[1][r] *= alpha;
        }
      }
    }
    if (run[0]) finish_pv(s0, vt, 0);
    if (run[1]) finish_pv(s1, vt, 1);
  };

  // Ring of two 128-key slots: the DMAs of slot i+1 are issued right after
  // the barrier that opens slot i, so they have the compute of slot i (four
  // 32-key blocks) to land, and one barrier serves 128 keys.
  auto issue_slot = [&](int i, int e0, int e1, char* slot) {
    if (2 * i < nsteps) issue(e0, slot);
    if (2 * i + 1 < nsteps) issue(e1, slot + kStageBytes);
  };
  const int nslots = (nsteps + 1) >> 1;
  // The list entries a pair of slots needs (steps 2i .. 2i+5) arrive in one
  // scalar load of eight, issued before the pair's first wait.  The read may
  // run up to 7 entries past the list's end, into the plan's next section
  // (query lists are followed by the key-tile counts); entries at or past
  // nsteps are never used.
  {
    const i32x8u e = ld_const8(list, 0);
    issue_slot(0, e[0], e[1], slotA);
  }
  // Whole pairs of slots; a slot past the end is skipped whole (its wait,
  // barrier and computes; nslots is uniform over the workgroup) rather than
  // leaving the loop mid-pair (a mid-pair exit gives the accumulators two
  // exit paths, resolved with register copies).
  for (int i = 0; i < nslots; i += 2) {
    const i32x8u e = ld_const8(list, 2 * i);
    wait_vmcnt<0>();
    barrier();
    issue_slot(i + 1, e[2], e[3], slotB);
    compute(2 * i, e[0], slotA);
    if (2 * i + 1 < nsteps) compute(2 * i + 1, e[1], slotA + kStageBytes);
    if (i + 1 < nslots) {
      wait_vmcnt<0>();
      barrier();
      issue_slot(i + 2, e[4], e[5], slotA);
      compute(2 * i + 2, e[2], slotB);
      if (2 * i + 3 < nsteps) compute(2 * i + 3, e[3], slotB + kStageBytes);
    }
  }
  wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS at exit

  // the lane's query position and half again from the lane id: recomputing
  // them is cheaper than keeping them (the compiler would spill them) across
  // the loop
  const int elane = fresh_lane_id();
  const int ehalf = elane >> 5;
  const int eqpos = qt * kTile + (wave & 3) * 32 + (elane & 31);
  const bool eqvalid = eqpos < a.T;
  const bool qactive = eqvalid && myqid != 0;
  const float lt = halves_sum(l0 + l1);
  const bool has = qactive && lt > 0.f;
  const float inv = has ? 1.f / lt : 0.f;
  if (eqvalid) {
    // natural-log LSE: shift / log2(e) + ln(l)
    if (ehalf == 0)
      a.lse[((size_t)b * a.Hq + head) * a.T + eqpos] = has ? fmaf(shift, kLn2, __logf(lt)) : kPosInf;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = db * 32 + 8 * g4 + 4 * ehalf;
        const bf16x4 o = scaled_bf16x4(oacc[db], g4 * 4, inv, has);
        *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(a.out) +
                                   (((size_t)b * a.T + eqpos) * a.Hq + head) * kD + d0) = o;
      }
  }
}

// Arguments of one forward launch: operands, the plan's sections, shapes and
// the workgroup shape (heads per workgroup: 2 when the GQA group splits into
// pairs, else 1).
static FwdArgs fwd_args(const void* q, const void* k, const void* v, int batch, int T, int S,
                        int Hq, int Hkv, int mode, float scale, const void* plan, void* out,
                        float* lse, int* hpw) {
  FwdArgs a = {};
  const PlanLayout lay = plan_layout(batch, T, S);
  const char* p = reinterpret_cast<const char*>(plan);
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.lse = lse;
  a.qid = reinterpret_cast<const int*>(p + lay.qid);
  a.kid = reinterpret_cast<const int*>(p + lay.kid);
  a.qcnt = reinterpret_cast<const int*>(p + lay.qcnt);
  a.qlist = reinterpret_cast<const int*>(p + lay.qlist);
  a.qorder = reinterpret_cast<const int*>(p + lay.qorder);
  a.T = T;
  a.S = S;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  *hpw = (a.G % 2 == 0) ? 2 : 1;
  a.hchunks = a.G / *hpw;
  a.nq = lay.nq;
  a.nk = lay.nk;
  a.tq_pad = lay.tq_pad;
  a.tk_pad = lay.tk_pad;
  a.causal = mode == 0;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.div_nh = make_fastdiv(a.Hkv * a.hchunks);
  a.div_hchunks = make_fastdiv(a.hchunks);
  a.div_nq = make_fastdiv(a.nq);
  return a;
}

hipError_t launch_attn_fwd(const void* q, const void* k, const void* v, bool f32, int batch,
                           int T, int S, int Hq, int Hkv, int mode, float scale,
                           const void* plan, void* out, float* lse, hipStream_t stream) {
  int hpw;
  const FwdArgs a = fwd_args(q, k, v, batch, T, S, Hq, Hkv, mode, scale, plan, out, lse, &hpw);
  const dim3 grid(Hkv * a.hchunks * batch * a.nq);
  if (f32) {
    if (hpw == 2)
      hipLaunchKernelGGL((attn_fwd_f32_kernel<2>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_f32_kernel<1>), grid, dim3(256), 0, stream, a);
  } else {
    if (hpw == 2)
      hipLaunchKernelGGL((attn_fwd_bf16_kernel<2, false>), grid, dim3(512), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_bf16_kernel<1, false>), grid, dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

// cos and sin of each token's 32 angles f32(position) * freq[i], rounded to
// bf16 and packed (cos in the low half): the values qk_norm_rope_kernel
// computes for the token (the same position, the same sincosf of the same
// single-precision product) and rounds before use.
__global__ __launch_bounds__(256) void rope_table_kernel(FwdArgs a, uint32_t* table, size_t n) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n * (kD / 2)) return;
  const size_t tok = idx / (kD / 2);
  const int i = (int)(idx % (kD / 2));
  const float pos = (float)(a.positions ? a.positions[tok] : (int)(tok % a.T));
  float f = a.freq[0];
#pragma unroll
  for (int j = 1; j < kD / 2; ++j) f = i == j ? a.freq[j] : f;  // no per-lane argument indexing
  float sv, cv;
  sincosf(pos * f, &sv, &cv);
  table[idx] = round_bf16_pair(cv, sv);
}

size_t rope_table_bytes(int B, int T) { return sizeof(uint32_t) * (kD / 2) * (size_t)B * T; }

hipError_t launch_attn_fwd_rope_q(const void* q_raw, const void* k, const void* v,
                                  const void* q_gain, const int32_t* positions, int batch, int T,
                                  int S, int Hq, int Hkv, int mode, float scale, float eps,
                                  float theta, const void* plan, void* table, void* out,
                                  float* lse, hipStream_t stream) {
  int hpw;
  FwdArgs a = fwd_args(q_raw, k, v, batch, T, S, Hq, Hkv, mode, scale, plan, out, lse, &hpw);
  a.q_gain = q_gain;
  a.positions = positions;
  a.rope_table = reinterpret_cast<const uint32_t*>(table);
  a.eps = eps;
  // theta ** (-arange(0, D, 2) / D) in single precision (rotary.py:33-35), as
  // the prologue's launcher computes them
  for (int i = 0; i < kD / 2; ++i) a.freq[i] = powf(theta, -((float)(2 * i) / (float)kD));
  const size_t tokens = (size_t)batch * T;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((tokens * (kD / 2) + 255) / 256)),
                     dim3(256), 0, stream, a, reinterpret_cast<uint32_t*>(table), tokens);
  const dim3 grid(Hkv * a.hchunks * batch * a.nq);
  if (hpw == 2)
    hipLaunchKernelGGL((attn_fwd_bf16_kernel<2, true>), grid, dim3(512), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_bf16_kernel<1, true>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mf
