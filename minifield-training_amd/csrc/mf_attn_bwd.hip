// Backward of the segment-masked flash forward on gfx950.
//
// Three deterministic launches (no atomics, fixed reduction order):
//   1. delta:  D[b,h,t] = sum_d dO * O   (fp32), one thread per (b, t, h);
//              the workspace keeps -D and lse2 = lse * log2(e) per row.
//   2. dq:     per 128-query tile (like the forward): recompute
//              S^T = K Q^T and dP^T = V dO^T over the tile's non-empty key
//              stages, P^T = exp2(c S^T - lse2), dS^T = P^T (dP^T - D), and
//              dQ^T += K^T dS^T, with dS^T fed from its accumulator
//              registers as the B operand and K^T read from the natural K
//              tile in LDS by transposing reads.
//   3. dkdv:   per 128-key tile and KV head: K and V stay in registers;
//              for every non-empty query stage and every query head of the
//              GQA group, S = Q K^T and dP = dO V^T (accumulator column =
//              key), then dV^T += dO^T P and dK^T += Q^T dS with dO^T and
//              Q^T read transposed from the Q / dO tiles.  The group's heads
//              are summed in registers, which is the transpose of the
//              reference's jnp.repeat of K/V (kernels/attention.py:19-22).
// The fp32 kernels (parity tests, smoke) stage through registers and read
// single floats with v_mfma_f32_32x32x2_f32.
// Rows with no valid key have lse = +inf, so their P is exactly 0 and they
// contribute nothing; their dq is written as 0.
#include "mf_common.h"
#include "mf_lds.h"

namespace mf {

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const float* lse;
  float* ndelta;  // workspace: -D per row, [B, Hq, T]
  float* lse2;    // workspace: lse * log2(e) per row, [B, Hq, T]
  void* dq;
  void* dk;
  void* dv;
  const int* qid;
  const int* kid;
  const int* qcnt;
  const int* qlist;
  const int* kcnt;
  const int* klist;
  const int* qorder;
  const int* korder;
  int T, S, Hq, Hkv, G, hchunks;
  int nq, nk, tq_pad, tk_pad;
  int causal;
  int fuse_delta;  // bf16 dq computes D = rowsum(dO * O) itself and writes -D and lse2
  float scale, scale_log2;
  FastDiv div_nh, div_hchunks, div_nq, div_hkv, div_nk, div_g;  // Hkv * hchunks, hchunks, nq, Hkv, nk, G
};

constexpr int kStep = 64;
constexpr int kRowF = kD + 1;  // fp32 LDS row pitch

// ---------------------------------------------------------------------------
// 1. delta
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdArgs a, int B) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // (b, t, h)
  const size_t total = (size_t)B * a.T * a.Hq;
  if (idx >= total) return;
  const int h = idx % a.Hq;
  const size_t bt = idx / a.Hq;
  const int t = bt % a.T;
  const int b = bt / a.T;
  float acc = 0.f;
  if constexpr (!F32) {
    const bf16* o = reinterpret_cast<const bf16*>(a.out) + idx * kD;
    const bf16* g = reinterpret_cast<const bf16*>(a.dout) + idx * kD;
#pragma unroll
    for (int c8 = 0; c8 < 8; ++c8) {
      const bf16x8 x = ld_bf16x8(o + c8 * 8);
      const bf16x8 y = ld_bf16x8(g + c8 * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf((float)x[e], (float)y[e], acc);
    }
  } else {
    const float* o = reinterpret_cast<const float*>(a.out) + idx * kD;
    const float* g = reinterpret_cast<const float*>(a.dout) + idx * kD;
#pragma unroll
    for (int c4 = 0; c4 < 16; ++c4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(o + c4 * 4);
      const f32x4 y = *reinterpret_cast<const f32x4*>(g + c4 * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(x[e], y[e], acc);
    }
  }
  const size_t li = ((size_t)b * a.Hq + h) * a.T + t;
  a.ndelta[li] = -acc;
  a.lse2[li] = a.lse[li] * kLog2e;
}

// ---------------------------------------------------------------------------
// 2. dq (per query tile), fp32
// ---------------------------------------------------------------------------
struct DqLdsF32 {
  float k[2][kStep * kRowF];
  float v[2][kStep * kRowF];
  int kid[2][kStep];
};

struct StageF32 {
  u32x4 r[8];
};

// K and V rows kb .. kb+63 of one KV head (zero past S) into registers.
__device__ __forceinline__ void dq_load_f32(const BwdArgs& a, int b, int kvh, int kb, StageF32& st) {
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

__device__ __forceinline__ void dq_store_f32(const BwdArgs& a, int b, int kb, const StageF32& st,
                                             DqLdsF32& lds, int buf) {
  const int tid = threadIdx.x;
  if (tid < kStep) lds.kid[buf][tid] = a.kid[(size_t)b * a.tk_pad + kb + tid];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i;
    const int key = u >> 4, ch = u & 15;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds.k[buf][key * kRowF + ch * 4 + e] = __uint_as_float(st.r[i][e]);
      lds.v[buf][key * kRowF + ch * 4 + e] = __uint_as_float(st.r[4 + i][e]);
    }
  }
}

template <int HPW>
__global__ __launch_bounds__(256) void bwd_dq_f32_kernel(BwdArgs a) {
  __shared__ DqLdsF32 lds;
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
  const bool qactive = qvalid && myqid != 0;
  int head[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) head[j] = kvh * a.G + hc * HPW + j;

  float qf[HPW][32], gf[HPW][32];
  float lse2[HPW], dlt[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const size_t row = (((size_t)b * a.T + qpos) * a.Hq + head[j]) * kD;
    const float* qs = reinterpret_cast<const float*>(a.q) + row + half;
    const float* gs = reinterpret_cast<const float*>(a.dout) + row + half;
#pragma unroll
    for (int st = 0; st < 32; ++st) {
      qf[j][st] = qvalid ? qs[2 * st] : 0.f;
      gf[j][st] = qvalid ? gs[2 * st] : 0.f;
    }
    const size_t li = ((size_t)b * a.Hq + head[j]) * a.T + qpos;
    lse2[j] = qactive ? a.lse[li] * kLog2e : kPosInf;
    dlt[j] = qvalid ? -a.ndelta[li] : 0.f;
  }

  f32x16 dqacc[HPW][2];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    dqacc[j][0] = zero16();
    dqacc[j][1] = zero16();
  }

  const int count = ld_const(a.qcnt, b * a.nq + qt);
  const int* list = a.qlist + ((size_t)b * a.nq + qt) * 2 * a.nk;
  const int nsteps = count;  // one 64-key stage per list entry
  const float c = a.scale_log2;

  StageF32 stage;
  if (nsteps > 0) {
    const int kb0 = (list[0] >> 2) * kStep;
    dq_load_f32(a, b, kvh, kb0, stage);
    dq_store_f32(a, b, kb0, stage, lds, 0);
  }
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const int entry = list[step];
    const int kb = (entry >> 2) * kStep;
    const bool partial = (entry & 3) == 1;
    int next_kb = 0;
    if (step + 1 < nsteps) {
      next_kb = (list[step + 1] >> 2) * kStep;
      dq_load_f32(a, b, kvh, next_kb, stage);
    }

#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      f32x16 s[HPW], dp[HPW];
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        s[j] = zero16();
        dp[j] = zero16();
      }
      const float* krow = &lds.k[buf][(kb2 * 32 + (lane & 31)) * kRowF + half];
      const float* vrow = &lds.v[buf][(kb2 * 32 + (lane & 31)) * kRowF + half];
#pragma unroll
      for (int st = 0; st < 32; ++st) {
        const float kf = krow[2 * st];
        const float vf = vrow[2 * st];
#pragma unroll
        for (int j = 0; j < HPW; ++j) {
          s[j] = mfma32x32x2(kf, qf[j][st], s[j]);
          dp[j] = mfma32x32x2(vf, gf[j][st], dp[j]);
        }
      }
      // P^T and dS^T in place of s
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bool ok[4] = {true, true, true, true};
        if (partial) {
          const int kk0 = kb2 * 32 + 8 * g4 + 4 * half;
          const int4 kids = *reinterpret_cast<const int4*>(&lds.kid[buf][kk0]);
          const int kv[4] = {kids.x, kids.y, kids.z, kids.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) ok[i] = kv[i] == myqid && (!a.causal || kb + kk0 + i <= qpos);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = g4 * 4 + i;
#pragma unroll
          for (int j = 0; j < HPW; ++j) {
            const float p = ok[i] ? fast_exp2(fmaf(s[j][r], c, -lse2[j])) : 0.f;
            s[j][r] = p * (dp[j][r] - dlt[j]);
          }
        }
      }
      // dQ^T += K^T dS^T
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float af = lds.k[buf][(kb2 * 32 + acc_row(r, lane)) * kRowF + db * 32 + (lane & 31)];
#pragma unroll
          for (int j = 0; j < HPW; ++j) dqacc[j][db] = mfma32x32x2(af, s[j][r], dqacc[j][db]);
        }
    }

    if (step + 1 < nsteps) dq_store_f32(a, b, next_kb, stage, lds, buf ^ 1);
    __syncthreads();
  }

  if (!qvalid) return;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = db * 32 + 8 * g4 + 4 * half;
        const size_t off = (((size_t)b * a.T + qpos) * a.Hq + head[j]) * kD + d0;
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = qactive ? dqacc[j][db][g4 * 4 + i] * a.scale : 0.f;
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.dq) + off) = o;
      }
  }
}

// ---------------------------------------------------------------------------
// 3. dk, dv (per key tile and KV head), fp32
// ---------------------------------------------------------------------------
struct KvLdsF32 {
  float q[2][kStep * kRowF];
  float g[2][kStep * kRowF];
  float lse2[2][kStep];
  float dlt[2][kStep];
  int qid[2][kStep];
};

struct KvStageF32 {
  u32x4 r[8];
  float lse2, dlt;
  int qid;
};

// Iteration `it` of a key tile's loop -> (64-query stage entry, head in group).
__device__ __forceinline__ void kv_iter(const BwdArgs& a, const int* list, int it, int& qb,
                                        int& head_in_group, int& cls) {
  const int entry = list[it / a.G];
  head_in_group = it % a.G;
  qb = (entry >> 2) * kStep;
  cls = entry & 3;
}

__device__ __forceinline__ void kv_load_f32(const BwdArgs& a, int b, int h, int qb, KvStageF32& st) {
  const int tid = threadIdx.x;
  const float* qs = reinterpret_cast<const float*>(a.q);
  const float* gs = reinterpret_cast<const float*>(a.dout);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i;
    const int qq = qb + (u >> 4), ch = u & 15;
    const size_t off = (((size_t)b * a.T + qq) * a.Hq + h) * kD + ch * 4;
    st.r[i] = qq < a.T ? ld_u32x4(qs + off) : u32x4{0, 0, 0, 0};
    st.r[4 + i] = qq < a.T ? ld_u32x4(gs + off) : u32x4{0, 0, 0, 0};
  }
  if (tid < kStep) {
    const int qq = qb + tid;
    const int id = a.qid[(size_t)b * a.tq_pad + qq];
    const bool act = qq < a.T && id != 0;
    const size_t li = ((size_t)b * a.Hq + h) * a.T + qq;
    st.qid = id;
    st.lse2 = act ? a.lse[li] * kLog2e : kPosInf;
    st.dlt = act ? -a.ndelta[li] : 0.f;
  }
}

__device__ __forceinline__ void kv_store_f32(const KvStageF32& st, KvLdsF32& lds, int buf) {
  const int tid = threadIdx.x;
  if (tid < kStep) {
    lds.qid[buf][tid] = st.qid;
    lds.lse2[buf][tid] = st.lse2;
    lds.dlt[buf][tid] = st.dlt;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i;
    const int qq = u >> 4, ch = u & 15;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds.q[buf][qq * kRowF + ch * 4 + e] = __uint_as_float(st.r[i][e]);
      lds.g[buf][qq * kRowF + ch * 4 + e] = __uint_as_float(st.r[4 + i][e]);
    }
  }
}

__global__ __launch_bounds__(256) void bwd_dkdv_f32_kernel(BwdArgs a) {
  __shared__ KvLdsF32 lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = lane >> 5;
  // 1-D grid: (key-tile item in launch order, kvh), heads fastest
  const int slot = uniform(fast_div(blockIdx.x, a.div_hkv));
  const int kvh = uniform(blockIdx.x - slot * a.Hkv);
  const int item = ld_const(a.korder, slot);  // (row, key tile), longest first
  const int b = uniform(fast_div(item, a.div_nk));
  const int kt = uniform(item - b * a.nk);
  const int kpos = kt * kTile + wave * 32 + (lane & 31);
  const int mykid = a.kid[(size_t)b * a.tk_pad + kpos];
  const bool kvalid = kpos < a.S;

  // K, V as B operands of S = Q K^T and dP = dO V^T
  float kf[32], vf[32];
  {
    const size_t row = (((size_t)b * a.S + kpos) * a.Hkv + kvh) * kD;
    const float* ks = reinterpret_cast<const float*>(a.k) + row + half;
    const float* vs = reinterpret_cast<const float*>(a.v) + row + half;
#pragma unroll
    for (int st = 0; st < 32; ++st) {
      kf[st] = kvalid ? ks[2 * st] : 0.f;
      vf[st] = kvalid ? vs[2 * st] : 0.f;
    }
  }

  f32x16 dkacc[2], dvacc[2];
  dkacc[0] = dkacc[1] = dvacc[0] = dvacc[1] = zero16();

  const int count = ld_const(a.kcnt, b * a.nk + kt);
  const int* list = a.klist + ((size_t)b * a.nk + kt) * 2 * a.nq;
  const int niters = count * a.G;  // (64-query stage, head) iterations
  const float c = a.scale_log2;

  KvStageF32 stage;
  if (niters > 0) {
    int qb, hg, cls;
    kv_iter(a, list, 0, qb, hg, cls);
    kv_load_f32(a, b, kvh * a.G + hg, qb, stage);
    kv_store_f32(stage, lds, 0);
  }
  __syncthreads();

  for (int it = 0; it < niters; ++it) {
    const int buf = it & 1;
    int qb, hg, cls;
    kv_iter(a, list, it, qb, hg, cls);
    const bool partial = cls == 1;
    if (it + 1 < niters) {
      int qb2, hg2, cls2;
      kv_iter(a, list, it + 1, qb2, hg2, cls2);
      kv_load_f32(a, b, kvh * a.G + hg2, qb2, stage);
    }

#pragma unroll
    for (int qb2 = 0; qb2 < 2; ++qb2) {
      f32x16 s = zero16(), dp = zero16();
      const float* qrow = &lds.q[buf][(qb2 * 32 + (lane & 31)) * kRowF + half];
      const float* grow = &lds.g[buf][(qb2 * 32 + (lane & 31)) * kRowF + half];
#pragma unroll
      for (int st = 0; st < 32; ++st) {
        s = mfma32x32x2(qrow[2 * st], kf[st], s);
        dp = mfma32x32x2(grow[2 * st], vf[st], dp);
      }
      // rows of s/dp are queries qq = qb2*32 + acc_row(r, lane); column = my key
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int qq0 = qb2 * 32 + 8 * g4 + 4 * half;
        const float4 l4 = *reinterpret_cast<const float4*>(&lds.lse2[buf][qq0]);
        const float4 d4 = *reinterpret_cast<const float4*>(&lds.dlt[buf][qq0]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
        bool ok[4] = {true, true, true, true};
        if (partial) {
          const int4 ids = *reinterpret_cast<const int4*>(&lds.qid[buf][qq0]);
          const int iv[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) ok[i] = iv[i] == mykid && (!a.causal || kpos <= qb + qq0 + i);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = g4 * 4 + i;
          const float p = ok[i] ? fast_exp2(fmaf(s[r], c, -lv[i])) : 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - dv4[i]);
        }
      }
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qq = qb2 * 32 + acc_row(r, lane);
          dvacc[db] = mfma32x32x2(lds.g[buf][qq * kRowF + db * 32 + (lane & 31)], s[r], dvacc[db]);
          dkacc[db] = mfma32x32x2(lds.q[buf][qq * kRowF + db * 32 + (lane & 31)], dp[r], dkacc[db]);
        }
    }

    if (it + 1 < niters) kv_store_f32(stage, lds, buf ^ 1);
    __syncthreads();
  }

  if (!kvalid) return;
  const bool kactive = mykid != 0;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = db * 32 + 8 * g4 + 4 * half;
      const size_t off = (((size_t)b * a.S + kpos) * a.Hkv + kvh) * kD + d0;
      f32x4 ok, ov;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok[i] = kactive ? dkacc[db][g4 * 4 + i] * a.scale : 0.f;
        ov[i] = kactive ? dvacc[db][g4 * 4 + i] : 0.f;
      }
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.dk) + off) = ok;
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.dv) + off) = ov;
    }
}

// ---------------------------------------------------------------------------
// bf16 dq: the structure of the bf16 forward (one head per wave, 4*HPW
// waves, K/V tiles DMA'd into a two-slot LDS ring of 128-key slots).
// dQ^T += K^T dS^T takes its K^T operand from the K tile through
// transposing LDS reads.
// ---------------------------------------------------------------------------
template <int HPW>
__global__ __launch_bounds__(256 * HPW) __attribute__((amdgpu_waves_per_eu(2 * HPW)))
void bwd_dq_bf16_kernel(BwdArgs a) {
  constexpr int W = 4 * HPW;
  // two ring slots of 128 keys, each two 64-key stages
  __shared__ __attribute__((aligned(16))) char slotA[2 * kStageBytes], slotB[2 * kStageBytes];
  const int lane = threadIdx.x & 63;
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
  const bool qvalid = qpos < a.T;
  const bool qactive = qvalid && myqid != 0;

  bf16x8 qf[4], gf[4];  // query and output-gradient fragments (loaded below)
  float lse2 = 0.f, dlt = 0.f;
  uint64_t ndlt2 = 0;  // (-D, -D) of the lane's row, the start of each dP^T block
  f32x16 dqacc[2] = {zero16(), zero16()};
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

  // (the precomputed-offset form of kv_dma measured 2-5% slower here while
  // its offsets made dq spill; without spills, at 128 VGPRs, it measures
  // within 0.6%)
  auto issue = [&](int entry, char* stage) {
    kv_dma<W>(kg, vg, row_stride, a.S, kid_row, (entry >> 2) * kKvStep, wave, stage);
  };

  // Sub-block classification inside PARTIAL tiles, as in the forward: a
  // wave's 32 queries against one 32-key block are skipped when no pair can
  // be valid and run without id masks when every id matches.
  const int q0 = qt * kTile + (wave & 3) * 32;
  const int u = uniform(myqid);
  const bool quni = __all(myqid == u);

  auto block = [&](const char* kt, const char* vt, const int* kids_lds, int kb, int kb2,
                   bool mask_ids, bool diag) {
    f32x16 s = zero16();
    f32x16 dp;
    {
      // dP^T starts from -D (per lane: one query row), so the MFMA chain
      // yields dP - D and the 16 subtractions per block go: eight 64-bit
      // moves of the lane's (-D, -D) pair, in asm because the compiler either
      // hoists a sixteen-register splat out of the loop (spilling at 128
      // VGPRs) or emits sixteen 32-bit moves.  s_nop 1 gives the two wait
      // states between a VALU write and an MFMA reading it as SrcC.  The
      // registers written are the block's dP accumulators, which no MFMA in
      // flight reads as SrcC (the previous block's dP chain finished before
      // its probabilities were formed).
      uint64_t p0, p1, p2, p3, p4, p5, p6, p7;
      asm volatile(
          "v_mov_b64 %0, %8\n\tv_mov_b64 %1, %8\n\tv_mov_b64 %2, %8\n\tv_mov_b64 %3, %8\n\t"
          "v_mov_b64 %4, %8\n\tv_mov_b64 %5, %8\n\tv_mov_b64 %6, %8\n\tv_mov_b64 %7, %8\n\t"
          "s_nop 1"
          : "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3), "=&v"(p4), "=&v"(p5), "=&v"(p6),
            "=&v"(p7)
          : "v"(ndlt2));
      typedef uint64_t u64x8 __attribute__((ext_vector_type(8)));
      dp = __builtin_bit_cast(f32x16, (u64x8){p0, p1, p2, p3, p4, p5, p6, p7});
    }
    const int krow = kb2 * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s = mfma32x32x16(tile_chunk(kt, krow, 2 * ks + half), qf[ks], s);
      dp = mfma32x32x16(tile_chunk(vt, krow, 2 * ks + half), gf[ks], dp);
    }
    if (mask_ids) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int4 kids = *reinterpret_cast<const int4*>(&kids_lds[kb2 * 32 + 8 * g4 + 4 * half]);
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
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], c, -lse2)) * dp[r];
    const bf16x8 ds0 = pack8(s, 0), ds1 = pack8(s, 8);
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const bf16x8 k0 = tile_tr_operand(kt, kb2 * 32 + tr_row, db * 32 + tr_col);
      const bf16x8 k1 = tile_tr_operand(kt, kb2 * 32 + 16 + tr_row, db * 32 + tr_col);
      dqacc[db] = mfma32x32x16(k0, ds0, dqacc[db]);
      dqacc[db] = mfma32x32x16(k1, ds1, dqacc[db]);
    }
  };

  auto compute = [&](int entry, const char* stage) {
    const int kb = (entry >> 2) * kKvStep;
    const bool partial = (entry & 3) == 1;
    const char* kt = stage;
    const char* vt = stage + kTileBytes;
    const int* kids_lds = reinterpret_cast<const int*>(stage + 2 * kTileBytes);
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      bool run = true, mask_ids = false, diag = false;
      if (partial) {
        const int k0 = kb + kb2 * 32;
        const bool above = a.causal && k0 > q0 + 31;
        diag = a.causal && k0 + 31 > q0;
        if (quni) {
          const uint64_t m = __ballot(kids_lds[kb2 * 32 + (lane & 31)] == u);
          run = !above && u != 0 && m != 0;
          mask_ids = m != ~0ull;
        } else {
          run = !above;
          mask_ids = true;
        }
      }
      if (run) block(kt, vt, kids_lds, kb, kb2, mask_ids, diag);
    }
  };

  // Ring of two 128-key slots (as in the forward): slot i+1's DMAs are issued
  // right after the barrier that opens slot i; whole pairs of slots, with the
  // computes past the end skipped.
  auto issue_slot = [&](int i, int e0, int e1, char* slot) {
    if (2 * i < nsteps) issue(e0, slot);
    if (2 * i + 1 < nsteps) issue(e1, slot + kStageBytes);
  };
  const int nslots = (nsteps + 1) >> 1;
  // Both slots and the query-side rows (q, dO, lse, O for D) are in flight
  // together before the first wait; after that slot i+1's DMAs are issued
  // when slot i opens.  The list entries a pair of slots needs (steps
  // 2i .. 2i+5) arrive in one scalar load of eight; the read may run up to 7
  // entries past the list's end, into the plan's next section (query lists
  // are followed by the key-tile counts), and entries at or past nsteps are
  // never used.
  {
    const i32x8u e = ld_const8(list, 0);
    issue_slot(0, e[0], e[1], slotA);
    issue_slot(1, e[2], e[3], slotB);
  }
  {
    const size_t row = (((size_t)b * a.T + min(qpos, a.T - 1)) * a.Hq + head) * kD + 8 * half;
    const bf16* qs = reinterpret_cast<const bf16*>(a.q) + row;
    const bf16* gs = reinterpret_cast<const bf16*>(a.dout) + row;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = ld_bf16x8(qs + ks * 16);
      gf[ks] = ld_bf16x8(gs + ks * 16);
    }
  }
  const size_t li = ((size_t)b * a.Hq + head) * a.T + min(qpos, a.T - 1);
  const float lse_raw = a.lse[li];
  float dlt_raw;
  if (a.fuse_delta) {
    // D = rowsum(dO * O): this lane holds half of the row's 64 dims
    const bf16* os = reinterpret_cast<const bf16*>(a.out) +
                     (((size_t)b * a.T + min(qpos, a.T - 1)) * a.Hq + head) * kD + 8 * half;
    float part = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 ow = ld_u32x4(os + ks * 16);
      const u32x4 gw = __builtin_bit_cast(u32x4, gf[ks]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // through scalars: __builtin_bit_cast of a vector element reads
        // element 0 whatever the index (clang 22)
        const uint32_t oj = ow[j], gj = gw[j];
        part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, oj),
                                               __builtin_bit_cast(bf16x2, gj), part, false);
      }
    }
    dlt_raw = halves_sum(part);
  } else {
    dlt_raw = -a.ndelta[li];
  }
  drain_memory();
  lse2 = qactive ? lse_raw * kLog2e : kPosInf;
  dlt = qactive ? dlt_raw : 0.f;
  {
    const uint32_t nd = __builtin_bit_cast(uint32_t, -dlt);
    ndlt2 = ((uint64_t)nd << 32) | nd;
  }
  // (a slot past the end is skipped whole, as in the forward)
  for (int i = 0; i < nslots; i += 2) {
    const i32x8u e = ld_const8(list, 2 * i);
    wait_vmcnt<0>();
    barrier();
    if (i > 0) issue_slot(i + 1, e[2], e[3], slotB);
    compute(e[0], slotA);
    if (2 * i + 1 < nsteps) compute(e[1], slotA + kStageBytes);
    if (i + 1 < nslots) {
      wait_vmcnt<0>();
      barrier();
      issue_slot(i + 2, e[4], e[5], slotA);
      compute(e[2], slotB);
      if (2 * i + 3 < nsteps) compute(e[3], slotB + kStageBytes);
    }
  }
  wait_vmcnt<0>();

  // the lane's query position and half again from a fresh lane id
  // (cheaper than keeping them across the loop)
  const int elane = fresh_lane_id();
  const int ehalf = elane >> 5;
  const int eqpos = qt * kTile + (wave & 3) * 32 + (elane & 31);
  if (eqpos >= a.T) return;
  // -D and lse * log2(e) for the dk/dv kernel, stored after the loop rather
  // than before it (a store in flight would hold up the first stage's wait).
  // The values the loop used: an inactive row's are 0 and +inf, which dk/dv
  // never combines with a non-zero probability.
  if (a.fuse_delta && ehalf == 0) {
    const size_t lj = ((size_t)b * a.Hq + head) * a.T + eqpos;
    a.ndelta[lj] = -dlt;
    a.lse2[lj] = lse2;
  }
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = db * 32 + 8 * g4 + 4 * ehalf;
      const bf16x4 o = scaled_bf16x4(dqacc[db], g4 * 4, a.scale, qactive);
      *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(a.dq) +
                                 (((size_t)b * a.T + eqpos) * a.Hq + head) * kD + d0) = o;
    }
}

// ---------------------------------------------------------------------------
// bf16 dk/dv: 4 waves per workgroup for one 128-key tile of one KV head; each
// wave owns 32 keys (K, V as B operands in registers) and walks the GQA
// group's query heads in turn, summing their dK/dV in the same accumulators.
// Q, dO, lse, D and the query ids are DMA'd into a three-stage LDS ring of
// 64-query stages, two steps ahead of use; dV^T += dO^T P and dK^T += Q^T dS
// read their transposed operands from the Q / dO tiles.  Each 32-query block
// runs its scores, VALU and accumulation before the next block starts: that
// keeps the kernel within 168 VGPRs and 51 KB of LDS, i.e. three workgroups
// (12 waves) per CU, which measured 10% faster at C2 and C3 than two
// workgroups with both blocks' scores issued first and the two-slot ring of
// the forward.
// ---------------------------------------------------------------------------
struct QDma {
  static constexpr int W = 4;
  static constexpr int kTiles = 2;                           // Q, dO
  static constexpr int kGroupsPerWave = kTiles * 8 / W;      // 8-row groups
  static constexpr int kWordArrays = 3;                      // lse, D, ids
  // stage layout: tiles [Q, dO], then lse[64], D[64], ids[64]
  static constexpr int kLseOff = kTiles * kTileBytes;
  static constexpr int kDltOff = kLseOff + 256;
  static constexpr int kIdOff = kDltOff + 256;
  static constexpr int kStageBytes = kIdOff + 256;
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void bwd_dkdv_bf16_kernel(BwdArgs a) {
  using Q = QDma;
  constexpr int W = Q::W;
  __shared__ __attribute__((aligned(16))) char stage0[Q::kStageBytes], stage1[Q::kStageBytes],
      stage2[Q::kStageBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int half = lane >> 5;
  // 1-D grid: (key-tile item in launch order, kvh), heads fastest
  const int slot = uniform(fast_div(blockIdx.x, a.div_hkv));
  const int kvh = uniform(blockIdx.x - slot * a.Hkv);
  const int item = ld_const(a.korder, slot);  // (row, key tile), longest first
  const int b = uniform(fast_div(item, a.div_nk));
  const int kt = uniform(item - b * a.nk);
  const int kpos = kt * kTile + (wave & 3) * 32 + (lane & 31);
  const int mykid = a.kid[(size_t)b * a.tk_pad + kpos];
  const bool kvalid = kpos < a.S;

  bf16x8 kf[4], vf[4];
  {
    const size_t row = (((size_t)b * a.S + min(kpos, a.S - 1)) * a.Hkv + kvh) * kD + 8 * half;
    const bf16* ks = reinterpret_cast<const bf16*>(a.k) + row;
    const bf16* vs = reinterpret_cast<const bf16*>(a.v) + row;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kf[i] = ld_bf16x8(ks + i * 16);
      vf[i] = ld_bf16x8(vs + i * 16);
    }
  }
  drain_memory();
  f32x16 dkacc[2] = {zero16(), zero16()}, dvacc[2] = {zero16(), zero16()};

  const int count = ld_const(a.kcnt, b * a.nk + kt);
  const int* list = a.klist + ((size_t)b * a.nk + kt) * 2 * a.nq;
  const int hps = a.G;             // heads of the group, walked in turn
  const int niters = count * hps;  // (64-query stage, head) iterations
  const float c = a.scale_log2;
  const uint32_t qrow_stride = (uint32_t)a.Hq * kD * sizeof(bf16);

  const char* const qbase = reinterpret_cast<const char*>(a.q);
  const char* const gbase = reinterpret_cast<const char*>(a.dout);
  // DMA of iteration `it` (query rows qb .. qb+63 of one head) into a stage.
  auto issue = [&](int it, char* stage) {
    it = min(it, niters - 1);
    const int si = fast_div(it, a.div_g);  // hps == G
    const int entry = ld_const(list, si);
    const int hj = it - si * hps;
    const int qb = (entry >> 2) * kKvStep;
    // the word arrays first, so the short step wait covers them
    if (wave < Q::kWordArrays) {
      // rows past T re-read row T-1 (finite values); their ids are 0, so
      // every pair they form is masked or belongs to a zeroed inactive key
      const size_t row = ((size_t)b * a.Hq + kvh * a.G + hj) * a.T;
      const void* sbase = wave == 2 ? (const void*)(a.qid + (size_t)b * a.tq_pad + qb)
                          : (wave & 1) ? (const void*)(a.ndelta + row)
                                       : (const void*)(a.lse2 + row);
      const uint32_t voff = 4u * (wave == 2 ? lane : min(qb + lane, a.T - 1));
      char* dst = wave == 2 ? stage + Q::kIdOff
                  : (wave & 1) ? stage + Q::kDltOff
                               : stage + Q::kLseOff;
      dma_word64(sbase, voff, dst);
    }
#pragma unroll
    for (int j = 0; j < Q::kGroupsPerWave; ++j) {
      // 8-row group wave + W j: its tile (W j) / 8 is a compile-time
      // constant, so the Q / dO choice is a register select rather than a
      // reload of the argument
      const int tile = (W * j) >> 3, r0 = 8 * ((wave + W * j) & 7);
      const int h = kvh * a.G + hj;
      const char* base = ((tile & 1) ? gbase : qbase) + ((size_t)b * a.T * a.Hq + h) * kD * sizeof(bf16);
      dma_rows8(base, qrow_stride, qb, r0, a.T - 1, stage + tile * kTileBytes);
    }
  };

  // Sub-block classification inside PARTIAL tiles (mirror of the forward's,
  // with the roles of queries and keys swapped): the wave's 32 keys against
  // one 32-query block are skipped when no pair can be valid and run without
  // id masks when every id matches.
  const int k0 = kt * kTile + (wave & 3) * 32;
  const int uk = uniform(mykid);
  const bool kuni = __all(mykid == uk);

  // One 32-query block in three parts: S = Q K^T and dP - D = dO V^T - D
  // (MFMA, the accumulator starting from the stage's -D), P and dS (VALU),
  // dV^T += dO^T P and dK^T += Q^T dS (MFMA).
  auto scores = [&](const char* qt, const char* gt, const float* ndlt_l, int qb2, f32x16& s,
                    f32x16& dp) {
    s = zero16();
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const float4 d4 = *reinterpret_cast<const float4*>(&ndlt_l[qb2 * 32 + 8 * g4 + 4 * half]);
      dp[g4 * 4 + 0] = d4.x;
      dp[g4 * 4 + 1] = d4.y;
      dp[g4 * 4 + 2] = d4.z;
      dp[g4 * 4 + 3] = d4.w;
    }
    const int qrow = qb2 * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s = mfma32x32x16(tile_chunk(qt, qrow, 2 * ks + half), kf[ks], s);
      dp = mfma32x32x16(tile_chunk(gt, qrow, 2 * ks + half), vf[ks], dp);
    }
  };
  auto probs = [&](f32x16& s, f32x16& dp, const float* lse_l, const int* qid_l, int qb, int qb2,
                   bool mask_ids, bool diag,
                   bf16x8 (&pf)[2], bf16x8 (&sf)[2]) {
    if (mask_ids) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int4 ids = *reinterpret_cast<const int4*>(&qid_l[qb2 * 32 + 8 * g4 + 4 * half]);
        const int iv[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) s[g4 * 4 + i] = iv[i] == mykid ? s[g4 * 4 + i] : kNegInf;
      }
    }
    if (diag) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        s[r] = kpos <= qb + qb2 * 32 + acc_row(r, lane) ? s[r] : kNegInf;
    }
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const float4 l4 = *reinterpret_cast<const float4*>(&lse_l[qb2 * 32 + 8 * g4 + 4 * half]);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = g4 * 4 + i;
        // lse_l holds lse * log2(e); masked scores are -inf and inactive
        // rows have lse = +inf: p = 0
        const float p = fast_exp2(fmaf(s[r], c, -lv[i]));
        s[r] = p;
        dp[r] *= p;
      }
    }
    pf[0] = pack8(s, 0);
    pf[1] = pack8(s, 8);
    sf[0] = pack8(dp, 0);
    sf[1] = pack8(dp, 8);
  };
  auto accumulate = [&](const char* qt, const char* gt, int qb2, const bf16x8 (&pf)[2],
                        const bf16x8 (&sf)[2]) {
    const int r0 = qb2 * 32 + tr_row_of(lane);
    const int cb = tr_col_of(lane);
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const bf16x8 g0 = tile_tr_operand(gt, r0, db * 32 + cb);
      const bf16x8 g1 = tile_tr_operand(gt, r0 + 16, db * 32 + cb);
      dvacc[db] = mfma32x32x16(g0, pf[0], dvacc[db]);
      dvacc[db] = mfma32x32x16(g1, pf[1], dvacc[db]);
      const bf16x8 q0 = tile_tr_operand(qt, r0, db * 32 + cb);
      const bf16x8 q1 = tile_tr_operand(qt, r0 + 16, db * 32 + cb);
      dkacc[db] = mfma32x32x16(q0, sf[0], dkacc[db]);
      dkacc[db] = mfma32x32x16(q1, sf[1], dkacc[db]);
    }
  };

  auto compute = [&](int it, const char* stage) {
    const int entry = ld_const(list, fast_div(it, a.div_g));
    const int qb = (entry >> 2) * kKvStep;
    const bool partial = (entry & 3) == 1;
    const char* qt = stage;
    const char* gt = stage + kTileBytes;
    const float* lse_l = reinterpret_cast<const float*>(stage + Q::kLseOff);
    const float* ndlt_l = reinterpret_cast<const float*>(stage + Q::kDltOff);
    const int* qid_l = reinterpret_cast<const int*>(stage + Q::kIdOff);
    bool run[2] = {true, true}, mask_ids[2] = {false, false}, diag[2] = {false, false};
    if (partial) {
#pragma unroll
      for (int qb2 = 0; qb2 < 2; ++qb2) {
        const int q0 = qb + qb2 * 32;
        const bool above = a.causal && k0 > q0 + 31;
        diag[qb2] = a.causal && k0 + 31 > q0;
        if (kuni) {
          const uint64_t m = __ballot(qid_l[qb2 * 32 + (lane & 31)] == uk);
          run[qb2] = !above && uk != 0 && m != 0;
          mask_ids[qb2] = m != ~0ull;
        } else {
          run[qb2] = !above;
          mask_ids[qb2] = true;
        }
      }
    }
    f32x16 s0, dp0, s1, dp1;
    bf16x8 pf[2], sf[2];
    if (run[0]) {
      scores(qt, gt, ndlt_l, 0, s0, dp0);
      probs(s0, dp0, lse_l, qid_l, qb, 0, mask_ids[0], diag[0], pf, sf);
      accumulate(qt, gt, 0, pf, sf);
    }
    if (run[1]) {
      scores(qt, gt, ndlt_l, 1, s1, dp1);
      probs(s1, dp1, lse_l, qid_l, qb, 1, mask_ids[1], diag[1], pf, sf);
      accumulate(qt, gt, 1, pf, sf);
    }
  };

  // Whole groups of three steps; the computes past the end are skipped
  // rather than leaving the loop mid-group (a mid-group exit gives the
  // accumulators three exit paths, resolved with 64-register copies).  Waves
  // below kWordArrays issue one more DMA per step than the others; the step
  // wait uses the tile count, which for them also covers the oldest DMA of
  // the stage issued one step earlier.  (Skipping the steps past the end
  // whole -- their waits, barriers and clamped re-issues of the last stage --
  // measured 1.7-2.2% slower at C2 and within 1% at C3 and C5.)
  constexpr int G = Q::kGroupsPerWave;
  if (niters > 0) {
    issue(0, stage0);
    issue(1, stage1);
  }
  for (int it = 0; it < niters; it += 3) {
    wait_vmcnt<G>();
    barrier();
    issue(it + 2, stage2);
    compute(it, stage0);
    wait_vmcnt<G>();
    barrier();
    issue(it + 3, stage0);
    if (it + 1 < niters) compute(it + 1, stage1);
    wait_vmcnt<G>();
    barrier();
    issue(it + 4, stage1);
    if (it + 2 < niters) compute(it + 2, stage2);
  }
  wait_vmcnt<0>();

  if (!kvalid) return;
  const bool kactive = mykid != 0;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = db * 32 + 8 * g4 + 4 * half;
      const size_t off = (((size_t)b * a.S + kpos) * a.Hkv + kvh) * kD + d0;
      const bf16x4 ok = scaled_bf16x4(dkacc[db], g4 * 4, a.scale, kactive);
      const bf16x4 ov = scaled_bf16x4(dvacc[db], g4 * 4, 1.f, kactive);
      *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(a.dk) + off) = ok;
      *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(a.dv) + off) = ov;
    }
}

hipError_t launch_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                           const void* dout, const float* lse, bool f32, int batch, int T, int S,
                           int Hq, int Hkv, int mode, float scale, const void* plan, void* dq,
                           void* dk, void* dv, float* workspace, int phases, hipStream_t stream) {
  BwdArgs a;
  const PlanLayout lay = plan_layout(batch, T, S);
  const char* p = reinterpret_cast<const char*>(plan);
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.dout = dout;
  a.lse = lse;
  a.ndelta = workspace;
  a.lse2 = workspace + (size_t)batch * Hq * T;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.qid = reinterpret_cast<const int*>(p + lay.qid);
  a.kid = reinterpret_cast<const int*>(p + lay.kid);
  a.qcnt = reinterpret_cast<const int*>(p + lay.qcnt);
  a.qlist = reinterpret_cast<const int*>(p + lay.qlist);
  a.kcnt = reinterpret_cast<const int*>(p + lay.kcnt);
  a.klist = reinterpret_cast<const int*>(p + lay.klist);
  a.qorder = reinterpret_cast<const int*>(p + lay.qorder);
  a.korder = reinterpret_cast<const int*>(p + lay.korder);
  a.T = T;
  a.S = S;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  const int hpw = (a.G % 2 == 0) ? 2 : 1;
  a.hchunks = a.G / hpw;
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
  a.div_hkv = make_fastdiv(a.Hkv);
  a.div_nk = make_fastdiv(a.nk);
  a.div_g = make_fastdiv(a.G);
  const size_t rows = (size_t)batch * T * Hq;
  const unsigned dgrid = (unsigned)((rows + 255) / 256);
  // bf16 with both the delta and the dq phase: the dq kernel, which holds
  // the dO rows of its queries in registers anyway, also loads O and writes
  // D; the separate delta pass (a full read of O and dO) is skipped
  a.fuse_delta = !f32 && (phases & 3) == 3;
  if ((phases & 1) && !a.fuse_delta) {
    if (f32)
      hipLaunchKernelGGL((bwd_delta_kernel<true>), dim3(dgrid), dim3(256), 0, stream, a, batch);
    else
      hipLaunchKernelGGL((bwd_delta_kernel<false>), dim3(dgrid), dim3(256), 0, stream, a, batch);
  }
  const dim3 qgrid(Hkv * a.hchunks * batch * lay.nq);
  if (!(phases & 2)) {
  } else if (f32) {
    if (hpw == 2)
      hipLaunchKernelGGL((bwd_dq_f32_kernel<2>), qgrid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((bwd_dq_f32_kernel<1>), qgrid, dim3(256), 0, stream, a);
  } else {
    if (hpw == 2)
      hipLaunchKernelGGL((bwd_dq_bf16_kernel<2>), qgrid, dim3(512), 0, stream, a);
    else
      hipLaunchKernelGGL((bwd_dq_bf16_kernel<1>), qgrid, dim3(256), 0, stream, a);
  }
  const dim3 kgrid(Hkv * batch * lay.nk);
  if (phases & 4) {
    // 4-wave workgroups, one head at a time: measured 11-32% faster at
    // C2/C3/C5 than 8-wave workgroups whose halves took different heads and
    // summed through LDS, because the workgroups of a CU share no barriers.
    if (f32)
      hipLaunchKernelGGL(bwd_dkdv_f32_kernel, kgrid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(bwd_dkdv_bf16_kernel, kgrid, dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace mf
