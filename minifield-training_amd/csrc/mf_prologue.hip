// Attention prologue on gfx950: per-head RMS normalisation of q and k with
// per-dimension gains, then rotary position embeddings, in one pass over q
// and k (the reference runs rms_norm twice and apply_rotary twice, each a
// full read and write of the tensor).
//
// Semantics (reference: src/minifield_training/layers/attention.py:62-97,
// kernels/normalization.py:7-22, kernels/rotary.py:7-39):
//   n   = dtype(f32(x) * rsqrt(mean(f32(x)^2) + eps)) * dtype(gain)
//   out = n * dtype(cos(a)) + rotate_half(n) * dtype(sin(a)),
//   a_i = f32(position) * f32(theta^(-2i/D)),  rotate_half(n) = (-n[D/2:], n[:D/2])
// with the frequencies computed on the host (single precision, as the
// reference).  In bf16 every operation rounds to bf16 as the reference's
// declared dtypes do (its tests pin them with xla_allow_excess_precision
// off): the normalised value, its product with the gain, cos and sin, the
// two rotation products and their sum.
//
// Layout: one wave per token.  Lane (g = lane / 8, dl = lane % 8) owns dims
// 8 dl .. 8 dl + 7 of head g of a group of 8 heads, so a 16-byte (bf16) or
// two 16-byte (fp32) loads per lane move 8 whole head rows, the sum of
// squares reduces over 8 lanes with DPP, and the rotation partner (dims
// +- 32) is lane dl ^ 4 of the same head.  Lanes j and j + 32 evaluate the
// token's angle j; the lanes read their dims' cos/sin by shuffle.
#include <algorithm>
#include <type_traits>

#include "mf_common.h"

namespace mf {

struct RopeArgs {
  const void* q;
  const void* k;
  const void* q_gain;
  const void* k_gain;
  const int32_t* positions;  // [B, T] or null (0 .. T-1 on every row)
  void* q_out;
  void* k_out;
  int B, T, Hq, Hkv;
  float eps;
  float freq[kD / 2];
};

__device__ __forceinline__ float dpp_xor_sum8(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
  return x;
}

// ---------------------------------------------------------------------------
// Rows as loaded: one 8-head group of a token (16 bytes per lane in bf16, 32
// in fp32), kept raw until the group is computed, so that every load of a
// token is in flight before the first use.
// ---------------------------------------------------------------------------
template <bool F32> struct RopeRow;
template <> struct RopeRow<false> { bf16x8 v; };
template <> struct RopeRow<true> { f32x4 a, b; };

template <bool F32>
__device__ __forceinline__ RopeRow<F32> load_rope_row(const void* src, size_t base) {
  RopeRow<F32> r;
  if constexpr (F32) {
    const float* p = reinterpret_cast<const float*>(src) + base;
    r.a = *reinterpret_cast<const f32x4*>(p);
    r.b = *reinterpret_cast<const f32x4*>(p + 4);
  } else {
    r.v = ld_bf16x8(reinterpret_cast<const bf16*>(src) + base);
  }
  return r;
}

template <bool F32>
__device__ __forceinline__ void rope_row_floats(const RopeRow<F32>& r, float (&x)[8]) {
  if constexpr (F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = r.a[i], x[4 + i] = r.b[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (float)r.v[i];
  }
}

// The gains (cast to the tensor dtype) of the lane's 8 dims.
template <bool F32>
__device__ __forceinline__ void load_gains(const void* gain, int dl, float (&w)[8]) {
  typedef typename std::conditional<F32, float, bf16>::type T;
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = (float)reinterpret_cast<const T*>(gain)[8 * dl + i];
}

// The token's position as a float: positions[tok], or its index in the row
// when there are no positions.
__device__ __forceinline__ float token_position(const int32_t* positions, size_t tok, int T) {
  return (float)(positions ? positions[tok] : (int)(tok % T));
}

// cos and sin of the token's angles for the lane's dims 8 dl .. 8 dl + 7.
// `freq` is the lane's freq[lane mod 32], so lanes j and j + 32 evaluate
// angle j = f32(position) * freq[j]; each lane reads its dims' angles
// (d mod 32) by shuffle.  The fused forward's rope table evaluates the same
// sincosf of the same product.
template <bool F32>
__device__ __forceinline__ void token_cos_sin(float pos, float freq, int dl, float (&c)[8],
                                              float (&s)[8]) {
  float sv, cv;
  sincosf(pos * freq, &sv, &cv);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = __shfl(cv, (8 * dl + i) & 31);
    s[i] = __shfl(sv, (8 * dl + i) & 31);
    if constexpr (!F32) {
      c[i] = round_bf16(c[i]);
      s[i] = round_bf16(s[i]);
    }
  }
}

// Norm and rotation of one loaded group: lane (g, dl) holds dims 8 dl ..
// 8 dl + 7 of head g.  Every lane takes part (the 8-lane sum and the
// rotation shuffle); only live lanes store.
template <bool F32>
__device__ __forceinline__ void norm_rope_store(const RopeRow<F32>& xin, void* dst, size_t base,
                                                bool live, const float (&w)[8],
                                                const float (&c)[8], const float (&s)[8], int dl,
                                                float eps) {
  float x[8];
  rope_row_floats<F32>(xin, x);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rsqrtf(dpp_xor_sum8(ss) * (1.f / kD) + eps);
  float n[8], r[8];
  if constexpr (F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = x[i] * inv * w[i];
  } else {
    // the normalised value, then its product with the gain, each rounded to
    // bf16; two elements per conversion
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const uint32_t y = round_bf16_pair(x[i] * inv, x[i + 1] * inv);
      const uint32_t z = round_bf16_pair(bf16_lo(y) * w[i], bf16_hi(y) * w[i + 1]);
      n[i] = bf16_lo(z);
      n[i + 1] = bf16_hi(z);
    }
  }
  // rotate_half: dims d < 32 take -n[d + 32], dims d >= 32 take n[d - 32]
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float o = __shfl_xor(n[i], 4);
    r[i] = dl < 4 ? -o : o;
  }
  if (!live) return;
  if constexpr (F32) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = fmaf(n[i], c[i], r[i] * s[i]);
      b[i] = fmaf(n[4 + i], c[4 + i], r[4 + i] * s[4 + i]);
    }
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(dst) + base) = a;
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(dst) + base + 4) = b;
  } else {
    // the two rotation products rounded to bf16 by one conversion and added
    // by one dot product with (1, 1) (exact products, one fp32 rounding)
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t pq = round_bf16_pair(n[i] * c[i], r[i] * s[i]);
      o[i] = (bf16)__builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pq), ones, 0.f, false);
    }
    *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(dst) + base) = o;
  }
}

// 8-head groups of one token (q groups first, then k) loaded per batch
// before any of them is computed.
constexpr int kRopeFwdBatch = 4;

// One wave per token, no LDS and no barrier: the token's row loads (all of
// them when the q and k heads fill at most four groups) are issued first,
// the angles are evaluated while they are in flight, then each group is
// normalised, rotated and stored.
template <bool F32>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 3, dl = lane & 7;
  const size_t tok = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // b * T + t
  if (tok >= (size_t)a.B * a.T) return;
  const int gq = (a.Hq + 7) >> 3;  // Hq == 0: the key half only (no query operands)
  const int groups = gq + ((a.Hkv + 7) >> 3);
  auto locate = [&](int i, const void*& src, void*& dst, size_t& base, bool& live) {
    const bool isq = i < gq;
    const int H = isq ? a.Hq : a.Hkv;
    const int h = 8 * (isq ? i : i - gq) + g;
    live = h < H;
    base = (tok * H + min(h, H - 1)) * kD + 8 * dl;
    src = isq ? a.q : a.k;
    dst = isq ? a.q_out : a.k_out;
  };
  // the small operands first (position, the lane's frequency, the gains):
  // loads complete in issue order, so anything loaded after the rows could
  // only be read once every row had arrived
  const float pos = token_position(a.positions, tok, a.T);
  const float fq = a.freq[lane & 31];
  const RopeRow<F32> gq_raw = load_rope_row<F32>(gq > 0 ? a.q_gain : a.k_gain, 8 * dl);
  const RopeRow<F32> gk_raw = load_rope_row<F32>(a.k_gain, 8 * dl);
  RopeRow<F32> x[kRopeFwdBatch];
  auto load_batch = [&](int i0) {
#pragma unroll
    for (int j = 0; j < kRopeFwdBatch; ++j) {
      if (i0 + j < groups) {
        const void* src;
        void* dst;
        size_t base;
        bool live;
        locate(i0 + j, src, dst, base, live);
        x[j] = load_rope_row<F32>(src, base);
      }
    }
  };
  float wq[8], wk[8], c[8], s[8];
  auto store_batch = [&](int i0) {
#pragma unroll
    for (int j = 0; j < kRopeFwdBatch; ++j) {
      if (i0 + j < groups) {
        const void* src;
        void* dst;
        size_t base;
        bool live;
        locate(i0 + j, src, dst, base, live);
        norm_rope_store<F32>(x[j], dst, base, live, i0 + j < gq ? wq : wk, c, s, dl, a.eps);
      }
    }
  };
  load_batch(0);
  // the angles and gains only after the first rows are in flight (they would
  // otherwise be hoisted above them as loop invariants)
  __builtin_amdgcn_sched_barrier(0);
  rope_row_floats<F32>(gq_raw, wq);  // gains cast to the tensor dtype (read in it)
  rope_row_floats<F32>(gk_raw, wk);
  token_cos_sin<F32>(pos, fq, dl, c, s);
  store_batch(0);
  for (int i0 = kRopeFwdBatch; i0 < groups; i0 += kRopeFwdBatch) {
    load_batch(i0);
    store_batch(i0);
  }
}

// ---------------------------------------------------------------------------
// Backward (the VJP JAX autodiff derives for the reference's prologue).  Per
// head row, with y = x * inv, inv = rsqrt(mean(x^2) + eps), n = y * w and
// out = n * C + rot(n) * S:
//   dn_j = g_j C_j + (j < 32 ? g_{j+32} : -g_{j-32}) S_j      (rot^T)
//   dw  += dn * y   (y as the forward rounded it: y cast to the dtype)
//   dy   = dn * w
//   dx   = inv * (dy - y * mean(dy * y))
// everything in fp32 from the tensor-dtype operands, dx rounded once.  The
// gain gradients sum over every token and head: each wave accumulates its
// tokens' terms in registers, the workgroup adds its four waves, and a second
// launch adds the per-workgroup partials in workgroup order (deterministic,
// no atomics).
// ---------------------------------------------------------------------------
struct RopeBwdArgs {
  const void* q;
  const void* k;
  const void* q_gain;
  const void* k_gain;
  const int32_t* positions;
  const void* dq_out;
  const void* dk_out;
  void* dq;
  void* dk;
  float* partials;  // [gridDim.x][2][64]
  int B, T, Hq, Hkv;
  float eps;
  float freq[kD / 2];
};

constexpr int kRopeBwdBlocks = 1024;  // workgroups of the backward (fewer for short inputs)
constexpr int kRopeBatch = 3;          // (token, head group) rows loaded before any is computed

// The VJP of one loaded group: lane (g, dl) holds dims 8 dl .. 8 dl + 7 of
// head g.  Every lane takes part (shuffles and the 8-lane sums); only live
// lanes store and accumulate the gain gradient.
template <bool F32>
__device__ __forceinline__ void norm_rope_bwd_store(const RopeRow<F32>& xin,
                                                    const RopeRow<F32>& gin, void* dst,
                                                    size_t base, bool live, const float (&w)[8],
                                                    const float (&c)[8], const float (&s)[8],
                                                    int dl, float eps, float (&dw)[8]) {
  float x[8], go[8];
  rope_row_floats<F32>(xin, x);
  rope_row_floats<F32>(gin, go);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rsqrtf(dpp_xor_sum8(ss) * (1.f / kD) + eps);
  float dy[8], y[8], dot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // rot^T: dims d < 32 take +g[d + 32], dims d >= 32 take -g[d - 32]
    const float o = __shfl_xor(go[i], 4);
    const float dn = fmaf(go[i], c[i], (dl < 4 ? o : -o) * s[i]);
    y[i] = x[i] * inv;
    const float yr = F32 ? y[i] : round_bf16(y[i]);
    if (live) dw[i] = fmaf(dn, yr, dw[i]);
    dy[i] = dn * w[i];
    dot = fmaf(dy[i], y[i], dot);
  }
  const float mean = dpp_xor_sum8(dot) * (1.f / kD);
  if (!live) return;
  if constexpr (F32) {
    f32x4 oa, ob;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      oa[i] = inv * fmaf(-y[i], mean, dy[i]);
      ob[i] = inv * fmaf(-y[4 + i], mean, dy[4 + i]);
    }
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(dst) + base) = oa;
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(dst) + base + 4) = ob;
  } else {
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (bf16)(inv * fmaf(-y[i], mean, dy[i]));
    *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(dst) + base) = o;
  }
}

// Sum of x over the 8 lanes l, l ^ 8, ..., l ^ 56 (the 8 heads of a group
// that hold the same dims).
__device__ __forceinline__ float heads_sum8(float x) {
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

template <bool F32>
__global__ __launch_bounds__(256) void qk_norm_rope_bwd_kernel(RopeBwdArgs a) {
  __shared__ float part[4][2][kD];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 3, dl = lane & 7;
  const size_t total = (size_t)a.B * a.T;
  const size_t stride = (size_t)gridDim.x * 4;
  const int gq = (a.Hq + 7) >> 3;
  const int groups = gq + ((a.Hkv + 7) >> 3);  // 8-head groups of a token, q first
  float wq[8], wk[8];
  load_gains<F32>(a.q_gain, dl, wq);
  load_gains<F32>(a.k_gain, dl, wk);
  float dwq[8] = {0, 0, 0, 0, 0, 0, 0, 0}, dwk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // (token, group) of this wave's rows; no barrier inside the loop, so the
  // waves of a block need not run the same number of tokens
  auto locate = [&](size_t tok, int i, const void*& src, const void*& gsrc, void*& dst,
                    size_t& base, bool& live) {
    const bool isq = i < gq;
    const int H = isq ? a.Hq : a.Hkv;
    const int h = 8 * (isq ? i : i - gq) + g;
    live = h < H;
    base = (tok * H + min(h, H - 1)) * kD + 8 * dl;
    src = isq ? a.q : a.k;
    gsrc = isq ? a.dq_out : a.dk_out;
    dst = isq ? a.dq : a.dk;
  };
  for (size_t tok = (size_t)blockIdx.x * 4 + wave; tok < total; tok += stride) {
    // position and frequency loaded before the rows
    const float pos = token_position(a.positions, tok, a.T);
    const float fq = a.freq[lane & 31];
    float c[8], s[8];
    for (int i0 = 0; i0 < groups; i0 += kRopeBatch) {
      RopeRow<F32> x[kRopeBatch], go[kRopeBatch];
#pragma unroll
      for (int j = 0; j < kRopeBatch; ++j) {
        if (i0 + j < groups) {
          const void *src, *gsrc;
          void* dst;
          size_t base;
          bool live;
          locate(tok, i0 + j, src, gsrc, dst, base, live);
          x[j] = load_rope_row<F32>(src, base);
          go[j] = load_rope_row<F32>(gsrc, base);
        }
      }
      // the token's angles, evaluated while its loads are in flight
      if (i0 == 0) token_cos_sin<F32>(pos, fq, dl, c, s);
#pragma unroll
      for (int j = 0; j < kRopeBatch; ++j) {
        if (i0 + j < groups) {
          const void *src, *gsrc;
          void* dst;
          size_t base;
          bool live;
          locate(tok, i0 + j, src, gsrc, dst, base, live);
          if (i0 + j < gq)
            norm_rope_bwd_store<F32>(x[j], go[j], dst, base, live, wq, c, s, dl, a.eps, dwq);
          else
            norm_rope_bwd_store<F32>(x[j], go[j], dst, base, live, wk, c, s, dl, a.eps, dwk);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float sq = heads_sum8(dwq[i]), sk = heads_sum8(dwk[i]);
    if (lane < 8) {
      part[wave][0][8 * dl + i] = sq;
      part[wave][1][8 * dl + i] = sk;
    }
  }
  __syncthreads();
  if (threadIdx.x < 2 * kD) {
    const int which = threadIdx.x / kD, d = threadIdx.x % kD;
    const float v = ((part[0][which][d] + part[1][which][d]) + part[2][which][d]) + part[3][which][d];
    a.partials[((size_t)blockIdx.x * 2 + which) * kD + d] = v;
  }
}

// Sum of the per-workgroup gain partials in a fixed order: one block per
// column (2 gains x 64 dims); thread j adds workgroups j, j + 256, ... and
// the 256 sums are added as a tree in LDS.
constexpr int kRopeReduceThreads = 256;

__global__ __launch_bounds__(kRopeReduceThreads) void rope_gain_reduce_kernel(
    const float* partials, int blocks, float* dq_gain, float* dk_gain) {
  __shared__ float acc_l[kRopeReduceThreads];
  const int col = blockIdx.x;
  float acc = 0.f;
  for (int b = threadIdx.x; b < blocks; b += kRopeReduceThreads)
    acc += partials[(size_t)b * 2 * kD + col];
  acc_l[threadIdx.x] = acc;
  __syncthreads();
  for (int n = kRopeReduceThreads / 2; n > 0; n >>= 1) {
    if (threadIdx.x < n) acc_l[threadIdx.x] += acc_l[threadIdx.x + n];
    __syncthreads();
  }
  if (threadIdx.x == 0) (col >= kD ? dk_gain : dq_gain)[col % kD] = acc_l[0];
}

// Packer positions from segment ids: the offset of each token inside its run
// of equal nonzero ids, 0 for padding (batching/packing.py:92-100 writes
// arange(len) over each placed sequence and leaves padding at 0).  One
// workgroup per row: run starts by a max-scan.
__global__ __launch_bounds__(1024) void segment_positions_kernel(const int32_t* seg, int T,
                                                                 int32_t* pos) {
  __shared__ int carry_start;
  __shared__ int part[1024];
  const int b = blockIdx.x;
  const int32_t* s = seg + (size_t)b * T;
  int32_t* p = pos + (size_t)b * T;
  if (threadIdx.x == 0) carry_start = 0;
  __syncthreads();
  for (int base = 0; base < T; base += 1024) {
    const int t = base + threadIdx.x;
    const bool in = t < T;
    const int id = in ? s[t] : 0;
    const int start = (in && (t == 0 || s[t - 1] != id)) ? t : 0;
    part[threadIdx.x] = start;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int x = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
      __syncthreads();
      part[threadIdx.x] = max(part[threadIdx.x], x);
      __syncthreads();
    }
    const int run = max(part[threadIdx.x], carry_start);
    if (in) p[t] = id == 0 ? 0 : t - run;
    __syncthreads();
    if (threadIdx.x == 1023) carry_start = max(carry_start, part[1023]);
    __syncthreads();
  }
}

hipError_t launch_qk_norm_rope(const void* q, const void* k, const void* q_gain,
                               const void* k_gain, const int32_t* positions, bool f32, int B,
                               int T, int Hq, int Hkv, float eps, float theta, void* q_out,
                               void* k_out, hipStream_t stream) {
  RopeArgs a;
  a.q = q;
  a.k = k;
  a.q_gain = q_gain;
  a.k_gain = k_gain;
  a.positions = positions;
  a.q_out = q_out;
  a.k_out = k_out;
  a.B = B;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.eps = eps;
  // theta ** (-arange(0, D, 2) / D) in single precision (rotary.py:33-35)
  for (int i = 0; i < kD / 2; ++i) a.freq[i] = powf(theta, -((float)(2 * i) / (float)kD));
  const size_t total = (size_t)B * T;
  const dim3 grid((unsigned)((total + 3) / 4));
  if (f32)
    hipLaunchKernelGGL((qk_norm_rope_kernel<true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_kernel<false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

size_t rope_bwd_blocks(int B, int T) {
  const size_t total = (size_t)B * T;
  return std::min<size_t>((total + 3) / 4, kRopeBwdBlocks);
}

size_t rope_bwd_workspace_bytes(int B, int T) {
  return rope_bwd_blocks(B, T) * 2 * kD * sizeof(float);
}

hipError_t launch_qk_norm_rope_bwd(const void* q, const void* k, const void* q_gain,
                                   const void* k_gain, const int32_t* positions,
                                   const void* dq_out, const void* dk_out, bool f32, int B, int T,
                                   int Hq, int Hkv, float eps, float theta, void* dq, void* dk,
                                   float* dq_gain, float* dk_gain, void* workspace,
                                   hipStream_t stream) {
  RopeBwdArgs a;
  a.q = q;
  a.k = k;
  a.q_gain = q_gain;
  a.k_gain = k_gain;
  a.positions = positions;
  a.dq_out = dq_out;
  a.dk_out = dk_out;
  a.dq = dq;
  a.dk = dk;
  a.partials = static_cast<float*>(workspace);
  a.B = B;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.eps = eps;
  for (int i = 0; i < kD / 2; ++i) a.freq[i] = powf(theta, -((float)(2 * i) / (float)kD));
  const int blocks = (int)rope_bwd_blocks(B, T);
  if (f32)
    hipLaunchKernelGGL((qk_norm_rope_bwd_kernel<true>), dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_bwd_kernel<false>), dim3(blocks), dim3(256), 0, stream, a);
  hipLaunchKernelGGL(rope_gain_reduce_kernel, dim3(2 * kD), dim3(kRopeReduceThreads), 0, stream,
                     a.partials, blocks, dq_gain, dk_gain);
  return hipGetLastError();
}

hipError_t launch_segment_positions(const int32_t* seg, int B, int T, int32_t* pos,
                                    hipStream_t stream) {
  hipLaunchKernelGGL(segment_positions_kernel, dim3(B), dim3(1024), 0, stream, seg, T, pos);
  return hipGetLastError();
}

}  // namespace mf
