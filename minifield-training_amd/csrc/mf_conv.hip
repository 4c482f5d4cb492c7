// Segmented short convolutions of the packed layers on gfx950.
//
//   causal   (kernels/convolution.py:25-53, gated_depthwise_convolution_segmented):
//     out[t] = c[t] * sum_i (b*v)[t - (K-1) + i] * w[:, i] * same(t - (K-1) + i, t)
//   centered (kernels/bidirectional.py:38-58, centered_convolution, as the
//     encoder calls it at models/lfm2_5/encoder.py:80-85):
//     out[t] = c[t] * sum_i (b*v)[t + i - K/2] * w[:, i] * same(t + i - K/2, t)
// where same(s, t) = 0 <= s < T && seg[s] == seg[t] && seg[t] != 0 (without
// segment ids: 0 <= s < T, the zero padding of the unsegmented versions).
// b and c may be absent (1).  Depthwise: channel c uses taps w[c, :].
//
// dtype contract: b*v, every tap product, every partial tap sum (in tap
// order) and c*mixed are rounded to the tensor dtype, the reference's
// declared dtypes (bidirectional.py:48-57, convolution.py:41-52), so the bf16
// result is the reference's bit for bit.  [B, T, C] row-major, C a multiple
// of 8.
//
// Thread = (row, 8 channels, 32 consecutive output tokens): a sliding window
// of the K gated inputs lives in registers, so every input element is read
// from HBM once (16-byte loads, 128 lanes per 1024-channel token row).
#include <type_traits>

#include "mf_common.h"

namespace mf {

struct ConvArgs {
  const void* b;
  const void* c;
  const void* v;
  const void* w;            // [C, K]
  const int32_t* seg;       // [B, T] or null
  void* out;
  int B, T, C, centered;
};

constexpr int kConvTile = 32;  // output tokens per thread

// 8 elements of one token row as loaded: raw tensor words, converted when used.
template <typename T>
struct Raw8 {
  bf16x8 v;
  __device__ __forceinline__ void load(const T* p) { v = ld_bf16x8(p); }
  __device__ __forceinline__ float operator[](int e) const { return (float)v[e]; }
};
template <>
struct Raw8<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float operator[](int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
};

// x and y rounded to bf16 (to nearest even) by one conversion: the packed
// pair (x in the low half), and both values back in fp32.
__device__ __forceinline__ uint32_t pack_pair(float x, float y) {
  const bf16x2 p = {(bf16)x, (bf16)y};
  return __builtin_bit_cast(uint32_t, p);
}
__device__ __forceinline__ uint32_t round_pair(float x, float y, float& rx, float& ry) {
  const uint32_t u = pack_pair(x, y);
  rx = __builtin_bit_cast(float, u << 16);
  ry = __builtin_bit_cast(float, u & 0xffff0000u);
  return u;
}

constexpr int conv_gcd(int x, int y) { return y ? conv_gcd(y, x % y) : x; }


// Thread = (row, 8 channels, kConvTile consecutive output tokens).  Input
// token u of the tile (u = 0 .. kConvTile + K - 2, token t0 + lo + u) is
// loaded kAhead steps before it is gated, into ring slot u % kAhead; at step
// u the output token u - (K - 1) is formed from a sliding window of the last
// K gated inputs and stored.  For bf16, the rounded tap products of a pair of
// taps are packed by one conversion and added to the fp32 sum by one dot
// product with (1, 1).
template <typename T, int K>
__global__ __launch_bounds__(256) void segmented_conv_kernel(ConvArgs a) {
  // input tokens whose v, b and c loads are in flight ahead of the one in use
  // (fewer for fp32, whose rows are twice as wide), chosen so that
  // lcm(K, kAhead) stays small enough to unroll
  constexpr int kAhead = std::is_same<T, float>::value ? 2 : (K <= 4 || K == 8) ? 4 : K;
  constexpr int kIn = kConvTile + K - 1;
  constexpr bool kBf16 = !std::is_same<T, float>::value;
  constexpr int kUnroll = K * kAhead / conv_gcd(K, kAhead);
  const int chunks = a.C / 8;
  const int tiles = (a.T + kConvTile - 1) / kConvTile;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)a.B * tiles * chunks) return;
  const int ch = (int)(gid % chunks);
  const int tile = (int)((gid / chunks) % tiles);
  const int b = (int)(gid / ((long long)chunks * tiles));
  const int c0 = ch * 8;
  const int lo = a.centered ? -(K / 2) : -(K - 1);  // offset of tap 0
  const int ctr = -lo;                              // the tap that reads the output token itself
  const int t0 = tile * kConvTile;

  float w[K][8];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) w[i][e] = (float)reinterpret_cast<const T*>(a.w)[(size_t)(c0 + e) * K + i];

  const size_t row = (size_t)b * a.T;
  const T* vp = reinterpret_cast<const T*>(a.v);
  const T* bp = reinterpret_cast<const T*>(a.b);
  const T* cp = reinterpret_cast<const T*>(a.c);
  // ring slot k: input u's v, b and segment id, and the c gate of output
  // u - (K - 1); tokens outside the row read token 0 or T - 1 and get id 0
  Raw8<T> vin[kAhead], bin[kAhead], cin[kAhead];
  int sin_[kAhead];
  auto issue = [&](int u, int k) {
    const int s = t0 + lo + u;
    const int sc = min(max(s, 0), a.T - 1);
    const size_t off = (row + sc) * a.C + c0;
    vin[k].load(vp + off);
    if (a.b) bin[k].load(bp + off);
    sin_[k] = s != sc ? 0 : a.seg ? a.seg[row + sc] : 1;
    const int j = u - (K - 1);
    if (a.c && j >= 0) cin[k].load(cp + (row + min(t0 + j, a.T - 1)) * a.C + c0);
  };
#pragma unroll
  for (int k = 0; k < kAhead; ++k)
    if (k < kIn) issue(k, k);

  // window: input u in slot u % K; the step loop is unrolled by a multiple
  // of both K and kAhead, so window and ring slots are compile-time indices
  float g[K][8];
  int sid[K];
  for (int u0 = 0; u0 < kIn; u0 += kUnroll) {
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int u = u0 + k;
      if (u >= kIn) break;
      const int slot = k % kAhead;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float x0 = vin[slot][e], x1 = vin[slot][e + 1];
        if (a.b) {
          x0 *= bin[slot][e];
          x1 *= bin[slot][e + 1];
          if constexpr (kBf16) round_pair(x0, x1, x0, x1);
        }
        g[k % K][e] = x0;
        g[k % K][e + 1] = x1;
      }
      sid[k % K] = sin_[slot];
      const int j = u - (K - 1);
      float cu[8];
      if (a.c && j >= 0)
#pragma unroll
        for (int e = 0; e < 8; ++e) cu[e] = cin[slot][e];
      if (u + kAhead < kIn) issue(u + kAhead, slot);
      if (j < 0 || t0 + j >= a.T) continue;
      // tap i of output j reads input j + i, window slot (k - (K - 1) + i) mod K
      auto win = [&](int i) { return ((k - (K - 1) + i) % K + K) % K; };
      const int me = sid[win(ctr)];
      const size_t off = (row + t0 + j) * a.C + c0;  // output element
      if constexpr (kBf16) {
        // the reference's declared-dtype order: each tap product rounded, the
        // taps added one at a time in tap order with every partial sum
        // rounded (taps outside the token's segment add an exact zero); two
        // channels share each conversion
        bool on[K];
#pragma unroll
        for (int i = 0; i < K; ++i) on[i] = me != 0 && sid[win(i)] == me;
        uint32_t words[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float m0 = 0.f, m1 = 0.f;
#pragma unroll
          for (int i = 0; i < K; ++i) {
            float p0, p1;
            round_pair(g[win(i)][e] * w[i][e], g[win(i)][e + 1] * w[i][e + 1], p0, p1);
            if (!on[i]) p0 = p1 = 0.f;
            if (i == 0) {
              m0 = p0;
              m1 = p1;
            } else {
              round_pair(m0 + p0, m1 + p1, m0, m1);
            }
          }
          words[e / 2] = a.c ? pack_pair(cu[e] * m0, cu[e + 1] * m1) : pack_pair(m0, m1);
        }
        const u32x4 x = {words[0], words[1], words[2], words[3]};
        *reinterpret_cast<u32x4*>(reinterpret_cast<bf16*>(a.out) + off) = x;
      } else {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
        for (int i = 0; i < K; ++i) {
          const bool on = me != 0 && sid[win(i)] == me;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += on ? g[win(i)][e] * w[i][e] : 0.f;
        }
        f32x4 x0, x1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x0[e] = a.c ? cu[e] * acc[e] : acc[e];
          x1[e] = a.c ? cu[4 + e] * acc[4 + e] : acc[4 + e];
        }
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + off) = x0;
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + off + 4) = x1;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward (the VJP of out[t] = c[t] * m[t], m[t] = sum_i u[t + o_i] w_i
// keep(t, t + o_i), u = b * v, o_i = lo + i).  With h = g * c:
//   dc[t] = g[t] * m[t]
//   du[s] = sum_i h[s - o_i] w_i keep(s - o_i, s)     (keep is symmetric)
//   db = du * v,  dv = du * b,  dw_i = sum_{b,t} h[t] u[t + o_i] keep(t, t + o_i)
// in fp32 from the tensor-dtype operands (u and m rounded as the forward
// rounds them), each gradient rounded once.  Thread = (row, 8 channels, 16
// output tokens), streaming its input rows once through a register ring; a
// workgroup holds 8 channel chunks x 32 token tiles, so the tap-gradient
// terms of its 32 tiles are added inside it (lanes, then waves) and written
// as one partial per (workgroup row, channel, tap); a second launch adds the
// partials in a fixed order (deterministic, no atomics).
// ---------------------------------------------------------------------------
struct ConvBwdArgs {
  const void* b;
  const void* c;
  const void* v;
  const void* w;
  const int32_t* seg;
  const void* g;   // d out
  void* db;
  void* dc;
  void* dv;
  float* partials;  // [B * tile groups][C][K]
  int B, T, C, K, centered;
};

constexpr int kConvBwdTile = 16;    // output tokens per thread of the backward
constexpr int kConvBwdTiles = 32;   // token tiles per workgroup
constexpr int kConvBwdChunks = 8;   // channel chunks per workgroup

// Channels per thread of the backward.  A thread holds a ring of W + 1 slots
// of four input rows (W = 2K - 1 causal, K or K + 1 centered) plus K taps and
// K tap gradients per channel.  At 8 channels that exceeds the register file
// beyond K = 4 (K = 5 centered still fits): the compiler spilled up to 2 KB
// per lane to scratch, 4-6x slower, so wider filters take 4 channels.
template <typename T, int K, bool CENTERED>
constexpr int conv_bwd_channels() {
  return K <= 4 || (K == 5 && CENTERED && !std::is_same<T, float>::value) ? 8 : 4;
}

// CW elements of one token row of the backward as loaded.
template <typename T, int CW>
struct RawC : Raw8<T> {};
template <>
struct RawC<bf16, 4> {
  bf16x4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x4*>(p); }
  __device__ __forceinline__ float operator[](int e) const { return (float)v[e]; }
};
template <>
struct RawC<float, 4> {
  f32x4 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const f32x4*>(p); }
  __device__ __forceinline__ float operator[](int e) const { return v[e]; }
};

template <typename T, int CW>
__device__ __forceinline__ void store_row(T* p, const float (&x)[CW]) {
  if constexpr (std::is_same<T, float>::value) {
#pragma unroll
    for (int h = 0; h < CW; h += 4) {
      const f32x4 v = {x[h], x[h + 1], x[h + 2], x[h + 3]};
      *reinterpret_cast<f32x4*>(p + h) = v;
    }
  } else if constexpr (CW == 8) {
    uint32_t words[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) words[e / 2] = pack_pair(x[e], x[e + 1]);
    const u32x4 v = {words[0], words[1], words[2], words[3]};
    *reinterpret_cast<u32x4*>(p) = v;
  } else {
    const u32x2 v = {pack_pair(x[0], x[1]), pack_pair(x[2], x[3])};
    *reinterpret_cast<u32x2*>(p) = v;
  }
}

// One thread's output tokens t0 .. t0 + kConvBwdTile - 1 for tap offsets
// LO .. LO + K - 1.  m[t] reads u at t + LO + i and du[t] reads h at
// t - LO - i, so output t needs input tokens t + SMIN .. t + SMAX.  Input q
// (token t0 + SMIN + q) goes to ring slot q % R (R = W + kAhead, W the window
// width) kAhead steps before it is used; at step q output q - (W - 1) is
// formed from the W newest slots, so every row is loaded once per thread.
// The step loop is unrolled by R, so all slot indices are compile-time.
template <typename T, int K, int LO, int CW>
__device__ __forceinline__ void conv_bwd_tile(const ConvBwdArgs& a, size_t row, int t0, int c0,
                                              const float (&w)[K][CW], float (&dw)[K][CW]) {
  constexpr bool kBf16 = !std::is_same<T, float>::value;
  constexpr int SMIN = LO < -LO - (K - 1) ? LO : -LO - (K - 1);
  constexpr int SMAX = LO + K - 1 > -LO ? LO + K - 1 : -LO;
  constexpr int W = SMAX - SMIN + 1;
  constexpr int kAhead = 1;
  constexpr int R = W + kAhead;
  constexpr int kSteps = kConvBwdTile + W - 1;
  const T* vp = reinterpret_cast<const T*>(a.v);
  const T* bp = reinterpret_cast<const T*>(a.b);
  const T* cp = reinterpret_cast<const T*>(a.c);
  const T* gp = reinterpret_cast<const T*>(a.g);
  RawC<T, CW> rv[R], rb[R], rg[R], rc[R];
  int sg[R];
  auto issue = [&](int q, int slot) {
    const int s = t0 + SMIN + q;
    const int sc = min(max(s, 0), a.T - 1);
    const size_t off = (row + sc) * a.C + c0;
    rv[slot].load(vp + off);
    if (a.b) rb[slot].load(bp + off);
    rg[slot].load(gp + off);
    if (a.c) rc[slot].load(cp + off);
    sg[slot] = s != sc ? 0 : a.seg ? a.seg[row + sc] : 1;
  };
#pragma unroll
  for (int q = 0; q < kAhead; ++q) issue(q, q);
  const int tend = min(kConvBwdTile, a.T - t0);
#pragma unroll 1
  for (int q0 = 0; q0 < kSteps; q0 += R) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int q = q0 + k;
      if (q >= kSteps) break;
      // the slot of input q - W left the window last step
      if (q + kAhead < kSteps) issue(q + kAhead, (k + kAhead) % R);
      const int j = q - (W - 1);
      if (j < 0 || j >= tend) continue;
      auto slot = [&](int d) { return ((k - SMAX + d) % R + R) % R; };  // input at t + d
      const int s0 = slot(0);
      const int me = sg[s0];
      float m[CW], du[CW], h0[CW];
#pragma unroll
      for (int e = 0; e < CW; ++e) {
        m[e] = 0.f;
        du[e] = 0.f;
        h0[e] = a.c ? rg[s0][e] * rc[s0][e] : rg[s0][e];
      }
#pragma unroll
      for (int i = 0; i < K; ++i) {
        // forward tap: u at t + LO + i feeds m[t] (rounded in tap order as
        // the forward does); transposed tap: h at t - LO - i feeds du[t]
        const int su = slot(LO + i), sh = slot(-LO - i);
        if (me != 0 && sg[su] == me) {
#pragma unroll
          for (int e = 0; e < CW; ++e) {
            float u = rv[su][e];
            if (a.b) u = kBf16 ? round_bf16(u * rb[su][e]) : u * rb[su][e];
            const float p = u * w[i][e];
            m[e] = kBf16 ? round_bf16(round_bf16(p) + m[e]) : m[e] + p;
            dw[i][e] = fmaf(h0[e], u, dw[i][e]);
          }
        }
        if (me != 0 && sg[sh] == me) {
#pragma unroll
          for (int e = 0; e < CW; ++e) {
            const float hn = a.c ? rg[sh][e] * rc[sh][e] : rg[sh][e];
            du[e] = fmaf(hn, w[i][e], du[e]);
          }
        }
      }
      const size_t off = (row + t0 + j) * a.C + c0;
      if (a.dc) {
        float dc[CW];
#pragma unroll
        for (int e = 0; e < CW; ++e) dc[e] = rg[s0][e] * m[e];
        store_row<T, CW>(reinterpret_cast<T*>(a.dc) + off, dc);
      }
      float dv[CW];
      if (a.b) {
        float db[CW];
#pragma unroll
        for (int e = 0; e < CW; ++e) dv[e] = du[e] * rb[s0][e], db[e] = du[e] * rv[s0][e];
        store_row<T, CW>(reinterpret_cast<T*>(a.db) + off, db);
      } else {
#pragma unroll
        for (int e = 0; e < CW; ++e) dv[e] = du[e];
      }
      store_row<T, CW>(reinterpret_cast<T*>(a.dv) + off, dv);
    }
  }
}

template <typename T, int K, bool CENTERED>
__global__ __launch_bounds__(256) void segmented_conv_bwd_kernel(ConvBwdArgs a) {
  constexpr int CW = conv_bwd_channels<T, K, CENTERED>();
  __shared__ float red[4][kConvBwdChunks][K * CW];
  const int chunks = a.C / CW;
  const int tiles = (a.T + kConvBwdTile - 1) / kConvBwdTile;
  const int cgroups = (chunks + kConvBwdChunks - 1) / kConvBwdChunks;
  const int tgroups = (tiles + kConvBwdTiles - 1) / kConvBwdTiles;
  const int cg = blockIdx.x % cgroups;
  const int tg = (blockIdx.x / cgroups) % tgroups;
  const int b = blockIdx.x / (cgroups * tgroups);
  const int lc = threadIdx.x % kConvBwdChunks, lt = threadIdx.x / kConvBwdChunks;
  const int ch = cg * kConvBwdChunks + lc;
  const int tile = tg * kConvBwdTiles + lt;
  const bool on = ch < chunks && tile < tiles;
  const int c0 = min(ch, chunks - 1) * CW;
  const size_t row = (size_t)b * a.T;

  float w[K][CW];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int e = 0; e < CW; ++e) w[i][e] = (float)reinterpret_cast<const T*>(a.w)[(size_t)(c0 + e) * K + i];
  float dw[K][CW];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int e = 0; e < CW; ++e) dw[i][e] = 0.f;

  if (on) {
    const int t0 = tile * kConvBwdTile;
    conv_bwd_tile<T, K, CENTERED ? -(K / 2) : -(K - 1), CW>(a, row, t0, c0, w, dw);
  }
  // tap gradients: add the 8 tiles of each wave (lanes lc, lc + 8, ... hold
  // the same channels), then the 4 waves, in a fixed order
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int e = 0; e < CW; ++e) {
      float x = dw[i][e];
      x += __shfl_xor(x, 8);
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      if (lane < kConvBwdChunks) red[wave][lane][i * CW + e] = x;
    }
  __syncthreads();
  for (int j = threadIdx.x; j < kConvBwdChunks * K * CW; j += blockDim.x) {
    const int jc = j / (K * CW), ie = j % (K * CW), i = ie / CW, e = ie % CW;
    const int chj = cg * kConvBwdChunks + jc;
    if (chj >= chunks) continue;
    const float x = ((red[0][jc][ie] + red[1][jc][ie]) + red[2][jc][ie]) + red[3][jc][ie];
    a.partials[((size_t)(b * tgroups + tg) * a.C + chj * CW + e) * K + i] = x;
  }
}

// d taps [C][K] fp32: the partials of every (row, tile group) added in a
// fixed order.  A block takes 32 columns; thread (slice, column) adds parts
// slice, slice + 8, ..., and the 8 slice sums are added in slice order.
constexpr int kTapCols = 32, kTapSlices = 8;

__global__ __launch_bounds__(kTapCols * kTapSlices) void conv_taps_reduce_kernel(
    const float* partials, int parts, int n, float* dw) {
  __shared__ float acc_l[kTapSlices][kTapCols];
  const int c = threadIdx.x % kTapCols, sl = threadIdx.x / kTapCols;
  const int j = blockIdx.x * kTapCols + c;
  float acc = 0.f;
  if (j < n)
    for (int p = sl; p < parts; p += kTapSlices) acc += partials[(size_t)p * n + j];
  acc_l[sl][c] = acc;
  __syncthreads();
  if (sl == 0 && j < n) {
    float v = acc_l[0][c];
#pragma unroll
    for (int k = 1; k < kTapSlices; ++k) v += acc_l[k][c];
    dw[j] = v;
  }
}

size_t conv_bwd_parts(int B, int T) {
  const int tiles = (T + kConvBwdTile - 1) / kConvBwdTile;
  return (size_t)B * ((tiles + kConvBwdTiles - 1) / kConvBwdTiles);
}

size_t conv_bwd_workspace_bytes(int B, int T, int C, int K) {
  return conv_bwd_parts(B, T) * (size_t)C * K * sizeof(float);
}

template <typename T>
hipError_t launch_conv_bwd_t(const ConvBwdArgs& a, hipStream_t stream) {
  const int tiles = (a.T + kConvBwdTile - 1) / kConvBwdTile;
  const long long tgroups = (tiles + kConvBwdTiles - 1) / kConvBwdTiles;
  // one workgroup per (row, tile group, group of kConvBwdChunks channel chunks)
  auto grid_for = [&](int cw) {
    const int chunks = a.C / cw;
    return dim3((unsigned)(a.B * tgroups * ((chunks + kConvBwdChunks - 1) / kConvBwdChunks)));
  };
#define MF_CONV_BWD_CASE(KK)                                                                     \
    case KK: {                                                                                    \
      if (a.centered)                                                                             \
        hipLaunchKernelGGL((segmented_conv_bwd_kernel<T, KK, true>),                              \
                           grid_for(conv_bwd_channels<T, KK, true>()), dim3(256), 0, stream, a);  \
      else                                                                                        \
        hipLaunchKernelGGL((segmented_conv_bwd_kernel<T, KK, false>),                             \
                           grid_for(conv_bwd_channels<T, KK, false>()), dim3(256), 0, stream, a); \
      break;                                                                                      \
    }
  switch (a.K) {
    MF_CONV_BWD_CASE(1)
    MF_CONV_BWD_CASE(2)
    MF_CONV_BWD_CASE(3)
    MF_CONV_BWD_CASE(4)
    MF_CONV_BWD_CASE(5)
    MF_CONV_BWD_CASE(6)
    MF_CONV_BWD_CASE(7)
    MF_CONV_BWD_CASE(8)
#undef MF_CONV_BWD_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_segmented_conv_bwd(const void* b, const void* c, const void* v, const void* w,
                                     const int32_t* seg, const void* g, bool centered, bool f32,
                                     int B, int T, int C, int K, void* db, void* dc, void* dv,
                                     float* dw, void* workspace, hipStream_t stream) {
  ConvBwdArgs a;
  a.b = b;
  a.c = c;
  a.v = v;
  a.w = w;
  a.seg = seg;
  a.g = g;
  a.db = db;
  a.dc = dc;
  a.dv = dv;
  a.partials = static_cast<float*>(workspace);
  a.B = B;
  a.T = T;
  a.C = C;
  a.K = K;
  a.centered = centered;
  const hipError_t e = f32 ? launch_conv_bwd_t<float>(a, stream) : launch_conv_bwd_t<bf16>(a, stream);
  if (e != hipSuccess) return e;
  const int n = C * K;
  hipLaunchKernelGGL(conv_taps_reduce_kernel, dim3((n + kTapCols - 1) / kTapCols),
                     dim3(kTapCols * kTapSlices), 0, stream, a.partials, (int)conv_bwd_parts(B, T),
                     n, dw);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_conv_t(const ConvArgs& a, int K, hipStream_t stream) {
  const long long threads = (long long)a.B * ((a.T + kConvTile - 1) / kConvTile) * (a.C / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  switch (K) {
    case 1: hipLaunchKernelGGL((segmented_conv_kernel<T, 1>), grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((segmented_conv_kernel<T, 2>), grid, dim3(256), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((segmented_conv_kernel<T, 3>), grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((segmented_conv_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
    case 5: hipLaunchKernelGGL((segmented_conv_kernel<T, 5>), grid, dim3(256), 0, stream, a); break;
    case 6: hipLaunchKernelGGL((segmented_conv_kernel<T, 6>), grid, dim3(256), 0, stream, a); break;
    case 7: hipLaunchKernelGGL((segmented_conv_kernel<T, 7>), grid, dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((segmented_conv_kernel<T, 8>), grid, dim3(256), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_segmented_conv(const void* b, const void* c, const void* v, const void* w,
                                 const int32_t* seg, bool centered, bool f32, int B, int T, int C,
                                 int K, void* out, hipStream_t stream) {
  ConvArgs a;
  a.b = b;
  a.c = c;
  a.v = v;
  a.w = w;
  a.seg = seg;
  a.out = out;
  a.B = B;
  a.T = T;
  a.C = C;
  a.centered = centered;
  return f32 ? launch_conv_t<float>(a, K, stream) : launch_conv_t<bf16>(a, K, stream);
}

}  // namespace mf
