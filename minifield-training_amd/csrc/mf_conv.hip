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
// dtype contract: b*v, every tap product and c*mixed are rounded to the
// tensor dtype as in the reference; the tap sum accumulates in fp32 and is
// rounded once.  [B, T, C] row-major, C a multiple of 8.
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

// acc + lo + hi of a packed bf16 pair (products with 1 are exact).
__device__ __forceinline__ float dot2_ones(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                         __builtin_bit_cast(bf16x2, 0x3F803F80u), acc, false);
}

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
        // taps in pairs (2p, 2p + 1): both rounded products packed by one
        // conversion, the halves of taps outside the token's segment masked
        // off, and the pair added to the fp32 sum by a dot product with (1, 1)
        constexpr int kPairs = (K + 1) / 2;
        uint32_t keep[kPairs];
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
          const bool on0 = me != 0 && sid[win(2 * q)] == me;
          const bool on1 = 2 * q + 1 < K && me != 0 && sid[win(2 * q + 1)] == me;
          keep[q] = (on0 ? 0x0000ffffu : 0u) | (on1 ? 0xffff0000u : 0u);
        }
        uint32_t words[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float sum[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q < kPairs; ++q) {
              const float p0 = g[win(2 * q)][e + h] * w[2 * q][e + h];
              const float p1 = 2 * q + 1 < K ? g[win(2 * q + 1)][e + h] * w[2 * q + 1][e + h] : 0.f;
              acc = dot2_ones(pack_pair(p0, p1) & keep[q], acc);
            }
            sum[h] = acc;
          }
          float m0, m1;
          uint32_t word = round_pair(sum[0], sum[1], m0, m1);
          if (a.c) word = pack_pair(cu[e] * m0, cu[e + 1] * m1);
          words[e / 2] = word;
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
