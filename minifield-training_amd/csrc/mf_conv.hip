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

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* x) {
  if constexpr (std::is_same<T, float>::value) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = a[i], x[4 + i] = b[i];
  } else {
    const bf16x8 a = ld_bf16x8(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (float)a[i];
  }
}

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (std::is_same<T, float>::value) return x;
  else return (float)(bf16)x;
}

template <typename T, int K>
__global__ __launch_bounds__(256) void segmented_conv_kernel(ConvArgs a) {
  const int chunks = a.C / 8;
  const int tiles = (a.T + kConvTile - 1) / kConvTile;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)a.B * tiles * chunks) return;
  const int ch = (int)(gid % chunks);
  const int tile = (int)((gid / chunks) % tiles);
  const int b = (int)(gid / ((long long)chunks * tiles));
  const int c0 = ch * 8;
  const int lo = a.centered ? -(K / 2) : -(K - 1);  // offset of tap 0
  const int t0 = tile * kConvTile;
  const int t1 = min(t0 + kConvTile, a.T);

  float w[K][8];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) w[i][e] = (float)reinterpret_cast<const T*>(a.w)[(size_t)(c0 + e) * K + i];

  const size_t row = (size_t)b * a.T;
  auto gated = [&](int s, float* g) {  // round(b*v) at token s (0 outside the row)
    if (s < 0 || s >= a.T) {
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = 0.f;
      return;
    }
    const size_t off = (row + s) * a.C + c0;
    load8(reinterpret_cast<const T*>(a.v) + off, g);
    if (a.b) {
      float bb[8];
      load8(reinterpret_cast<const T*>(a.b) + off, bb);
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = round_to<T>(g[e] * bb[e]);
    }
  };
  auto seg_at = [&](int s) { return (a.seg && s >= 0 && s < a.T) ? a.seg[row + s] : (s >= 0 && s < a.T ? 1 : 0); };

  // window[i] = gated input at t + lo + i for the current output token t
  float win[K][8];
  int sid[K];
#pragma unroll
  for (int i = 0; i < K - 1; ++i) {
    gated(t0 + lo + i, win[i + 1]);
    sid[i + 1] = seg_at(t0 + lo + i);
  }
  for (int t = t0; t < t1; ++t) {
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = win[i + 1][e];
      sid[i] = sid[i + 1];
    }
    gated(t + lo + K - 1, win[K - 1]);
    sid[K - 1] = seg_at(t + lo + K - 1);
    const int me = seg_at(t);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const bool on = me != 0 && sid[i] == me;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += on ? round_to<T>(win[i][e] * w[i][e]) : 0.f;
    }
    const size_t off = (row + t) * a.C + c0;
    float cc[8];
    if (a.c) load8(reinterpret_cast<const T*>(a.c) + off, cc);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float m = round_to<T>(acc[e]);
      o[e] = a.c ? round_to<T>(cc[e] * m) : m;
    }
    if constexpr (std::is_same<T, float>::value) {
      f32x4 x0, x1;
#pragma unroll
      for (int e = 0; e < 4; ++e) x0[e] = o[e], x1[e] = o[4 + e];
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + off) = x0;
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + off + 4) = x1;
    } else {
      bf16x8 x;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16)o[e];
      *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(a.out) + off) = x;
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
