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
// reference).  In bf16 the products with the gain and the rotation are
// rounded once each (the final combination at fp32, as XLA's fused
// elementwise code does).
//
// Layout: one wave per token.  Lanes 0..31 compute the token's 32 angles'
// cos/sin into LDS; then lane (g = lane / 8, dl = lane % 8) owns dims
// 8 dl .. 8 dl + 7 of head g of a group of 8 heads, so a 16-byte (bf16) or
// two 16-byte (fp32) loads per lane move 8 whole head rows, the sum of
// squares reduces over 8 lanes with DPP, and the rotation partner (dims
// +- 32) is lane dl ^ 4 of the same head.
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

template <bool F32>
__device__ __forceinline__ void norm_rope_rows(const void* src, void* dst, const void* gain, int H,
                                               size_t token, int lane, const float* cs,
                                               const float* sn, float eps) {
  typedef typename std::conditional<F32, float, bf16>::type T;
  const int g = lane >> 3, dl = lane & 7;
  float w[8], c[8], s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = 8 * dl + i;
    w[i] = (float)reinterpret_cast<const T*>(gain)[d];  // gain cast to the tensor dtype
    c[i] = cs[d & 31];
    s[i] = sn[d & 31];
    if constexpr (!F32) {
      c[i] = (float)(bf16)c[i];
      s[i] = (float)(bf16)s[i];
    }
  }
  for (int h0 = 0; h0 < H; h0 += 8) {
    const int h = h0 + g;
    const bool live = h < H;
    const size_t base = (token * H + min(h, H - 1)) * kD + 8 * dl;
    float x[8];
    if constexpr (F32) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(src) + base);
      const f32x4 b = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(src) + base + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = a[i], x[4 + i] = b[i];
    } else {
      const bf16x8 a = ld_bf16x8(reinterpret_cast<const bf16*>(src) + base);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = (float)a[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
    const float inv = rsqrtf(dpp_xor_sum8(ss) * (1.f / kD) + eps);
    float n[8], r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = x[i] * inv;
      if constexpr (!F32) v = (float)(bf16)v;
      v *= w[i];
      if constexpr (!F32) v = (float)(bf16)v;
      n[i] = v;
    }
    // rotate_half: dims d < 32 take -n[d + 32], dims d >= 32 take n[d - 32]
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float o = __shfl_xor(n[i], 4);
      r[i] = dl < 4 ? -o : o;
    }
    if (!live) continue;
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
      bf16x8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (bf16)fmaf(n[i], c[i], r[i] * s[i]);
      *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(dst) + base) = o;
    }
  }
}

template <bool F32>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  __shared__ float cs_l[4][kD / 2], sn_l[4][kD / 2];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t token = (size_t)blockIdx.x * 4 + wave;  // b * T + t
  const size_t total = (size_t)a.B * a.T;
  const size_t tok = token < total ? token : total - 1;  // tail waves redo the last token, no store
  const int t = (int)(tok % a.T);
  const float pos = (float)(a.positions ? a.positions[tok] : t);
  if (lane < kD / 2) {
    float sv, cv;
    sincosf(pos * a.freq[lane], &sv, &cv);
    cs_l[wave][lane] = cv;
    sn_l[wave][lane] = sv;
  }
  __syncthreads();
  if (token >= total) return;
  norm_rope_rows<F32>(a.q, a.q_out, a.q_gain, a.Hq, tok, lane, cs_l[wave], sn_l[wave], a.eps);
  norm_rope_rows<F32>(a.k, a.k_out, a.k_gain, a.Hkv, tok, lane, cs_l[wave], sn_l[wave], a.eps);
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

hipError_t launch_segment_positions(const int32_t* seg, int B, int T, int32_t* pos,
                                    hipStream_t stream) {
  hipLaunchKernelGGL(segment_positions_kernel, dim3(B), dim3(1024), 0, stream, seg, T, pos);
  return hipGetLastError();
}

}  // namespace mf
