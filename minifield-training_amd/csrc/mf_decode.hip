// Ragged KV-cached decode (one query token per row) on gfx950.
//
// Split-K over the cache: the valid prefix of every row is cut into chunks
// of C tokens; a work item is (row, chunk) for one KV head.  A tiny prep
// kernel turns the per-row lengths into chunk offsets (a prefix sum on the
// device, so the host never reads the lengths back), then a persistent grid
// walks the flattened item list.  Each item streams its chunk of K and V for
// one KV head into LDS with fully coalesced 16-byte loads (8 lanes cover one
// 128-byte key row), scores the G query heads of the group against it, and
// writes a partial (max, sum, unnormalised output).  A combine kernel merges
// a row's partials with the usual log-sum-exp rescaling.
//
// Reference semantics: kernels/attention.py:264-282 -- slot j of row b is
// valid iff j < valid_length[b]; a length above the capacity reads every
// slot; a length <= 0 leaves every slot masked, which the reference turns
// into a uniform average over all slots (the softmax of a constant row).
#include <type_traits>

#include "mf_common.h"

namespace mf {

struct DecArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* lengths;
  // decode-step append: the step's key/value rows and per-row cache slots;
  // null for a plain decode
  const void* k_new;
  const void* v_new;
  const int32_t* positions;
  int32_t* step_lengths;  // positions + 1, the lengths the step attends over
  void* k_cache;          // writable views of k / v for the append
  void* v_cache;
  void* out;
  int* offsets;    // [B + 1] chunk offsets
  float* partial;  // [B][Hq][maxc][2 + D]: (scaled max, sum, acc[D])
  int B, cap, Hq, Hkv, G, maxc, chunk;
  float scale_log2;
};

constexpr int kPitch = kD + 8;    // bf16 LDS row pitch (144 B)
constexpr int kPitchF = kD + 4;   // fp32 LDS row pitch (272 B)
constexpr int kMaxG = 8;          // query heads per KV head served by decode

__device__ __forceinline__ int eff_len(int len, int cap) {
  return len <= 0 ? cap : (len > cap ? cap : len);
}

// Row b's length as given: lengths[b], or positions[b] + 1 for a decode step
// with an append (saturated to int32).
__device__ __forceinline__ int raw_length(const int32_t* lengths, const int32_t* positions, int b) {
  if (positions) {
    const long long len = (long long)positions[b] + 1;
    return (int)(len > INT32_MAX ? INT32_MAX : len);
  }
  return lengths[b];
}

// Decode-step append (dynamic_update_slice of one token per row): row b's
// key/value go to slot clamp(positions[b], 0, cap - 1) -- the start index
// clamping of dynamic_update_slice -- and the step attends over
// positions[b] + 1 slots.  16-byte copies; the decode kernels of the same
// stream read the cache after this kernel.
template <int ELEM>
__device__ void append_rows(const DecArgs& a) {
  constexpr int kChunks = kD * ELEM / 16;  // 16-byte chunks per (row, head)
  const int total = a.B * a.Hkv * kChunks;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int ch = i % kChunks;
    const int bh = i / kChunks;
    const int b = bh / a.Hkv, h = bh % a.Hkv;
    const int slot = min(max(a.positions[b], 0), a.cap - 1);
    const size_t src = ((size_t)bh * kD) * ELEM + ch * 16;
    const size_t dst = ((((size_t)b * a.cap + slot) * a.Hkv + h) * kD) * ELEM + ch * 16;
    st_u32x4(reinterpret_cast<char*>(a.k_cache) + dst, ld_u32x4(reinterpret_cast<const char*>(a.k_new) + src));
    st_u32x4(reinterpret_cast<char*>(a.v_cache) + dst, ld_u32x4(reinterpret_cast<const char*>(a.v_new) + src));
  }
}

template <int ELEM>
__global__ __launch_bounds__(256) void decode_prep_kernel(DecArgs a) {
  if (a.positions) {
    append_rows<ELEM>(a);
    for (int b = threadIdx.x; b < a.B; b += blockDim.x) {
      const long long len = (long long)a.positions[b] + 1;
      a.step_lengths[b] = (int)min(max(len, (long long)INT32_MIN), (long long)INT32_MAX);
    }
    __syncthreads();
    a.lengths = a.step_lengths;
  }
  // Block-wide exclusive scan of per-row chunk counts (B may exceed 256).
  __shared__ int part[256];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < a.B; base += 256) {
    const int b = base + threadIdx.x;
    const int n = b < a.B ? (eff_len(a.lengths[b], a.cap) + a.chunk - 1) / a.chunk : 0;
    part[threadIdx.x] = n;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int x = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
      __syncthreads();
      part[threadIdx.x] += x;
      __syncthreads();
    }
    if (b < a.B) a.offsets[b] = carry + part[threadIdx.x] - n;
    __syncthreads();
    if (threadIdx.x == 255) carry += part[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.offsets[a.B] = carry;
}

template <bool F32>
struct DecLds;

template <>
struct DecLds<false> {
  bf16 k[256 * kPitch];
  bf16 v[256 * kPitch];
  float p[kMaxG][256];
  float q[kMaxG][kD];
  float red[kMaxG][4];
  float acc[4][kMaxG][kD];
};

template <>
struct DecLds<true> {
  float k[128 * kPitchF];
  float v[128 * kPitchF];
  float p[kMaxG][256];
  float q[kMaxG][kD];
  float red[kMaxG][4];
  float acc[4][kMaxG][kD];
};

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <bool F32>
__global__ __launch_bounds__(256) void decode_kernel(DecArgs a) {
  __shared__ DecLds<F32> lds;
  constexpr int C = F32 ? 128 : 256;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kvh = blockIdx.y;
  const int total = a.offsets[a.B];
  const float c = a.scale_log2;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    // row of this item: last b with offsets[b] <= item
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.offsets[mid] <= item) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int chunk = item - a.offsets[b];
    const int raw = a.lengths[b];
    const bool uniform = raw <= 0;
    const int len = eff_len(raw, a.cap);
    const int t0 = chunk * C;
    const int n = min(C, len - t0);

    // ---- stage K, V chunk and the group's queries -------------------------
    if constexpr (!F32) {
      const bf16* ks = reinterpret_cast<const bf16*>(a.k);
      const bf16* vs = reinterpret_cast<const bf16*>(a.v);
      u32x4 kr[8], vr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = tid + 256 * i;
        const int t = u >> 3, ch = u & 7;
        const size_t off = (((size_t)b * a.cap + t0 + t) * a.Hkv + kvh) * kD + ch * 8;
        kr[i] = t < n ? ld_u32x4(ks + off) : u32x4{0, 0, 0, 0};
        vr[i] = t < n ? ld_u32x4(vs + off) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = tid + 256 * i;
        st_u32x4(&lds.k[(u >> 3) * kPitch + (u & 7) * 8], kr[i]);
        st_u32x4(&lds.v[(u >> 3) * kPitch + (u & 7) * 8], vr[i]);
      }
    } else {
      const float* ks = reinterpret_cast<const float*>(a.k);
      const float* vs = reinterpret_cast<const float*>(a.v);
      u32x4 kr[8], vr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = tid + 256 * i;
        const int t = u >> 4, ch = u & 15;
        const size_t off = (((size_t)b * a.cap + t0 + t) * a.Hkv + kvh) * kD + ch * 4;
        kr[i] = t < n ? ld_u32x4(ks + off) : u32x4{0, 0, 0, 0};
        vr[i] = t < n ? ld_u32x4(vs + off) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = tid + 256 * i;
        st_u32x4(&lds.k[(u >> 4) * kPitchF + (u & 15) * 4], kr[i]);
        st_u32x4(&lds.v[(u >> 4) * kPitchF + (u & 15) * 4], vr[i]);
      }
    }

    // The group's query heads in chunks of kMaxG, each against the staged
    // K and V (any number of query heads per KV head).
    for (int g0 = 0; g0 < a.G; g0 += kMaxG) {
    const int gc = min(kMaxG, a.G - g0);
    for (int e = tid; e < gc * kD; e += 256) {
      const int g = e / kD, d = e % kD;
      const size_t qi = ((size_t)b * a.Hq + kvh * a.G + g0 + g) * kD + d;
      if constexpr (F32) lds.q[g][d] = reinterpret_cast<const float*>(a.q)[qi];
      else lds.q[g][d] = (float)reinterpret_cast<const bf16*>(a.q)[qi];
    }
    __syncthreads();

    // ---- scores: thread t owns token t ---------------------------------------
    float sc[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) sc[g] = 0.f;
    if (tid < n && !uniform) {
      if constexpr (!F32) {
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const bf16x8 kx = ld_bf16x8(&lds.k[tid * kPitch + c8 * 8]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float kv = (float)kx[e];
#pragma unroll
            for (int g = 0; g < kMaxG; ++g)
              if (g < gc) sc[g] = fmaf(lds.q[g][c8 * 8 + e], kv, sc[g]);
          }
        }
      } else {
#pragma unroll
        for (int c4 = 0; c4 < 16; ++c4) {
          const f32x4 kx = *reinterpret_cast<const f32x4*>(&lds.k[tid * kPitchF + c4 * 4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int g = 0; g < kMaxG; ++g)
              if (g < gc) sc[g] = fmaf(lds.q[g][c4 * 4 + e], kx[e], sc[g]);
        }
      }
    }
    // chunk max and exponentials per head (log2 domain)
    float mx2[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      if (g >= gc) break;
      const float s2 = tid < n ? sc[g] * c : kNegInf;
      const float wm = wave_max(s2);
      if (lane == 0) lds.red[g][wave] = wm;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      if (g >= gc) break;
      mx2[g] = fmaxf(fmaxf(lds.red[g][0], lds.red[g][1]), fmaxf(lds.red[g][2], lds.red[g][3]));
      const float p = tid < n ? fast_exp2(fmaf(sc[g], c, -mx2[g])) : 0.f;
      if (tid < C) lds.p[g][tid] = p;
    }
    __syncthreads();
    float lsum[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      if (g >= gc) break;
      const float ws = wave_sum(tid < C ? lds.p[g][tid] : 0.f);
      lsum[g] = ws;
    }
    __syncthreads();  // everyone has read red[] for the max
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      if (g >= gc) break;
      if (lane == 0) lds.red[g][wave] = lsum[g];
    }

    // ---- PV: thread (d = lane, token group = wave) ---------------------------
    float acc[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) acc[g] = 0.f;
    for (int t = wave; t < n; t += 4) {
      float vv;
      if constexpr (!F32) vv = (float)lds.v[t * kPitch + lane];
      else vv = lds.v[t * kPitchF + lane];
#pragma unroll
      for (int g = 0; g < kMaxG; ++g)
        if (g < gc) acc[g] = fmaf(lds.p[g][t], vv, acc[g]);
    }
#pragma unroll
    for (int g = 0; g < kMaxG; ++g)
      if (g < gc) lds.acc[wave][g][lane] = acc[g];
    __syncthreads();
    if (wave == 0) {
      for (int g = 0; g < gc; ++g) {
        const float o = lds.acc[0][g][lane] + lds.acc[1][g][lane] + lds.acc[2][g][lane] +
                        lds.acc[3][g][lane];
        const int h = kvh * a.G + g0 + g;
        float* dst = a.partial + (((size_t)b * a.Hq + h) * a.maxc + chunk) * (2 + kD);
        dst[2 + lane] = o;
        if (lane == 0) dst[0] = mx2[g];
        if (lane == 1) dst[1] = lds.red[g][0] + lds.red[g][1] + lds.red[g][2] + lds.red[g][3];
      }
    }
    __syncthreads();  // q, p, red and acc are rewritten by the next chunk
    }
    __syncthreads();  // LDS reused by the next item
  }
}

// ---------------------------------------------------------------------------
// bf16 decode: one wave per (row, 256-token chunk, KV head) item, no LDS.
// Lane = (key kg = lane / 8 of an 8-key group, d-slice dl = lane % 8 of 8
// dims), so one 16-byte load per lane covers 8 whole 128-byte key rows and a
// wave streams 32 keys of K and V (8 KiB) per iteration, the next
// iteration's loads in flight while this one is scored.  Scores are 4-term
// bf16 dot products (v_dot2) reduced over the 8 lanes of a key with DPP;
// P V packs pairs of probabilities and the matching V elements of two keys
// into bf16 pairs for v_dot2 as well.  The online softmax keeps one running
// max per query head (wave-uniform) and rescales lazily like the prefill
// forward.  The chunk's (max, sum, unnormalised output) go to the same
// partial buffer the combine kernel reads.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// sum over the 8 lanes of a key group (lanes 8j .. 8j+7)
__device__ __forceinline__ float group8_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));  // quad xor 1
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));  // quad xor 2
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false)); // half-row mirror
  return x;
}

// combine over the 8 key groups (lanes with equal lane % 8): the lane ^ 8,
// lane ^ 16 and lane ^ 32 exchanges
template <bool MAX>
__device__ __forceinline__ float across_groups(float x) {
  const float m = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xF, 0xF, false));  // row_ror:8 = lane ^ 8 in a row of 16
  x = MAX ? fmaxf(x, m) : x + m;
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = MAX ? fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]))
          : __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return MAX ? fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]))
             : __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

constexpr int kDecChunk = 256;  // tokens per work item (bf16)

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_prefix(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  return x;
}

// Chunk count of the rows base + lane (0 past the batch).
__device__ __forceinline__ int row_chunks(const DecArgs& a, int base) {
  const int r = base + (threadIdx.x & 63);
  return r < a.B ? (eff_len(raw_length(a.lengths, a.positions, r), a.cap) + kDecChunk - 1) / kDecChunk
                 : 0;
}

template <int G>
__global__ __launch_bounds__(512) void decode_bf16_kernel(DecArgs a) {
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 3, dl = lane & 7;
  const int wpb = blockDim.x >> 6;  // waves per block
  const int nwaves = gridDim.x * wpb;
  const float c = a.scale_log2;
  const float tau = 8.f / c;
  const bf16* ks = reinterpret_cast<const bf16*>(a.k);
  const bf16* vs = reinterpret_cast<const bf16*>(a.v);
  // The (row, chunk) list is walked without a prefix-sum launch: every wave
  // scans the rows' chunk counts itself (one 64-row block per step).
  int total_chunks = 0;
  for (int base = 0; base < a.B; base += 64) total_chunks += __shfl(wave_prefix(row_chunks(a, base)), 63);
  const int total = uniform(total_chunks) * a.Hkv;

  for (int item = uniform(blockIdx.x * wpb + (threadIdx.x >> 6)); item < total; item += nwaves) {
    const int kvh = item % a.Hkv;
    const int ci = item / a.Hkv;  // chunk item over all rows
    int b = 0, first = 0;         // row of chunk item ci and its first item
    for (int base = 0, carry = 0; base < a.B; base += 64) {
      const int incl = wave_prefix(row_chunks(a, base));
      const int tot = __shfl(incl, 63);
      if (ci < carry + tot) {
        const int k = __popcll(__ballot(carry + incl <= ci));  // rows of the block before ci's
        b = base + k;
        first = carry + (k > 0 ? __shfl(incl, k - 1) : 0);
        break;
      }
      carry += tot;
    }
    b = uniform(b);
    const int chunk = uniform(ci - first);
    const int raw = uniform(raw_length(a.lengths, a.positions, b));
    const bool flat = raw <= 0;  // every slot masked: uniform weights
    const int len = eff_len(raw, a.cap);
    const int t0 = chunk * kDecChunk;
    const int n = min(kDecChunk, len - t0);
    const int last = t0 + n - 1;
    // decode step with an append: slot `slot` reads the new row, and the
    // wave whose chunk holds it writes that row to the cache (no other wave
    // reads the slot)
    const int slot = a.positions ? uniform(min(max(a.positions[b], 0), a.cap - 1)) : -1;

    u32x4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
      qv[g] = ld_u32x4(reinterpret_cast<const bf16*>(a.q) + ((size_t)b * a.Hq + kvh * G + g) * kD + 8 * dl);
    const size_t head_off = (size_t)kvh * kD + 8 * dl;
    const size_t new_off = ((size_t)b * a.Hkv + kvh) * kD + 8 * dl;
    auto row_ptr = [&](const bf16* base, const void* fresh, int t) {
      const int tt = min(t, last);
      return tt == slot ? reinterpret_cast<const bf16*>(fresh) + new_off
                        : base + ((size_t)b * a.cap + tt) * a.Hkv * kD + head_off;
    };
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegInf;
      l[g] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    }
    const int iters = (n + 31) >> 5;
    u32x4 kc[4], vc[4], kn[4], vn[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kc[u] = ld_u32x4(row_ptr(ks, a.k_new, t0 + 8 * u + kg));
      vc[u] = ld_u32x4(row_ptr(vs, a.v_new, t0 + 8 * u + kg));
    }
    for (int it = 0; it < iters; ++it) {
      const int tb = t0 + 32 * it;
      // prefetch the next 32 keys (clamped into the chunk, so always in bounds)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kn[u] = ld_u32x4(row_ptr(ks, a.k_new, tb + 32 + 8 * u + kg));
        vn[u] = ld_u32x4(row_ptr(vs, a.v_new, tb + 32 + 8 * u + kg));
      }
      float s[G][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool valid = tb + 8 * u + kg <= last;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float x = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) x = dot2_bf16(qv[g][j], kc[u][j], x);
          x = group8_sum(x);
          s[g][u] = valid ? (flat ? 0.f : x) : kNegInf;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3]));
        mx = across_groups<true>(mx);
        if (mx > m[g] + tau) {  // wave-uniform
          const float alpha = m[g] == kNegInf ? 0.f : fast_exp2((m[g] - mx) * c);
          m[g] = mx;
          l[g] *= alpha;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
        }
        const float mc = m[g] * c;
        float p[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          p[u] = fast_exp2(fmaf(s[g][u], c, -mc));
          l[g] += p[u];
        }
        // P V: bf16 pairs over keys (u, u + 1)
#pragma unroll
        for (int up = 0; up < 2; ++up) {
          const bf16x2_t pp = {(bf16)p[2 * up], (bf16)p[2 * up + 1]};
          const uint32_t pw = __builtin_bit_cast(uint32_t, pp);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t va = vc[2 * up][j], vb = vc[2 * up + 1][j];
            // (va.lo, vb.lo) and (va.hi, vb.hi)
            const uint32_t lo16 = __builtin_amdgcn_perm(vb, va, 0x05040100u);
            const uint32_t hi16 = __builtin_amdgcn_perm(vb, va, 0x07060302u);
            acc[g][2 * j] = dot2_bf16(pw, lo16, acc[g][2 * j]);
            acc[g][2 * j + 1] = dot2_bf16(pw, hi16, acc[g][2 * j + 1]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kc[u] = kn[u];
        vc[u] = vn[u];
      }
    }
    if (slot >= t0 && slot <= last && kg == 0) {
      const size_t dst = ((size_t)b * a.cap + slot) * a.Hkv * kD + head_off;
      st_u32x4(reinterpret_cast<bf16*>(a.k_cache) + dst,
               ld_u32x4(reinterpret_cast<const bf16*>(a.k_new) + new_off));
      st_u32x4(reinterpret_cast<bf16*>(a.v_cache) + dst,
               ld_u32x4(reinterpret_cast<const bf16*>(a.v_new) + new_off));
    }
    // reduce over the 8 key groups; lanes 0..7 hold the chunk's result
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float lt = across_groups<false>(l[g]);
      const int h = kvh * G + g;
      float* dst = a.partial + (((size_t)b * a.Hq + h) * a.maxc + chunk) * (2 + kD);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o = across_groups<false>(acc[g][i]);
        if (kg == 0) dst[2 + 8 * dl + i] = o;
      }
      if (lane == 0) {
        dst[0] = m[g] * c;
        dst[1] = lt;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 decode over whole token rows: one wave per (row, 128-token chunk)
// item covering every KV head.  A token's K (or V) row -- Hkv heads x 128 B,
// contiguous in the [B, cap, Hkv, 64] cache -- is read by 8 * Hkv lanes with
// one non-temporal 16-byte load each, so a wave streams the chunk's rows as
// one contiguous range (the access pattern that reaches the HBM read
// ceiling on this part, where one wave per (row, chunk, head) reads 8
// separate 128-byte pieces per instruction).  Lane = (token j of the TPL =
// 8 / Hkv tokens a load covers, head h, 8-dim slice dl).  Per token the
// lane's 8 dims of the G query heads of group h are dotted with its K slice
// (v_dot2) and reduced over the 8 lanes of (j, h) with DPP, so every lane of
// the group holds the same score; the online softmax state (max, sum) and
// the P V accumulator of its 8 dims live in the lane.  8 tokens of K and V
// are in flight per lane (16 loads).  Lanes of different j merge their
// states at the end (log-sum-exp), and the (max, sum, acc) of the chunk go
// to the partial buffer the combine kernel reads.
// ---------------------------------------------------------------------------
constexpr int kRowChunk = 128;  // tokens per work item of the row kernel
constexpr int kRowUnroll = 8;   // tokens per lane in flight (K and V)

__device__ __forceinline__ u32x4 ld_nt(const bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// merge two online-softmax states (max in log2 units m2, sum l, acc[8])
template <int G>
__device__ __forceinline__ void merge_lanes(float (&m2)[G], float (&l)[G], float (&acc)[G][8],
                                            int xor_mask) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mo = __shfl_xor(m2[g], xor_mask);
    const float lo = __shfl_xor(l[g], xor_mask);
    const float mn = fmaxf(m2[g], mo);
    // a state with no key yet has max -inf and zero sum/acc: weight 0
    const float wa = m2[g] == kNegInf ? 0.f : fast_exp2(m2[g] - mn);
    const float wb = mo == kNegInf ? 0.f : fast_exp2(mo - mn);
    l[g] = l[g] * wa + lo * wb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ao = __shfl_xor(acc[g][i], xor_mask);
      acc[g][i] = acc[g][i] * wa + ao * wb;
    }
    m2[g] = mn;
  }
}

// Chunk count of rows base + lane for the row kernel (0 past the batch).
__device__ __forceinline__ int row_chunks_c(const DecArgs& a, int base, int chunk) {
  const int r = base + (threadIdx.x & 63);
  return r < a.B ? (eff_len(raw_length(a.lengths, a.positions, r), a.cap) + chunk - 1) / chunk : 0;
}

template <int G, int TPL>
__global__ __launch_bounds__(256) void decode_rows_kernel(DecArgs a) {
  constexpr int kHkv = 8 / TPL;
  const int lane = threadIdx.x & 63;
  const int j = lane / (8 * kHkv);           // token of a load
  const int h = (lane >> 3) % kHkv;          // KV head
  const int dl = lane & 7;                   // 8-dim slice
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  // (row, chunk) of this item: rows' chunk counts scanned 64 rows at a time
  int b = -1, chunk = 0;
  for (int base = 0, carry = 0; base < a.B; base += 64) {
    const int incl = wave_prefix(row_chunks_c(a, base, kRowChunk));
    const int tot = __shfl(incl, 63);
    if (item < carry + tot) {
      const int k = __popcll(__ballot(carry + incl <= item));
      b = base + k;
      chunk = item - carry - (k > 0 ? __shfl(incl, k - 1) : 0);
      break;
    }
    carry += tot;
  }
  b = uniform(b);
  if (b < 0) return;  // past the last item (the grid is sized for full rows)
  chunk = uniform(chunk);
  const float c = a.scale_log2;
  const float tau2 = 8.f;  // lazy rescale threshold, log2 units
  const int raw = uniform(raw_length(a.lengths, a.positions, b));
  const bool flat = raw <= 0;  // every slot masked: uniform weights
  const int len = eff_len(raw, a.cap);
  const int t0 = chunk * kRowChunk;
  const int last = t0 + min(kRowChunk, len - t0) - 1;
  const int slot = a.positions ? uniform(min(max(a.positions[b], 0), a.cap - 1)) : -1;
  const size_t row_elems = (size_t)kHkv * kD;  // one token's row
  const bf16* kbase = reinterpret_cast<const bf16*>(a.k) + (size_t)b * a.cap * row_elems;
  const bf16* vbase = reinterpret_cast<const bf16*>(a.v) + (size_t)b * a.cap * row_elems;
  const size_t lane_off = (size_t)h * kD + 8 * dl;
  const bf16* knew = reinterpret_cast<const bf16*>(a.k_new) + (size_t)b * row_elems + lane_off;
  const bf16* vnew = reinterpret_cast<const bf16*>(a.v_new) + (size_t)b * row_elems + lane_off;

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = ld_u32x4(reinterpret_cast<const bf16*>(a.q) + ((size_t)b * a.Hq + h * G + g) * kD + 8 * dl);
  float m2[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m2[g] = kNegInf;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }
  // this lane's tokens: t0 + j + TPL * u; loads clamp past the chunk's end
  // (always in bounds), and the token at the append slot reads the new row
  constexpr int kStep = TPL * kRowUnroll;  // tokens per iteration over the wave
  for (int tb = t0; tb <= last; tb += kStep) {
    u32x4 kr[kRowUnroll], vr[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int t = min(tb + j + TPL * u, last);
      if (t == slot) {
        kr[u] = ld_u32x4(knew);
        vr[u] = ld_u32x4(vnew);
      } else {
        kr[u] = ld_nt(kbase + (size_t)t * row_elems + lane_off);
        vr[u] = ld_nt(vbase + (size_t)t * row_elems + lane_off);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[kRowUnroll];
      float mx = kNegInf;
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        float x = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) x = dot2_bf16(qv[g][i], kr[u][i], x);
        x = group8_sum(x) * c;  // log2 units
        s[u] = tb + j + TPL * u <= last ? (flat ? 0.f : x) : kNegInf;
        mx = fmaxf(mx, s[u]);
      }
      if (mx > m2[g] + tau2) {
        const float alpha = m2[g] == kNegInf ? 0.f : fast_exp2(m2[g] - mx);
        m2[g] = mx;
        l[g] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
      }
      // a lane that has seen no valid token yet keeps max -inf: shift by 0
      const float shift = m2[g] == kNegInf ? 0.f : m2[g];
      float p[kRowUnroll];
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        p[u] = fast_exp2(s[u] - shift);
        l[g] += p[u];
      }
      // P V: bf16 pairs over tokens (u, u + 1)
#pragma unroll
      for (int up = 0; up < kRowUnroll / 2; ++up) {
        const bf16x2_t pp = {(bf16)p[2 * up], (bf16)p[2 * up + 1]};
        const uint32_t pw = __builtin_bit_cast(uint32_t, pp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t va = vr[2 * up][i], vb = vr[2 * up + 1][i];
          const uint32_t lo16 = __builtin_amdgcn_perm(vb, va, 0x05040100u);
          const uint32_t hi16 = __builtin_amdgcn_perm(vb, va, 0x07060302u);
          acc[g][2 * i] = dot2_bf16(pw, lo16, acc[g][2 * i]);
          acc[g][2 * i + 1] = dot2_bf16(pw, hi16, acc[g][2 * i + 1]);
        }
      }
    }
  }
  if (slot >= t0 && slot <= last && j == 0) {
    // the append: this item's chunk holds the slot; write the new row
    const size_t dst = ((size_t)b * a.cap + slot) * row_elems + lane_off;
    st_u32x4(reinterpret_cast<bf16*>(a.k_cache) + dst, ld_u32x4(knew));
    st_u32x4(reinterpret_cast<bf16*>(a.v_cache) + dst, ld_u32x4(vnew));
  }
  // lanes of different tokens j hold partial states of the same heads
  if constexpr (TPL >= 2) merge_lanes<G>(m2, l, acc, 32);
  if constexpr (TPL >= 4) merge_lanes<G>(m2, l, acc, 16);
  if constexpr (TPL >= 8) merge_lanes<G>(m2, l, acc, 8);
  if (j != 0) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float* dst = a.partial + (((size_t)b * a.Hq + h * G + g) * a.maxc + chunk) * (2 + kD);
    f32x4 lo = {acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
    f32x4 hi = {acc[g][4], acc[g][5], acc[g][6], acc[g][7]};
    *reinterpret_cast<f32x4*>(dst + 2 + 8 * dl) = lo;
    *reinterpret_cast<f32x4*>(dst + 2 + 8 * dl + 4) = hi;
    if (dl == 0) {
      dst[0] = m2[g];
      dst[1] = l[g];
    }
  }
}

// One block of kCombineWaves waves per (row, query head).  Every wave
// combines the chunk maxima and sums lane-parallel over chunks (the same
// values in every wave); wave w then accumulates the weighted partial outputs
// of chunks w, w + kCombineWaves, ... with lane = d, and the waves' sums are
// added in wave order through LDS.  Splitting the chunks over waves shortens
// the chain of dependent loads each lane waits on.
constexpr int kCombineWaves = 4;

template <bool F32>
__global__ __launch_bounds__(64 * kCombineWaves) void decode_combine_kernel(DecArgs a) {
  __shared__ float part[kCombineWaves][kD];
  const int bh = blockIdx.x;
  const int b = bh / a.Hq;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nch = (eff_len(raw_length(a.lengths, a.positions, b), a.cap) + a.chunk - 1) / a.chunk;
  const float* src = a.partial + (size_t)bh * a.maxc * (2 + kD);
  float M = kNegInf;
  for (int ch = lane; ch < nch; ch += 64) M = fmaxf(M, src[ch * (2 + kD)]);
  M = wave_max(M);
  float L = 0.f;
  for (int ch = lane; ch < nch; ch += 64)
    L = fmaf(src[ch * (2 + kD) + 1], fast_exp2(src[ch * (2 + kD)] - M), L);
  L = wave_sum(L);
  float acc = 0.f;
#pragma unroll 4
  for (int ch = wave; ch < nch; ch += kCombineWaves)
    acc = fmaf(src[ch * (2 + kD) + 2 + lane], fast_exp2(src[ch * (2 + kD)] - M), acc);
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kCombineWaves; ++w) total += part[w][lane];
  const float o = total / L;
  if constexpr (!F32) reinterpret_cast<bf16*>(a.out)[(size_t)bh * kD + lane] = (bf16)o;
  else reinterpret_cast<float*>(a.out)[(size_t)bh * kD + lane] = o;
}

// workspace: chunk offsets [B + 1], step lengths [B], partials
size_t decode_workspace_bytes(int batch, int cap, int Hq, int chunk) {
  const int maxc = (cap + chunk - 1) / chunk;
  return align256(sizeof(int) * (size_t)(batch + 1)) + align256(sizeof(int) * (size_t)batch) +
         sizeof(float) * (size_t)batch * Hq * maxc * (2 + kD);
}

// Tokens per partial of the path a call takes: the row kernel (bf16, G and
// Hkv in {1, 2, 4, 8}), the older bf16 streaming kernel (other power-of-two
// G), or the LDS-staged kernels (fp32, other G).
int decode_chunk(bool f32) { return f32 ? 128 : kDecChunk; }

bool decode_rows_path(bool f32, int G, int Hkv) {
  return !f32 && (G == 1 || G == 2 || G == 4 || G == 8) &&
         (Hkv == 1 || Hkv == 2 || Hkv == 4 || Hkv == 8);
}

// workspace bytes that serve every path (the smallest chunk has the most
// partials)
size_t decode_workspace_bytes_any(int batch, int cap, int Hq) {
  return decode_workspace_bytes(batch, cap, Hq, kRowChunk < 128 ? kRowChunk : 128);
}

hipError_t launch_decode(const void* q, const void* k, const void* v, const int32_t* lengths,
                         bool f32, int batch, int cap, int Hq, int Hkv, float scale, void* out,
                         void* workspace, hipStream_t stream, const void* k_new,
                         const void* v_new, const int32_t* positions) {
  DecArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.lengths = lengths;
  a.k_new = k_new;
  a.v_new = v_new;
  a.positions = positions;
  a.k_cache = const_cast<void*>(k);
  a.v_cache = const_cast<void*>(v);
  a.out = out;
  a.B = batch;
  a.cap = cap;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  const bool rows = decode_rows_path(f32, a.G, Hkv);
  a.chunk = rows ? kRowChunk : decode_chunk(f32);
  a.maxc = (cap + a.chunk - 1) / a.chunk;
  a.scale_log2 = scale * kLog2e;
  char* ws = reinterpret_cast<char*>(workspace);
  a.offsets = reinterpret_cast<int*>(ws);
  a.step_lengths = reinterpret_cast<int32_t*>(ws + align256(sizeof(int) * (size_t)(batch + 1)));
  a.partial = reinterpret_cast<float*>(ws + align256(sizeof(int) * (size_t)(batch + 1)) +
                                       align256(sizeof(int) * (size_t)batch));
  // The register-streaming bf16 kernel walks the chunks and appends itself;
  // the LDS-staged kernels (fp32, other head groups) need the prep pass.
  const bool streaming = !f32 && (a.G == 1 || a.G == 2 || a.G == 4 || a.G == 8);
  if (!streaming) {
    if (f32)
      hipLaunchKernelGGL((decode_prep_kernel<4>), dim3(1), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((decode_prep_kernel<2>), dim3(1), dim3(256), 0, stream, a);
    if (positions) a.lengths = a.step_lengths;  // the kernels below attend over positions + 1
  }
  const int upper = batch * a.maxc;
  int gx = (1024 + Hkv - 1) / Hkv;
  if (gx > upper) gx = upper;
  if (gx < 1) gx = 1;
  if (f32) {
    hipLaunchKernelGGL((decode_kernel<true>), dim3(gx, Hkv), dim3(256), 0, stream, a);
    hipLaunchKernelGGL((decode_combine_kernel<true>), dim3(batch * Hq), dim3(64 * kCombineWaves), 0,
                       stream, a);
    return hipGetLastError();
  }
  if (rows) {
    // one wave per (row, chunk) item; the grid covers full rows, waves past
    // the last item exit at once
    const long long waves = (long long)batch * a.maxc;
    const dim3 grid((unsigned)((waves + 3) / 4));
    switch (a.G * 16 + Hkv) {
#define MF_ROWS(GG, HH) \
  case GG * 16 + HH: hipLaunchKernelGGL((decode_rows_kernel<GG, 8 / HH>), grid, dim3(256), 0, stream, a); break;
      MF_ROWS(1, 1) MF_ROWS(1, 2) MF_ROWS(1, 4) MF_ROWS(1, 8)
      MF_ROWS(2, 1) MF_ROWS(2, 2) MF_ROWS(2, 4) MF_ROWS(2, 8)
      MF_ROWS(4, 1) MF_ROWS(4, 2) MF_ROWS(4, 4) MF_ROWS(4, 8)
      MF_ROWS(8, 1) MF_ROWS(8, 2) MF_ROWS(8, 4) MF_ROWS(8, 8)
#undef MF_ROWS
      default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL((decode_combine_kernel<false>), dim3(batch * Hq), dim3(64 * kCombineWaves),
                       0, stream, a);
    return hipGetLastError();
  }
  // bf16: persistent grid of 4-wave blocks over (chunk item, KV head)
  const int items = upper * Hkv;
  int blocks = (items + 3) / 4;
  if (blocks > 2048) blocks = 2048;
  switch (a.G) {
    case 1: hipLaunchKernelGGL((decode_bf16_kernel<1>), dim3(blocks), dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((decode_bf16_kernel<2>), dim3(blocks), dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((decode_bf16_kernel<4>), dim3(blocks), dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((decode_bf16_kernel<8>), dim3(blocks), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((decode_kernel<false>), dim3(gx, Hkv), dim3(256), 0, stream, a); break;
  }
  hipLaunchKernelGGL((decode_combine_kernel<false>), dim3(batch * Hq), dim3(64 * kCombineWaves), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace mf
