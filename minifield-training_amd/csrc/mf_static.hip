// The decode entry point that allocates nothing: mf_decode's kernels with
// their workspace in a file-scope device array instead of a caller buffer,
// for callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).
//
// Every GPU the library runs on holds its own copy of `scratch` (kScratchBytes)
// until the process ends.  Its device address differs per GPU, so it is looked
// up once per device with hipGetSymbolAddress (with that device current) and
// kept; host code passes only that address to the kernels, never the
// array's name (a host-side stand-in).  All calls on one GPU share the array:
// calls that overlap on one GPU (different streams, or different host threads
// without ordering) race on it.  The decode kernels write every scratch word
// they read within a call, so nothing needs clearing between calls.
#include <mutex>

#include "../../include/mfattn.h"
#include "mf_common.h"

namespace mf {
size_t decode_workspace_bytes_any(int batch, int cap, int Hq);
hipError_t launch_decode(const void* q, const void* k, const void* v, const int32_t* lengths,
                         bool f32, int batch, int cap, int Hq, int Hkv, float scale, void* out,
                         void* workspace, hipStream_t stream, const void* k_new,
                         const void* v_new, const int32_t* positions);
int abi_fail(int code, const char* fmt, ...);
int abi_check_hip(hipError_t e, const char* what);
int abi_check_scale(float scale);
int abi_check_decode_shape(int dtype, int batch, int capacity, int q_heads, int kv_heads,
                           int head_dim);
}  // namespace mf

namespace {

constexpr size_t kScratchBytes = MF_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device (null until looked up)

// The address of the current device's `scratch`, looked up on the first call
// on that device.
int device_scratch(void** out) {
  int dev = -1;
  if (int rc = mf::abi_check_hip(hipGetDevice(&dev), "mf_decode_static: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return mf::abi_fail(MF_ERR_INVALID_ARGUMENT, "mf_decode_static: device %d beyond %d", dev,
                        kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (int rc = mf::abi_check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                                   "mf_decode_static: hipGetSymbolAddress(scratch)"))
      return rc;
    if (!ptr)
      return mf::abi_fail(MF_ERR_HIP, "mf_decode_static: no device address for the scratch array");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MF_OK;
}

}  // namespace

extern "C" {

size_t mf_static_scratch_bytes(void) { return kScratchBytes; }

int mf_decode_static(const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* lengths, int dtype, int batch, int capacity, int q_heads,
                     int kv_heads, int head_dim, float scale, void* out, void* stream) {
  if (int rc = mf::abi_check_decode_shape(dtype, batch, capacity, q_heads, kv_heads, head_dim))
    return rc;
  if (int rc = mf::abi_check_scale(scale)) return rc;
  const bool f32 = dtype == MF_DTYPE_F32;
  const size_t need = mf::decode_workspace_bytes_any(batch, capacity, q_heads);
  if (need > kScratchBytes)
    return mf::abi_fail(MF_ERR_WORKSPACE,
                        "mf_decode_static needs %zu bytes of scratch; the static array holds %zu "
                        "(use mf_decode with a workspace)",
                        need, kScratchBytes);
  if (!q || !k_cache || !v_cache || !lengths || !out)
    return mf::abi_fail(MF_ERR_INVALID_ARGUMENT, "every tensor pointer must be non-null");
  void* ws = nullptr;
  if (int rc = device_scratch(&ws)) return rc;
  return mf::abi_check_hip(mf::launch_decode(q, k_cache, v_cache, lengths, f32, batch, capacity,
                                             q_heads, kv_heads, scale, out, ws,
                                             static_cast<hipStream_t>(stream), nullptr, nullptr,
                                             nullptr),
                           "mf_decode_static launch");
}

}  // extern "C"
