// C ABI of the mfattn library: argument validation, error reporting and the
// launches.  Every check here runs on the host before anything is enqueued,
// so a malformed call returns an MF_ERR_* code (and leaves a message for
// mf_last_error) without touching the GPU.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/mfattn.h"
#include "mf_common.h"

namespace mf {
hipError_t launch_block_map(const int32_t* seg, const void* mask, int mask_u8, int mode, int batch,
                            int q_len, int kv_len, void* plan, hipStream_t stream);
hipError_t launch_attn_fwd(const void* q, const void* k, const void* v, bool f32, int batch, int T,
                           int S, int Hq, int Hkv, int mode, float scale, const void* plan,
                           void* out, float* lse, hipStream_t stream);
hipError_t launch_attn_fwd_rope_q(const void* q_raw, const void* k, const void* v,
                                  const void* q_gain, const int32_t* positions, int batch, int T,
                                  int S, int Hq, int Hkv, int mode, float scale, float eps,
                                  float theta, const void* plan, void* table, void* out,
                                  float* lse, hipStream_t stream);
size_t rope_table_bytes(int B, int T);
hipError_t launch_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                           const void* dout, const float* lse, bool f32, int batch, int T, int S,
                           int Hq, int Hkv, int mode, float scale, const void* plan, void* dq,
                           void* dk, void* dv, float* workspace, int phases, hipStream_t stream);
size_t decode_workspace_bytes(int batch, int cap, int Hq, int chunk);
size_t decode_workspace_bytes_any(int batch, int cap, int Hq);
int decode_chunk(bool f32);
hipError_t launch_decode(const void* q, const void* k, const void* v, const int32_t* lengths,
                         bool f32, int batch, int cap, int Hq, int Hkv, float scale, void* out,
                         void* workspace, hipStream_t stream, const void* k_new = nullptr,
                         const void* v_new = nullptr, const int32_t* positions = nullptr);
hipError_t launch_qk_norm_rope(const void* q, const void* k, const void* q_gain,
                               const void* k_gain, const int32_t* positions, bool f32, int B,
                               int T, int Hq, int Hkv, float eps, float theta, void* q_out,
                               void* k_out, hipStream_t stream);
size_t rope_bwd_workspace_bytes(int B, int T);
hipError_t launch_qk_norm_rope_bwd(const void* q, const void* k, const void* q_gain,
                                   const void* k_gain, const int32_t* positions,
                                   const void* dq_out, const void* dk_out, bool f32, int B, int T,
                                   int Hq, int Hkv, float eps, float theta, void* dq, void* dk,
                                   float* dq_gain, float* dk_gain, void* workspace,
                                   hipStream_t stream);
hipError_t launch_segment_positions(const int32_t* seg, int B, int T, int32_t* pos,
                                    hipStream_t stream);
hipError_t launch_block_map_placements(const int32_t* placements, int count, int mode, int batch,
                                       int length, void* plan, int32_t* seg_out, int32_t* pos_out,
                                       hipStream_t stream);
hipError_t launch_segmented_conv(const void* b, const void* c, const void* v, const void* w,
                                 const int32_t* seg, bool centered, bool f32, int B, int T, int C,
                                 int K, void* out, hipStream_t stream);
size_t conv_bwd_workspace_bytes(int B, int T, int C, int K);
hipError_t launch_segmented_conv_bwd(const void* b, const void* c, const void* v, const void* w,
                                     const int32_t* seg, const void* g, bool centered, bool f32,
                                     int B, int T, int C, int K, void* db, void* dc, void* dv,
                                     float* dw, void* workspace, hipStream_t stream);
}  // namespace mf

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return MF_OK;
}

int check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

int check_mode(int mode) {
  if (mode != MF_MODE_PACKED_CAUSAL && mode != MF_MODE_PACKED_BIDIR && mode != MF_MODE_KEYMASK_BIDIR)
    return fail(MF_ERR_MODE, "Unknown mask mode %d", mode);
  return MF_OK;
}

// The logit scale: finite and positive (the reference scales by
// head_dim ** -0.5, attention.py:23-25).  The forward takes each query's
// running maximum on the raw scores and scales it once, which relies on it.
int check_scale(float scale) {
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(MF_ERR_INVALID_ARGUMENT, "scale must be finite and positive (got %g)", (double)scale);
  return MF_OK;
}

// Shape checks shared by forward and backward.
int check_attn(int dtype, int batch, int q_len, int kv_len, int q_heads, int kv_heads,
               int head_dim, int mode, size_t plan_bytes) {
  if (dtype != MF_DTYPE_F32 && dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_DTYPE, "Unsupported dtype code %d", dtype);
  if (int rc = check_mode(mode)) return rc;
  if (batch < 1 || q_len < 1 || kv_len < 1 || q_heads < 1 || kv_heads < 1)
    return fail(MF_ERR_INVALID_ARGUMENT,
                "Sizes must be positive (batch=%d q_len=%d kv_len=%d q_heads=%d kv_heads=%d)",
                batch, q_len, kv_len, q_heads, kv_heads);
  if (mode != MF_MODE_KEYMASK_BIDIR && q_len != kv_len)
    return fail(MF_ERR_SHAPE, "Packed attention query/KV shapes are incompatible");
  if (q_heads % kv_heads) return fail(MF_ERR_HEADS, "Query heads must be divisible by KV heads");
  if (head_dim != mf::kD)
    return fail(MF_ERR_HEAD_DIM, "head_dim %d is not supported (kernels serve head_dim 64)", head_dim);
  // the bf16 kernels address one batch row of q/dO and of k/v with 32-bit
  // byte offsets (fp32 rows are twice as long; both are checked)
  if ((size_t)q_len * q_heads * head_dim * 4 >= (size_t(1) << 32) ||
      (size_t)kv_len * kv_heads * head_dim * 4 >= (size_t(1) << 32))
    return fail(MF_ERR_SHAPE, "A batch row of q or k/v exceeds 4 GiB (q_len=%d kv_len=%d)", q_len,
                kv_len);
  const size_t need = mf::plan_layout(batch, q_len, kv_len).total;
  if (plan_bytes < need)
    return fail(MF_ERR_WORKSPACE, "plan holds %zu bytes, %zu needed", plan_bytes, need);
  return MF_OK;
}

}  // namespace


extern "C" {

void mf_plan_layout(int batch, int q_len, int kv_len, size_t offsets[11]) {
  const mf::PlanLayout p = mf::plan_layout(batch, q_len, kv_len);
  offsets[0] = p.qid;
  offsets[1] = p.kid;
  offsets[2] = p.tmap;
  offsets[3] = p.qcnt;
  offsets[4] = p.qlist;
  offsets[5] = p.kcnt;
  offsets[6] = p.klist;
  offsets[7] = p.qorder;
  offsets[8] = p.korder;
  offsets[9] = p.runs;
  offsets[10] = p.total;
}

size_t mf_plan_bytes(int batch, int q_len, int kv_len) {
  if (batch < 1 || q_len < 1 || kv_len < 1) return 0;
  return mf::plan_layout(batch, q_len, kv_len).total;
}

int mf_block_map(const int32_t* segment_ids, const void* mask, int mask_dtype, int mode, int batch,
                 int q_len, int kv_len, void* plan, size_t plan_bytes, void* stream) {
  if (int rc = check_mode(mode)) return rc;
  if (mask_dtype != MF_MASK_I32 && mask_dtype != MF_MASK_U8)
    return fail(MF_ERR_DTYPE, "Unsupported mask dtype code %d", mask_dtype);
  if (batch < 1 || q_len < 1 || kv_len < 1)
    return fail(MF_ERR_INVALID_ARGUMENT, "Sizes must be positive (batch=%d q_len=%d kv_len=%d)",
                batch, q_len, kv_len);
  if (mode != MF_MODE_KEYMASK_BIDIR) {
    if (q_len != kv_len)
      return fail(MF_ERR_SHAPE, "Packed attention query/KV shapes are incompatible");
    if (!segment_ids) return fail(MF_ERR_INVALID_ARGUMENT, "segment_ids is required in packed modes");
  }
  if (!mask || !plan) return fail(MF_ERR_INVALID_ARGUMENT, "mask and plan must be non-null");
  const size_t need = mf::plan_layout(batch, q_len, kv_len).total;
  if (plan_bytes < need)
    return fail(MF_ERR_WORKSPACE, "plan holds %zu bytes, %zu needed", plan_bytes, need);
  return check_hip(mf::launch_block_map(segment_ids, mask, mask_dtype == MF_MASK_U8, mode, batch,
                                        q_len, kv_len, plan, static_cast<hipStream_t>(stream)),
                   "mf_block_map launch");
}

int mf_block_map_placements(const int32_t* placements, int count, int mode, int batch,
                            int length, void* plan, size_t plan_bytes, int32_t* segment_ids_out,
                            int32_t* positions_out, void* stream) {
  if (mode != MF_MODE_PACKED_CAUSAL && mode != MF_MODE_PACKED_BIDIR)
    return fail(MF_ERR_MODE, "placements describe packed rows (mode %d or %d), got %d",
                MF_MODE_PACKED_CAUSAL, MF_MODE_PACKED_BIDIR, mode);
  if (batch < 1 || length < 1 || count < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "Sizes must be positive (batch=%d length=%d count=%d)",
                batch, length, count);
  if ((count > 0 && !placements) || !plan)
    return fail(MF_ERR_INVALID_ARGUMENT, "placements and plan must be non-null");
  const size_t need = mf::plan_layout(batch, length, length).total;
  if (plan_bytes < need)
    return fail(MF_ERR_WORKSPACE, "plan holds %zu bytes, %zu needed", plan_bytes, need);
  return check_hip(mf::launch_block_map_placements(placements, count, mode, batch, length, plan,
                                                   segment_ids_out, positions_out,
                                                   static_cast<hipStream_t>(stream)),
                   "mf_block_map_placements launch");
}

int mf_attn_fwd(const void* q, const void* k, const void* v, int dtype, int batch, int q_len,
                int kv_len, int q_heads, int kv_heads, int head_dim, int mode, float scale,
                const void* plan, size_t plan_bytes, void* out, float* lse, void* stream) {
  if (int rc = check_attn(dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, mode, plan_bytes))
    return rc;
  if (int rc = check_scale(scale)) return rc;
  if (!q || !k || !v || !plan || !out || !lse)
    return fail(MF_ERR_INVALID_ARGUMENT, "q, k, v, plan, out and lse must be non-null");
  return check_hip(mf::launch_attn_fwd(q, k, v, dtype == MF_DTYPE_F32, batch, q_len, kv_len,
                                       q_heads, kv_heads, mode, scale, plan, out, lse,
                                       static_cast<hipStream_t>(stream)),
                   "mf_attn_fwd launch");
}

size_t mf_attn_bwd_workspace_bytes(int batch, int q_len, int q_heads) {
  if (batch < 1 || q_len < 1 || q_heads < 1) return 0;
  return 2 * sizeof(float) * (size_t)batch * q_len * q_heads;  // -D and lse2 per row
}

namespace {

// Shared validation + launch of the backward phases (1 delta, 2 dq, 4 dkdv).
int attn_bwd_phases(const void* q, const void* k, const void* v, const void* out,
                    const void* dout, const float* lse, int dtype, int batch, int q_len,
                    int kv_len, int q_heads, int kv_heads, int head_dim, int mode, float scale,
                    const void* plan, size_t plan_bytes, void* dq, void* dk, void* dv,
                    void* workspace, size_t workspace_bytes, int phases, void* stream,
                    const char* what) {
  if (int rc = check_attn(dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, mode, plan_bytes))
    return rc;
  if (int rc = check_scale(scale)) return rc;
  const bool need_qkv = phases & 6;
  if ((need_qkv && (!q || !k || !v || !plan)) || !lse || !dout || !workspace ||
      ((phases & 1) && !out) || ((phases & 2) && !dq) || ((phases & 4) && (!dk || !dv)))
    return fail(MF_ERR_INVALID_ARGUMENT, "%s: a required tensor pointer or the workspace is null",
                what);
  const size_t need = mf_attn_bwd_workspace_bytes(batch, q_len, q_heads);
  if (workspace_bytes < need)
    return fail(MF_ERR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  return check_hip(mf::launch_attn_bwd(q, k, v, out, dout, lse, dtype == MF_DTYPE_F32, batch, q_len,
                                       kv_len, q_heads, kv_heads, mode, scale, plan, dq, dk, dv,
                                       static_cast<float*>(workspace), phases,
                                       static_cast<hipStream_t>(stream)),
                   what);
}

}  // namespace

int mf_attn_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                const float* lse, int dtype, int batch, int q_len, int kv_len, int q_heads,
                int kv_heads, int head_dim, int mode, float scale, const void* plan,
                size_t plan_bytes, void* dq, void* dk, void* dv, void* workspace,
                size_t workspace_bytes, void* stream) {
  return attn_bwd_phases(q, k, v, out, dout, lse, dtype, batch, q_len, kv_len, q_heads, kv_heads,
                         head_dim, mode, scale, plan, plan_bytes, dq, dk, dv, workspace,
                         workspace_bytes, 7, stream, "mf_attn_bwd launch");
}

int mf_attn_bwd_delta(const void* out, const void* dout, const float* lse, int dtype, int batch,
                      int q_len, int q_heads, int head_dim, void* workspace,
                      size_t workspace_bytes, void* stream) {
  // the delta phase reads no plan; validate it against a minimal one
  return attn_bwd_phases(nullptr, nullptr, nullptr, out, dout, lse, dtype, batch, q_len, q_len,
                         q_heads, 1, head_dim, MF_MODE_PACKED_BIDIR, 1.f, nullptr,
                         mf::plan_layout(batch, q_len, q_len).total, nullptr, nullptr, nullptr,
                         workspace, workspace_bytes, 1, stream, "mf_attn_bwd_delta launch");
}

int mf_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                   const float* lse, int dtype, int batch, int q_len, int kv_len, int q_heads,
                   int kv_heads, int head_dim, int mode, float scale, const void* plan,
                   size_t plan_bytes, void* dq, const void* workspace, size_t workspace_bytes,
                   void* stream) {
  return attn_bwd_phases(q, k, v, nullptr, dout, lse, dtype, batch, q_len, kv_len, q_heads,
                         kv_heads, head_dim, mode, scale, plan, plan_bytes, dq, nullptr, nullptr,
                         const_cast<void*>(workspace), workspace_bytes, 2, stream,
                         "mf_attn_bwd_dq launch");
}

int mf_attn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, int dtype, int batch, int q_len, int kv_len, int q_heads,
                     int kv_heads, int head_dim, int mode, float scale, const void* plan,
                     size_t plan_bytes, void* dk, void* dv, const void* workspace,
                     size_t workspace_bytes, void* stream) {
  return attn_bwd_phases(q, k, v, nullptr, dout, lse, dtype, batch, q_len, kv_len, q_heads,
                         kv_heads, head_dim, mode, scale, plan, plan_bytes, nullptr, dk, dv,
                         const_cast<void*>(workspace), workspace_bytes, 4, stream,
                         "mf_attn_bwd_dkdv launch");
}

size_t mf_decode_workspace_bytes(int batch, int capacity, int q_heads, int head_dim) {
  if (batch < 1 || capacity < 1 || q_heads < 1 || head_dim != mf::kD) return 0;
  return mf::decode_workspace_bytes_any(batch, capacity, q_heads);
}

namespace {

int check_decode_shape(int dtype, int batch, int capacity, int q_heads, int kv_heads,
                       int head_dim) {
  if (dtype != MF_DTYPE_F32 && dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_DTYPE, "Unsupported dtype code %d", dtype);
  if (batch < 1 || capacity < 1 || q_heads < 1 || kv_heads < 1)
    return fail(MF_ERR_INVALID_ARGUMENT,
                "Sizes must be positive (batch=%d capacity=%d q_heads=%d kv_heads=%d)", batch,
                capacity, q_heads, kv_heads);
  if (head_dim != mf::kD)
    return fail(MF_ERR_SHAPE, "Cached attention query/KV shapes are incompatible");
  if (q_heads % kv_heads) return fail(MF_ERR_HEADS, "Query heads must be divisible by KV heads");
  return MF_OK;
}

int check_decode(int dtype, int batch, int capacity, int q_heads, int kv_heads, int head_dim,
                 size_t workspace_bytes) {
  if (int rc = check_decode_shape(dtype, batch, capacity, q_heads, kv_heads, head_dim)) return rc;
  const size_t need = mf_decode_workspace_bytes(batch, capacity, q_heads, head_dim);
  if (workspace_bytes < need)
    return fail(MF_ERR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  return MF_OK;
}

}  // namespace

int mf_decode_append(const void* q, const void* k_new, const void* v_new,
                     const int32_t* positions, int dtype, int batch, int capacity, int q_heads,
                     int kv_heads, int head_dim, float scale, void* k_cache, void* v_cache,
                     void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k_new || !v_new || !positions || !k_cache || !v_cache || !out || !workspace)
    return fail(MF_ERR_INVALID_ARGUMENT, "every tensor pointer and the workspace must be non-null");
  if (int rc = check_decode(dtype, batch, capacity, q_heads, kv_heads, head_dim, workspace_bytes))
    return rc;
  if (int rc = check_scale(scale)) return rc;
  return check_hip(mf::launch_decode(q, k_cache, v_cache, nullptr, dtype == MF_DTYPE_F32, batch,
                                     capacity, q_heads, kv_heads, scale, out, workspace,
                                     static_cast<hipStream_t>(stream), k_new, v_new, positions),
                   "mf_decode_append launch");
}

int mf_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* lengths,
              int dtype, int batch, int capacity, int q_heads, int kv_heads, int head_dim,
              float scale, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_decode_shape(dtype, batch, capacity, q_heads, kv_heads, head_dim)) return rc;
  if (!q || !k_cache || !v_cache || !lengths || !out || !workspace)
    return fail(MF_ERR_INVALID_ARGUMENT, "every tensor pointer and the workspace must be non-null");
  if (int rc = check_decode(dtype, batch, capacity, q_heads, kv_heads, head_dim, workspace_bytes))
    return rc;
  if (int rc = check_scale(scale)) return rc;
  return check_hip(mf::launch_decode(q, k_cache, v_cache, lengths, dtype == MF_DTYPE_F32, batch,
                                     capacity, q_heads, kv_heads, scale, out, workspace,
                                     static_cast<hipStream_t>(stream)),
                   "mf_decode launch");
}

namespace {

int check_rope(int dtype, int batch, int seq_len, int q_heads, int kv_heads, int head_dim,
               float rope_theta) {
  if (dtype != MF_DTYPE_F32 && dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_DTYPE, "Unsupported dtype code %d", dtype);
  if (batch < 1 || seq_len < 1 || q_heads < 1 || kv_heads < 1)
    return fail(MF_ERR_INVALID_ARGUMENT,
                "Sizes must be positive (batch=%d seq_len=%d q_heads=%d kv_heads=%d)", batch,
                seq_len, q_heads, kv_heads);
  if (head_dim != mf::kD)
    return fail(MF_ERR_HEAD_DIM, "head_dim must be %d (got %d)", mf::kD, head_dim);
  if (!(rope_theta > 0.f)) return fail(MF_ERR_INVALID_ARGUMENT, "rope_theta must be positive");
  return MF_OK;
}

}  // namespace

int mf_qk_norm_rope(const void* q, const void* k, const void* q_gain, const void* k_gain,
                    const int32_t* positions, int dtype, int batch, int seq_len, int q_heads,
                    int kv_heads, int head_dim, float eps, float rope_theta, void* q_out,
                    void* k_out, void* stream) {
  // q_heads == 0 with null q, q_gain and q_out: the key half only
  const bool keys_only = q_heads == 0 && !q && !q_gain && !q_out;
  if (int rc = check_rope(dtype, batch, seq_len, keys_only ? 1 : q_heads, kv_heads, head_dim,
                          rope_theta))
    return rc;
  if ((!keys_only && (!q || !q_gain || !q_out)) || !k || !k_gain || !k_out)
    return fail(MF_ERR_INVALID_ARGUMENT, "a required tensor pointer is null");
  return check_hip(mf::launch_qk_norm_rope(q, k, q_gain, k_gain, positions, dtype == MF_DTYPE_F32,
                                           batch, seq_len, q_heads, kv_heads, eps, rope_theta,
                                           q_out, k_out, static_cast<hipStream_t>(stream)),
                   "mf_qk_norm_rope launch");
}

size_t mf_rope_table_bytes(int batch, int q_len) {
  if (batch < 1 || q_len < 1) return 0;
  return mf::rope_table_bytes(batch, q_len);
}

int mf_attn_fwd_rope_q(const void* q_raw, const void* k, const void* v, const void* q_gain,
                       const int32_t* positions, int dtype, int batch, int q_len, int kv_len,
                       int q_heads, int kv_heads, int head_dim, int mode, float scale, float eps,
                       float rope_theta, const void* plan, size_t plan_bytes, void* table,
                       size_t table_bytes, void* out, float* lse, void* stream) {
  if (int rc = check_attn(dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, mode, plan_bytes))
    return rc;
  if (int rc = check_rope(dtype, batch, q_len, q_heads, kv_heads, head_dim, rope_theta)) return rc;
  if (int rc = check_scale(scale)) return rc;
  if (dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_DTYPE, "mf_attn_fwd_rope_q serves bf16 tensors (dtype code %d)", dtype);
  if (!q_raw || !k || !v || !q_gain || !plan || !table || !out || !lse)
    return fail(MF_ERR_INVALID_ARGUMENT, "q_raw, k, v, q_gain, plan, table, out and lse must be non-null");
  const size_t need = mf_rope_table_bytes(batch, q_len);
  if (table_bytes < need)
    return fail(MF_ERR_WORKSPACE, "table holds %zu bytes, %zu needed", table_bytes, need);
  if (reinterpret_cast<uintptr_t>(table) % 16)
    return fail(MF_ERR_INVALID_ARGUMENT, "table must be 16-byte aligned");
  return check_hip(mf::launch_attn_fwd_rope_q(q_raw, k, v, q_gain, positions, batch, q_len, kv_len,
                                              q_heads, kv_heads, mode, scale, eps, rope_theta,
                                              plan, table, out, lse,
                                              static_cast<hipStream_t>(stream)),
                   "mf_attn_fwd_rope_q launch");
}

size_t mf_qk_norm_rope_bwd_workspace_bytes(int batch, int seq_len) {
  if (batch < 1 || seq_len < 1) return 0;
  return mf::rope_bwd_workspace_bytes(batch, seq_len);
}

int mf_qk_norm_rope_bwd(const void* q, const void* k, const void* q_gain, const void* k_gain,
                        const int32_t* positions, const void* dq_out, const void* dk_out,
                        int dtype, int batch, int seq_len, int q_heads, int kv_heads,
                        int head_dim, float eps, float rope_theta, void* dq, void* dk,
                        float* dq_gain, float* dk_gain, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (int rc = check_rope(dtype, batch, seq_len, q_heads, kv_heads, head_dim, rope_theta))
    return rc;
  if (!q || !k || !q_gain || !k_gain || !dq_out || !dk_out || !dq || !dk || !dq_gain ||
      !dk_gain || !workspace)
    return fail(MF_ERR_INVALID_ARGUMENT, "a required tensor pointer or the workspace is null");
  const size_t need = mf_qk_norm_rope_bwd_workspace_bytes(batch, seq_len);
  if (workspace_bytes < need)
    return fail(MF_ERR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  return check_hip(mf::launch_qk_norm_rope_bwd(q, k, q_gain, k_gain, positions, dq_out, dk_out,
                                               dtype == MF_DTYPE_F32, batch, seq_len, q_heads,
                                               kv_heads, eps, rope_theta, dq, dk, dq_gain,
                                               dk_gain, workspace,
                                               static_cast<hipStream_t>(stream)),
                   "mf_qk_norm_rope_bwd launch");
}

int mf_segment_positions(const int32_t* segment_ids, int batch, int seq_len, int32_t* positions,
                         void* stream) {
  if (batch < 1 || seq_len < 1)
    return fail(MF_ERR_INVALID_ARGUMENT, "Sizes must be positive (batch=%d seq_len=%d)", batch,
                seq_len);
  if (!segment_ids || !positions)
    return fail(MF_ERR_INVALID_ARGUMENT, "segment_ids and positions must be non-null");
  return check_hip(mf::launch_segment_positions(segment_ids, batch, seq_len, positions,
                                                static_cast<hipStream_t>(stream)),
                   "mf_segment_positions launch");
}

namespace {

int check_conv(int mode, int dtype, int batch, int seq_len, int channels, int kernel_size) {
  if (dtype != MF_DTYPE_F32 && dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_DTYPE, "Unsupported dtype code %d", dtype);
  if (mode != MF_CONV_CAUSAL && mode != MF_CONV_CENTERED)
    return fail(MF_ERR_MODE, "Unsupported convolution mode %d", mode);
  if (batch < 1 || seq_len < 1 || channels < 1)
    return fail(MF_ERR_INVALID_ARGUMENT, "Sizes must be positive (batch=%d seq_len=%d channels=%d)",
                batch, seq_len, channels);
  if (channels % 8)
    return fail(MF_ERR_SHAPE, "channels must be a multiple of 8 (got %d)", channels);
  if (kernel_size < 1 || kernel_size > 8)
    return fail(MF_ERR_SHAPE, "kernel_size must be in [1, 8] (got %d)", kernel_size);
  return MF_OK;
}

}  // namespace

int mf_segmented_conv(const void* b_gate, const void* c_gate, const void* values,
                      const void* taps, const int32_t* segment_ids, int mode, int dtype,
                      int batch, int seq_len, int channels, int kernel_size, void* out,
                      void* stream) {
  if (int rc = check_conv(mode, dtype, batch, seq_len, channels, kernel_size)) return rc;
  if (!values || !taps || !out)
    return fail(MF_ERR_INVALID_ARGUMENT, "values, taps and out must be non-null");
  return check_hip(mf::launch_segmented_conv(b_gate, c_gate, values, taps, segment_ids,
                                             mode == MF_CONV_CENTERED, dtype == MF_DTYPE_F32,
                                             batch, seq_len, channels, kernel_size, out,
                                             static_cast<hipStream_t>(stream)),
                   "mf_segmented_conv launch");
}

size_t mf_segmented_conv_bwd_workspace_bytes(int batch, int seq_len, int channels,
                                             int kernel_size) {
  if (batch < 1 || seq_len < 1 || channels < 1 || kernel_size < 1) return 0;
  return mf::conv_bwd_workspace_bytes(batch, seq_len, channels, kernel_size);
}

int mf_segmented_conv_bwd(const void* b_gate, const void* c_gate, const void* values,
                          const void* taps, const int32_t* segment_ids, const void* d_out,
                          int mode, int dtype, int batch, int seq_len, int channels,
                          int kernel_size, void* d_b_gate, void* d_c_gate, void* d_values,
                          float* d_taps, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_conv(mode, dtype, batch, seq_len, channels, kernel_size)) return rc;
  if (!values || !taps || !d_out || !d_values || !d_taps || !workspace)
    return fail(MF_ERR_INVALID_ARGUMENT,
                "values, taps, d_out, d_values, d_taps and the workspace must be non-null");
  if ((b_gate == nullptr) != (d_b_gate == nullptr) || (c_gate == nullptr) != (d_c_gate == nullptr))
    return fail(MF_ERR_INVALID_ARGUMENT,
                "a gate and its gradient must both be given or both be null");
  const size_t need = mf_segmented_conv_bwd_workspace_bytes(batch, seq_len, channels, kernel_size);
  if (workspace_bytes < need)
    return fail(MF_ERR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  return check_hip(mf::launch_segmented_conv_bwd(b_gate, c_gate, values, taps, segment_ids, d_out,
                                                 mode == MF_CONV_CENTERED, dtype == MF_DTYPE_F32,
                                                 batch, seq_len, channels, kernel_size, d_b_gate,
                                                 d_c_gate, d_values, d_taps, workspace,
                                                 static_cast<hipStream_t>(stream)),
                   "mf_segmented_conv_bwd launch");
}

const char* mf_last_error(void) { return g_last_error.c_str(); }

const char* mf_version(void) { return "mfattn 0.1.0 (gfx950)"; }

}  // extern "C"

// Validation and error reporting shared with the other C-ABI source files.
namespace mf {

int abi_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int abi_check_hip(hipError_t e, const char* what) { return check_hip(e, what); }

int abi_check_scale(float scale) { return check_scale(scale); }

int abi_check_decode_shape(int dtype, int batch, int capacity, int q_heads, int kv_heads,
                           int head_dim) {
  return check_decode_shape(dtype, batch, capacity, q_heads, kv_heads, head_dim);
}

}  // namespace mf
