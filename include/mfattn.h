/* mfattn: MI355X (gfx950) packed-sequence attention -- C ABI.
 *
 * Plain C declarations: device pointers, sizes, an opaque HIP stream.  No
 * allocation happens inside any entry point; callers pass every buffer,
 * including the plan and workspace whose sizes the *_bytes queries return.
 * Every entry point is stream-ordered on `stream` (a hipStream_t, NULL =
 * default stream) and never synchronises the host.  Every entry point but
 * mf_decode_static keeps no mutable global state, so it is safe to call
 * from several host threads; mf_decode_static keeps its workspace in one
 * library-owned device array per GPU (and a per-device table of its
 * address), so its calls on one GPU race unless ordered on one stream.
 *
 * Status: 0 on success, a negative MF_ERR_* code otherwise; the message of
 * the calling thread's last failure is returned by mf_last_error().
 *
 * Tensor layouts (row-major, last dimension fastest):
 *   query    [B, T, Hq, D]     key/value [B, S, Hkv, D]     (BTHD)
 *   out      [B, T, Hq, D]     lse       [B, Hq, T] fp32 (natural log;
 *                                         +inf for rows with no valid key)
 *   segment_ids [B, T] int32 (0 = padding); mask [B, T] (or [B, S] in
 *   MF_MODE_KEYMASK_BIDIR) int32 or uint8/bool.
 * Query head h reads KV head h / (Hq / Hkv).
 */
#ifndef MFATTN_H
#define MFATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MF_OK 0
#define MF_ERR_INVALID_ARGUMENT (-1) /* null pointer, non-positive size   */
#define MF_ERR_SHAPE (-2)            /* query/KV shapes incompatible      */
#define MF_ERR_HEADS (-3)            /* Hq not divisible by Hkv           */
#define MF_ERR_HEAD_DIM (-4)         /* head_dim other than 64            */
#define MF_ERR_DTYPE (-5)            /* unknown dtype / mask dtype        */
#define MF_ERR_MODE (-6)             /* unknown mask mode                 */
#define MF_ERR_WORKSPACE (-7)        /* plan/workspace smaller than needed */
#define MF_ERR_HIP (-9)              /* a HIP launch failed               */

/* element types of query/key/value/out (and gradients) */
#define MF_DTYPE_F32 0
#define MF_DTYPE_BF16 1

/* mask element types */
#define MF_MASK_I32 0
#define MF_MASK_U8 1

/* mask semantics */
#define MF_MODE_PACKED_CAUSAL 0 /* kernels/attention.py:79-108, :245-261     */
#define MF_MODE_PACKED_BIDIR 1  /* kernels/bidirectional.py:24-31 (with ids) */
#define MF_MODE_KEYMASK_BIDIR 2 /* kernels/bidirectional.py:21-23 (no ids)   */

/* tile classes stored in the plan's tile map */
#define MF_TILE_EMPTY 0
#define MF_TILE_PARTIAL 1
#define MF_TILE_FULL 2

/* tile edge (queries and keys) of the block map */
#define MF_TILE 128

/* Offsets (bytes) of the plan's sections, for callers that inspect it:
 * [0] qid int32 [B][nQ*128]   canonical query ids (segment id; 0 = inactive
 *                             token or padding past the sequence end)
 * [1] kid int32 [B][nK*128]   canonical key ids (same convention)
 * [2] tile map uint8 [B][nQ][nK]
 * [3] q_count int32 [B][nQ]    [4] q_list int32 [B][nQ][2*nK]: the 64-key
 *                              stages s (keys 64s .. 64s+63) a query tile
 *                              attends to, as s*4 + class
 * [5] k_count int32 [B][nK]    [6] k_list int32 [B][nK][2*nQ]: the 64-query
 *                              stages of a key tile, s*4 + class
 * [7] q_order int32 [B*nQ]     [8] k_order int32 [B*nK]: the items b*nQ + qi
 *                              (b*nK + kj) by decreasing list length, the
 *                              attention kernels' launch order
 * [9] run scratch              [10] total size
 * with nQ = ceil(T/128), nK = ceil(S/128). */
void mf_plan_layout(int batch, int q_len, int kv_len, size_t offsets[11]);
size_t mf_plan_bytes(int batch, int q_len, int kv_len);

/* Block-mask builder.  Replaces the dense validity grids of
 * kernels/attention.py:79-108 (_packed_valid_mask) and
 * kernels/bidirectional.py:21-31 with a per-(row, 128-query tile, 128-key
 * tile) EMPTY/PARTIAL/FULL map plus compacted work lists of 64-row stages.
 * segment_ids may be NULL only in MF_MODE_KEYMASK_BIDIR; there `mask` is the
 * [B, kv_len] key mask and q_len may differ from kv_len.  In the packed
 * modes q_len must equal kv_len. */
int mf_block_map(const int32_t* segment_ids, const void* mask, int mask_dtype,
                 int mode, int batch, int q_len, int kv_len, void* plan,
                 size_t plan_bytes, void* stream);

/* The block map built from the packer's placements instead of [B, T] id and
 * mask arrays: `placements` is [count][3] int32 (row, start, length), the
 * i-th placed sequence getting segment id i + 1 and positions
 * 0 .. length-1 -- the PackedRows of batching/packing.py:74-102, whose
 * attention mask is segment_ids != 0.  Placements must not overlap (the
 * packer's guarantee).  Optionally also writes the [B, length] segment ids
 * and positions (either pointer may be NULL).  Modes MF_MODE_PACKED_*. */
int mf_block_map_placements(const int32_t* placements, int count, int mode,
                            int batch, int length, void* plan,
                            size_t plan_bytes, int32_t* segment_ids_out,
                            int32_t* positions_out, void* stream);

/* Forward.  Replaces _dense_attention with its callers
 * dense_packed_causal_attention (kernels/attention.py:245-261, mode 0) and
 * bidirectional.attention (kernels/bidirectional.py:7-35, modes 1 and 2).
 * Rows with no valid key (inactive queries) are written as exact zeros.
 * `scale` multiplies the logits (the reference uses head_dim ** -0.5,
 * attention.py:23-25); it must be finite and positive in every attention
 * and decode entry point (MF_ERR_INVALID_ARGUMENT otherwise).  `plan` must
 * come from mf_block_map with the same batch/q_len/kv_len and the mode the
 * caller intends. */
int mf_attn_fwd(const void* q, const void* k, const void* v, int dtype,
                int batch, int q_len, int kv_len, int q_heads, int kv_heads,
                int head_dim, int mode, float scale, const void* plan,
                size_t plan_bytes, void* out, float* lse, void* stream);

/* Backward of mf_attn_fwd (the JAX-autodiff VJP the reference relies on):
 * dq, dk, dv in the element type of q/k/v; dk/dv summed over each GQA group.
 * `workspace` holds two fp32 values per (batch, head, query) row
 * (mf_attn_bwd_workspace_bytes): -rowsum(dO * O) and lse * log2(e).
 * Deterministic: no atomics, fixed reduction order. */
size_t mf_attn_bwd_workspace_bytes(int batch, int q_len, int q_heads);
int mf_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                const void* dout, const float* lse, int dtype, int batch,
                int q_len, int kv_len, int q_heads, int kv_heads, int head_dim,
                int mode, float scale, const void* plan, size_t plan_bytes,
                void* dq, void* dk, void* dv, void* workspace,
                size_t workspace_bytes, void* stream);

/* The three launches of mf_attn_bwd as separate entry points, for callers
 * that schedule them themselves (e.g. dq and dk/dv on two streams) and for
 * per-kernel timing.  mf_attn_bwd_delta writes the workspace (from O, dO
 * and the forward's lse); mf_attn_bwd_dq and mf_attn_bwd_dkdv read it, so
 * both must be ordered after it.  Arguments mean what they mean in
 * mf_attn_bwd. */
int mf_attn_bwd_delta(const void* out, const void* dout, const float* lse,
                      int dtype, int batch, int q_len, int q_heads,
                      int head_dim, void* workspace, size_t workspace_bytes,
                      void* stream);
int mf_attn_bwd_dq(const void* q, const void* k, const void* v,
                   const void* dout, const float* lse, int dtype, int batch,
                   int q_len, int kv_len, int q_heads, int kv_heads,
                   int head_dim, int mode, float scale, const void* plan,
                   size_t plan_bytes, void* dq, const void* workspace,
                   size_t workspace_bytes, void* stream);
int mf_attn_bwd_dkdv(const void* q, const void* k, const void* v,
                     const void* dout, const float* lse, int dtype, int batch,
                     int q_len, int kv_len, int q_heads, int kv_heads,
                     int head_dim, int mode, float scale, const void* plan,
                     size_t plan_bytes, void* dk, void* dv,
                     const void* workspace, size_t workspace_bytes,
                     void* stream);

/* Ragged KV-cached decode.  Replaces dense_cached_attention
 * (kernels/attention.py:264-282) / cudnn_cached_attention (:366-396): one
 * query token per row attends to cache slots [0, lengths[b]) of a
 * [B, capacity, Hkv, D] cache.  lengths[b] > capacity reads the whole cache;
 * lengths[b] <= 0 reproduces the reference's unguarded result (a uniform
 * average over all `capacity` slots).  Split-K over the cache with a
 * log-sum-exp merge; `workspace` holds the partials. */
size_t mf_decode_workspace_bytes(int batch, int capacity, int q_heads,
                                 int head_dim);
int mf_decode(const void* q, const void* k_cache, const void* v_cache,
              const int32_t* lengths, int dtype, int batch, int capacity,
              int q_heads, int kv_heads, int head_dim, float scale, void* out,
              void* workspace, size_t workspace_bytes, void* stream);

/* Decode step with the ragged KV-cache append: writes row b's new key and
 * value (k_new, v_new: [B, 1, Hkv, 64]) into slot
 * clamp(positions[b], 0, capacity - 1) of k_cache / v_cache IN PLACE, then
 * attends q over positions[b] + 1 slots with mf_decode's semantics (so a
 * position at or past the capacity reads every slot, and a negative one gives
 * the uniform average).  Replaces the scalar
 * `dynamic_update_slice` + `cached_attention(valid_length=position + 1)` of
 * layers/attention.py:309-317 (called from models/lfm2_5/decode.py:249-258)
 * with one slot per row; the append runs in the decode's first launch, so a
 * step costs no extra kernel.  Workspace as mf_decode. */
int mf_decode_append(const void* q, const void* k_new, const void* v_new,
                     const int32_t* positions, int dtype, int batch,
                     int capacity, int q_heads, int kv_heads, int head_dim,
                     float scale, void* k_cache, void* v_cache, void* out,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Attention prologue: RMS-normalise every q and k head over its 64 dims with
 * per-dimension gains (q_gain, k_gain: [64] in the tensor dtype), then apply
 * rotary embeddings at per-token positions ([B, T] int32; NULL means
 * 0 .. T-1 on every row), in one pass.  Replaces the two rms_norm and two
 * apply_rotary calls of layers/attention.py:62-97 (kernels/normalization.py:7-22,
 * kernels/rotary.py:7-39) on the packed path, where positions restart at
 * every segment (layers/attention.py:224-227).  q_out / k_out may alias q /
 * k.  Layout [B, T, H, 64]; eps and rope_theta as the reference's.  With
 * q_heads = 0 and q, q_gain, q_out null only the key half runs (the key
 * operand of mf_attn_fwd_rope_q). */
int mf_qk_norm_rope(const void* q, const void* k, const void* q_gain,
                    const void* k_gain, const int32_t* positions, int dtype,
                    int batch, int seq_len, int q_heads, int kv_heads,
                    int head_dim, float eps, float rope_theta, void* q_out,
                    void* k_out, void* stream);

/* Packed attention forward (mf_attn_fwd) with the query half of
 * mf_qk_norm_rope fused into the kernel's query loads, for callers that
 * need no gradient (prefill, evaluation).  Replaces the composition
 * rms_norm + apply_rotary of q (kernels/normalization.py:7-22,
 * kernels/rotary.py:7-39, as layers/attention.py:62-97 applies them) feeding
 * packed_causal_attention / bidirectional.attention (layers/attention.py:
 * 224-243): q_raw is the query projection [B, T, Hq, 64] before RMS norm
 * and RoPE, q_gain its per-dimension gain in the tensor dtype, positions
 * [B, T] or null as for mf_qk_norm_rope, and k the key after
 * mf_qk_norm_rope (its tiles reach the kernel by DMA, which cannot transform
 * them).  out and lse equal those of mf_qk_norm_rope followed by
 * mf_attn_fwd bit for bit.  bf16 only.  `table` (16-byte aligned,
 * mf_rope_table_bytes(batch, q_len)) receives each token's bf16 cos/sin
 * (a first launch), which the attention launch reads. */
size_t mf_rope_table_bytes(int batch, int q_len);
int mf_attn_fwd_rope_q(const void* q_raw, const void* k, const void* v,
                       const void* q_gain, const int32_t* positions, int dtype,
                       int batch, int q_len, int kv_len, int q_heads,
                       int kv_heads, int head_dim, int mode, float scale,
                       float eps, float rope_theta, const void* plan,
                       size_t plan_bytes, void* table, size_t table_bytes,
                       void* out, float* lse, void* stream);

/* Backward of mf_qk_norm_rope (the VJP JAX autodiff derives for the
 * reference's rms_norm + apply_rotary, kernels/normalization.py:7-22,
 * kernels/rotary.py:7-39, as layers/attention.py:62-97 composes them):
 * given dq_out / dk_out (the gradients of q_out / k_out), writes dq / dk in
 * the tensor dtype and the gain gradients dq_gain / dk_gain ([64] fp32,
 * summed over every token and head in a fixed order: deterministic).  Inputs
 * and positions as for the forward call; dq / dk may alias dq_out / dk_out.
 * `workspace` holds per-workgroup gain partials
 * (mf_qk_norm_rope_bwd_workspace_bytes). */
size_t mf_qk_norm_rope_bwd_workspace_bytes(int batch, int seq_len);
int mf_qk_norm_rope_bwd(const void* q, const void* k, const void* q_gain,
                        const void* k_gain, const int32_t* positions,
                        const void* dq_out, const void* dk_out, int dtype,
                        int batch, int seq_len, int q_heads, int kv_heads,
                        int head_dim, float eps, float rope_theta, void* dq,
                        void* dk, float* dq_gain, float* dk_gain,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Per-token positions from segment ids on the device: the offset of each
 * token inside its run of equal nonzero ids, 0 for padding -- the positions
 * batching/packing.py:92-100 builds on the host for packed rows. */
int mf_segment_positions(const int32_t* segment_ids, int batch, int seq_len,
                         int32_t* positions, void* stream);

/* Segmented short (depthwise) convolution of the packed conv layers, gates
 * fused:  out = c_gate * conv(b_gate * values)  over [B, T, C] (C a multiple
 * of 8), taps [C, kernel_size] (kernel_size <= 8) in the tensor dtype.  A tap
 * at token s contributes to token t only when 0 <= s < T and, with segment
 * ids, segment_ids[s] == segment_ids[t] != 0 -- segment boundaries act as the
 * zero padding of an independently processed sequence.
 *   MF_CONV_CAUSAL:   taps at t-(K-1) .. t  (kernels/convolution.py:25-53)
 *   MF_CONV_CENTERED: taps at t-K/2 .. t+K-1-K/2 (kernels/bidirectional.py:38-58,
 *                     as models/lfm2_5/encoder.py:80-85 calls it)
 * b_gate, c_gate and segment_ids may be NULL (no gate / no segments). */
#define MF_CONV_CAUSAL 0
#define MF_CONV_CENTERED 1
int mf_segmented_conv(const void* b_gate, const void* c_gate, const void* values,
                      const void* taps, const int32_t* segment_ids, int mode,
                      int dtype, int batch, int seq_len, int channels,
                      int kernel_size, void* out, void* stream);

/* Backward of mf_segmented_conv (the VJP JAX autodiff derives for
 * kernels/bidirectional.py:38-58 and kernels/convolution.py:25-53 with the
 * gate products of models/lfm2_5/encoder.py:80-85): given d_out, writes
 * d_values, d_b_gate and d_c_gate in the tensor dtype (each gate gradient
 * only when that gate is given; pass NULL for both or neither) and the tap
 * gradients d_taps ([channels, kernel_size] fp32, summed over rows and tokens
 * in a fixed order: deterministic).  `workspace` holds per-workgroup tap
 * partials (mf_segmented_conv_bwd_workspace_bytes). */
size_t mf_segmented_conv_bwd_workspace_bytes(int batch, int seq_len,
                                             int channels, int kernel_size);
int mf_segmented_conv_bwd(const void* b_gate, const void* c_gate,
                          const void* values, const void* taps,
                          const int32_t* segment_ids, const void* d_out,
                          int mode, int dtype, int batch, int seq_len,
                          int channels, int kernel_size, void* d_b_gate,
                          void* d_c_gate, void* d_values, float* d_taps,
                          void* workspace, size_t workspace_bytes, void* stream);

/* mf_decode without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference.  The same kernels as mf_decode
 * run on a static device array of MF_STATIC_SCRATCH_BYTES that every GPU the
 * library runs on holds until the process ends; calls whose decode workspace
 * (mf_decode_workspace_bytes) exceeds it return MF_ERR_WORKSPACE before
 * anything is enqueued.  Calls that overlap on one GPU share the
 * array and race: order them on one stream.  Nothing is allocated. */
#define MF_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
size_t mf_static_scratch_bytes(void);
int mf_decode_static(const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* lengths, int dtype, int batch, int capacity,
                     int q_heads, int kv_heads, int head_dim, float scale,
                     void* out, void* stream);

/* Message of the calling thread's most recent failure ("" if none). */
const char* mf_last_error(void);

/* Library version string. */
const char* mf_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MFATTN_H */
