"""Host-side argument checks of the Python binding (no GPU needed).

Every check here raises before a tensor's device is looked at, so malformed
calls are rejected before anything is enqueued: mixed dtypes (the kernels
index every operand with one element size), mismatched mask / id / batch
shapes (the block map reads B x S mask entries and B x T ids, and the plan is
indexed with the query's batch), and plans built for another call.
"""

import pytest
import torch

from mfattn import ops
from mfattn.kernels import attention, bidirectional


def _qkv(b=2, t=8, s=None, hq=4, hkv=2, dtype=torch.bfloat16):
    s = t if s is None else s
    return (torch.zeros(b, t, hq, 64, dtype=dtype), torch.zeros(b, s, hkv, 64, dtype=dtype),
            torch.zeros(b, s, hkv, 64, dtype=dtype))


def test_decode_rejects_mixed_dtypes_before_any_launch():
    q = torch.zeros(2, 1, 4, 64, dtype=torch.float32)
    kc = torch.zeros(2, 16, 2, 64, dtype=torch.bfloat16)
    lengths = torch.tensor([3, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="share one dtype"):
        ops.decode(q, kc, kc.clone(), lengths, 0.125)
    kn = torch.zeros(2, 1, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="share one dtype"):
        ops.decode_append(q, kn, kn.clone(), kc, kc.clone(), lengths, 0.125)
    with pytest.raises(ValueError, match="share one dtype"):
        attention.cached_attention_step(q, kn, kn.clone(), kc, kc.clone(), 3)


def test_decode_rejects_bad_shapes_and_lengths():
    q = torch.zeros(2, 1, 4, 64)
    kc = torch.zeros(2, 16, 2, 64)
    with pytest.raises(ValueError, match="Cached attention query/KV shapes are incompatible"):
        ops.decode(q, kc, torch.zeros(2, 15, 2, 64), torch.tensor([3, 4], dtype=torch.int32), 1.0)
    with pytest.raises(ValueError, match="Cached attention query/KV shapes are incompatible"):
        ops.decode(torch.zeros(3, 1, 4, 64), kc, kc.clone(), torch.tensor([3, 4, 5], dtype=torch.int32), 1.0)
    with pytest.raises(ValueError, match="int32"):
        ops.decode(q, kc, kc.clone(), torch.tensor([3, 4], dtype=torch.int64), 1.0)
    with pytest.raises(ValueError, match="int32"):
        ops.decode(q, kc, kc.clone(), torch.tensor([3], dtype=torch.int32), 1.0)
    kn = torch.zeros(2, 1, 2, 64)
    with pytest.raises(ValueError, match="new key/value rows"):
        ops.decode_append(q, kn[:, :, :1], kn[:, :, :1], kc, kc.clone(),
                          torch.tensor([3, 4], dtype=torch.int32), 1.0)


def test_packed_attention_rejects_mixed_dtypes_at_the_op_level():
    q, k, v = _qkv()
    seg = torch.ones(2, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="share one dtype"):
        ops.packed_attention(q.float(), k, v, seg, seg, 1, 0.125)


def test_drop_in_functions_promote_mixed_dtypes_like_the_reference():
    # a float32 query over bfloat16 keys is promoted to float32 (the reference's einsum
    # promotes); with host tensors the call then stops at the device check, not a dtype error
    q, k, v = _qkv()
    seg = torch.ones(2, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU only"):
        bidirectional.attention(q.float(), k, v, seg, seg)
    with pytest.raises(ValueError, match="GPU only"):
        attention.dense_cached_attention(q[:, :1].float(), k, v, 4)


@pytest.mark.parametrize("mask_shape, seg_shape", [((2, 1), (2, 8)), ((3, 8), (3, 8)),
                                                   ((2, 8), (2, 7)), ((2, 8), (1, 8))])
def test_block_map_requires_exact_mask_and_id_shapes(mask_shape, seg_shape):
    q, k, v = _qkv()
    mask = torch.ones(mask_shape, dtype=torch.int32)
    seg = torch.ones(seg_shape, dtype=torch.int32)
    with pytest.raises(ValueError, match="must be"):
        ops.packed_attention(q, k, v, mask, seg, 1, 0.125)
    with pytest.raises(ValueError, match="must be"):
        ops.block_map(seg, mask, 1, 8, 8, batch=2)


def test_query_and_kv_batches_must_agree():
    q, k, v = _qkv()
    seg = torch.ones(2, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="Packed attention query/KV shapes are incompatible"):
        ops.packed_attention(q, k[:1], v[:1], seg, seg, 1, 0.125)
    with pytest.raises(ValueError, match="Packed attention query/KV shapes are incompatible"):
        ops.packed_attention(q, k, v[:, :, :1], seg, seg, 1, 0.125)


def test_a_plan_for_another_call_is_rejected():
    q, k, v = _qkv()
    plan = ops.Plan(torch.zeros(1, dtype=torch.uint8), 2, 16, 16, 1)
    with pytest.raises(ValueError, match="plan was built for batch 2, lengths 16/16"):
        ops.attn_fwd(q, k, v, plan, 1, 0.125)
    plan = ops.Plan(torch.zeros(1, dtype=torch.uint8), 2, 8, 8, 0)
    with pytest.raises(ValueError, match="mask mode 0"):
        ops.attn_fwd(q, k, v, plan, 1, 0.125)


def test_strided_views_are_refused_before_any_launch():
    """The kernels read operands as dense arrays from their data pointers: a slice or a
    transposed view is refused by every op that takes raw tensors (the drop-in functions
    pass contiguous copies)."""
    q, k, v = _qkv(t=16)
    plan = ops.Plan(torch.zeros(1, dtype=torch.uint8), 2, 16, 16, 1)
    strided_q = torch.zeros(2, 16, 8, 64, dtype=q.dtype)[:, :, ::2]
    transposed_k = torch.zeros(2, 2, 16, 64, dtype=k.dtype).transpose(1, 2)
    assert not strided_q.is_contiguous() and not transposed_k.is_contiguous()
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_fwd(strided_q, k, v, plan, 1, 0.125)
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_fwd(q, transposed_k, v, plan, 1, 0.125)
    lse = torch.zeros(2, 4, 16)
    out = torch.zeros_like(q)
    dout_view = torch.zeros(2, 16, 8, 64, dtype=q.dtype)[:, :, 4:]
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_bwd(q, k, v, out, dout_view, lse, plan, 1, 0.125)
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_bwd(q, k, v, out, torch.zeros_like(q), lse.transpose(1, 2).contiguous()
                     .transpose(1, 2), plan, 1, 0.125)
    ws = ops.bwd_workspace(q)
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_bwd_dq(q, k, v, torch.zeros_like(q), lse, plan, 1, 0.125, ws,
                        torch.zeros(2, 16, 8, 64, dtype=q.dtype)[:, :, ::2])
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.attn_bwd_dkdv(q, k, v, torch.zeros_like(q), lse, plan, 1, 0.125, ws, transposed_k,
                          torch.zeros_like(v))
    with pytest.raises(ValueError, match="at least"):
        ops.attn_bwd_dkdv(q, k, v, torch.zeros_like(q), lse, plan, 1, 0.125, ws[:8],
                          torch.zeros_like(k), torch.zeros_like(v))
    with pytest.raises(ValueError, match="lse must be"):
        ops.attn_bwd_delta(out, torch.zeros_like(q), torch.zeros(2, 4, 15), ws)
