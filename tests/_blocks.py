"""The reference's block callers of the hot path, restated in torch over mfattn.

These are ``layers/attention.py:61-137, :214-243, :246-322`` and
``models/lfm2_5/encoder.py:64-110`` written with torch for the projections,
norms and SwiGLU tail, and the drop-in ``mfattn`` functions for the path
itself: ``kernels.prologue.qk_norm_rope`` (QK RMS norm + RoPE),
``kernels.attention.packed_causal_attention`` / ``cached_attention_step``,
``kernels.bidirectional.attention`` and ``kernels.convolution``.  The GPU
tests run them to show the drop-in composes the way the reference's layers
call it.  Weights are dicts of tensors named as in ``oracle.blocks``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from mfattn.kernels import attention, bidirectional, convolution, prologue


def rms_norm(x, gain, eps):
    """``kernels/normalization.py:19-22``: fp32 statistics, cast, then the gain."""
    value = x.float()
    value = value * torch.rsqrt((value * value).mean(-1, keepdim=True) + eps)
    return value.to(x.dtype) * gain.to(x.dtype)


def full_linear(x, weight):
    return x @ weight.to(x.dtype).T


def swiglu(x, ffn, eps):
    n = rms_norm(x, ffn["norm"], eps)
    return x + full_linear(F.silu(full_linear(n, ffn["gate"])) * full_linear(n, ffn["up"]),
                           ffn["down"])


def rope_qkv(x, w, positions, *, head_dim, rope_theta, eps):
    """``layers/attention.py:61-97`` with the fused HIP prologue for q and k."""
    b, t, _ = x.shape
    hidden = rms_norm(x, w["operator_norm"], eps)
    q = full_linear(hidden, w["query"]).reshape(b, t, -1, head_dim)
    k = full_linear(hidden, w["key"]).reshape(b, t, -1, head_dim)
    v = full_linear(hidden, w["value"]).reshape(b, t, -1, head_dim)
    q, k = prologue.qk_norm_rope(q, k, w["query_norm"], w["key_norm"], positions, eps=eps,
                                 rope_theta=rope_theta)
    return q, k, v


def _residual(x, attended, w, ffn, eps):
    return swiglu(x + full_linear(attended.reshape(x.shape[0], x.shape[1], -1), w["out"]), ffn, eps)


def attention_block_packed(x, w, ffn, attention_mask, segment_ids, positions, *, head_dim,
                           rope_theta, eps, backend):
    """``layers/attention.py:214-243``."""
    q, k, v = rope_qkv(x, w, positions, head_dim=head_dim, rope_theta=rope_theta, eps=eps)
    attended = attention.packed_causal_attention(q, k, v, attention_mask, segment_ids,
                                                 backend=backend)
    return _residual(x, attended, w, ffn, eps)


def attention_block_prefill(x, w, ffn, attention_mask, *, capacity, head_dim, rope_theta, eps,
                            backend):
    """``layers/attention.py:246-278``: the block plus mask-zeroed keys/values padded to a
    ``capacity``-slot cache.  Rows are causal over their valid prefix (one segment per row)."""
    q, k, v = rope_qkv(x, w, None, head_dim=head_dim, rope_theta=rope_theta, eps=eps)
    ids = (attention_mask != 0).to(torch.int32)
    attended = attention.packed_causal_attention(q, k, v, attention_mask, ids, backend=backend)
    padding = capacity - k.shape[1]
    if padding < 0:
        raise ValueError("Prompt length exceeds attention cache capacity")
    keep = attention_mask[:, :, None, None].to(k.dtype)
    pad = (0, 0, 0, 0, 0, padding)
    return _residual(x, attended, w, ffn, eps), F.pad(k * keep, pad), F.pad(v * keep, pad)


def attention_block_step(x, w, ffn, cache_key, cache_value, position, *, head_dim, rope_theta,
                         eps, backend):
    """``layers/attention.py:281-322`` with one cache slot per row: ``position`` ([B]) is
    each row's slot and RoPE position; the step attends over ``position + 1`` slots."""
    q, k, v = rope_qkv(x, w, position[:, None], head_dim=head_dim, rope_theta=rope_theta, eps=eps)
    attended, cache_key, cache_value = attention.cached_attention_step(
        q, k, v, cache_key, cache_value, position, backend=backend)
    return _residual(x, attended, w, ffn, eps), cache_key, cache_value


def encoder_block(x, params, ffn, mask, segment_ids, positions, *, kind, head_dim, rope_theta,
                  eps):
    """``models/lfm2_5/encoder.py:64-110`` (packed ids and per-segment positions)."""
    norm = rms_norm(x, params["operator_norm"], eps)
    if kind == "conv":
        hidden = norm * mask[..., None].to(norm.dtype)
        b_gate, c_gate, values = torch.split(full_linear(hidden, params["in_proj"]),
                                             params["conv"].shape[0], dim=-1)
        mixed = convolution.gated_centered_convolution(b_gate, c_gate, values,
                                                       params["conv"].to(x.dtype), segment_ids)
        return swiglu(x + full_linear(mixed, params["out"]), ffn, eps)
    b, t, _ = x.shape
    q = full_linear(norm, params["query"]).reshape(b, t, -1, head_dim)
    k = full_linear(norm, params["key"]).reshape(b, t, -1, head_dim)
    v = full_linear(norm, params["value"]).reshape(b, t, -1, head_dim)
    q, k = prologue.qk_norm_rope(q, k, params["query_norm"], params["key_norm"], positions,
                                 eps=eps, rope_theta=rope_theta)
    mixed = bidirectional.attention(q, k, v, mask, segment_ids)
    return swiglu(x + full_linear(mixed.reshape(b, t, -1), params["out"]), ffn, eps)
