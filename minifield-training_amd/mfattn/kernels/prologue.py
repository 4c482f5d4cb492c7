"""Attention prologue: QK RMS norm + rotary embeddings in one device pass.

Mirrors the q/k part of ``_rope_qkv`` (``layers/attention.py:62-97``):
``rms_norm`` of the query and key heads with their per-dimension gains
(``kernels/normalization.py:7-22``), then ``apply_rotary`` at per-token
positions (``kernels/rotary.py:7-39``; on the packed path the positions
restart at every segment).  ``segment_positions`` builds those positions on
the device from segment ids, as ``batching/packing.py:92-100`` does on the host.
"""

from __future__ import annotations

import torch

from .. import _lib
from .. import ops
from ..ops import _ptr, _stream, dtype_code, require_device


def _positions(positions, batch: int, length: int, device: torch.device) -> torch.Tensor | None:
    """The reference's scalar / [T] / [B, T] forms, as [B, T] int32 (rotary.py:18-31)."""
    if positions is None:
        return None
    pos = positions.to(device=device, dtype=torch.int32) if isinstance(positions, torch.Tensor) \
        else torch.tensor(positions, dtype=torch.int32, device=device)
    if pos.dim() == 0:
        pos = pos.expand(batch, length)
    elif pos.dim() == 1:
        pos = pos[None, :].expand(batch, pos.shape[0])
    elif pos.dim() != 2:
        raise ValueError("RoPE positions must be scalar, [T], or [B, T]")
    if tuple(pos.shape) != (batch, length):
        raise ValueError("RoPE positions must match the token dimensions")
    return pos.contiguous()


def _launch_forward(q, k, qg, kg, pos, eps, theta, q_out, k_out):
    _lib.check(_lib.LIB.mf_qk_norm_rope(_ptr(q), _ptr(k), _ptr(qg), _ptr(kg), _ptr(pos),
                                        dtype_code(q), q.shape[0], q.shape[1], q.shape[2],
                                        k.shape[2], q.shape[3], float(eps), float(theta),
                                        _ptr(q_out), _ptr(k_out), _stream(q.device)))


class QKNormRope(torch.autograd.Function):
    """The fused prologue with a HIP forward and a HIP backward (``mf_qk_norm_rope_bwd``).

    Gradients reach q, k and both gains; positions are integers (no gradient).
    """

    @staticmethod
    def forward(ctx, q, k, qg, kg, pos, eps, theta):
        q_out, k_out = torch.empty_like(q), torch.empty_like(k)
        _launch_forward(q, k, qg, kg, pos, eps, theta, q_out, k_out)
        ctx.save_for_backward(q, k, qg, kg, pos)
        ctx.eps, ctx.theta = eps, theta
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq_out, dk_out):
        q, k, qg, kg, pos = ctx.saved_tensors
        dq_out = torch.zeros_like(q) if dq_out is None else dq_out.contiguous()
        dk_out = torch.zeros_like(k) if dk_out is None else dk_out.contiguous()
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        dqg = torch.empty(q.shape[-1], dtype=torch.float32, device=q.device)
        dkg = torch.empty_like(dqg)
        b, t = q.shape[:2]
        ws_bytes = _lib.LIB.mf_qk_norm_rope_bwd_workspace_bytes(b, t)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        _lib.check(_lib.LIB.mf_qk_norm_rope_bwd(
            _ptr(q), _ptr(k), _ptr(qg), _ptr(kg), _ptr(pos), _ptr(dq_out), _ptr(dk_out),
            dtype_code(q), b, t, q.shape[2], k.shape[2], q.shape[3], float(ctx.eps),
            float(ctx.theta), _ptr(dq), _ptr(dk), _ptr(dqg), _ptr(dkg), _ptr(ws), ws_bytes,
            _stream(q.device)))
        return dq, dk, dqg.to(qg.dtype), dkg.to(kg.dtype), None, None, None


def qk_norm_rope(query: torch.Tensor, key: torch.Tensor, query_gain: torch.Tensor,
                 key_gain: torch.Tensor, positions=None, *, eps: float, rope_theta: float,
                 inplace: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """RMS-normalise and rotate ``query [B,T,Hq,D]`` and ``key [B,T,Hkv,D]``.

    Gains are cast to the tensors' dtype (``weight.astype(x.dtype)`` in the
    reference).  ``positions=None`` means ``0 .. T-1`` on every row.
    Differentiable in q, k and the gains (HIP backward); ``inplace=True``
    overwrites q and k and is only allowed when no gradient is being recorded.
    """
    device = require_device(query, key)
    if query.shape[:2] != key.shape[:2] or query.shape[-1] != key.shape[-1] or query.dtype != key.dtype:
        raise ValueError("query and key must share batch, length, head_dim and dtype")
    b, t, hq, d = query.shape
    pos = _positions(positions, b, t, device)
    q, k = query.contiguous(), key.contiguous()
    qg = query_gain.to(device=device, dtype=query.dtype).contiguous()
    kg = key_gain.to(device=device, dtype=query.dtype).contiguous()
    needs_grad = torch.is_grad_enabled() and any(
        x.requires_grad for x in (query, key, query_gain, key_gain))
    if inplace:
        if needs_grad:
            raise ValueError("qk_norm_rope(inplace=True) cannot record gradients; "
                             "call it out of place or under torch.no_grad()")
        _launch_forward(q, k, qg, kg, pos, eps, rope_theta, q, k)
        return q, k
    if not needs_grad:
        q_out, k_out = torch.empty_like(q), torch.empty_like(k)
        _launch_forward(q, k, qg, kg, pos, eps, rope_theta, q_out, k_out)
        return q_out, k_out
    return QKNormRope.apply(q, k, qg, kg, pos, float(eps), float(rope_theta))


def key_norm_rope(key: torch.Tensor, key_gain: torch.Tensor, positions=None, *, eps: float,
                  rope_theta: float) -> torch.Tensor:
    """The key half of :func:`qk_norm_rope` alone (``mf_qk_norm_rope`` with no query heads):
    the key operand of :func:`packed_attention_normed_query`.  Forward only."""
    if torch.is_grad_enabled() and (key.requires_grad or key_gain.requires_grad):
        raise ValueError("key_norm_rope has no backward; call qk_norm_rope to record gradients")
    device = require_device(key)
    b, t, hkv, d = key.shape
    pos = _positions(positions, b, t, device)
    k = key.contiguous()
    kg = key_gain.to(device=device, dtype=key.dtype).contiguous()
    k_out = torch.empty_like(k)
    _lib.check(_lib.LIB.mf_qk_norm_rope(None, _ptr(k), None, _ptr(kg), _ptr(pos), dtype_code(k), b,
                                        t, 0, hkv, d, float(eps), float(rope_theta), None,
                                        _ptr(k_out), _stream(device)))
    return k_out


def segment_positions(segment_ids: torch.Tensor) -> torch.Tensor:
    """Offset of every token in its run of equal nonzero ids; 0 on padding."""
    device = require_device(segment_ids)
    seg = segment_ids.to(torch.int32).contiguous()
    b, t = seg.shape
    out = torch.empty_like(seg)
    _lib.check(_lib.LIB.mf_segment_positions(_ptr(seg), b, t, _ptr(out), _stream(device)))
    return out


def packed_attention_normed_query(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                  query_gain: torch.Tensor, attention_mask: torch.Tensor,
                                  segment_ids: torch.Tensor | None, positions=None, *,
                                  eps: float, rope_theta: float, causal: bool = True,
                                  plan=None) -> torch.Tensor:
    """Packed attention of the RMS-normalised, rotated query, the query's norm and RoPE applied
    in the attention kernel's query loads (``mf_attn_fwd_rope_q``).

    Equal bit for bit to ``qk_norm_rope`` of the query followed by the packed attention
    (``packed_causal_attention`` when ``causal``, else ``bidirectional.attention`` with segment
    ids): the composition ``layers/attention.py:214-243`` runs, without the normalised query
    ever reaching memory.  ``key`` must already be normalised and rotated (``qk_norm_rope``'s
    key output), ``query`` is the query projection; ``causal=False`` without segment ids is the
    key-mask mode of ``bidirectional.attention``.  bfloat16, head_dim 64, forward only: inputs
    that record gradients raise (training calls ``qk_norm_rope`` and the attention).
    """
    if torch.is_grad_enabled() and any(
            x.requires_grad for x in (query, key, value, query_gain)):
        raise ValueError("packed_attention_normed_query has no backward; call qk_norm_rope and "
                         "the packed attention to record gradients")
    device = require_device(query, key, value, attention_mask)
    b, t, _, d = query.shape
    mode = (_lib.MODE_PACKED_CAUSAL if causal else
            _lib.MODE_PACKED_BIDIR if segment_ids is not None else _lib.MODE_KEYMASK_BIDIR)
    if plan is None:
        plan = ops.PLANS.get(segment_ids, attention_mask, mode, t, key.shape[1], b)
    q, k, v = query.contiguous(), key.contiguous(), value.contiguous()
    qg = query_gain.to(device=device, dtype=query.dtype)
    pos = _positions(positions, b, t, device)
    out, _ = ops.attn_fwd_rope_q(q, k, v, qg, pos, plan, mode, d ** -0.5, eps=eps,
                                 rope_theta=rope_theta)
    return out
