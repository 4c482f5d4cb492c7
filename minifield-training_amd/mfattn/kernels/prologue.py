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


def qk_norm_rope(query: torch.Tensor, key: torch.Tensor, query_gain: torch.Tensor,
                 key_gain: torch.Tensor, positions=None, *, eps: float, rope_theta: float,
                 inplace: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """RMS-normalise and rotate ``query [B,T,Hq,D]`` and ``key [B,T,Hkv,D]``.

    Gains are cast to the tensors' dtype (``weight.astype(x.dtype)`` in the
    reference).  ``positions=None`` means ``0 .. T-1`` on every row.
    """
    device = require_device(query, key)
    if query.shape[:2] != key.shape[:2] or query.shape[-1] != key.shape[-1] or query.dtype != key.dtype:
        raise ValueError("query and key must share batch, length, head_dim and dtype")
    b, t, hq, d = query.shape
    pos = _positions(positions, b, t, device)
    q, k = query.contiguous(), key.contiguous()
    qg = query_gain.to(device=device, dtype=query.dtype).contiguous()
    kg = key_gain.to(device=device, dtype=query.dtype).contiguous()
    q_out = q if inplace else torch.empty_like(q)
    k_out = k if inplace else torch.empty_like(k)
    _lib.check(_lib.LIB.mf_qk_norm_rope(_ptr(q), _ptr(k), _ptr(qg), _ptr(kg), _ptr(pos),
                                        dtype_code(q), b, t, hq, key.shape[2], d, float(eps),
                                        float(rope_theta), _ptr(q_out), _ptr(k_out),
                                        _stream(device)))
    return q_out, k_out


def segment_positions(segment_ids: torch.Tensor) -> torch.Tensor:
    """Offset of every token in its run of equal nonzero ids; 0 on padding."""
    device = require_device(segment_ids)
    seg = segment_ids.to(torch.int32).contiguous()
    b, t = seg.shape
    out = torch.empty_like(seg)
    _lib.check(_lib.LIB.mf_segment_positions(_ptr(seg), b, t, _ptr(out), _stream(device)))
    return out
