"""Segmented short convolutions of the packed layers (HIP).

Mirrors ``kernels/bidirectional.py:38-58`` (``centered_convolution``) and
``kernels/convolution.py:7-53`` (``gated_depthwise_convolution`` and its
segmented variant).  Channels must be a multiple of 8; kernel sizes up to 8.
Taps are cast to the activations' dtype (the reference's callers pass
``weights.conv.astype(hidden.dtype)``, ``models/lfm2_5/encoder.py:84``).
"""

from __future__ import annotations

import torch

from .. import _lib
from ..ops import _ptr, _stream, dtype_code, require_device


def _launch_forward(bg, cg, v, w, seg, mode, out):
    b, t, c = v.shape
    _lib.check(_lib.LIB.mf_segmented_conv(_ptr(bg), _ptr(cg), _ptr(v), _ptr(w), _ptr(seg), mode,
                                          dtype_code(v), b, t, c, w.shape[1], _ptr(out),
                                          _stream(v.device)))


class SegmentedConv(torch.autograd.Function):
    """``c * conv(b * v)`` with a HIP forward and a HIP backward (``mf_segmented_conv_bwd``).

    Gradients reach the values, both gates (when given) and the taps; segment
    ids are integers (no gradient).
    """

    @staticmethod
    def forward(ctx, bg, cg, v, w, seg, mode):
        out = torch.empty_like(v)
        _launch_forward(bg, cg, v, w, seg, mode, out)
        ctx.save_for_backward(bg, cg, v, w, seg)
        ctx.mode = mode
        return out

    @staticmethod
    def backward(ctx, d_out):
        bg, cg, v, w, seg = ctx.saved_tensors
        g = d_out.contiguous()
        b, t, c = v.shape
        k = w.shape[1]
        dv = torch.empty_like(v)
        db = None if bg is None else torch.empty_like(v)
        dc = None if cg is None else torch.empty_like(v)
        dw = torch.empty((c, k), dtype=torch.float32, device=v.device)
        ws_bytes = _lib.LIB.mf_segmented_conv_bwd_workspace_bytes(b, t, c, k)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=v.device)
        _lib.check(_lib.LIB.mf_segmented_conv_bwd(
            _ptr(bg), _ptr(cg), _ptr(v), _ptr(w), _ptr(seg), _ptr(g), ctx.mode, dtype_code(v),
            b, t, c, k, _ptr(db), _ptr(dc), _ptr(dv), _ptr(dw), _ptr(ws), ws_bytes,
            _stream(v.device)))
        return db, dc, dv, dw.to(w.dtype), None, None


def _run(b_gate, c_gate, values, taps, segment_ids, mode: int) -> torch.Tensor:
    device = require_device(values)
    if taps.dim() != 2 or taps.shape[0] != values.shape[-1]:
        raise ValueError("Convolution taps must be [channels, kernel_size]")
    # the casts below are differentiable: gradients flow back to the callers' dtypes
    v = values.contiguous()
    w = taps.to(device=device, dtype=v.dtype).contiguous()
    bg = None if b_gate is None else b_gate.to(v.dtype).contiguous()
    cg = None if c_gate is None else c_gate.to(v.dtype).contiguous()
    for gate in (bg, cg):
        if gate is not None and gate.shape != v.shape:
            raise ValueError("Convolution gates must match the values' shape")
    seg = None if segment_ids is None else segment_ids.to(device=device, dtype=torch.int32).contiguous()
    b, t, c = v.shape
    if seg is not None and tuple(seg.shape) != (b, t):
        raise ValueError("segment_ids must be [batch, tokens]")
    needs_grad = torch.is_grad_enabled() and any(
        x is not None and x.requires_grad for x in (b_gate, c_gate, values, taps))
    if not needs_grad:
        out = torch.empty_like(v)
        _launch_forward(bg, cg, v, w, seg, mode, out)
        return out
    return SegmentedConv.apply(bg, cg, v, w, seg, mode)


def centered_convolution(gated: torch.Tensor, taps: torch.Tensor,
                         segment_ids: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped conv1d with padding ``k // 2`` and right crop, segment-masked."""
    return _run(None, None, gated, taps, segment_ids, _lib.CONV_CENTERED)


def gated_centered_convolution(b_gate, c_gate, values, taps, segment_ids=None) -> torch.Tensor:
    """``c_gate * centered_convolution(b_gate * values, taps, segment_ids)`` in one pass."""
    return _run(b_gate, c_gate, values, taps, segment_ids, _lib.CONV_CENTERED)


def gated_depthwise_convolution(b_gate, c_gate, values, weights, *, kernel_size: int) -> torch.Tensor:
    if weights.shape[-1] != kernel_size:
        raise ValueError("Convolution weights must hold kernel_size taps")
    return _run(b_gate, c_gate, values, weights, None, _lib.CONV_CAUSAL)


def gated_depthwise_convolution_segmented(b_gate, c_gate, values, weights, segment_ids, *,
                                          kernel_size: int) -> torch.Tensor:
    if weights.shape[-1] != kernel_size:
        raise ValueError("Convolution weights must hold kernel_size taps")
    return _run(b_gate, c_gate, values, weights, segment_ids, _lib.CONV_CAUSAL)
