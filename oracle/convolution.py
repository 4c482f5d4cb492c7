"""CPU restatement of the segmented short convolutions (test infrastructure).

* ``centered`` follows ``src/minifield_training/kernels/bidirectional.py:38-58``
  (``centered_convolution``): zero padding of ``K // 2`` on both sides, right
  crop, and with segment ids a tap counts only inside the token's nonzero
  segment.
* ``causal`` follows ``kernels/convolution.py:25-53``
  (``gated_depthwise_convolution_segmented``): left padding ``K - 1``, the
  same segment rule, gates ``c * conv(b * v)``.
Both evaluate in float64; the dtype casts are the caller's.

* ``centered_cast`` / ``causal_cast`` are the same convolutions in torch on
  the CPU with the reference's declared dtypes: ``b * v``, every tap product
  and every partial sum (in tap order) rounded to the tensor dtype, then the
  ``c`` product (``bidirectional.py:48-57``, ``convolution.py:41-52``).  Pinned
  by the reference fixtures and by a hand-derived bf16 case in which each of
  those roundings changes the result.
* ``centered_vjp`` / ``causal_vjp`` are the analytic VJPs (the reference takes
  them from JAX autodiff) of ``c * conv(b * v)``: with ``h = g * c``,
  ``dc = g * conv(b * v)``, ``d(b*v)[s] = sum_i h[s - o_i] w_i keep``,
  ``db = d(b*v) * v``, ``dv = d(b*v) * b``, ``dw_i = sum h[t] (b*v)[t + o_i] keep``.
  Pinned by the reference's gradient fixtures
  (``tests/kernels/test_bidirectional.py:35-38``, ``:75-78``) and by central
  differences of the forward.
"""

from __future__ import annotations

import numpy as np


def _conv(x, taps, segment_ids, offsets):
    x = np.asarray(x, np.float64)
    taps = np.asarray(taps, np.float64)
    b, t, c = x.shape
    out = np.zeros_like(x)
    seg = None if segment_ids is None else np.asarray(segment_ids)
    for i, off in enumerate(offsets):
        src = np.arange(t) + off
        inside = (src >= 0) & (src < t)
        srcc = np.clip(src, 0, t - 1)
        contrib = x[:, srcc, :] * taps[None, None, :, i]
        if seg is None:
            keep = np.broadcast_to(inside[None, :], (b, t))
        else:
            keep = inside[None, :] & (seg[:, srcc] == seg) & (seg != 0)
        out += contrib * keep[..., None]
    return out


def centered(gated, taps, segment_ids=None):
    k = np.asarray(taps).shape[-1]
    return _conv(gated, taps, segment_ids, [i - k // 2 for i in range(k)])


def causal(b_gate, c_gate, values, weights, segment_ids=None):
    k = np.asarray(weights).shape[-1]
    gated = np.asarray(b_gate, np.float64) * np.asarray(values, np.float64)
    mixed = _conv(gated, weights, segment_ids, [i - (k - 1) for i in range(k)])
    return np.asarray(c_gate, np.float64) * mixed


def _offsets(k: int, centered: bool) -> list[int]:
    return [i - k // 2 for i in range(k)] if centered else [i - (k - 1) for i in range(k)]


def _vjp(b_gate, c_gate, values, taps, segment_ids, d_out, centered: bool, with_abs=False):
    v = np.asarray(values, np.float64)
    b = np.ones_like(v) if b_gate is None else np.asarray(b_gate, np.float64)
    c = np.ones_like(v) if c_gate is None else np.asarray(c_gate, np.float64)
    w = np.asarray(taps, np.float64)
    g = np.asarray(d_out, np.float64)
    bsz, t, ch = v.shape
    k = w.shape[-1]
    seg = None if segment_ids is None else np.asarray(segment_ids)
    u = b * v
    h = g * c
    mixed = np.zeros_like(v)
    du = np.zeros_like(v)
    dw = np.zeros_like(w)
    dw_abs = np.zeros_like(w)
    for i, off in enumerate(_offsets(k, centered)):
        for tt in range(t):
            s = tt + off
            if not 0 <= s < t:
                continue
            if seg is None:
                keep = np.ones(bsz, bool)
            else:
                keep = (seg[:, s] == seg[:, tt]) & (seg[:, tt] != 0)
            kk = keep[:, None].astype(np.float64)
            mixed[:, tt] += u[:, s] * w[None, :, i] * kk      # forward tap t <- s
            du[:, s] += h[:, tt] * w[None, :, i] * kk         # its transpose s <- t
            dw[:, i] += (h[:, tt] * u[:, s] * kk).sum(0)
            dw_abs[:, i] += np.abs(h[:, tt] * u[:, s] * kk).sum(0)
    dc = g * mixed
    if with_abs:
        return du * v, dc, du * b, dw, dw_abs
    return du * v, dc, du * b, dw


def centered_vjp(b_gate, c_gate, values, taps, d_out, segment_ids=None, with_abs=False):
    """``(db, dc, dv, dw)`` of ``c * centered(b * values, taps, segment_ids)``.

    ``with_abs`` appends ``sum |h u|`` per (channel, tap): the scale a rounding of
    each tap-gradient term is relative to."""
    return _vjp(b_gate, c_gate, values, taps, segment_ids, d_out, True, with_abs)


def causal_vjp(b_gate, c_gate, values, weights, d_out, segment_ids=None, with_abs=False):
    """``(db, dc, dv, dw)`` of ``causal(b_gate, c_gate, values, weights, segment_ids)``."""
    return _vjp(b_gate, c_gate, values, weights, segment_ids, d_out, False, with_abs)


def _torch():
    import torch  # local import: only the cast-order restatement needs it
    return torch


def _conv_cast(gated, taps, segment_ids, offsets):
    torch = _torch()
    t = gated.shape[1]
    result = None
    for i, off in enumerate(offsets):
        src = torch.arange(t) + off
        inside = (src >= 0) & (src < t)
        srcc = src.clamp(0, t - 1)
        tap = gated[:, srcc, :] * taps[:, i]
        if segment_ids is None:
            keep = inside[None, :].expand(gated.shape[0], t)
        else:
            seg = torch.as_tensor(segment_ids)
            keep = inside[None, :] & (seg[:, srcc] == seg) & (seg != 0)
        tap = tap * keep[..., None].to(tap.dtype)
        result = tap if result is None else result + tap
    return result


def centered_cast(gated, taps, segment_ids=None):
    """``centered_convolution`` on torch tensors, rounding as the reference's dtypes."""
    k = taps.shape[-1]
    return _conv_cast(gated, taps, segment_ids, [i - k // 2 for i in range(k)])


def causal_cast(b_gate, c_gate, values, weights, segment_ids=None):
    """``gated_depthwise_convolution[_segmented]`` on torch tensors, rounding as the reference."""
    k = weights.shape[-1]
    mixed = _conv_cast(b_gate * values, weights, segment_ids, [i - (k - 1) for i in range(k)])
    return c_gate * mixed
