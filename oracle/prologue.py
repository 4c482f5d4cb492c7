"""CPU restatement of the attention prologue: QK RMS norm and rotary embeddings.

Test infrastructure only (the product never imports ``oracle``).

* ``rms_norm`` follows ``src/minifield_training/kernels/normalization.py:7-22``
  (fp32 statistics; the normalised value is cast to the tensor dtype before
  the gain multiply).
* ``apply_rotary`` follows ``kernels/rotary.py:7-39``: single-precision
  frequencies ``theta ** (-arange(0, D, 2) / D)`` (correctly rounded) and angles
  ``f32(position) * freq``, split-half rotation ``(-x[D/2:], x[:D/2])``.
  Evaluated in float64 from those single-precision angles.
* ``rotate_pairs`` is an independent restatement: a 2x2 rotation matrix per
  dimension pair (i, i + D/2), the method of ``tests/layers/test_blocks.py:116-121``.
* ``qk_norm_rope_cast`` is the same prologue with the reference's dtype cast
  order, evaluated in torch on the CPU (NumPy has no bfloat16): fp32
  statistics, the normalised value cast to the tensor dtype before the gain
  product (``normalization.py:19-22``), cos/sin cast to the tensor dtype and
  every product and the sum rounded to it (``rotary.py:37-39``; the declared
  dtypes, as the reference's own tests enforce with
  ``xla_allow_excess_precision=False``, ``tests/models/lfm2_5/test_encoder.py:190-192``).
  Pinned by hand-derived bf16 cases in which each of those cast points
  changes the result, and equal to the FP64 restatement in float32.
* ``qk_norm_rope_vjp`` is the analytic VJP of the FP64 prologue (the
  reference takes it from JAX autodiff): for each head row, with
  ``y = x * inv``, ``n = y * w``, ``out = n * cos + rot(n) * sin``:
  ``dn = g * cos + rot^T(g * sin)``, ``dw = sum dn * y``, ``dy = dn * w``,
  ``dx = inv * (dy - y * mean(dy * y))``.  Pinned by central differences.
* ``segment_positions`` restates the packer's positions
  (``batching/packing.py:92-100``): ``arange(len)`` inside each placed
  sequence, 0 on padding -- here the offset inside each run of equal
  nonzero ids.
"""

from __future__ import annotations

import numpy as np


def rms_norm(x, weight, eps: float):
    """fp64 value of the fp32 computation; the dtype casts are the caller's."""
    v = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps)
    return v * inv * np.asarray(weight, np.float64)


def frequencies(rope_theta: float, head_dim: int) -> np.ndarray:
    """``rope_theta ** (-arange(0, D, 2) / D)`` in float32 (rotary.py:33-35), correctly
    rounded: the float64 power rounded once.  (NumPy's float32 power is up to ~0.9 ulp off,
    and a one-ulp frequency difference moves the angle of position p by p * 6e-8 of it.)"""
    exps = -(np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    return (np.float64(np.float32(rope_theta)) ** exps).astype(np.float32)


def angles(positions, rope_theta: float, head_dim: int) -> np.ndarray:
    """float32 ``position * frequency`` per (row, token, pair)."""
    pos = np.asarray(positions, np.float32)
    return (pos[..., None] * frequencies(rope_theta, head_dim)).astype(np.float32)


def apply_rotary(x, rope_theta: float, positions) -> np.ndarray:
    """Split-half rotary embedding of ``[B, T, H, D]`` at ``positions [B, T]``."""
    x = np.asarray(x, np.float64)
    d = x.shape[-1]
    a = angles(positions, rope_theta, d).astype(np.float64)[:, :, None, :]
    a = np.concatenate((a, a), axis=-1)
    first, second = x[..., : d // 2], x[..., d // 2 :]
    rotated = np.concatenate((-second, first), axis=-1)
    return x * np.cos(a) + rotated * np.sin(a)


def rotate_pairs(x, rope_theta: float, positions) -> np.ndarray:
    """The same map written as a rotation of each pair (x_i, x_{i+D/2})."""
    x = np.asarray(x, np.float64)
    b, t, h, d = x.shape
    a = angles(positions, rope_theta, d).astype(np.float64)
    out = np.empty_like(x)
    for i in range(d // 2):
        c, s = np.cos(a[..., i])[:, :, None], np.sin(a[..., i])[:, :, None]
        u, w = x[..., i], x[..., i + d // 2]
        out[..., i] = c * u - s * w
        out[..., i + d // 2] = s * u + c * w
    return out


def qk_norm_rope(q, k, q_gain, k_gain, positions, eps: float, rope_theta: float):
    """The prologue: RMS-normalise q and k heads, then rotate (fp64)."""
    return (apply_rotary(rms_norm(q, q_gain, eps), rope_theta, positions),
            apply_rotary(rms_norm(k, k_gain, eps), rope_theta, positions))


def _head_vjp(x, gain, eps, positions, rope_theta, d_out):
    x = np.asarray(x, np.float64)
    g = np.asarray(d_out, np.float64)
    d = x.shape[-1]
    a = angles(positions, rope_theta, d).astype(np.float64)[:, :, None, :]
    a = np.concatenate((a, a), axis=-1)
    cos, sin = np.cos(a), np.sin(a)
    gs = g * sin
    # rot(n) = (-n[D/2:], n[:D/2]); its transpose maps u to (u[D/2:], -u[:D/2])
    dn = g * cos + np.concatenate((gs[..., d // 2 :], -gs[..., : d // 2]), axis=-1)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * inv
    w = np.asarray(gain, np.float64)
    dw = (dn * y).reshape(-1, d).sum(0)
    dy = dn * w
    dx = inv * (dy - y * np.mean(dy * y, axis=-1, keepdims=True))
    return dx, dw, np.abs(dn * y).reshape(-1, d).sum(0)


def qk_norm_rope_vjp(q, k, q_gain, k_gain, positions, eps: float, rope_theta: float, dq_out,
                     dk_out, with_abs: bool = False):
    """``(dq, dk, dq_gain, dk_gain)`` of ``qk_norm_rope`` for upstream ``dq_out, dk_out``.

    ``with_abs`` also returns the sums of the gain gradients' absolute terms
    (``sum |dn * y|`` per dim), the scale a rounding of each term is relative to.
    """
    dq, dqg, aq = _head_vjp(q, q_gain, eps, positions, rope_theta, dq_out)
    dk, dkg, ak = _head_vjp(k, k_gain, eps, positions, rope_theta, dk_out)
    if with_abs:
        return dq, dk, dqg, dkg, aq, ak
    return dq, dk, dqg, dkg


def _torch():
    import torch  # local import: only the cast-order restatement needs it
    return torch


def rms_norm_cast(x, weight, eps: float):
    """``normalization.py:19-22`` for a torch tensor ``x`` of any float dtype."""
    torch = _torch()
    value = x.float()
    value = value * torch.rsqrt((value * value).mean(-1, keepdim=True) + eps)
    return value.to(x.dtype) * torch.as_tensor(weight).to(x.dtype)


def apply_rotary_cast(x, rope_theta: float, positions):
    """``rotary.py:16-39`` for a torch ``[B, T, H, D]`` tensor at ``positions [B, T]``."""
    torch = _torch()
    d = x.shape[-1]
    a = torch.tensor(angles(positions, rope_theta, d))[:, :, None, :]
    a = torch.cat((a, a), dim=-1)
    first, second = x[..., : d // 2], x[..., d // 2 :]
    rotated = torch.cat((-second, first), dim=-1)
    return x * torch.cos(a).to(x.dtype) + rotated * torch.sin(a).to(x.dtype)


def qk_norm_rope_cast(q, k, q_gain, k_gain, positions, eps: float, rope_theta: float):
    """The prologue on torch tensors in their own dtype, cast points as the reference."""
    return (apply_rotary_cast(rms_norm_cast(q, q_gain, eps), rope_theta, positions),
            apply_rotary_cast(rms_norm_cast(k, k_gain, eps), rope_theta, positions))


def segment_positions(segment_ids) -> np.ndarray:
    seg = np.asarray(segment_ids)
    pos = np.zeros(seg.shape, np.int32)
    for row in range(seg.shape[0]):
        start = 0
        for t in range(seg.shape[1]):
            if t == 0 or seg[row, t] != seg[row, t - 1]:
                start = t
            pos[row, t] = 0 if seg[row, t] == 0 else t - start
    return pos
