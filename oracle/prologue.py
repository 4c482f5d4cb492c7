"""CPU restatement of the attention prologue: QK RMS norm and rotary embeddings.

Test infrastructure only (the product never imports ``oracle``).

* ``rms_norm`` follows ``src/minifield_training/kernels/normalization.py:7-22``
  (fp32 statistics; the normalised value is cast to the tensor dtype before
  the gain multiply).
* ``apply_rotary`` follows ``kernels/rotary.py:7-39``: single-precision
  frequencies ``theta ** (-arange(0, D, 2) / D)`` and angles
  ``f32(position) * freq``, split-half rotation ``(-x[D/2:], x[:D/2])``.
  Evaluated in float64 from those single-precision angles.
* ``rotate_pairs`` is an independent restatement: a 2x2 rotation matrix per
  dimension pair (i, i + D/2), the method of ``tests/layers/test_blocks.py:116-121``.
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
    """``rope_theta ** (-arange(0, D, 2) / D)`` in float32 (rotary.py:33-35)."""
    exps = -(np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim))
    return (np.float32(rope_theta) ** exps).astype(np.float32)


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
