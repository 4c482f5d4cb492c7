"""CPU restatement of the segmented short convolutions (test infrastructure).

* ``centered`` follows ``src/minifield_training/kernels/bidirectional.py:38-58``
  (``centered_convolution``): zero padding of ``K // 2`` on both sides, right
  crop, and with segment ids a tap counts only inside the token's nonzero
  segment.
* ``causal`` follows ``kernels/convolution.py:25-53``
  (``gated_depthwise_convolution_segmented``): left padding ``K - 1``, the
  same segment rule, gates ``c * conv(b * v)``.
Both evaluate in float64; the dtype casts are the caller's.
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
