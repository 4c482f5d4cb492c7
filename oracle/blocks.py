"""FP64 restatement of the reference's attention and conv blocks around this path.

Test infrastructure only (the product never imports ``oracle``).  These are
the callers of the hot path (§ a11 of the scope), composed from the pinned
oracle pieces so the GPU tests can check the HIP ops in the context the
reference calls them in:

* ``attention_block`` / ``attention_block_packed`` -- ``layers/attention.py:110-137``
  and ``:214-243``: pre-norm, q/k/v projections, QK RMS norm + RoPE
  (``oracle.prologue``), causal (packed: same-segment) attention
  (``oracle.attention``), the out projection and residual, then the SwiGLU
  tail (``layers/feed_forward.py:25-40``).
* ``encoder_block`` -- ``models/lfm2_5/encoder.py:64-110``: the same pre-norm
  block with bidirectional packed attention, or the gated centered
  convolution (``layers/convolution.py:29-37`` input projection with the
  attention mask, ``oracle.convolution``).
* ``loop_attention_block`` -- an independent evaluation with token/head loops
  and 2x2 rotation matrices per dimension pair, the method of the reference
  test's own reference (``tests/layers/test_blocks.py:98-134``); it pins the
  composed ``attention_block``.

Weights are plain dicts of float64 arrays: ``operator_norm [H]``, ``query
[Hq*D, H]``, ``key``/``value [Hkv*D, H]``, ``out [H, Hq*D]``, ``query_norm``,
``key_norm [D]``; conv: ``operator_norm``, ``in_proj [3C, H]``, ``conv [C, K]``,
``out [H, C]``; SwiGLU: ``norm [H]``, ``gate``/``up [F, H]``, ``down [H, F]``.
"""

from __future__ import annotations

import numpy as np

from . import attention as _att
from . import convolution as _conv
from . import masks as _masks
from . import prologue as _pro


def rms(x, gain, eps):
    """``kernels/normalization.py:7-22`` in FP64."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(gain, np.float64)


def swiglu(x, ffn, eps):
    """``layers/feed_forward.py:25-40``: ``x + down(silu(gate(n)) * up(n))``, ``n = rms(x)``."""
    n = rms(x, ffn["norm"], eps)
    g = n @ ffn["gate"].T
    return x + ((g / (1 + np.exp(-g))) * (n @ ffn["up"].T)) @ ffn["down"].T


def project_qkv(x, w, head_dim, eps, positions, rope_theta):
    """``layers/attention.py:61-97``: normed, projected, QK-normed and rotated q/k, raw v."""
    b, t, _ = x.shape
    hidden = rms(x, w["operator_norm"], eps)
    q = (hidden @ w["query"].T).reshape(b, t, -1, head_dim)
    k = (hidden @ w["key"].T).reshape(b, t, -1, head_dim)
    v = (hidden @ w["value"].T).reshape(b, t, -1, head_dim)
    if positions is None:
        positions = np.broadcast_to(np.arange(t), (b, t))
    q, k = _pro.qk_norm_rope(q, k, w["query_norm"], w["key_norm"], positions, eps, rope_theta)
    return q, k, v


def _residual(x, attended, w, ffn, eps):
    return swiglu(x + attended.reshape(x.shape[0], x.shape[1], -1) @ w["out"].T, ffn, eps)


def attention_block(x, w, ffn, attention_mask, *, head_dim, rope_theta, eps, positions=None):
    """Full-sequence causal block (``layers/attention.py:110-137``): the packed block
    with one segment per row."""
    ones = np.ones(np.asarray(x).shape[:2], np.int32)
    return attention_block_packed(x, w, ffn, attention_mask, ones, positions, head_dim=head_dim,
                                  rope_theta=rope_theta, eps=eps)


def attention_block_packed(x, w, ffn, attention_mask, segment_ids, positions, *, head_dim,
                           rope_theta, eps):
    """``layers/attention.py:214-243``."""
    x = np.asarray(x, np.float64)
    q, k, v = project_qkv(x, w, head_dim, eps, positions, rope_theta)
    attended = _att.grouped_fp64(_masks.MODE_PACKED_CAUSAL, q, k, v, attention_mask, segment_ids)
    return _residual(x, attended, w, ffn, eps)


def encoder_block(x, params, ffn, mask, segment_ids, positions, *, kind, head_dim, rope_theta,
                  eps):
    """``models/lfm2_5/encoder.py:64-110`` with packed ids (kind ``"conv"`` or ``"attention"``)."""
    x = np.asarray(x, np.float64)
    if kind == "conv":
        norm = rms(x, params["operator_norm"], eps)
        hidden = norm * np.asarray(mask, np.float64)[..., None]
        b_gate, c_gate, values = np.split(hidden @ params["in_proj"].T, 3, axis=-1)
        mixed = c_gate * _conv.centered(b_gate * values, params["conv"], segment_ids)
        return swiglu(x + mixed @ params["out"].T, ffn, eps)
    q, k, v = project_qkv(x, params, head_dim, eps, positions, rope_theta)
    attended = _att.grouped_fp64(_masks.MODE_PACKED_BIDIR, q, k, v, mask, segment_ids)
    return _residual(x, attended, params, ffn, eps)


def loop_attention_block(x, w, ffn, *, head_dim, rope_theta, eps):
    """Causal block over an all-valid row by token/head loops (one row, no padding)."""
    x = np.asarray(x, np.float64)
    _, t, _ = x.shape
    hq = w["query"].shape[0] // head_dim
    hkv = w["key"].shape[0] // head_dim
    half = head_dim // 2
    freq = _pro.frequencies(rope_theta, head_dim).astype(np.float64)
    hidden = rms(x, w["operator_norm"], eps)[0]
    q = rms((hidden @ w["query"].T).reshape(t, hq, head_dim), w["query_norm"], eps)
    k = rms((hidden @ w["key"].T).reshape(t, hkv, head_dim), w["key_norm"], eps)
    v = (hidden @ w["value"].T).reshape(t, hkv, head_dim)
    for token in range(t):
        for i in range(half):
            angle = float(np.float32(np.float32(token) * np.float32(freq[i])))
            rot = np.array([[np.cos(angle), -np.sin(angle)], [np.sin(angle), np.cos(angle)]])
            for arr in (q, k):
                pair = arr[token][:, [i, i + half]] @ rot.T
                arr[token][:, i], arr[token][:, i + half] = pair[:, 0], pair[:, 1]
    attended = np.zeros_like(q)
    for token in range(t):
        for head in range(hq):
            kv = head // (hq // hkv)
            scores = np.array([q[token, head] @ k[src, kv] / np.sqrt(head_dim)
                               for src in range(token + 1)])
            p = np.exp(scores - scores.max())
            attended[token, head] = (p / p.sum()) @ v[: token + 1, kv]
    return swiglu(x + (attended.reshape(1, t, -1) @ w["out"].T), ffn, eps)


def random_weights(rng, hidden, q_heads, kv_heads, head_dim, ffn_dim, channels=None,
                   kernel_size=3):
    """Seeded attention (or conv) and SwiGLU weights of the shapes above."""
    def normal(*shape, s=0.3):
        return rng.normal(0.0, s, shape)
    attn = {"operator_norm": 1 + 0.1 * normal(hidden), "query": normal(q_heads * head_dim, hidden, s=hidden ** -0.5),
            "key": normal(kv_heads * head_dim, hidden, s=hidden ** -0.5),
            "value": normal(kv_heads * head_dim, hidden, s=hidden ** -0.5),
            "out": normal(hidden, q_heads * head_dim, s=(q_heads * head_dim) ** -0.5),
            "query_norm": 1 + 0.1 * normal(head_dim), "key_norm": 1 + 0.1 * normal(head_dim)}
    ffn = {"norm": 1 + 0.1 * normal(hidden), "gate": normal(ffn_dim, hidden, s=hidden ** -0.5),
           "up": normal(ffn_dim, hidden, s=hidden ** -0.5),
           "down": normal(hidden, ffn_dim, s=ffn_dim ** -0.5)}
    if channels is None:
        return attn, ffn
    conv = {"operator_norm": 1 + 0.1 * normal(hidden), "in_proj": normal(3 * channels, hidden, s=hidden ** -0.5),
            "conv": normal(channels, kernel_size, s=0.5), "out": normal(hidden, channels, s=channels ** -0.5)}
    return attn, ffn, conv
