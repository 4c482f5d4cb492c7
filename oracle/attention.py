"""Masked softmax attention: FP64 forward/VJP and bf16 cast-point emulation.

Test infrastructure only (see ``oracle/__init__.py``).

Restated from (``/root/reference`` paths):

* ``dense_fp64``      -- ``src/minifield_training/kernels/attention.py:12-34``
  and the reference's own FP64 oracle ``tests/kernels/test_attention.py:40-58``
  (GQA by ``repeat``: query head ``h`` reads KV head ``h // (Hq/Hkv)``; logits
  scaled by ``D ** -0.5``; masked entries filled with the float minimum).
* ``packed_causal_fp64`` -- ``attention.py:245-261`` (inactive rows times 0).
* ``bidirectional_fp64`` -- ``kernels/bidirectional.py:7-35`` (``where(present,
  result, 0)``).
* ``cached_fp64``      -- ``attention.py:264-282``.
* ``vjp_fp64``         -- the analytic VJP of the above (the reference takes it
  from JAX autodiff): ``dV = P^T dO``, ``dS = P * (dO V^T - rowsum(dO * O))``,
  ``dQ = s dS K``, ``dK = s dS^T Q``, GQA gradients summed over the group.
* ``dense_bf16_einsum`` -- the bf16 cast points of ``attention.py:23-33``:
  bf16 logits, scaled in bf16, fp32 masked softmax, bf16 probabilities, bf16
  output.
* ``sdpa_bf16``        -- XLA SDPA's cast points used by
  ``bidirectional.py:32-34`` (jax 0.7.2, upstream, not vendored): fp32 logits,
  fp32 softmax, probabilities cast to the value dtype, bf16 output.

Pinned by: the analytical fixtures of ``tests/kernels/test_bidirectional.py:12-26``
and ``:41-65`` (zero q/k averages and their dV gradients), central differences
of the forward (method of ``tests/layers/test_blocks.py:156-174``), the
packed-equals-independent-rows invariant (``tests/layers/test_blocks.py:342-382``),
segment-id permutation invariance, a single-segment case equal to a textbook
``scipy.special.softmax`` attention, and the grouped (per-segment) evaluation
agreeing with the dense grid.  The two bf16 emulations are pinned by closed
forms that move when a cast point moves: rounded probabilities (zero q/k over
six keys: ``bf16(1/6) * 100`` rounds to 16.75 where ``100/6`` rounds to 16.625),
the einsum's bf16 logits against SDPA's fp32 logits (raw logits 100 and 100.25
give P1 = 0.5 against 0.5078125), the rounded output, single-key rows and the
two agreeing bit for bit when every logit is representable in bf16.
"""

from __future__ import annotations

import numpy as np

from . import masks as _masks

F64_MIN = float(np.finfo(np.float64).min)
F32_MIN = float(np.finfo(np.float32).min)


def _expand_kv(x: np.ndarray, q_heads: int) -> np.ndarray:
    return np.repeat(x, q_heads // x.shape[2], axis=2)


def dense_fp64(query, key, value, valid, scale=None):
    """Masked softmax attention over a ``[B, (1|H), T, S]`` validity grid.

    Returns ``(out [B,T,H,D], probabilities [B,H,T,S])`` in float64.
    """
    q = np.asarray(query, np.float64)
    k = _expand_kv(np.asarray(key, np.float64), q.shape[2])
    v = _expand_kv(np.asarray(value, np.float64), q.shape[2])
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    scores = np.einsum("bthd,bshd->bhts", q, k) * scale
    scores = np.where(valid, scores, F64_MIN)
    shifted = scores - scores.max(-1, keepdims=True)
    e = np.exp(shifted)
    probs = e / e.sum(-1, keepdims=True)
    return np.einsum("bhts,bshd->bthd", probs, v), probs


def packed_causal_fp64(query, key, value, attention_mask, segment_ids):
    valid, active = _masks.packed_valid(attention_mask, segment_ids)
    out, probs = dense_fp64(query, key, value, valid[:, None])
    return out * active[:, :, None, None], probs, active


def bidirectional_fp64(query, key, value, mask, segment_ids=None):
    valid, present = _masks.bidirectional_valid(
        mask, segment_ids, np.asarray(query).shape[1])
    out, probs = dense_fp64(query, key, value, valid[:, None])
    return np.where(present[:, :, None, None], out, 0.0), probs, present


def cached_fp64(query, key, value, valid_length):
    b, s = np.asarray(key).shape[:2]
    valid = _masks.cached_valid(valid_length, b, s)
    out, probs = dense_fp64(query, key, value, valid[:, None, None, :])
    return out, probs


def vjp_fp64(query, key, value, probs, row_keep, d_out, scale=None):
    """Gradients of ``out = keep * softmax(s QK^T) V`` w.r.t. q, k, v.

    ``row_keep [B, T]`` is the active/present indicator that multiplies (or
    selects) each output row; rows it drops receive no gradient.
    """
    q = np.asarray(query, np.float64)
    kvh = np.asarray(key).shape[2]
    k = _expand_kv(np.asarray(key, np.float64), q.shape[2])
    v = _expand_kv(np.asarray(value, np.float64), q.shape[2])
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    do = np.asarray(d_out, np.float64) * np.asarray(row_keep, np.float64)[:, :, None, None]
    out = np.einsum("bhts,bshd->bthd", probs, v)
    dv = np.einsum("bhts,bthd->bshd", probs, do)
    dp = np.einsum("bthd,bshd->bhts", do, v)
    delta = np.einsum("bthd,bthd->bht", do, out)
    ds = probs * (dp - delta[..., None])
    dq = np.einsum("bhts,bshd->bthd", ds, k) * scale
    dk = np.einsum("bhts,bthd->bshd", ds, q) * scale
    b, s, h, d = dk.shape
    dk = dk.reshape(b, s, kvh, h // kvh, d).sum(3)
    dv = dv.reshape(b, s, kvh, h // kvh, d).sum(3)
    return dq, dk, dv


# --------------------------------------------------------------------------
# Grouped evaluation: every useful pair shares one canonical id, so each id's
# token set can be attended on its own.  O(sum L^2) instead of O(T^2).
# --------------------------------------------------------------------------


def grouped_fp64(mode, query, key, value, mask, segment_ids, d_out=None):
    """Forward (and optional VJP) evaluated id-group by id-group.

    Exact restatement of the dense grid for the three packed modes: pairs
    with different canonical ids never interact and rows with no useful key
    produce 0.  Returns ``out`` or ``(out, dq, dk, dv)`` in float64.
    """
    q = np.asarray(query, np.float64)
    k = np.asarray(key, np.float64)
    v = np.asarray(value, np.float64)
    b, t, hq, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = d ** -0.5
    qid, kid = _masks._token_ids(mode, mask, segment_ids, t)
    causal = mode == _masks.MODE_PACKED_CAUSAL
    out = np.zeros_like(q)
    grads = d_out is not None
    if grads:
        do_all = np.asarray(d_out, np.float64)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for row in range(b):
        for ident in np.unique(qid[row][qid[row] != _masks.Q_INACTIVE]):
            qi = np.flatnonzero(qid[row] == ident)
            kj = np.flatnonzero(kid[row] == ident)
            if kj.size == 0:
                continue
            allowed = (kj[None, :] <= qi[:, None]) if causal else np.ones((qi.size, kj.size), bool)
            has = allowed.any(1)
            for h in range(hq):
                kh = h // g
                sc = q[row, qi, h] @ k[row, kj, kh].T * scale
                sc = np.where(allowed, sc, -np.inf)
                m = np.where(has, sc.max(1), 0.0)
                e = np.where(allowed, np.exp(sc - m[:, None]), 0.0)
                den = e.sum(1)
                p = e / np.where(den > 0, den, 1.0)[:, None]
                o = p @ v[row, kj, kh]
                out[row, qi, h] = o
                if grads:
                    go = do_all[row, qi, h]
                    dv[row, kj, kh] += p.T @ go
                    dp = go @ v[row, kj, kh].T
                    delta = (go * o).sum(1)
                    ds = p * (dp - delta[:, None])
                    dq[row, qi, h] += ds @ k[row, kj, kh] * scale
                    dk[row, kj, kh] += ds.T @ q[row, qi, h] * scale
    if grads:
        return out, dq, dk, dv
    return out


# --------------------------------------------------------------------------
# bf16 cast-point emulation (torch on CPU; NumPy has no bfloat16)
# --------------------------------------------------------------------------


def _torch():
    import torch  # local import: only the bf16 emulation needs it
    return torch


def dense_bf16_einsum(query, key, value, valid):
    """``attention.py:23-33`` for bf16 operands (all tensors torch-CPU)."""
    torch = _torch()
    hq = query.shape[2]
    g = hq // key.shape[2]
    k = key.repeat_interleave(g, dim=2).float()
    v = value.repeat_interleave(g, dim=2).float()
    scores = torch.einsum("bthd,bshd->bhts", query.float(), k).to(torch.bfloat16)
    scores = scores * torch.tensor(query.shape[-1] ** -0.5, dtype=torch.bfloat16)
    scores = torch.where(valid, scores.float(), torch.tensor(F32_MIN))
    probs = torch.softmax(scores, dim=-1).to(torch.bfloat16)
    return torch.einsum("bhts,bshd->bthd", probs.float(), v).to(torch.bfloat16)


def sdpa_bf16(query, key, value, valid):
    """XLA SDPA cast points (fp32 logits and softmax, bf16 probabilities)."""
    torch = _torch()
    hq = query.shape[2]
    g = hq // key.shape[2]
    k = key.repeat_interleave(g, dim=2).float()
    v = value.repeat_interleave(g, dim=2).float()
    logits = torch.einsum("bthd,bshd->bhts", query.float(), k) * (query.shape[-1] ** -0.5)
    logits = torch.where(valid, logits, torch.tensor(-0.7 * float(np.finfo(np.float32).max)))
    probs = torch.softmax(logits, dim=-1).to(value.dtype)
    return torch.einsum("bhts,bshd->bthd", probs.float(), v).to(value.dtype)
