"""Useful-work accounting for the roofline (CPU, NumPy).

Test infrastructure only (see ``oracle/__init__.py``).

Definitions follow the BASELINE accounting:

* useful pairs ``P`` = number of true entries of ``masks.useful_grid`` (per
  head); for contiguous segments that is ``sum L(L+1)/2`` (causal) or
  ``sum L^2`` (bidirectional).
* FLOPs: forward ``4 D Hq P``, backward ``8 D Hq P``, forward+backward
  ``12 D Hq P`` (the FlashAttention-2 ``14 D Hq P`` convention is reported
  separately and labelled).
* attention bytes: forward ``2(|q|+|k|+|v|+|o|) + 4|lse|``; backward
  ``2(|q|+|k|+|v|+|o|+|dO|+|dq|+|dk|+|dv|) + 4|lse|`` (bf16 element = 2 B).
* decode bytes: ``sum_b len_b * Hkv * D * 2 B * 2 + 2 * B * Hq * D * 2 + 4 B``.

Pinned by: ``useful_pairs_closed_form`` (the ``L(L+1)/2`` / ``L^2`` sums over
contiguous runs) equals the count of the brute-force grid on every BASELINE
layout (``tests/test_oracle_masks.py``).
"""

from __future__ import annotations

import numpy as np

from . import masks as _masks
from . import packing as _packing


def useful_pairs(mode, mask, segment_ids, query_length=None) -> int:
    """Count of useful (query, key) pairs per head, counted id group by id
    group (exact for non-contiguous ids too)."""
    qid, kid = _masks._token_ids(mode, mask, segment_ids, query_length)
    total = 0
    for row in range(qid.shape[0]):
        qs, kc = np.unique(qid[row][qid[row] != _masks.Q_INACTIVE], return_counts=True)
        for ident, nq in zip(qs, kc):
            kpos = np.flatnonzero(kid[row] == ident)
            if mode == _masks.MODE_PACKED_CAUSAL:
                qpos = np.flatnonzero(qid[row] == ident)
                total += int(np.searchsorted(kpos, qpos, side="right").sum())
            else:
                total += int(nq) * int(kpos.size)
    return total


def useful_pairs_closed_form(segment_ids, causal: bool) -> int:
    total = 0
    for runs in _packing.segment_runs(segment_ids):
        for _, start, stop in runs:
            n = stop - start
            total += n * (n + 1) // 2 if causal else n * n
    return total


def attention_flops(pairs: int, head_dim: int, q_heads: int) -> dict:
    unit = head_dim * q_heads * pairs
    return {"fwd": 4 * unit, "bwd": 8 * unit, "fwd_bwd": 12 * unit,
            "fwd_bwd_fa2": 14 * unit}


def attention_bytes(batch, length, q_heads, kv_heads, head_dim, elem=2) -> dict:
    q = batch * length * q_heads * head_dim
    k = batch * length * kv_heads * head_dim
    lse = batch * length * q_heads
    fwd = elem * (q + k + k + q) + 4 * lse
    bwd = elem * (q + k + k + q + q + q + k + k) + 4 * lse
    return {"fwd": fwd, "bwd": bwd, "fwd_bwd": fwd + bwd}


def decode_bytes(lengths, batch, q_heads, kv_heads, head_dim) -> int:
    lengths = np.asarray(lengths, np.int64)
    return int(lengths.sum()) * kv_heads * head_dim * 2 * 2 + 2 * batch * q_heads * head_dim * 2 + 4 * batch
