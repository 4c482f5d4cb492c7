"""Validity grids and the brute-force tile map (CPU, NumPy, integer/bool).

Test infrastructure only (see ``oracle/__init__.py``).

Restated semantics (``/root/reference`` paths):

* ``packed_valid``   -- ``src/minifield_training/kernels/attention.py:79-108``
  (causal, same nonzero segment, both tokens active; inactive queries fall
  back to attending to themselves).
* ``bidirectional_valid`` -- ``src/minifield_training/kernels/bidirectional.py:21-31``
  (with segment ids: same segment, both active; without: key mask only and
  rows of examples with no active key are zeroed).
* ``cached_valid``   -- ``attention.py:280-281`` (``j < valid_length[b]``).
* ``useful_grid``    -- the grid whose entries are real work: ``valid`` with
  the self-fallback rows of inactive queries removed (their outputs are
  multiplied by 0 at ``attention.py:261``).
* ``tile_map``       -- brute-force reduction of ``useful_grid`` over
  ``tile_q x tile_k`` tiles: 0 EMPTY (no useful entry), 2 FULL (every entry
  useful), 1 PARTIAL.  The grid is padded to whole tiles with invalid
  entries, so a tile reaching past the sequence end is never FULL.

Pinned by: the reference's fixture layouts (``tests/kernels/test_attention.py:316-319``,
``tests/batching/test_packing.py:24-26``, ``:87-89``,
``tests/batching/test_pointer.py:155-157``, ``tests/kernels/test_bidirectional.py:48``)
whose grids are checked element by element against per-pair loops written from
the reference's prose, plus tile maps checked against a per-tile Python loop.
"""

from __future__ import annotations

import numpy as np

EMPTY, PARTIAL, FULL = 0, 1, 2

MODE_PACKED_CAUSAL = 0  # dense_packed_causal_attention
MODE_PACKED_BIDIR = 1  # bidirectional.attention with segment_ids
MODE_KEYMASK_BIDIR = 2  # bidirectional.attention without segment_ids


def packed_valid(attention_mask: np.ndarray, segment_ids: np.ndarray):
    """``(valid [B,T,T], active [B,T])`` of ``attention.py:94-108``."""
    seg = np.asarray(segment_ids)
    t = seg.shape[1]
    pos = np.arange(t)
    causal = pos[:, None] >= pos[None, :]
    active = (np.asarray(attention_mask) > 0) & (seg != 0)
    same = seg[:, :, None] == seg[:, None, :]
    valid = (
        causal[None]
        & same
        & (seg[:, :, None] != 0)
        & active[:, None, :]
        & active[:, :, None]
    )
    valid = valid | ((~active)[:, :, None] & (pos[:, None] == pos[None, :])[None])
    return valid, active


def bidirectional_valid(mask: np.ndarray, segment_ids: np.ndarray | None,
                        query_length: int | None = None):
    """``(valid [B,T,S], present [B,T])`` of ``bidirectional.py:21-31``."""
    mask = np.asarray(mask)
    if segment_ids is None:
        b, s = mask.shape
        t = s if query_length is None else query_length
        valid = np.broadcast_to(mask.astype(bool)[:, None, :], (b, t, s))
        present = np.broadcast_to(mask.astype(bool).any(-1)[:, None], (b, t))
        return valid.copy(), present.copy()
    seg = np.asarray(segment_ids)
    active = mask.astype(bool) & (seg != 0)
    valid = (seg[:, :, None] == seg[:, None, :]) & active[:, :, None] & active[:, None, :]
    return valid, active


def cached_valid(valid_length, batch: int, capacity: int) -> np.ndarray:
    """``[B, S]`` of ``attention.py:280-281``; scalar or ``[B]`` lengths."""
    lengths = np.broadcast_to(np.asarray(valid_length).reshape(-1), (batch,))
    return np.arange(capacity)[None, :] < lengths[:, None]


def useful_grid(mode: int, mask: np.ndarray, segment_ids: np.ndarray | None,
                query_length: int | None = None) -> np.ndarray:
    """Head-independent grid of pairs that carry work (``[B, T, S]``)."""
    if mode == MODE_PACKED_CAUSAL:
        valid, active = packed_valid(mask, segment_ids)
        return valid & active[:, :, None]
    if mode == MODE_PACKED_BIDIR:
        valid, _ = bidirectional_valid(mask, segment_ids)
        return valid
    if mode == MODE_KEYMASK_BIDIR:
        valid, present = bidirectional_valid(mask, None, query_length)
        return valid & present[:, :, None]
    raise ValueError(mode)


# Sentinels of inactive tokens: outside the int32 range of segment ids, and
# different for queries and keys, so they never match anything.
Q_INACTIVE = -(1 << 40)
K_INACTIVE = -(1 << 41)


def _token_ids(mode: int, mask: np.ndarray, segment_ids, query_length):
    """Canonical per-token ids (int64): a query attends to a key iff the ids
    match (plus causality).  Inactive queries get ``Q_INACTIVE``, inactive
    keys ``K_INACTIVE``."""
    mask = np.asarray(mask)
    if mode == MODE_KEYMASK_BIDIR:
        b, s = mask.shape
        t = s if query_length is None else query_length
        present = mask.astype(bool).any(-1)
        qid = np.where(present[:, None], 1, Q_INACTIVE) * np.ones((b, t), np.int64)
        kid = np.where(mask.astype(bool), 1, K_INACTIVE).astype(np.int64)
        return qid, kid
    seg = np.asarray(segment_ids).astype(np.int64)
    if mode == MODE_PACKED_CAUSAL:
        active = (mask > 0) & (seg != 0)
    else:
        active = mask.astype(bool) & (seg != 0)
    return np.where(active, seg, Q_INACTIVE), np.where(active, seg, K_INACTIVE)


def tile_map(mode: int, mask: np.ndarray, segment_ids: np.ndarray | None,
             tile_q: int, tile_k: int, query_length: int | None = None) -> np.ndarray:
    """Brute-force EMPTY/PARTIAL/FULL map ``[B, nQ, nK]`` (uint8).

    Evaluated one query tile at a time over the padded grid so the largest
    BASELINE row (32768 tokens) never materialises more than
    ``tile_q x S`` booleans.
    """
    qid, kid = _token_ids(mode, mask, segment_ids, query_length)
    b, t = qid.shape
    s = kid.shape[1]
    nq, nk = -(-t // tile_q), -(-s // tile_k)
    qid = np.pad(qid, ((0, 0), (0, nq * tile_q - t)), constant_values=Q_INACTIVE)
    kid = np.pad(kid, ((0, 0), (0, nk * tile_k - s)), constant_values=K_INACTIVE)
    causal = mode == MODE_PACKED_CAUSAL
    kpos = np.arange(nk * tile_k)
    out = np.zeros((b, nq, nk), dtype=np.uint8)
    for row in range(b):
        for qi in range(nq):
            qs = slice(qi * tile_q, (qi + 1) * tile_q)
            grid = qid[row, qs, None] == kid[row, None, :]
            if causal:
                grid &= kpos[None, :] <= np.arange(qi * tile_q, (qi + 1) * tile_q)[:, None]
            tiles = grid.reshape(tile_q, nk, tile_k)
            anyv = tiles.any(axis=(0, 2))
            allv = tiles.all(axis=(0, 2))
            out[row, qi] = np.where(allv, FULL, np.where(anyv, PARTIAL, EMPTY))
    return out


def tile_map_loops(grid: np.ndarray, tile_q: int, tile_k: int) -> np.ndarray:
    """Per-tile Python loop over an explicit ``[B, T, S]`` grid (tiny inputs);
    the independent check of ``tile_map``."""
    b, t, s = grid.shape
    nq, nk = -(-t // tile_q), -(-s // tile_k)
    out = np.zeros((b, nq, nk), dtype=np.uint8)
    for row in range(b):
        for qi in range(nq):
            for kj in range(nk):
                seen = full = 0
                total = 0
                for i in range(qi * tile_q, (qi + 1) * tile_q):
                    for j in range(kj * tile_k, (kj + 1) * tile_k):
                        total += 1
                        inside = i < t and j < s and bool(grid[row, i, j])
                        seen |= inside
                        full += inside
                out[row, qi, kj] = FULL if full == total else (PARTIAL if seen else EMPTY)
    return out
