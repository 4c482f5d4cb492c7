"""Seeded synthetic packed batches of the benchmark configurations.

Layout generators for the BASELINE configurations (C1, C2, C3, C5 packed
attention; C4 ragged decode) and their useful-work accounting.  ``bench.py``
and the smoke run use them; the test suite checks that they reproduce the
independently written generators of the CPU oracle bit for bit.
"""

from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass(frozen=True)
class Packed:
    name: str
    batch: int
    length: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: str
    causal: bool
    segment_ids: np.ndarray
    attention_mask: np.ndarray
    qkv_scale: float
    seed: int
    description: str


@dataclasses.dataclass(frozen=True)
class Decode:
    name: str
    batch: int
    capacity: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: str
    valid_length: np.ndarray
    seed: int
    description: str


def _fill_rows(draw, rows, length):
    seg = np.zeros((rows, length), dtype=np.int32)
    for row in range(rows):
        cursor, ident = 0, 1
        while True:
            size = int(draw())
            if cursor + size > length:
                break
            seg[row, cursor : cursor + size] = ident
            cursor += size
            ident += 1
    return seg


def _first_fit(draw, rows, length):
    fill = [0] * rows
    seg = np.zeros((rows, length), dtype=np.int32)
    ident = 1
    while True:
        size = int(draw())
        row = next((r for r in range(rows) if fill[r] + size <= length), None)
        if row is None:
            return seg
        seg[row, fill[row] : fill[row] + size] = ident
        fill[row] += size
        ident += 1


def packed(name: str) -> Packed:
    if name == "C1":
        rng = np.random.default_rng(101)
        seg = np.zeros((2, 256), dtype=np.int32)
        for row in range(2):
            cursor = 0
            for index, size in enumerate(rng.integers(1, 65, size=4)):
                seg[row, cursor : cursor + size] = index + 1
                cursor += int(size)
        return Packed("C1", 2, 256, 4, 2, 64, "float32", True, seg, (seg != 0).astype(np.int32),
                      1.0, 101, "tiny packed causal: 2x256, 4 segments/row, 4/2 heads, D=64, fp32")
    if name == "C2":
        rng = np.random.default_rng(202)
        lo, hi = np.log(32.0), np.log(2048.0)
        seg = _first_fit(lambda: np.floor(np.exp(rng.uniform(lo, hi))), 8, 4096)
        return Packed("C2", 8, 4096, 16, 8, 64, "bfloat16", False, seg,
                      (seg != 0).astype(np.int32), 0.5, 202,
                      "LFM2.5-350M encoder shape: 8x4096 packed, segments log-uniform 32-2048, "
                      "bidirectional within segment, 16/8 heads, D=64, bf16")
    if name == "C3":
        rng = np.random.default_rng(303)
        seg = _fill_rows(lambda: max(16, rng.geometric(1.0 / 512.0)), 4, 8192)
        return Packed("C3", 4, 8192, 16, 8, 64, "bfloat16", True, seg,
                      (seg != 0).astype(np.int32), 1.0, 303,
                      "causal packed training: 4x8192, geometric lengths mean 512, 16/8 heads, bf16")
    if name == "C5":
        rng = np.random.default_rng(505)
        seg = _fill_rows(lambda: rng.integers(16, 129), 1, 32768)
        return Packed("C5", 1, 32768, 16, 8, 64, "bfloat16", True, seg,
                      (seg != 0).astype(np.int32), 1.0, 505,
                      "long-row stress: 1x32768, lengths U[16,128], causal, 16/8 heads, bf16")
    raise KeyError(name)


def decode(name: str = "C4") -> Decode:
    if name != "C4":
        raise KeyError(name)
    rng = np.random.default_rng(404)
    lengths = rng.integers(128, 8193, size=64).astype(np.int32)
    return Decode("C4", 64, 8192, 16, 8, 64, "bfloat16", lengths, 404,
                  "ragged KV-cached decode: 64 rows x 1 token, cache lengths U[128,8192] of 8192, "
                  "16/8 heads, D=64, bf16")


def useful_pairs(segment_ids: np.ndarray, causal: bool) -> int:
    """Useful (query, key) pairs per head of contiguous runs of equal ids."""
    total = 0
    for row in np.asarray(segment_ids):
        edges = np.flatnonzero(np.diff(row)) + 1
        starts = np.concatenate(([0], edges))
        stops = np.concatenate((edges, [len(row)]))
        for a, b in zip(starts, stops):
            if row[a] != 0:
                n = int(b - a)
                total += n * (n + 1) // 2 if causal else n * n
    return total


def attention_flops(w: Packed) -> dict:
    unit = w.head_dim * w.q_heads * useful_pairs(w.segment_ids, w.causal)
    return {"fwd": 4 * unit, "dq": 2 * unit, "dkdv": 6 * unit, "bwd": 8 * unit,
            "fwd_bwd": 12 * unit, "fwd_bwd_fa2": 14 * unit}


def attention_bytes(w: Packed, elem: int = 2) -> dict:
    q = w.batch * w.length * w.q_heads * w.head_dim
    k = w.batch * w.length * w.kv_heads * w.head_dim
    lse = w.batch * w.length * w.q_heads
    fwd = elem * (2 * q + 2 * k) + 4 * lse
    bwd = elem * (4 * q + 4 * k) + 4 * lse
    return {"fwd": fwd, "bwd": bwd, "fwd_bwd": fwd + bwd}


def decode_bytes(d: Decode) -> int:
    lengths = np.minimum(np.asarray(d.valid_length, np.int64), d.capacity)
    return (int(lengths.sum()) * d.kv_heads * d.head_dim * 2 * 2
            + 2 * d.batch * d.q_heads * d.head_dim * 2 + 4 * d.batch)
