"""Row packing and the seeded BASELINE workload generators (CPU, NumPy).

Test infrastructure only (see ``oracle/__init__.py``).

``pack`` restates the reference packer's contract:

* ``_first_fit_decreasing``  -- ``src/minifield_training/batching/packing.py:34-66``
  (longest first, ties in input order, first row with room, overflow raises).
* ``pack``                   -- ``packing.py:74-102`` (segment id ``index + 1``,
  0 for padding, positions restart at 0 in every sequence).

Pinned by the hand-derived layouts of ``tests/batching/test_packing.py:11-29``,
``:44-48`` and ``:74-88`` (restated in ``tests/test_oracle_packing.py``) and by
round-trip/invariant checks on random inputs.

The workload generators follow the BASELINE configuration text (C1..C5); their
seeds are fixed here so every test, the bench and the smoke run draw the same
inputs.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Sequence

import numpy as np


@dataclasses.dataclass(frozen=True)
class Placement:
    row: int
    start: int
    length: int


@dataclasses.dataclass(frozen=True)
class PackedRows:
    input_ids: np.ndarray
    segment_ids: np.ndarray
    positions: np.ndarray
    placements: tuple[Placement, ...]


def first_fit_decreasing(
    lengths: Sequence[int], length: int, rows: int | None
) -> tuple[list[tuple[int, int]], int]:
    """(row, start) per sequence and the number of rows used.

    Follows ``batching/packing.py:34-66``: visit sequences by decreasing
    length (stable, so ties keep input order) and put each in the first row
    whose fill plus the size fits.
    """
    if length < 1:
        raise ValueError("Packed row length must be positive")
    if any(size < 1 or size > length for size in lengths):
        raise ValueError(
            f"Every packed sequence needs 1 to {length} tokens; got "
            f"{min(lengths)} to {max(lengths)}"
        )
    order = sorted(range(len(lengths)), key=lambda i: -lengths[i])
    fill: list[int] = []
    where = [(0, 0)] * len(lengths)
    for index in order:
        size = lengths[index]
        target = len(fill)
        for row, used in enumerate(fill):
            if used + size <= length:
                target = row
                break
        if target == len(fill):
            if rows is not None and target == rows:
                raise ValueError(
                    f"Sequences need more than {rows} packed rows of "
                    f"{length} tokens"
                )
            fill.append(0)
        where[index] = (target, fill[target])
        fill[target] += size
    return where, len(fill)


def rows_required(lengths: Sequence[int], length: int) -> int:
    return first_fit_decreasing(lengths, length, None)[1]


def pack(
    sequences: Sequence[Sequence[int]], rows: int, length: int, *, pad_token_id: int
) -> PackedRows:
    """Pack whole sequences into fixed rows (``batching/packing.py:74-102``)."""
    if rows < 1:
        raise ValueError("Packed row count must be positive")
    sizes = [len(s) for s in sequences]
    where, _ = first_fit_decreasing(sizes, length, rows)
    ids = np.full((rows, length), pad_token_id, dtype=np.int32)
    seg = np.zeros((rows, length), dtype=np.int32)
    pos = np.zeros((rows, length), dtype=np.int32)
    placed = []
    for index, (tokens, (row, start)) in enumerate(zip(sequences, where)):
        stop = start + len(tokens)
        ids[row, start:stop] = tokens
        seg[row, start:stop] = index + 1
        pos[row, start:stop] = np.arange(len(tokens))
        placed.append(Placement(row, start, len(tokens)))
    return PackedRows(ids, seg, pos, tuple(placed))


# --------------------------------------------------------------------------
# Seeded BASELINE workloads
# --------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class Workload:
    """One attention workload: integer layout plus shape metadata."""

    name: str
    batch: int
    length: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: str  # "float32" | "bfloat16"
    causal: bool
    segment_ids: np.ndarray  # [B, T] int32, 0 = padding
    attention_mask: np.ndarray  # [B, T] int32
    qkv_scale: float
    seed: int


def _rows_sequential(
    draw, rows: int, length: int, first_id: int = 1
) -> np.ndarray:
    """Fill each row left to right with drawn lengths; the first draw that
    does not fit ends the row and the rest is tail padding."""
    seg = np.zeros((rows, length), dtype=np.int32)
    for row in range(rows):
        cursor, ident = 0, first_id
        while True:
            size = int(draw())
            if cursor + size > length:
                break
            seg[row, cursor : cursor + size] = ident
            cursor += size
            ident += 1
    return seg


def _rows_first_fit(draw, rows: int, length: int) -> np.ndarray:
    """Greedy first-fit in draw order: each drawn segment goes to the first
    row with room; the first segment that fits nowhere stops packing.  Ids
    are global draw order + 1 (as ``pack`` numbers input order)."""
    fill = [0] * rows
    seg = np.zeros((rows, length), dtype=np.int32)
    ident = 1
    while True:
        size = int(draw())
        row = next((r for r in range(rows) if fill[r] + size <= length), None)
        if row is None:
            break
        seg[row, fill[row] : fill[row] + size] = ident
        fill[row] += size
        ident += 1
    return seg


def make_workload(name: str) -> Workload:
    """The five BASELINE configurations with fixed seeds."""
    if name == "C1":
        rng = np.random.default_rng(101)
        rows, length = 2, 256
        seg = np.zeros((rows, length), dtype=np.int32)
        for row in range(rows):
            sizes = rng.integers(1, 65, size=4)  # 4 segments, sum <= 256
            cursor = 0
            for index, size in enumerate(sizes):
                seg[row, cursor : cursor + size] = index + 1
                cursor += int(size)
        return Workload("C1", rows, length, 4, 2, 64, "float32", True, seg,
                        (seg != 0).astype(np.int32), 1.0, 101)
    if name == "C2":
        rng = np.random.default_rng(202)
        lo, hi = np.log(32.0), np.log(2048.0)
        seg = _rows_first_fit(lambda: np.floor(np.exp(rng.uniform(lo, hi))), 8, 4096)
        return Workload("C2", 8, 4096, 16, 8, 64, "bfloat16", False, seg,
                        (seg != 0).astype(np.int32), 0.5, 202)
    if name == "C3":
        rng = np.random.default_rng(303)
        seg = _rows_sequential(lambda: max(16, rng.geometric(1.0 / 512.0)), 4, 8192)
        return Workload("C3", 4, 8192, 16, 8, 64, "bfloat16", True, seg,
                        (seg != 0).astype(np.int32), 1.0, 303)
    if name == "C5":
        rng = np.random.default_rng(505)
        seg = _rows_sequential(lambda: rng.integers(16, 129), 1, 32768)
        return Workload("C5", 1, 32768, 16, 8, 64, "bfloat16", True, seg,
                        (seg != 0).astype(np.int32), 1.0, 505)
    raise KeyError(name)


@dataclasses.dataclass(frozen=True)
class DecodeWorkload:
    name: str
    batch: int
    capacity: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: str
    valid_length: np.ndarray  # [B] int32
    seed: int


def make_decode_workload(name: str = "C4") -> DecodeWorkload:
    if name != "C4":
        raise KeyError(name)
    rng = np.random.default_rng(404)
    lengths = rng.integers(128, 8193, size=64).astype(np.int32)
    return DecodeWorkload("C4", 64, 8192, 16, 8, 64, "bfloat16", lengths, 404)


def segment_runs(segment_ids: np.ndarray) -> list[list[tuple[int, int, int]]]:
    """Per row, the maximal runs ``(id, start, stop)`` of equal nonzero ids."""
    out = []
    for row in np.asarray(segment_ids):
        runs, start = [], 0
        for pos in range(1, len(row) + 1):
            if pos == len(row) or row[pos] != row[start]:
                if row[start] != 0:
                    runs.append((int(row[start]), start, pos))
                start = pos
        out.append(runs)
    return out
