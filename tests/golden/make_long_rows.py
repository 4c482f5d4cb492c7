"""Digests of the oracle's block maps for rows longer than one list round.

The block map classifies a tile's stages in rounds of at most 1024 threads, so
rows of more than 65536 tokens (over 1024 64-row stages) take several rounds;
the BASELINE configurations stop at 32768 tokens.  The oracle needs about a
minute per such row (``oracle.masks.tile_map`` walks one query tile at a
time), too long for a GPU test, so this script evaluates it here once and
stores SHA-256 digests of every plan section (tile map, work-list counts and
entries, launch orders) in ``long_rows.json``.  The GPU test rebuilds the same
seeded layouts with ``long_row_layout`` and compares the digests of the
device's plan, section by section, with ``digest_sections``.

Run from the repository root: ``python tests/golden/make_long_rows.py``.
"""

from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import masks  # noqa: E402

OUT = HERE / "long_rows.json"
LAYOUTS = ("causal_98304", "bidir_131072", "keymask_65600x131149")


def _segments(rng, t, lo, hi, log_uniform):
    lens, tot = [], 0
    while tot < t:
        if log_uniform:
            n = int(np.exp(rng.uniform(np.log(lo), np.log(hi))))
        else:
            n = int(rng.integers(lo, hi + 1))
        lens.append(min(n, t - tot))
        tot += lens[-1]
    return np.array(lens)


def long_row_layout(name: str):
    """``(mode, mask [B, S], segment_ids [B, T] or None, T, S)`` of one seeded layout."""
    if name == "causal_98304":
        # LFM2.5-like lengths, every 9th segment padding, scattered masked tokens
        rng = np.random.default_rng(98304)
        t = 98304
        lens = _segments(rng, t, 32, 2048, True)
        ids = np.arange(1, lens.size + 1)
        ids[8::9] = 0
        seg = np.repeat(ids, lens)[None].astype(np.int32)
        mask = ((seg != 0) & (rng.random((1, t)) > 0.002)).astype(np.int32)
        return masks.MODE_PACKED_CAUSAL, mask, seg, t, t
    if name == "bidir_131072":
        # ids drawn from a small pool (negative ones included), so distant
        # segments share an id and far-off tiles are PARTIAL
        rng = np.random.default_rng(131072)
        t = 131072
        lens = _segments(rng, t, 16, 4096, False)
        pool = np.array([i for i in range(-40, 41) if i != 0])
        ids = rng.choice(pool, size=lens.size)
        ids[rng.random(lens.size) < 0.1] = 0
        seg = np.repeat(ids, lens)[None].astype(np.int32)
        mask = (rng.random((1, t)) > 0.01).astype(np.int32)
        return masks.MODE_PACKED_BIDIR, mask, seg, t, t
    if name == "keymask_65600x131149":
        # two rows of keys, masked in runs; query length not a tile multiple
        rng = np.random.default_rng(65600)
        t, s = 65600, 131149
        runs = _segments(rng, s, 1, 3000, True)
        on = (np.arange(runs.size) % 2).astype(bool)
        row0 = np.repeat(on, runs)
        row1 = rng.random(s) > 0.5
        row1[: 70000] = False
        mask = np.stack([row0, row1]).astype(np.int32)
        return masks.MODE_KEYMASK_BIDIR, mask, None, t, s
    raise KeyError(name)


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def digest_sections(tmap, qcnt, qlist, kcnt, klist, qorder, korder) -> dict:
    """SHA-256 of each plan section: the tile map (uint8 ``[B, nq, nk]``), the
    list counts (int32 ``[B, nq]``, ``[B, nk]``), the valid list entries of
    every tile concatenated in order (the padded tails are not part of the
    plan's contract), and the launch orders."""
    b, nq, nk = tmap.shape
    qv = [qlist[r, i, : qcnt[r, i]] for r in range(b) for i in range(nq)]
    kv = [klist[r, j, : kcnt[r, j]] for r in range(b) for j in range(nk)]
    cat = lambda parts: np.concatenate(parts).astype("<i4")  # noqa: E731
    return {
        "tmap": _sha(tmap.astype(np.uint8)),
        "qcnt": _sha(qcnt.astype("<i4")),
        "qlist": _sha(cat(qv)),
        "kcnt": _sha(kcnt.astype("<i4")),
        "klist": _sha(cat(kv)),
        "qorder": _sha(qorder.astype("<i4")),
        "korder": _sha(korder.astype("<i4")),
    }


def oracle_plan(mode, mask, seg, t, s):
    """The plan sections as the oracle defines them: stage maps of 128x64 and
    64x128 tiles give the work lists (entry = stage * 4 + class), and the
    launch orders sort items by list length, longest first, lengths of 63 and
    more tied, stably."""
    tm = masks.tile_map(mode, mask, seg, 128, 128, query_length=t)
    sq = masks.tile_map(mode, mask, seg, 128, 64, query_length=t)
    sk = masks.tile_map(mode, mask, seg, 64, 128, query_length=t)
    b, nq, nk = tm.shape
    qcnt = np.count_nonzero(sq, axis=2).astype(np.int32)
    kcnt = np.count_nonzero(sk, axis=1).astype(np.int32)
    qlist = np.zeros((b, nq, 2 * nk), np.int32)
    klist = np.zeros((b, nk, 2 * nq), np.int32)
    for r in range(b):
        for i in range(nq):
            nz = np.flatnonzero(sq[r, i])
            qlist[r, i, : nz.size] = nz * 4 + sq[r, i, nz]
        for j in range(nk):
            nz = np.flatnonzero(sk[r, :, j])
            klist[r, j, : nz.size] = nz * 4 + sk[r, nz, j]
    order = lambda c: np.argsort(63 - np.minimum(c.ravel(), 63), kind="stable")  # noqa: E731
    return tm, qcnt, qlist, kcnt, klist, order(qcnt), order(kcnt)


def main() -> None:
    out = {}
    for name in LAYOUTS:
        mode, mask, seg, t, s = long_row_layout(name)
        sections = oracle_plan(mode, mask, seg, t, s)
        out[name] = {"mode": mode, "batch": int(mask.shape[0]), "q_len": t, "kv_len": s,
                     "stages": int(sections[1].sum()), "digests": digest_sections(*sections)}
        print(name, out[name]["stages"], flush=True)
    OUT.write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
