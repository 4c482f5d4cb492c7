"""Validity grids and the brute-force tile map, pinned independently.

The grids are checked against per-pair loops written from the reference's
prose (attention.py:86-91 docstring, bidirectional.py:14-20 docstring) on the
reference's own fixture layouts; the vectorised tile map is checked against a
per-tile loop; pair counts against the closed form L(L+1)/2 / L^2.
"""

import itertools
import json
import pathlib

import numpy as np
import pytest

from oracle import masks, packing, workload

FIX = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())


def _layouts():
    lay = FIX["layouts"]
    yield np.array(lay["attention_packed"]["mask"]), np.array(lay["attention_packed"]["segment_ids"])
    for key in ("packing_rows", "packing_exact_fill", "pointer_row", "bidirectional_packed",
                "blocks_packed"):
        seg = np.array(lay[key])
        yield (seg != 0).astype(np.int32), seg


def _causal_loop(mask, seg):
    b, t = seg.shape
    valid = np.zeros((b, t, t), bool)
    for r, i, j in itertools.product(range(b), range(t), range(t)):
        ai = mask[r, i] > 0 and seg[r, i] != 0
        aj = mask[r, j] > 0 and seg[r, j] != 0
        if ai:
            valid[r, i, j] = aj and j <= i and seg[r, i] == seg[r, j]
        else:
            valid[r, i, j] = i == j  # inactive queries attend to themselves
    return valid


@pytest.mark.parametrize("index", range(6))
def test_packed_valid_matches_pair_loop(index):
    mask, seg = list(_layouts())[index]
    valid, active = masks.packed_valid(mask, seg)
    np.testing.assert_array_equal(valid, _causal_loop(mask, seg))
    np.testing.assert_array_equal(active, (mask > 0) & (seg != 0))


def test_packed_fixture_grid_by_hand():
    """attention.py fixture row 1: [1,1,2,0,0,0] with mask [1,1,1,0,0,0]."""
    lay = FIX["layouts"]["attention_packed"]
    valid, _ = masks.packed_valid(np.array(lay["mask"]), np.array(lay["segment_ids"]))
    expected = np.array([
        [1, 0, 0, 0, 0, 0],
        [1, 1, 0, 0, 0, 0],
        [0, 0, 1, 0, 0, 0],
        [0, 0, 0, 1, 0, 0],
        [0, 0, 0, 0, 1, 0],
        [0, 0, 0, 0, 0, 1],
    ], bool)
    np.testing.assert_array_equal(valid[1], expected)


def test_bidirectional_valid_by_hand():
    seg = np.array(FIX["layouts"]["bidirectional_packed"])
    valid, present = masks.bidirectional_valid(seg != 0, seg)
    blocks = np.zeros((6, 6), bool)
    blocks[:2, :2] = True
    blocks[2:5, 2:5] = True
    np.testing.assert_array_equal(valid[0], blocks)
    np.testing.assert_array_equal(present[0], [1, 1, 1, 1, 1, 0])
    keymask = np.array([[1, 1, 0]])
    valid, present = masks.bidirectional_valid(keymask, None, 3)
    np.testing.assert_array_equal(valid[0], [[1, 1, 0]] * 3)
    np.testing.assert_array_equal(present[0], [1, 1, 1])
    valid, present = masks.bidirectional_valid(np.zeros((1, 3)), None, 3)
    assert not present.any()


def _random_seg(rng, b, t, contiguous=True):
    if contiguous:
        seg = np.zeros((b, t), np.int32)
        for r in range(b):
            cur, ident = 0, 1
            while cur < t:
                n = int(rng.integers(1, 40))
                seg[r, cur : cur + n] = ident if rng.random() > 0.15 else 0
                cur += n
                ident += 1
        return seg
    return rng.integers(0, 4, size=(b, t)).astype(np.int32)


@pytest.mark.parametrize("mode", [masks.MODE_PACKED_CAUSAL, masks.MODE_PACKED_BIDIR,
                                  masks.MODE_KEYMASK_BIDIR])
@pytest.mark.parametrize("contiguous", [True, False])
def test_tile_map_matches_per_tile_loop(mode, contiguous):
    rng = np.random.default_rng(7 + mode)
    seg = _random_seg(rng, 2, 45, contiguous)
    mask = (rng.random((2, 45)) > 0.1).astype(np.int32)
    if mode == masks.MODE_KEYMASK_BIDIR:
        mask[1] = 0  # an example with no active key
        grid = masks.useful_grid(mode, mask, None, 37)
        tm = masks.tile_map(mode, mask, None, 8, 4, query_length=37)
    else:
        grid = masks.useful_grid(mode, mask, seg)
        tm = masks.tile_map(mode, mask, seg, 8, 4)
    np.testing.assert_array_equal(tm, masks.tile_map_loops(grid, 8, 4))


def test_full_tiles_exist_and_tail_tiles_are_never_full():
    seg = np.ones((1, 20), np.int32)
    tm = masks.tile_map(masks.MODE_PACKED_BIDIR, seg, seg, 8, 8)
    np.testing.assert_array_equal(tm[0], [[2, 2, 1], [2, 2, 1], [1, 1, 1]])
    tm = masks.tile_map(masks.MODE_PACKED_CAUSAL, seg, seg, 8, 8)
    np.testing.assert_array_equal(tm[0], [[1, 0, 0], [2, 1, 0], [1, 1, 1]])


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_useful_pairs_closed_form(name):
    w = packing.make_workload(name)
    mode = masks.MODE_PACKED_CAUSAL if w.causal else masks.MODE_PACKED_BIDIR
    assert workload.useful_pairs(mode, w.attention_mask, w.segment_ids) == \
        workload.useful_pairs_closed_form(w.segment_ids, w.causal)


def test_useful_pairs_counts_grid_on_random_layouts():
    rng = np.random.default_rng(3)
    for mode in (0, 1):
        seg = _random_seg(rng, 3, 50, contiguous=False)
        mask = (rng.random((3, 50)) > 0.2).astype(np.int32)
        assert workload.useful_pairs(mode, mask, seg) == int(masks.useful_grid(mode, mask, seg).sum())


def test_tile_map_of_baseline_c2_is_mostly_empty():
    w = packing.make_workload("C2")
    tm = masks.tile_map(masks.MODE_PACKED_BIDIR, w.attention_mask, w.segment_ids, 128, 128)
    assert 0.6 < (tm == 0).mean() < 0.85
    assert (tm == 2).any() and (tm == 1).any()
