"""The packer restatement against the reference's hand-derived layouts.

Fixtures: tests/golden/reference_fixtures.json (restated from the reference's
tests/batching/test_packing.py:11-88).
"""

import json
import pathlib

import numpy as np
import pytest

from oracle import packing

FIX = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())


def test_first_fit_decreasing_places_whole_sequences():
    f = FIX["packing"]["ffd_two_rows"]
    packed = packing.pack(f["sequences"], f["rows"], f["length"], pad_token_id=f["pad_token_id"])
    assert [(p.row, p.start, p.length) for p in packed.placements] == [tuple(x) for x in f["placements"]]
    np.testing.assert_array_equal(packed.input_ids, f["input_ids"])
    np.testing.assert_array_equal(packed.segment_ids, f["segment_ids"])
    np.testing.assert_array_equal(packed.positions, f["positions"])
    assert packing.rows_required([len(s) for s in f["sequences"]], f["length"]) == f["rows_required"]


def test_equal_lengths_keep_input_order():
    f = FIX["packing"]["ties_keep_input_order"]
    packed = packing.pack(f["sequences"], f["rows"], f["length"], pad_token_id=0)
    assert [p.row for p in packed.placements] == f["placement_rows"]
    assert [p.start for p in packed.placements] == f["placement_starts"]


def test_exact_fill_and_one_token_sequences():
    f = FIX["packing"]["exact_fill"]
    packed = packing.pack(f["sequences"], f["rows"], f["length"], pad_token_id=0)
    np.testing.assert_array_equal(packed.input_ids, f["input_ids"])
    np.testing.assert_array_equal(packed.segment_ids, f["segment_ids"])
    np.testing.assert_array_equal(packed.positions, f["positions"])


@pytest.mark.parametrize("case", FIX["packing"]["admission_errors"])
def test_admission_rejects_instead_of_truncating(case):
    with pytest.raises(ValueError, match=case["message"]):
        packing.pack(case["sequences"], case["rows"], case["length"], pad_token_id=0)


@pytest.mark.parametrize("seed", range(5))
def test_random_packing_round_trips(seed):
    """Every token lands once, in order, under its own id; positions restart."""
    rng = np.random.default_rng(seed)
    seqs = [list(rng.integers(1, 1000, size=int(n))) for n in rng.integers(1, 40, size=30)]
    rows = packing.rows_required([len(s) for s in seqs], 64)
    packed = packing.pack(seqs, rows, 64, pad_token_id=0)
    for index, (seq, p) in enumerate(zip(seqs, packed.placements)):
        np.testing.assert_array_equal(packed.input_ids[p.row, p.start : p.start + p.length], seq)
        assert (packed.segment_ids[p.row, p.start : p.start + p.length] == index + 1).all()
        np.testing.assert_array_equal(packed.positions[p.row, p.start : p.start + p.length],
                                      np.arange(len(seq)))
    assert (packed.segment_ids != 0).sum() == sum(len(s) for s in seqs)


def test_workload_generators_are_seeded_and_shaped():
    for name, shape in (("C1", (2, 256)), ("C2", (8, 4096)), ("C3", (4, 8192)), ("C5", (1, 32768))):
        a, b = packing.make_workload(name), packing.make_workload(name)
        assert a.segment_ids.shape == shape
        np.testing.assert_array_equal(a.segment_ids, b.segment_ids)
        np.testing.assert_array_equal(a.attention_mask, (a.segment_ids != 0).astype(np.int32))
    runs = packing.segment_runs(packing.make_workload("C5").segment_ids)[0]
    assert all(16 <= stop - start <= 128 for _, start, stop in runs)
    runs = packing.segment_runs(packing.make_workload("C2").segment_ids)
    assert all(32 <= stop - start <= 2048 for row in runs for _, start, stop in row)
    c1 = packing.segment_runs(packing.make_workload("C1").segment_ids)
    assert [len(r) for r in c1] == [4, 4]
    d = packing.make_decode_workload()
    assert d.valid_length.shape == (64,) and d.valid_length.min() >= 128 and d.valid_length.max() <= 8192
