"""GPU block-mask builder: bit-exact against the brute-force tile reduction.

Oracle: ``oracle.masks.tile_map`` (per-tile reduction of the reference's
validity grid, itself checked against per-pair loops in test_oracle_masks).
"""

import json
import pathlib

import numpy as np
import pytest
import torch

from _helpers import say
from mfattn import _lib, ops
from oracle import masks, packing

FIX = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())
pytestmark = pytest.mark.gpu


def _check(mode, mask, seg, t, s, device):
    say("block_map", "mode", mode, "shape", mask.shape, "T", t, "S", s)
    tm_ref = masks.tile_map(mode, mask, seg, 128, 128, query_length=t)
    mt = torch.tensor(mask, device=device)
    st = None if seg is None else torch.tensor(seg, dtype=torch.int32, device=device)
    plan = ops.block_map(st, mt, mode, t, s)
    torch.cuda.synchronize()
    tm = plan.tile_map().cpu().numpy()
    np.testing.assert_array_equal(tm, tm_ref)
    b, nq, nk = tm.shape
    qcnt = plan.section(3, torch.int32, (b, nq)).cpu().numpy()
    qlist = plan.section(4, torch.int32, (b, nq, 2 * nk)).cpu().numpy()
    kcnt = plan.section(5, torch.int32, (b, nk)).cpu().numpy()
    klist = plan.section(6, torch.int32, (b, nk, 2 * nq)).cpu().numpy()
    # work lists hold 64-row stages: query tiles x 64-key stages, 64-query stages x key tiles
    sq = masks.tile_map(mode, mask, seg, 128, 64, query_length=t)
    sk = masks.tile_map(mode, mask, seg, 64, 128, query_length=t)
    for r in range(b):
        for qi in range(nq):
            nz = np.flatnonzero(sq[r, qi])
            assert qcnt[r, qi] == nz.size
            np.testing.assert_array_equal(qlist[r, qi, : nz.size], nz * 4 + sq[r, qi, nz])
        for kj in range(nk):
            nz = np.flatnonzero(sk[r, :, kj])
            assert kcnt[r, kj] == nz.size
            np.testing.assert_array_equal(klist[r, kj, : nz.size], nz * 4 + sk[r, nz, kj])
    # launch orders: items by decreasing list length (lengths >= 63 tie), stable
    for sec, cnt in ((7, qcnt), (8, kcnt)):
        order = plan.section(sec, torch.int32, (cnt.size,)).cpu().numpy()
        want = np.argsort(63 - np.minimum(cnt.ravel(), 63), kind="stable")
        np.testing.assert_array_equal(order, want)
    qid, kid = masks._token_ids(mode, mask, seg, t)
    gq = plan.section(0, torch.int32, (b, nq * 128)).cpu().numpy()
    gk = plan.section(1, torch.int32, (b, nk * 128)).cpu().numpy()
    np.testing.assert_array_equal(gq[:, :t], np.where(qid != masks.Q_INACTIVE, qid, 0))
    np.testing.assert_array_equal(gk[:, :s], np.where(kid != masks.K_INACTIVE, kid, 0))
    assert (gq[:, t:] == 0).all() and (gk[:, s:] == 0).all()


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_baseline_configs(name, device):
    w = packing.make_workload(name)
    mode = masks.MODE_PACKED_CAUSAL if w.causal else masks.MODE_PACKED_BIDIR
    _check(mode, w.attention_mask, w.segment_ids, w.length, w.length, device)


@pytest.mark.parametrize("mode", [0, 1])
def test_reference_fixture_layouts(mode, device):
    lay = FIX["layouts"]
    cases = [(np.array(lay["attention_packed"]["mask"], np.int32),
              np.array(lay["attention_packed"]["segment_ids"], np.int32))]
    for key in ("packing_rows", "packing_exact_fill", "pointer_row", "bidirectional_packed",
                "blocks_packed"):
        seg = np.array(lay[key], np.int32)
        cases.append(((seg != 0).astype(np.int32), seg))
    for mask, seg in cases:
        _check(mode, mask, seg, seg.shape[1], seg.shape[1], device)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("mode", [0, 1])
def test_random_layouts(seed, mode, device):
    """Ragged lengths, non-contiguous and repeated ids, masked holes, negative ids."""
    rng = np.random.default_rng(seed)
    t = int(rng.integers(1, 700))
    b = int(rng.integers(1, 4))
    if seed % 2:
        seg = rng.integers(-2, 4, size=(b, t)).astype(np.int32)
    else:
        seg = np.repeat(rng.integers(0, 6, size=(b, t // 50 + 1)), 50, axis=1)[:, :t].astype(np.int32)
    mask = rng.integers(-1, 3, size=(b, t)).astype(np.int32)
    _check(mode, mask, seg, t, t, device)


def test_single_segment_rows_are_full_and_padding_rows_empty(device):
    seg = np.zeros((2, 512), np.int32)
    seg[0] = 1
    _check(1, (seg != 0).astype(np.int32), seg, 512, 512, device)
    _check(0, (seg != 0).astype(np.int32), seg, 512, 512, device)


@pytest.mark.parametrize("t, s", [(300, 77), (5, 1000), (128, 128)])
def test_key_mask_mode_cross_lengths(t, s, device):
    rng = np.random.default_rng(t + s)
    mask = (rng.random((3, s)) > 0.3).astype(np.int32)
    mask[2] = 0
    _check(2, mask, None, t, s, device)


def test_bool_mask_dtype(device):
    w = packing.make_workload("C1")
    mask = torch.tensor(w.attention_mask != 0, device=device)
    seg = torch.tensor(w.segment_ids, device=device)
    a = ops.block_map(seg, mask, 0, w.length, w.length).tile_map().cpu().numpy()
    np.testing.assert_array_equal(a, masks.tile_map(0, w.attention_mask, w.segment_ids, 128, 128))


@pytest.mark.parametrize("mode", [0, 1])
def test_placements_build_the_same_plan(mode, device):
    """mf_block_map_placements == mf_block_map over the packer's PackedRows."""
    rng = np.random.default_rng(50 + mode)
    for length in (256, 1000):
        seqs = [list(range(int(n))) for n in rng.integers(1, min(300, length) + 1, size=9)]
        rows = packing.rows_required([len(s) for s in seqs], length)
        packed = packing.pack(seqs, rows, length, pad_token_id=0)
        say("placements", mode, length, rows)
        pl = torch.tensor([[p.row, p.start, p.length] for p in packed.placements], device=device)
        plan, seg, pos = ops.block_map_from_placements(pl, mode, rows, length)
        np.testing.assert_array_equal(seg.cpu().numpy(), packed.segment_ids)
        np.testing.assert_array_equal(pos.cpu().numpy(), packed.positions)
        mask = (packed.segment_ids != 0).astype(np.int32)
        ref = ops.block_map(torch.tensor(packed.segment_ids, device=device),
                            torch.tensor(mask, device=device), mode, length, length)
        nq = nk = -(-length // 128)
        for sec, dt, shape in ((0, torch.int32, (rows, nq * 128)), (1, torch.int32, (rows, nk * 128)),
                               (2, torch.uint8, (rows, nq, nk)), (3, torch.int32, (rows, nq)),
                               (5, torch.int32, (rows, nk)), (7, torch.int32, (rows * nq,)),
                               (8, torch.int32, (rows * nk,))):
            assert torch.equal(plan.section(sec, dt, shape), ref.section(sec, dt, shape)), sec
        cnt = ref.section(3, torch.int32, (rows, nq)).cpu().numpy()
        a, r = plan.section(4, torch.int32, (rows, nq, 2 * nk)).cpu().numpy(), \
            ref.section(4, torch.int32, (rows, nq, 2 * nk)).cpu().numpy()
        for row in range(rows):
            for qi in range(nq):
                np.testing.assert_array_equal(a[row, qi, : cnt[row, qi]], r[row, qi, : cnt[row, qi]])


def _long_rows():
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).parent / "golden"))
    import make_long_rows  # noqa: E402

    gold = json.loads((pathlib.Path(__file__).parent / "golden" / "long_rows.json").read_text())
    return make_long_rows, gold


@pytest.mark.parametrize("name", ["causal_98304", "bidir_131072", "keymask_65600x131149"])
def test_long_rows_against_oracle_digests(name, device):
    """Rows of 65,600-131,149 tokens: over 1024 64-row stages per tile, so the work lists are
    classified in several rounds.  Every plan section is bit-exact with the oracle's, compared
    through the SHA-256 digests that tests/golden/make_long_rows.py stored; ids directly."""
    mlr, gold = _long_rows()
    mode, mask, seg, t, s = mlr.long_row_layout(name)
    want = gold[name]
    assert (want["mode"], want["batch"], want["q_len"], want["kv_len"]) == (mode, mask.shape[0], t, s)
    say("long block map", name, "T", t, "S", s)
    st = None if seg is None else torch.tensor(seg, device=device)
    plan = ops.block_map(st, torch.tensor(mask, device=device), mode, t, s)
    tm = plan.tile_map().cpu().numpy()
    b, nq, nk = tm.shape
    qcnt = plan.section(3, torch.int32, (b, nq)).cpu().numpy()
    kcnt = plan.section(5, torch.int32, (b, nk)).cpu().numpy()
    got = mlr.digest_sections(
        tm, qcnt, plan.section(4, torch.int32, (b, nq, 2 * nk)).cpu().numpy(),
        kcnt, plan.section(6, torch.int32, (b, nk, 2 * nq)).cpu().numpy(),
        plan.section(7, torch.int32, (b * nq,)).cpu().numpy(),
        plan.section(8, torch.int32, (b * nk,)).cpu().numpy())
    assert int(qcnt.sum()) == want["stages"]
    for key, digest in want["digests"].items():
        assert got[key] == digest, key
    qid, kid = masks._token_ids(mode, mask, seg, t)
    gq = plan.section(0, torch.int32, (b, nq * 128)).cpu().numpy()
    gk = plan.section(1, torch.int32, (b, nk * 128)).cpu().numpy()
    np.testing.assert_array_equal(gq[:, :t], np.where(qid != masks.Q_INACTIVE, qid, 0))
    np.testing.assert_array_equal(gk[:, :s], np.where(kid != masks.K_INACTIVE, kid, 0))
