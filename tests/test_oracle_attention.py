"""FP64 attention oracle: analytical fixtures, finite differences, invariants.

Pins (none of them re-types the oracle's formula):
* tests/kernels/test_bidirectional.py:12-26, :41-65 closed forms (zero q/k
  gives per-segment averages; their value gradients are 3 and 2);
* central differences of the forward against the analytic VJP (method of
  tests/layers/test_blocks.py:156-174);
* packed rows equal independently computed rows (tests/layers/test_blocks.py:342-382);
* invariance under a permutation of segment ids;
* a single full segment equals textbook softmax attention (scipy);
* the grouped O(sum L^2) evaluation equals the dense grid;
* the decode oracle reads only the valid prefix, and a zero length gives
  the uniform average over all slots.
"""

import json
import pathlib

import numpy as np
import pytest
import scipy.special
import torch

from oracle import attention as oatt
from oracle import masks

FIX = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())


def test_bidirectional_uniform_fixture():
    f = FIX["bidirectional"]["uniform"]
    q, k = np.zeros(f["query_shape"]), np.zeros(f["key_shape"])
    v = np.array(f["values"])
    mask = np.array(f["mask"])
    out, probs, present = oatt.bidirectional_fp64(q, k, v, mask)
    np.testing.assert_allclose(out, np.broadcast_to(f["output_row"], out.shape))
    _, _, dv = oatt.vjp_fp64(q, k, v, probs, present, np.ones_like(out))
    np.testing.assert_allclose(dv, f["value_grad_of_sum"])
    empty, _, _ = oatt.bidirectional_fp64(q, k, v, np.zeros_like(mask))
    np.testing.assert_array_equal(empty, 0)


def test_bidirectional_packed_fixture():
    f = FIX["bidirectional"]["packed"]
    q, k = np.zeros(f["query_shape"]), np.zeros(f["key_shape"])
    v = np.array(f["values"]).reshape(1, 6, 1, 2)
    seg = np.array(f["segment_ids"])
    out, probs, present = oatt.bidirectional_fp64(q, k, v, seg != 0, seg)
    expected = np.broadcast_to(np.array(f["output_rows"], float)[None, :, None], (1, 6, 2, 2))
    np.testing.assert_allclose(out, expected)
    _, _, dv = oatt.vjp_fp64(q, k, v, probs, present, np.ones_like(out))
    np.testing.assert_allclose(dv.reshape(6, 2), f["value_grad_of_sum"], rtol=1e-12)
    grouped = oatt.grouped_fp64(masks.MODE_PACKED_BIDIR, q, k, v, seg != 0, seg)
    np.testing.assert_allclose(grouped, expected)


def _operands(rng, b, t, hq, hkv, d, s=None):
    s = t if s is None else s
    return (rng.standard_normal((b, t, hq, d)), rng.standard_normal((b, s, hkv, d)),
            rng.standard_normal((b, s, hkv, d)))


def _forward(mode, q, k, v, mask, seg):
    if mode == masks.MODE_PACKED_CAUSAL:
        return oatt.packed_causal_fp64(q, k, v, mask, seg)
    return oatt.bidirectional_fp64(q, k, v, mask, seg)


@pytest.mark.parametrize("mode", [masks.MODE_PACKED_CAUSAL, masks.MODE_PACKED_BIDIR,
                                  masks.MODE_KEYMASK_BIDIR])
def test_vjp_matches_central_differences(mode):
    rng = np.random.default_rng(11)
    q, k, v = _operands(rng, 1, 5, 4, 2, 3)
    seg = np.array([[1, 1, 2, 2, 0]])
    mask = np.array([[1, 1, 1, 0, 1]])
    if mode == masks.MODE_KEYMASK_BIDIR:
        seg = None
    do = rng.standard_normal(q.shape)
    out, probs, keep = _forward(mode, q, k, v, mask, seg)
    grads = oatt.vjp_fp64(q, k, v, probs, keep, do)
    step = 1e-5
    for arg, analytic in zip(range(3), grads):
        base = [q, k, v]
        flat = analytic.reshape(-1)
        for idx in range(0, flat.size, 7):
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[arg].reshape(-1)[idx] += step
            minus[arg].reshape(-1)[idx] -= step
            fp = (_forward(mode, *plus, mask, seg)[0] * do).sum()
            fm = (_forward(mode, *minus, mask, seg)[0] * do).sum()
            np.testing.assert_allclose((fp - fm) / (2 * step), flat[idx], rtol=3e-5, atol=3e-6)


@pytest.mark.parametrize("causal", [True, False])
def test_packed_rows_equal_independent_rows(causal):
    rng = np.random.default_rng(5)
    q, k, v = _operands(rng, 1, 9, 4, 2, 6)
    seg = np.array([[1, 1, 1, 1, 2, 2, 2, 2, 0]])
    mask = (seg != 0).astype(int)
    fn = oatt.packed_causal_fp64 if causal else oatt.bidirectional_fp64
    packed = fn(q, k, v, mask, seg)[0]
    for lo, hi in ((0, 4), (4, 8)):
        one = np.ones((1, hi - lo), int)
        alone = fn(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], one, one)[0]
        np.testing.assert_allclose(packed[:, lo:hi], alone, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(packed[:, 8], 0)


def test_segment_id_permutation_invariance():
    rng = np.random.default_rng(6)
    q, k, v = _operands(rng, 2, 12, 4, 2, 5)
    seg = rng.integers(0, 4, size=(2, 12))
    mask = (rng.random((2, 12)) > 0.2).astype(int)
    perm = np.array([0, 7, 3, 9])  # 0 stays padding, ids relabelled
    for fn in (oatt.packed_causal_fp64, oatt.bidirectional_fp64):
        np.testing.assert_allclose(fn(q, k, v, mask, seg)[0], fn(q, k, v, mask, perm[seg])[0],
                                   rtol=1e-13, atol=1e-13)


def test_single_segment_is_textbook_softmax_attention():
    rng = np.random.default_rng(8)
    q, k, v = _operands(rng, 1, 7, 2, 2, 4)
    one = np.ones((1, 7), int)
    out = oatt.bidirectional_fp64(q, k, v, one, one)[0]
    for h in range(2):
        p = scipy.special.softmax(q[0, :, h] @ k[0, :, h].T / 2.0, axis=-1)
        np.testing.assert_allclose(out[0, :, h], p @ v[0, :, h], rtol=1e-12)
    causal = oatt.packed_causal_fp64(q, k, v, one, one)[0]
    for i in range(7):
        p = scipy.special.softmax(q[0, i, 0] @ k[0, : i + 1, 0].T / 2.0)
        np.testing.assert_allclose(causal[0, i, 0], p @ v[0, : i + 1, 0], rtol=1e-12)


@pytest.mark.parametrize("mode", [masks.MODE_PACKED_CAUSAL, masks.MODE_PACKED_BIDIR,
                                  masks.MODE_KEYMASK_BIDIR])
def test_grouped_evaluation_equals_dense_grid(mode):
    rng = np.random.default_rng(9 + mode)
    q, k, v = _operands(rng, 2, 20, 4, 2, 8)
    seg = rng.integers(0, 5, size=(2, 20))  # non-contiguous ids on purpose
    mask = (rng.random((2, 20)) > 0.25).astype(int)
    if mode == masks.MODE_KEYMASK_BIDIR:
        seg = None
        mask[1] = 0
    do = rng.standard_normal(q.shape)
    out, probs, keep = _forward(mode, q, k, v, mask, seg)
    dq, dk, dv = oatt.vjp_fp64(q, k, v, probs, keep, do)
    g = oatt.grouped_fp64(mode, q, k, v, mask, seg, d_out=do)
    for a, b in zip(g, (out, dq, dk, dv)):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_cached_oracle_reads_only_the_valid_prefix():
    rng = np.random.default_rng(3)
    q, k, v = _operands(rng, 2, 1, 4, 2, 8, s=6)
    out = oatt.cached_fp64(q, k, v, np.array(4))[0]
    k2, v2 = k.copy(), v.copy()
    k2[:, 4:] = 1e3
    v2[:, 4:] = -1e3
    np.testing.assert_allclose(oatt.cached_fp64(q, k2, v2, np.array(4))[0], out, rtol=1e-12)
    short = oatt.bidirectional_fp64(q, k[:, :4], v[:, :4], np.ones((2, 4), int), None)[0]
    np.testing.assert_allclose(out, short, rtol=1e-12)
    ragged = oatt.cached_fp64(q, k, v, np.array([2, 6]))[0]
    np.testing.assert_allclose(ragged[1], oatt.cached_fp64(q, k, v, np.array(6))[0][1], rtol=1e-12)
    # an unguarded zero length: every slot masked -> uniform average of all slots
    zero = oatt.cached_fp64(q, k, v, np.array(0))[0]
    np.testing.assert_allclose(zero, np.repeat(v.mean(axis=1, keepdims=True), 2, axis=2), rtol=1e-12)


def test_bf16_emulations_stay_within_tolerance_of_fp64():
    rng = np.random.default_rng(12)
    q, k, v = (x * 0.5 for x in _operands(rng, 1, 96, 4, 2, 64))
    seg = np.repeat([1, 2, 3, 0], [40, 30, 20, 6])[None]
    mask = (seg != 0).astype(int)
    ref = oatt.bidirectional_fp64(q, k, v, mask, seg)[0]
    valid, present = masks.bidirectional_valid(mask, seg)
    tq, tk, tv = (torch.tensor(x, dtype=torch.bfloat16) for x in (q, k, v))
    for fn in (oatt.dense_bf16_einsum, oatt.sdpa_bf16):
        out = fn(tq, tk, tv, torch.tensor(valid[:, None]))
        out = torch.where(torch.tensor(present[:, :, None, None]), out.float(), 0.0).numpy()
        assert np.abs(out - ref).max() < 2e-2


# bf16 cast points of the two emulations, pinned by closed forms that move when a cast
# point moves (one head, D = 64, scale 1/8; bf16 keeps 8 significant bits).


def _bf(x):
    return torch.tensor(np.asarray(x, np.float32)).to(torch.bfloat16)


def test_bf16_emulations_round_the_probabilities_and_the_output():
    """Zero q/k over 6 keys: P = bf16(1/6) = 0.1669921875 exactly.  With V = [100, 0, ...]
    the output is bf16(100 * 0.1669921875) = bf16(16.699...) = 16.75; unrounded
    probabilities would give bf16(16.666...) = 16.625."""
    q, k = _bf(np.zeros((1, 1, 1, 64))), _bf(np.zeros((1, 6, 1, 64)))
    v = np.zeros((1, 6, 1, 64), np.float32)
    v[0, 0, 0, 0] = 100.0
    valid = torch.ones(1, 1, 1, 6, dtype=torch.bool)
    for fn in (oatt.dense_bf16_einsum, oatt.sdpa_bf16):
        out = fn(q, k, _bf(v), valid)
        assert out.dtype == torch.bfloat16
        assert out[0, 0, 0, 0].item() == 16.75, fn.__name__
        assert out[0, 0, 0, 1].item() == 0.0


def test_einsum_emulation_rounds_the_logits_and_sdpa_does_not():
    """q = (1, 1, 0, ...), keys (100, 0, ...) and (100, 0.25, ...): raw logits 100 and 100.25.
    attention.py:23-25 makes the einsum result bf16, and bf16(100.25) = 100 (a tie, to
    even), so both scaled logits are 12.5 and P = (0.5, 0.5).  SDPA keeps fp32 logits 12.5
    and 12.53125: P1 = 1 / (1 + e^-0.03125) = 0.5078119..., bf16 0.5078125, and
    P0 = 0.4921881..., bf16 0.4921875.  V = (0, 1) in dimension 0 reads P1 off."""
    q = np.zeros((1, 1, 1, 64), np.float32)
    q[..., :2] = 1.0
    k = np.zeros((1, 2, 1, 64), np.float32)
    k[0, :, 0, 0] = 100.0
    k[0, 1, 0, 1] = 0.25
    v = np.zeros((1, 2, 1, 64), np.float32)
    v[0, 1, 0, 0] = 1.0
    valid = torch.ones(1, 1, 1, 2, dtype=torch.bool)
    dense = oatt.dense_bf16_einsum(_bf(q), _bf(k), _bf(v), valid)
    sdpa = oatt.sdpa_bf16(_bf(q), _bf(k), _bf(v), valid)
    assert dense[0, 0, 0, 0].item() == 0.5
    assert sdpa[0, 0, 0, 0].item() == 0.5078125


def test_bf16_emulations_on_single_keys_and_representable_logits():
    """A row with one valid key returns that key's value exactly (P = 1); with integer q/k
    every logit is exactly representable in bf16, so the two emulations agree bit for bit
    (they differ only in the logits' cast and the masked fill, which a row with a valid key
    never sees)."""
    rng = np.random.default_rng(5)
    q = rng.integers(-2, 3, size=(2, 9, 4, 64)).astype(np.float32)
    k = rng.integers(-2, 3, size=(2, 9, 2, 64)).astype(np.float32)
    v = rng.standard_normal((2, 9, 2, 64)).astype(np.float32)
    seg = np.array([[1, 1, 2, 2, 2, 3, 4, 4, 0], [5, 5, 5, 5, 5, 5, 5, 5, 6]])
    valid, present = masks.bidirectional_valid(seg != 0, seg)
    tv = torch.tensor(valid[:, None])
    dense = oatt.dense_bf16_einsum(_bf(q), _bf(k), _bf(v), tv)
    sdpa = oatt.sdpa_bf16(_bf(q), _bf(k), _bf(v), tv)
    assert torch.equal(dense[torch.tensor(present)], sdpa[torch.tensor(present)])
    vb = _bf(v)
    for row, t in ((0, 5), (1, 8)):  # single-token segments 3 and 6
        torch.testing.assert_close(dense[row, t], vb[row, t].repeat_interleave(2, dim=0),
                                   rtol=0, atol=0)
