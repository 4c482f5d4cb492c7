"""The prologue oracle (QK RMS norm + rotary, packer positions) pinned on the CPU."""

import numpy as np

from oracle import packing, prologue


def test_split_half_rotation_equals_pair_rotation_matrices():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 7, 3, 64))
    pos = rng.integers(0, 5000, size=(2, 7))
    np.testing.assert_allclose(prologue.apply_rotary(x, 10000.0, pos),
                               prologue.rotate_pairs(x, 10000.0, pos), rtol=1e-13, atol=1e-13)


def test_two_dims_rotate_by_the_position():
    """tests/layers/test_blocks.py:116-121: D=2 rotates by the token index."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 5, 1, 2))
    pos = np.arange(5)[None]
    out = prologue.apply_rotary(x, 10000.0, pos)
    for t in range(5):
        rot = np.array([[np.cos(t), -np.sin(t)], [np.sin(t), np.cos(t)]])
        np.testing.assert_allclose(out[0, t, 0], rot @ x[0, t, 0], rtol=1e-6, atol=1e-6)


def test_rotation_keeps_pair_norms_and_depends_on_relative_position():
    rng = np.random.default_rng(2)
    q, k = rng.standard_normal((2, 1, 1, 1, 64))
    rq = lambda p: prologue.apply_rotary(q, 500.0, np.array([[p]]))[0, 0, 0]  # noqa: E731
    rk = lambda p: prologue.apply_rotary(k, 500.0, np.array([[p]]))[0, 0, 0]  # noqa: E731
    pairs = lambda v: v[:32] ** 2 + v[32:] ** 2  # noqa: E731
    np.testing.assert_allclose(pairs(rq(123)), pairs(q[0, 0, 0]), rtol=1e-12)
    # <R(a) q, R(b) k> depends on a - b only (exact for angles a*f, b*f)
    assert abs(rq(40) @ rk(10) - rq(30) @ rk(0)) < 1e-4


def test_frequencies_are_single_precision_powers():
    f = prologue.frequencies(10000.0, 64)
    assert f.dtype == np.float32 and f[0] == 1.0
    np.testing.assert_allclose(f, 10000.0 ** (-np.arange(0, 64, 2) / 64), rtol=1e-6)


def test_rms_norm_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 4, 2, 64)) * 3
    w = rng.standard_normal(64)
    out = prologue.rms_norm(x, np.ones(64), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(out ** 2, axis=-1)), 1.0, rtol=1e-12)
    np.testing.assert_allclose(prologue.rms_norm(x, w, 0.01),
                               x / np.sqrt(np.mean(x ** 2, -1, keepdims=True) + 0.01) * w)


def test_segment_positions_match_the_packer():
    rng = np.random.default_rng(4)
    for _ in range(5):
        seqs = [list(range(int(n))) for n in rng.integers(1, 40, size=12)]
        rows = packing.rows_required([len(s) for s in seqs], 64)
        packed = packing.pack(seqs, rows, 64, pad_token_id=0)
        np.testing.assert_array_equal(prologue.segment_positions(packed.segment_ids),
                                      packed.positions)
