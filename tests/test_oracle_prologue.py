"""The prologue oracle (QK RMS norm + rotary, packer positions) pinned on the CPU."""

import numpy as np
import pytest

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


@pytest.mark.parametrize("theta", [500.0, 10000.0, 1000000.0])
def test_frequencies_are_correctly_rounded_single_precision_powers(theta):
    f = prologue.frequencies(theta, 64)
    exact = np.float64(theta) ** (-np.arange(0, 64, 2) / 64)
    assert f.dtype == np.float32 and f[0] == 1.0
    # within half a float32 ulp of the exact power: the nearest single-precision value
    assert bool((np.abs(f.astype(np.float64) - exact) <= 0.5 * np.spacing(f).astype(np.float64)).all())


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


# Hand cases for the bf16 cast order (one head of 64 dims; nonzero dims 0, 5 and 32;
# gains 1 except dims 0 and 32; eps 1e-6; frequency of pair 0 is theta**0 = 1, so pair
# (0, 32) rotates by the position itself).  Derivation, in exact arithmetic with
# round-to-nearest-even to 8 significant bits (bf16) or 24 (fp32):
#   inv = f32(rsqrt(mean(x^2) + eps)); n_i = bf16(bf16(f32(x_i * inv)) * g_i)
#   c, s = bf16(f32 cos p), bf16(f32 sin p)
#   out_0  = bf16(bf16(n_0 * c) + bf16(-n_32 * s));  out_32 = bf16(bf16(n_32 * c) + bf16(n_0 * s))
# Each case also records what dropping one cast point would give instead (the
# normalised value not rounded before the gain; cos/sin not rounded; the two products
# summed at fp32 and rounded once), so a restatement that misses any of them fails.
PROLOGUE_CASES = [
    # x_0, x_32, x_5, g_0, g_32, position, (out_0, out_32), {dropped cast: (out_0, out_32)}
    (2.375, 0.32421875, 1.71875, 0.8515625, 1.25, 17, (-0.453125, -5.5625),
     {"norm": (-0.4609375, -5.59375), "cos_sin": (-0.4453125, -5.5625),
      "products": (-0.447265625, -5.5625)}),
    (-2.046875, -1.828125, 1.5234375, 0.55078125, 0.7734375, 36, (-3.1875, 3.3125),
     {"norm": (-3.21875, 3.3125), "cos_sin": (-3.1875, 3.296875),
      "products": (-3.203125, 3.3125)}),
]


def test_cast_order_restatement_matches_hand_derived_bf16_cases():
    import torch

    x = torch.zeros(1, len(PROLOGUE_CASES), 1, 64)
    gains = torch.ones(len(PROLOGUE_CASES), 64)
    for t, (x0, x32, x5, g0, g32, _, _, _) in enumerate(PROLOGUE_CASES):
        x[0, t, 0, 0], x[0, t, 0, 32], x[0, t, 0, 5] = x0, x32, x5
        gains[t, 0], gains[t, 32] = g0, g32
    pos = np.array([[case[5] for case in PROLOGUE_CASES]])
    for t, case in enumerate(PROLOGUE_CASES):
        xb = x[:, t:t + 1].to(torch.bfloat16)
        out = prologue.apply_rotary_cast(prologue.rms_norm_cast(xb, gains[t], 1e-6), 10000.0,
                                         pos[:, t:t + 1])
        assert out.dtype == torch.bfloat16
        got = (out[0, 0, 0, 0].item(), out[0, 0, 0, 32].item())
        assert got == case[6], (t, got)
        for dropped, other in case[7].items():
            assert other != case[6], dropped  # the case does distinguish that cast point


def test_cast_order_restatement_in_float32_equals_the_fp64_prologue():
    import torch

    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 9, 4, 64)).astype(np.float32) * 2
    k = rng.standard_normal((2, 9, 2, 64)).astype(np.float32)
    qg, kg = (1 + 0.1 * rng.standard_normal((2, 64))).astype(np.float32)
    pos = rng.integers(0, 3000, size=(2, 9))
    got = prologue.qk_norm_rope_cast(torch.tensor(q), torch.tensor(k), torch.tensor(qg),
                                     torch.tensor(kg), pos, 1e-5, 1e6)
    want = prologue.qk_norm_rope(q, k, qg, kg, pos, 1e-5, 1e6)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a.numpy(), b, rtol=2e-6, atol=2e-6)


def test_prologue_vjp_matches_central_differences():
    """Method of tests/layers/test_blocks.py:156-174: a nonuniform output probe."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 3, 2, 64))
    k = rng.standard_normal((1, 3, 1, 64))
    qg, kg = 1 + 0.2 * rng.standard_normal((2, 64))
    pos = np.array([[0, 5, 77]])
    pq, pk = rng.standard_normal(q.shape), rng.standard_normal(k.shape)
    eps, theta = 1e-3, 10000.0

    def loss(q_, k_, qg_, kg_):
        a, b = prologue.qk_norm_rope(q_, k_, qg_, kg_, pos, eps, theta)
        return (a * pq).sum() + (b * pk).sum()

    dq, dk, dqg, dkg = prologue.qk_norm_rope_vjp(q, k, qg, kg, pos, eps, theta, pq, pk)
    step = 1e-6
    for got, arr, which in ((dq, q, 0), (dk, k, 1), (dqg, qg, 2), (dkg, kg, 3)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [q.copy(), k.copy(), qg.copy(), kg.copy()]
            args[which][idx] += step
            up = loss(*args)
            args[which][idx] -= 2 * step
            num[idx] = (up - loss(*args)) / (2 * step)
        np.testing.assert_allclose(got, num, rtol=1e-6, atol=1e-7)
