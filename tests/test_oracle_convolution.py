"""The segmented-convolution oracle pinned on the CPU."""

import numpy as np
import torch

from oracle import convolution as oconv


def test_reference_fixtures():
    """tests/kernels/test_bidirectional.py:29-37 and :66-77."""
    taps = np.array([[10.0, 100.0, 1000.0]])
    out = oconv.centered(np.array([[[1.0], [2.0], [3.0], [4.0]]]), taps)
    np.testing.assert_array_equal(out.ravel(), [2100, 3210, 4320, 430])
    out = oconv.centered(np.array([[[1.0], [2.0], [3.0], [4.0], [5.0]]]), taps,
                         np.array([[1, 1, 2, 2, 0]]))
    np.testing.assert_array_equal(out.ravel(), [2100, 210, 4300, 430, 0])


def test_centered_is_torch_grouped_conv1d():
    """The reference's docstring: grouped conv1d with padding k//2, right crop."""
    rng = np.random.default_rng(0)
    for k in (1, 2, 3, 4, 5):
        x = rng.standard_normal((2, 11, 6))
        taps = rng.standard_normal((6, k))
        ref = torch.nn.functional.conv1d(torch.tensor(x).permute(0, 2, 1), torch.tensor(taps)[:, None, :],
                                         padding=k // 2, groups=6)[..., : x.shape[1]].permute(0, 2, 1)
        np.testing.assert_allclose(oconv.centered(x, taps), ref.numpy(), rtol=1e-12, atol=1e-12)


def test_causal_is_a_left_padded_convolution_per_channel():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 9, 3))
    w = rng.standard_normal((3, 3))
    out = oconv.causal(np.ones_like(x), np.ones_like(x), x, w)
    for ch in range(3):
        full = np.convolve(x[0, :, ch], w[ch, ::-1])[: x.shape[1]]
        np.testing.assert_allclose(out[0, :, ch], full, rtol=1e-12, atol=1e-12)


def test_segments_act_as_independent_padding():
    rng = np.random.default_rng(2)
    seg = np.array([[1, 1, 1, 2, 2, 2, 2, 3, 0, 0]])
    x = rng.standard_normal((1, 10, 4))
    bg, cg = rng.standard_normal((2, 1, 10, 4))
    w = rng.standard_normal((4, 3))
    packed_c = oconv.centered(x, w, seg)
    packed_k = oconv.causal(bg, cg, x, w, seg)
    for sid in (1, 2, 3):
        idx = np.flatnonzero(seg[0] == sid)
        sl = slice(idx[0], idx[-1] + 1)
        np.testing.assert_allclose(packed_c[:, sl], oconv.centered(x[:, sl], w), atol=1e-12)
        np.testing.assert_allclose(packed_k[:, sl], oconv.causal(bg[:, sl], cg[:, sl], x[:, sl], w),
                                   atol=1e-12)
    assert (packed_c[0, 8:] == 0).all() and (packed_k[0, 8:] == 0).all()


def test_reference_gradient_fixtures():
    """tests/kernels/test_bidirectional.py:35-38 and :75-78: the gradient of the summed
    output with respect to the values."""
    taps = np.array([[10.0, 100.0, 1000.0]])
    x = np.array([[[1.0], [2.0], [3.0], [4.0]]])
    _, _, dv, _ = oconv.centered_vjp(None, None, x, taps, np.ones_like(x))
    np.testing.assert_array_equal(dv.ravel(), [110, 1110, 1110, 1100])
    x = np.array([[[1.0], [2.0], [3.0], [4.0], [5.0]]])
    _, _, dv, _ = oconv.centered_vjp(None, None, x, taps, np.ones_like(x), np.array([[1, 1, 2, 2, 0]]))
    np.testing.assert_array_equal(dv.ravel(), [110, 1100, 110, 1100, 0])


def _central(fn, x, probe, step=1e-6):
    grad = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        up, lo = x.copy(), x.copy()
        up[idx] += step
        lo[idx] -= step
        grad[idx] = ((fn(up) - fn(lo)) * probe).sum() / (2 * step)
    return grad


def test_vjps_match_central_differences():
    """Method of tests/layers/test_blocks.py:156-174: a nonuniform output probe."""
    rng = np.random.default_rng(3)
    seg = np.array([[1, 1, 1, 2, 2, 0, 3], [4, 4, 4, 4, 4, 4, 4]])
    for centered in (True, False):
        for k in (2, 3, 4):
            x, bg, cg = rng.standard_normal((3, 2, 7, 2))
            w = rng.standard_normal((2, k))
            probe = rng.standard_normal(x.shape)
            if centered:
                fwd = lambda b_, c_, x_, w_: c_ * oconv.centered(b_ * x_, w_, seg)  # noqa: E731
                vjp = oconv.centered_vjp
            else:
                fwd = lambda b_, c_, x_, w_: oconv.causal(b_, c_, x_, w_, seg)  # noqa: E731
                vjp = oconv.causal_vjp
            db, dc, dv, dw = vjp(bg, cg, x, w, probe, seg)
            np.testing.assert_allclose(db, _central(lambda z: fwd(z, cg, x, w), bg, probe), atol=1e-7)
            np.testing.assert_allclose(dc, _central(lambda z: fwd(bg, z, x, w), cg, probe), atol=1e-7)
            np.testing.assert_allclose(dv, _central(lambda z: fwd(bg, cg, z, w), x, probe), atol=1e-7)
            np.testing.assert_allclose(dw, _central(lambda z: fwd(bg, cg, x, z), w, probe), atol=1e-7)


def test_cast_order_restatement_matches_a_hand_derived_bf16_case():
    """One token with its two neighbours, K = 3, centered, gates b and c.  In exact
    arithmetic with round-to-nearest-even to 8 significant bits:
      u_i = bf16(b_i v_i), p_i = bf16(u_i w_i), m = bf16(bf16(p_0 + p_1) + p_2),
      out = bf16(c m) = -5.71875,
    where u unrounded gives -5.78125, unrounded products -5.75 and one rounding of the
    three-term sum -5.75."""
    b = [3.96875, -0.23828125, 2.6875]
    v = [-0.189453125, 1.109375, -2.796875]
    w = [[1.078125, 2.9375, 0.185546875]]
    c = 1.9296875
    bf = lambda x: torch.tensor(x, dtype=torch.float32).to(torch.bfloat16)  # noqa: E731
    tb, tv = bf(b)[None, :, None], bf(v)[None, :, None]
    tc = bf([c, c, c])[None, :, None]
    out = tc * oconv.centered_cast(tb * tv, bf(w))
    assert out.dtype == torch.bfloat16
    assert out[0, 1, 0].item() == -5.71875
    # the causal form with K = 3 reads tokens t-2, t-1, t: the same sum at t = 2
    causal = oconv.causal_cast(tb, tc, tv, bf(w))
    assert causal[0, 2, 0].item() == -5.71875


def test_cast_order_restatement_on_the_reference_fixtures_and_in_float32():
    taps = torch.tensor([[10.0, 100.0, 1000.0]])
    out = oconv.centered_cast(torch.tensor([[[1.0], [2.0], [3.0], [4.0]]]), taps)
    np.testing.assert_array_equal(out.numpy().ravel(), [2100, 3210, 4320, 430])
    out = oconv.centered_cast(torch.tensor([[[1.0], [2.0], [3.0], [4.0], [5.0]]]), taps,
                              torch.tensor([[1, 1, 2, 2, 0]]))
    np.testing.assert_array_equal(out.numpy().ravel(), [2100, 210, 4300, 430, 0])
    rng = np.random.default_rng(4)
    seg = np.array([[1, 1, 1, 2, 2, 0, 3, 3]])
    x, bg, cg = rng.standard_normal((3, 1, 8, 4))
    w = rng.standard_normal((4, 3))
    t = lambda a: torch.tensor(a)  # noqa: E731
    np.testing.assert_allclose(oconv.centered_cast(t(x), t(w), t(seg)).numpy(),
                               oconv.centered(x, w, seg), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oconv.causal_cast(t(bg), t(cg), t(x), t(w), t(seg)).numpy(),
                               oconv.causal(bg, cg, x, w, seg), rtol=1e-12, atol=1e-12)
