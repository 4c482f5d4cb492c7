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
