"""GPU parity of the segmented short convolutions (kernels/bidirectional.py:38-58,
kernels/convolution.py:25-53)."""

import numpy as np
import pytest
import torch

from _helpers import say
from mfattn.kernels import convolution as conv
from oracle import convolution as oconv
from oracle import packing

pytestmark = pytest.mark.gpu


def _scaled_error(a, r):
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return np.abs(a - r).max() / max(1.0, np.abs(r).max())


def test_reference_fixtures_on_the_device(device):
    """test_bidirectional.py:29-37, :66-77 (one channel, replicated to 8)."""
    say("conv fixtures")
    taps = torch.tensor([[10.0, 100.0, 1000.0]] * 8)
    x = torch.tensor([1.0, 2.0, 3.0, 4.0], device=device)[None, :, None].expand(1, 4, 8).contiguous()
    out = conv.centered_convolution(x, taps)
    np.testing.assert_array_equal(out[0, :, 0].cpu().numpy(), [2100, 3210, 4320, 430])
    x = torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0], device=device)[None, :, None].expand(1, 5, 8).contiguous()
    out = conv.centered_convolution(x, taps, torch.tensor([[1, 1, 2, 2, 0]], device=device))
    np.testing.assert_array_equal(out[0, :, 0].cpu().numpy(), [2100, 210, 4300, 430, 0])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("mode", ["centered", "causal"])
def test_random_layouts(dtype, k, mode, device):
    rng = np.random.default_rng(30 + k)
    b, t, c = 3, 77, 24
    say("conv", mode, k, dtype)
    seg = np.repeat(rng.integers(0, 4, size=(b, t // 6 + 1)), 6, axis=1)[:, :t].astype(np.int32)
    x, bg, cg = (rng.standard_normal((b, t, c)).astype(np.float32) for _ in range(3))
    w = rng.standard_normal((c, k)).astype(np.float32)
    td = lambda a: torch.tensor(a, device=device).to(dtype)  # noqa: E731
    cast = lambda a: torch.tensor(a).to(dtype).double().numpy()  # noqa: E731
    for use_seg in (False, True):
        s = seg if use_seg else None
        st = torch.tensor(seg, device=device) if use_seg else None
        if mode == "centered":
            got = conv.gated_centered_convolution(td(bg), td(cg), td(x), td(w), st)
            ref = cast(cg) * oconv.centered(cast(bg) * cast(x), cast(w), s)
            plain = conv.centered_convolution(td(x), td(w), st)
            ref_plain = oconv.centered(cast(x), cast(w), s)
        else:
            fn = conv.gated_depthwise_convolution_segmented if use_seg else conv.gated_depthwise_convolution
            args = (st,) if use_seg else ()
            got = fn(td(bg), td(cg), td(x), td(w), *args, kernel_size=k)
            ref = oconv.causal(cast(bg), cast(cg), cast(x), cast(w), s)
            plain = ref_plain = None
        for a, r in ((got, ref), (plain, ref_plain)):
            if a is None:
                continue
            if dtype == torch.float32:
                np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5)
            else:
                assert _scaled_error(a.float().cpu().numpy(), r) < 2e-2


def test_c2_shaped_encoder_convolution(device):
    """The encoder's conv call at the C2 layout: [8, 4096, 1024], K=3, centered."""
    w = packing.make_workload("C2")
    rng = np.random.default_rng(31)
    say("conv C2")
    shape = (w.batch, w.length, 1024)
    x, bg, cg = (torch.randn(shape, device=device, dtype=torch.bfloat16) for _ in range(3))
    taps = torch.tensor(rng.standard_normal((1024, 3)).astype(np.float32))
    seg = torch.tensor(w.segment_ids, device=device)
    got = conv.gated_centered_convolution(bg, cg, x, taps, seg).float().cpu().numpy()
    d = lambda a: a.double().cpu().numpy()  # noqa: E731
    ref = d(cg) * oconv.centered(d(bg) * d(x), taps.to(torch.bfloat16).double().numpy(),
                                 w.segment_ids)
    assert _scaled_error(got, ref) < 2e-2
