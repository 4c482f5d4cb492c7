"""GPU parity of the segmented short convolutions (kernels/bidirectional.py:38-58,
kernels/convolution.py:25-53)."""

import numpy as np
import pytest
import torch

from _helpers import check_bf16, check_bf16_sum, say
from mfattn.kernels import convolution as conv
from oracle import convolution as oconv
from oracle import packing

pytestmark = pytest.mark.gpu


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
    tc = lambda a: torch.tensor(a).to(dtype)  # noqa: E731
    for use_seg in (False, True):
        s = seg if use_seg else None
        st = torch.tensor(seg, device=device) if use_seg else None
        sc = torch.tensor(seg) if use_seg else None
        if mode == "centered":
            got = conv.gated_centered_convolution(td(bg), td(cg), td(x), td(w), st)
            ref = cast(cg) * oconv.centered(cast(bg) * cast(x), cast(w), s)
            emu = tc(cg) * oconv.centered_cast(tc(bg) * tc(x), tc(w), sc)
            plain = conv.centered_convolution(td(x), td(w), st)
            ref_plain = oconv.centered(cast(x), cast(w), s)
            emu_plain = oconv.centered_cast(tc(x), tc(w), sc)
        else:
            fn = conv.gated_depthwise_convolution_segmented if use_seg else conv.gated_depthwise_convolution
            args = (st,) if use_seg else ()
            got = fn(td(bg), td(cg), td(x), td(w), *args, kernel_size=k)
            ref = oconv.causal(cast(bg), cast(cg), cast(x), cast(w), s)
            emu = oconv.causal_cast(tc(bg), tc(cg), tc(x), tc(w), sc)
            plain = ref_plain = emu_plain = None
        for a, r, e in ((got, ref, emu), (plain, ref_plain, emu_plain)):
            if a is None:
                continue
            if dtype == torch.float32:
                np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5)
            else:
                # the reference's declared-dtype rounding, bit for bit
                assert torch.equal(a.cpu(), e), (mode, k, use_seg)


def test_c2_shaped_encoder_convolution(device):
    """The encoder's conv call at the C2 layout: [8, 4096, 1024], K=3, centered."""
    w = packing.make_workload("C2")
    rng = np.random.default_rng(31)
    say("conv C2")
    shape = (w.batch, w.length, 1024)
    x, bg, cg = (torch.randn(shape, device=device, dtype=torch.bfloat16) for _ in range(3))
    taps = torch.tensor(rng.standard_normal((1024, 3)).astype(np.float32))
    seg = torch.tensor(w.segment_ids, device=device)
    got = conv.gated_centered_convolution(bg, cg, x, taps, seg).cpu()
    emu = cg.cpu() * oconv.centered_cast(bg.cpu() * x.cpu(), taps.to(torch.bfloat16),
                                         torch.tensor(w.segment_ids))
    assert torch.equal(got, emu)


def test_reference_gradient_fixtures_on_the_device(device):
    """tests/kernels/test_bidirectional.py:35-38 and :75-78 (one channel, replicated to 8)."""
    say("conv gradient fixtures")
    taps = torch.tensor([[10.0, 100.0, 1000.0]] * 8)
    for vals, seg, want in (([1.0, 2.0, 3.0, 4.0], None, [110, 1110, 1110, 1100]),
                            ([1.0, 2.0, 3.0, 4.0, 5.0], [[1, 1, 2, 2, 0]], [110, 1100, 110, 1100, 0])):
        x = torch.tensor(vals, device=device)[None, :, None].expand(1, len(vals), 8).contiguous()
        x.requires_grad_(True)
        st = None if seg is None else torch.tensor(seg, device=device)
        conv.centered_convolution(x, taps, st).sum().backward()
        np.testing.assert_array_equal(x.grad[0, :, 0].cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("mode", ["centered", "causal"])
def test_backward_matches_the_fp64_vjp(dtype, k, mode, device):
    """mf_segmented_conv_bwd through autograd against the analytic FP64 VJP (pinned by
    the reference's gradient fixtures and central differences).  Every width runs, so
    each channels-per-thread form of the kernel does: 8 channels for K <= 4 and for bf16
    K = 5 centered, 4 channels for the other wide filters (up to the 15-slot ring of
    causal K = 8)."""
    rng = np.random.default_rng(40 + k)
    b, t, c = 3, 77, 24
    say("conv backward", mode, k, dtype)
    seg = np.repeat(rng.integers(0, 4, size=(b, t // 6 + 1)), 6, axis=1)[:, :t].astype(np.int32)
    x, bg, cg, g = (rng.standard_normal((b, t, c)).astype(np.float32) for _ in range(4))
    w = rng.standard_normal((c, k)).astype(np.float32)
    dev = lambda a: torch.tensor(a, device=device).to(dtype).requires_grad_(True)  # noqa: E731
    tx, tb, tcg, tw = dev(x), dev(bg), dev(cg), dev(w)
    st = torch.tensor(seg, device=device)
    if mode == "centered":
        out = conv.gated_centered_convolution(tb, tcg, tx, tw, st)
        vjp = oconv.centered_vjp
    else:
        out = conv.gated_depthwise_convolution_segmented(tb, tcg, tx, tw, st, kernel_size=k)
        vjp = oconv.causal_vjp
    out.backward(torch.tensor(g, device=device).to(dtype))
    cast = lambda a: torch.tensor(a).to(dtype).double().numpy()  # noqa: E731
    rdb, rdc, rdv, rdw, aw = vjp(cast(bg), cast(cg), cast(x), cast(w), cast(g), seg, with_abs=True)
    got = (tb.grad, tcg.grad, tx.grad, tw.grad)
    names = ("db", "dc", "dv", "dw")
    if dtype == torch.float32:
        for name, a, r in zip(names, got, (rdb, rdc, rdv, rdw)):
            scale = max(1.0, float(np.abs(r).max()))
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5 * scale,
                                       err_msg=name)
    else:
        # db, dv: fp32 sums rounded once.  dc = g * m carries the forward's rounded tap sum:
        # K rounded gated inputs, K rounded products and K - 1 rounded partial sums, each
        # within 2**-9 of |g| * sum_i |u w_i| (half of the 2**-8 unit of the sum bar), plus
        # the final rounding
        check_bf16(f"conv bwd {mode} K {k} db", got[0], rdb)
        check_bf16(f"conv bwd {mode} K {k} dv", got[2], rdv)
        scale = (1.5 * k + 1) * _dc_scale(vjp, cast(bg), cast(x), cast(w), cast(g), seg)
        check_bf16_sum(f"conv bwd {mode} K {k} dc", got[1], rdc, scale)
        check_bf16_sum(f"conv bwd {mode} K {k} dw", got[3], rdw, aw)


def _dc_scale(vjp, bg, x, w, g, seg):
    """|g| * sum_i |u_i w_i| over the token's taps: the FP64 dc of |b|, |v|, |w|, |g|."""
    _, dc, _, _ = vjp(np.abs(bg), None, np.abs(x), np.abs(w), np.abs(g), seg)
    return dc


def test_c2_shaped_backward(device):
    """The encoder's conv backward at the C2 layout: [8, 4096, 1024], K=3, centered, bf16:
    deterministic, and the values' gradient equal to a torch fp32 evaluation of the
    transposed convolution."""
    w = packing.make_workload("C2")
    say("conv backward C2")
    shape = (w.batch, w.length, 1024)
    gen = torch.Generator(device=device).manual_seed(5)
    x, bg, cg, g = (torch.randn(shape, device=device, generator=gen, dtype=torch.float32)
                    .to(torch.bfloat16) for _ in range(4))
    taps = (0.5 * torch.randn(1024, 3, device=device, generator=gen)).to(torch.bfloat16)
    seg = torch.tensor(w.segment_ids, device=device)
    grads = []
    for _ in range(2):
        tx = x.clone().requires_grad_(True)
        tw = taps.clone().requires_grad_(True)
        conv.gated_centered_convolution(bg, cg, tx, tw, seg).backward(g)
        grads.append((tx.grad, tw.grad))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    # dv[s] = b[s] * sum_i h[s - o_i] w_i keep, h = g * c, o_i = i - 1
    h = g.float() * cg.float()
    segf = seg
    du = torch.zeros_like(h)
    t = w.length
    for i, off in enumerate((-1, 0, 1)):
        src = torch.arange(t, device=device) - off        # the output token t = s - o_i
        inside = (src >= 0) & (src < t)
        srcc = src.clamp(0, t - 1)
        keep = inside[None, :] & (segf[:, srcc] == segf) & (segf != 0)
        du += h[:, srcc] * taps[:, i].float() * keep[..., None]
    ref = du * bg.float()
    check_bf16("conv bwd C2 dv", grads[0][0], ref)
