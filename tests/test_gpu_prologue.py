"""GPU parity of the attention prologue (layers/attention.py:62-97) and of the
device-side packer positions (batching/packing.py:92-100)."""

import numpy as np
import pytest
import torch

from _helpers import check_bf16, check_bf16_sum, say
from mfattn.kernels import prologue
from oracle import packing
from oracle import prologue as oprol

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("theta", [10000.0, 1000000.0])
def test_qk_norm_rope_matches_the_oracle(dtype, theta, device):
    """fp32 against the FP64 prologue; bf16 against the reference's cast order (every
    operation rounded to bf16), which already carries five roundings an FP64 evaluation
    does not have."""
    rng = np.random.default_rng(20)
    w = packing.make_workload("C1")
    b, t, hq, hkv, d = w.batch, w.length, 16, 8, 64
    say("qk norm rope", dtype, theta)
    pos = oprol.segment_positions(w.segment_ids)
    q = (rng.standard_normal((b, t, hq, d)) * 2).astype(np.float32)
    k = (rng.standard_normal((b, t, hkv, d)) * 2).astype(np.float32)
    qg, kg = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32), rng.standard_normal(d).astype(np.float32)
    tq, tk = (torch.tensor(x, device=device).to(dtype) for x in (q, k))
    gq, gk = prologue.qk_norm_rope(tq, tk, torch.tensor(qg), torch.tensor(kg),
                                   torch.tensor(pos), eps=1e-5, rope_theta=theta)
    if dtype == torch.float32:
        rq, rk = oprol.qk_norm_rope(q, k, qg, kg, pos, 1e-5, theta)
        for name, got, ref in (("q", gq, rq), ("k", gk, rk)):
            np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5, err_msg=name)
    else:
        # the reference's cast order (torch-CPU bf16): bit for bit almost everywhere; where
        # the kernel's fp32 cos/sin or rsqrt differ from torch's in the last bit, a rounded
        # cos, sin or normalised value moves by one bf16 ulp, which moves a rotation
        # product by at most 2**-7 of its operand's magnitude (and, after cancellation in
        # the sum, possibly several ulps of the result): the bar is two such steps
        eq = oprol.qk_norm_rope_cast(torch.tensor(q).to(dtype), torch.tensor(k).to(dtype),
                                     torch.tensor(qg), torch.tensor(kg), pos, 1e-5, theta)
        for name, got, ref, x, gain in (("q", gq, eq[0], q, qg), ("k", gk, eq[1], k, kg)):
            got = got.cpu()
            n = oprol.rms_norm_cast(torch.tensor(x).to(dtype), torch.tensor(gain), 1e-5).float()
            bound = 2.0 ** -6 * (n.abs() + torch.cat((n[..., 32:], n[..., :32]), -1).abs())
            diff = (got.float() - ref.float()).abs()
            exact = (got == ref).float().mean().item()
            say(f"prologue {name} vs cast order: exact {exact:.6f}, max diff {diff.max().item():.3e},"
                f" max diff / bound {(diff / bound.clamp_min(1e-30)).max().item():.3f}")
            assert bool((diff <= bound).all()), name
            assert exact > 0.999, name


def test_hand_derived_bf16_cases_on_the_device(device):
    """The cast-order cases of tests/test_oracle_prologue.py, through the kernel."""
    from test_oracle_prologue import PROLOGUE_CASES

    say("prologue hand cases")
    for x0, x32, x5, g0, g32, p, want, _ in PROLOGUE_CASES:
        x = torch.zeros(1, 1, 1, 64)
        x[0, 0, 0, 0], x[0, 0, 0, 32], x[0, 0, 0, 5] = x0, x32, x5
        gain = torch.ones(64)
        gain[0], gain[32] = g0, g32
        xb = x.to(device, torch.bfloat16)
        out, _ = prologue.qk_norm_rope(xb, xb.clone(), gain, gain, torch.tensor([[p]]), eps=1e-6,
                                       rope_theta=10000.0)
        assert (out[0, 0, 0, 0].item(), out[0, 0, 0, 32].item()) == want


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qk_norm_rope_backward_matches_the_fp64_vjp(dtype, device):
    """mf_qk_norm_rope_bwd through autograd against the analytic FP64 VJP (itself pinned
    by central differences): dq, dk element-wise; the gain gradients, sums over every
    token and head, with the reduction bar."""
    rng = np.random.default_rng(23)
    w = packing.make_workload("C1")
    b, t, hq, hkv, d = w.batch, w.length, 16, 8, 64
    say("prologue backward", dtype)
    pos = oprol.segment_positions(w.segment_ids)
    q = (rng.standard_normal((b, t, hq, d)) * 2).astype(np.float32)
    k = rng.standard_normal((b, t, hkv, d)).astype(np.float32)
    qg, kg = (1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32)
    gq, gk = rng.standard_normal((b, t, hq, d)).astype(np.float32), \
        rng.standard_normal((b, t, hkv, d)).astype(np.float32)
    dev = lambda x: torch.tensor(x, device=device).to(dtype).requires_grad_(True)  # noqa: E731
    tq, tk = dev(q), dev(k)
    tqg = torch.tensor(qg, device=device, requires_grad=True)
    tkg = torch.tensor(kg, device=device, requires_grad=True)
    oq, ok = prologue.qk_norm_rope(tq, tk, tqg, tkg, torch.tensor(pos), eps=1e-5, rope_theta=1e4)
    assert oq.grad_fn is not None and ok.grad_fn is not None
    torch.autograd.backward((oq, ok), (torch.tensor(gq, device=device).to(dtype),
                                       torch.tensor(gk, device=device).to(dtype)))
    cast = lambda x: torch.tensor(x).to(dtype).double().numpy()  # noqa: E731
    rdq, rdk, rdqg, rdkg, aq, ak = oprol.qk_norm_rope_vjp(
        cast(q), cast(k), cast(qg), cast(kg), pos, 1e-5, 1e4, cast(gq), cast(gk), with_abs=True)
    got = (tq.grad, tk.grad, tqg.grad, tkg.grad)
    if dtype == torch.float32:
        for name, a, r in zip(("dq", "dk", "dq_gain", "dk_gain"), got, (rdq, rdk, rdqg, rdkg)):
            scale = max(1.0, float(np.abs(r).max()))
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5 * scale,
                                       err_msg=name)
    else:
        check_bf16("prologue bwd dq", got[0], rdq)
        check_bf16("prologue bwd dk", got[1], rdk)
        check_bf16_sum("prologue bwd dq_gain", got[2], rdqg, aq)
        check_bf16_sum("prologue bwd dk_gain", got[3], rdkg, ak)


def test_backward_is_deterministic_and_in_place_refuses_gradients(device):
    rng = np.random.default_rng(24)
    say("prologue backward determinism")
    b, t = 2, 300
    q = torch.tensor(rng.standard_normal((b, t, 4, 64)), dtype=torch.bfloat16, device=device)
    k = torch.tensor(rng.standard_normal((b, t, 2, 64)), dtype=torch.bfloat16, device=device)
    g = torch.ones(64, device=device)
    runs = []
    for _ in range(2):
        tq, tk = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
        tg = g.clone().requires_grad_(True)
        oq, ok = prologue.qk_norm_rope(tq, tk, tg, tg, None, eps=1e-6, rope_theta=500.0)
        (oq.float().sum() + 2 * ok.float().sum()).backward()
        runs.append((tq.grad, tk.grad, tg.grad))
    for x, y in zip(*runs):
        assert torch.equal(x, y)
    with pytest.raises(ValueError, match="inplace"):
        prologue.qk_norm_rope(q.clone().requires_grad_(True), k, g, g, None, eps=1e-6,
                              rope_theta=500.0, inplace=True)


def test_positions_forms_and_in_place(device):
    rng = np.random.default_rng(21)
    b, t, hq, hkv = 3, 70, 4, 2
    say("rope position forms")
    q = torch.tensor(rng.standard_normal((b, t, hq, 64)), dtype=torch.float32, device=device)
    k = torch.tensor(rng.standard_normal((b, t, hkv, 64)), dtype=torch.float32, device=device)
    g = torch.ones(64)
    base = prologue.qk_norm_rope(q, k, g, g, None, eps=1e-6, rope_theta=500.0)
    arange = prologue.qk_norm_rope(q, k, g, g, torch.arange(t), eps=1e-6, rope_theta=500.0)
    full = prologue.qk_norm_rope(q, k, g, g, torch.arange(t).expand(b, t), eps=1e-6, rope_theta=500.0)
    for x, y in zip(base, arange):
        assert torch.equal(x, y)
    for x, y in zip(base, full):
        assert torch.equal(x, y)
    scalar = prologue.qk_norm_rope(q, k, g, g, 7, eps=1e-6, rope_theta=500.0)
    ref = oprol.qk_norm_rope(q.cpu().numpy(), k.cpu().numpy(), np.ones(64), np.ones(64),
                             np.full((b, t), 7), 1e-6, 500.0)
    for x, r in zip(scalar, ref):
        np.testing.assert_allclose(x.cpu().numpy(), r, rtol=1e-5, atol=1e-5)
    qc, kc = q.clone(), k.clone()
    out = prologue.qk_norm_rope(qc, kc, g, g, None, eps=1e-6, rope_theta=500.0, inplace=True)
    assert out[0] is qc and torch.equal(qc, base[0]) and torch.equal(kc, base[1])
    with pytest.raises(ValueError, match="RoPE positions must match the token dimensions"):
        prologue.qk_norm_rope(q, k, g, g, torch.arange(t + 1), eps=1e-6, rope_theta=500.0)
    with pytest.raises(ValueError, match=r"RoPE positions must be scalar, \[T\], or \[B, T\]"):
        prologue.qk_norm_rope(q, k, g, g, torch.zeros(1, b, t), eps=1e-6, rope_theta=500.0)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_segment_positions_on_the_device(name, device):
    w = packing.make_workload(name)
    say("segment positions", name)
    got = prologue.segment_positions(torch.tensor(w.segment_ids, device=device)).cpu().numpy()
    np.testing.assert_array_equal(got, oprol.segment_positions(w.segment_ids))


def test_segment_positions_ragged_and_repeated_ids(device):
    rng = np.random.default_rng(22)
    say("segment positions random")
    for length in (1, 5, 1023, 1024, 1025, 3000):
        seg = np.repeat(rng.integers(0, 4, size=(3, length // 7 + 1)), 7, axis=1)[:, :length]
        got = prologue.segment_positions(torch.tensor(seg.astype(np.int32), device=device))
        np.testing.assert_array_equal(got.cpu().numpy(), oprol.segment_positions(seg))


@pytest.mark.parametrize("name, hq, hkv, mode, pos_kind", [
    ("C1", 16, 8, 0, "segment"),
    ("C1", 8, 8, 1, "none"),      # G = 1: one head per workgroup
    ("C1", 12, 4, 0, "large"),    # G = 3; positions far beyond T (sincosf's long reduction)
    ("C1", 16, 2, 2, "none"),     # key-mask mode, G = 8
    ("C2", 16, 8, 1, "segment"),  # the bench shape
    ("C5", 16, 8, 0, "segment"),
])
def test_fused_query_prologue_equals_prologue_then_attention(name, hq, hkv, mode, pos_kind, device):
    """mf_attn_fwd_rope_q (norm and RoPE of q in the attention kernel's query loads) against
    mf_qk_norm_rope followed by mf_attn_fwd: output and lse bit for bit."""
    from mfattn import ops
    w = packing.make_workload(name)
    b, t, d = w.batch, w.length, 64
    say("fused query prologue", name, hq, hkv, mode, pos_kind)
    g = torch.Generator(device=device).manual_seed(w.seed)
    mk = lambda h, s: (torch.randn(b, t, h, d, generator=g, device=device) * s).bfloat16()
    q_raw, k_raw, v = mk(hq, 3.0), mk(hkv, 3.0), mk(hkv, 1.0)
    qg = (1 + 0.2 * torch.randn(d, generator=g, device=device)).bfloat16()
    kg = (1 + 0.2 * torch.randn(d, generator=g, device=device)).bfloat16()
    if pos_kind == "segment":
        pos = torch.tensor(oprol.segment_positions(w.segment_ids), device=device)
    elif pos_kind == "large":
        pos = torch.randint(0, 1 << 24, (b, t), generator=g, device=device, dtype=torch.int32)
    else:
        pos = None
    eps, theta, scale = 1e-5, 10000.0, d ** -0.5
    qn, kn = prologue.qk_norm_rope(q_raw, k_raw, qg, kg, pos, eps=eps, rope_theta=theta)
    mask = torch.tensor(w.attention_mask, device=device)
    seg = None if mode == 2 else torch.tensor(w.segment_ids, device=device)
    plan = ops.block_map(seg, mask, mode, t, t)
    ref_out, ref_lse = ops.attn_fwd(qn, kn, v, plan, mode, scale)
    out, lse = ops.attn_fwd_rope_q(q_raw, kn, v, qg, pos, plan, mode, scale, eps=eps,
                                   rope_theta=theta)
    torch.cuda.synchronize()
    same_out = (out.view(torch.int16) == ref_out.view(torch.int16)).float().mean().item()
    say(f"  out bit-equal fraction {same_out:.6f}")
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    assert torch.equal(lse, ref_lse)


def test_fused_query_prologue_at_the_layer_level(device):
    """The kernels-level entry equals qk_norm_rope + packed_causal_attention, and refuses
    inputs that record gradients."""
    from mfattn.kernels import attention
    w = packing.make_workload("C1")
    b, t, hq, hkv, d = w.batch, w.length, 8, 4, 64
    g = torch.Generator(device=device).manual_seed(7)
    mk = lambda h: (torch.randn(b, t, h, d, generator=g, device=device) * 2).bfloat16()
    q_raw, k_raw, v = mk(hq), mk(hkv), mk(hkv)
    qg, kg = torch.rand(d, generator=g, device=device) + 0.5, torch.rand(d, generator=g, device=device) + 0.5
    mask = torch.tensor(w.attention_mask, device=device)
    seg = torch.tensor(w.segment_ids, device=device)
    pos = prologue.segment_positions(seg)
    qn, kn = prologue.qk_norm_rope(q_raw, k_raw, qg, kg, pos, eps=1e-6, rope_theta=1e6)
    ref = attention.packed_causal_attention(qn, kn, v, mask, seg, backend="hip")
    got = prologue.packed_attention_normed_query(q_raw, kn, v, qg, mask, seg, pos, eps=1e-6,
                                                 rope_theta=1e6)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    # the key half alone equals the key output of the joint call
    assert torch.equal(prologue.key_norm_rope(k_raw, kg, pos, eps=1e-6, rope_theta=1e6).view(torch.int16),
                       kn.view(torch.int16))
    with pytest.raises(ValueError, match="no backward"):
        prologue.packed_attention_normed_query(q_raw.requires_grad_(), kn, v, qg, mask, seg, pos,
                                               eps=1e-6, rope_theta=1e6)


@pytest.mark.parametrize("hq, hkv", [(37, 5), (40, 16), (3, 1)])
def test_large_positions_and_head_counts(hq, hkv, device):
    """fp32 at 1e-5 against the FP64 prologue and its VJP with positions up to 2**20 (where a
    one-ulp difference in a rotary frequency would move an angle by ~0.06 rad: the kernel's
    host-side frequencies are the correctly rounded single-precision powers, as the oracle's)
    and head counts that are not multiples of 8 or exceed four 8-head groups per token (the
    forward loads a token's groups in batches of four, the backward in batches of three)."""
    rng = np.random.default_rng(100 + hq)
    b, t, d = 2, 61, 64
    say("prologue positions to 2**20", hq, hkv)
    pos = rng.integers(0, 1 << 20, size=(b, t)).astype(np.int32)
    q = (rng.standard_normal((b, t, hq, d)) * 2).astype(np.float32)
    k = (rng.standard_normal((b, t, hkv, d)) * 2).astype(np.float32)
    qg, kg = (1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32)
    gq, gk = rng.standard_normal((b, t, hq, d)).astype(np.float32), rng.standard_normal((b, t, hkv, d)).astype(np.float32)
    tq, tk = (torch.tensor(x, device=device).requires_grad_(True) for x in (q, k))
    tqg, tkg = (torch.tensor(x, device=device).requires_grad_(True) for x in (qg, kg))
    oq, ok = prologue.qk_norm_rope(tq, tk, tqg, tkg, torch.tensor(pos), eps=1e-5, rope_theta=1e4)
    torch.autograd.backward((oq, ok), (torch.tensor(gq, device=device), torch.tensor(gk, device=device)))
    rq, rk = oprol.qk_norm_rope(q, k, qg, kg, pos, 1e-5, 1e4)
    vjp = oprol.qk_norm_rope_vjp(*(x.astype(np.float64) for x in (q, k, qg, kg)), pos, 1e-5, 1e4,
                                 gq.astype(np.float64), gk.astype(np.float64))
    got = (oq, ok, tq.grad, tk.grad, tqg.grad, tkg.grad)
    for name, a, r in zip(("q", "k", "dq", "dk", "dq_gain", "dk_gain"), got, (rq, rk, *vjp)):
        scale = max(1.0, float(np.abs(r).max()))
        np.testing.assert_allclose(a.detach().cpu().numpy(), r, rtol=1e-5, atol=1e-5 * scale, err_msg=name)
