"""GPU parity of the packed attention forward and backward.

Bars: fp32 within 1e-5 (relative, with a 1e-5 floor) of
the FP64 oracle; bf16 outputs and gradients within 2e-2 of an exact (FP64, or
fp32 at the full shapes) evaluation of the same bf16 inputs, element-wise and
beyond the one bf16 rounding of the result (``max(|a - r| - 2**-8 |r|) <
2e-2``), and within 2e-2 of the reference's bf16 cast-point emulation where
that fits on the CPU.
"""

import json
import pathlib

import numpy as np
import pytest
import torch

from _helpers import (BF16_HALF_ULP, BF16_TOL, DT, check_bf16, check_bf16_sum, max_abs,
                      operands, say, short_segment_rows, torch_reference)
from mfattn import _lib, ops
from mfattn.kernels import attention, bidirectional
from oracle import attention as oatt
from oracle import masks, packing

GOLD = pathlib.Path(__file__).parent / "golden"
FIX = json.loads((GOLD / "reference_fixtures.json").read_text())
pytestmark = pytest.mark.gpu

def _grads(fn, q, k, v, do):
    q, k, v = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    out = fn(q, k, v)
    out.backward(do)
    return out.detach(), q.grad, k.grad, v.grad


def _c1_inputs(device):
    import sys
    sys.path.insert(0, str(GOLD))
    from make_golden import c1_inputs  # noqa: E402

    w, q, k, v, do = c1_inputs()
    t = lambda x: torch.tensor(x, device=device)  # noqa: E731
    return w, t(q), t(k), t(v), t(do)


def test_c1_fp32_forward_backward_matches_fp64_oracle_and_golden(device):
    say("C1 fp32 fwd+bwd packed causal")
    w, q, k, v, do = _c1_inputs(device)
    mask = torch.tensor(w.attention_mask, device=device)
    seg = torch.tensor(w.segment_ids, device=device)
    out, dq, dk, dv = _grads(
        lambda a, b, c: attention.packed_causal_attention(a, b, c, mask, seg, backend="dense"),
        q, k, v, do)
    gold = np.load(GOLD / "c1_fp64.npz")
    np.testing.assert_allclose(gold["checksums"], [x.double().sum().item() for x in (q, k, v, do)],
                               rtol=1e-12)
    ref = oatt.packed_causal_fp64(*(x.cpu().numpy() for x in (q, k, v)), w.attention_mask,
                                  w.segment_ids)
    ref_grads = oatt.vjp_fp64(*(x.cpu().numpy() for x in (q, k, v)), ref[1], ref[2], do.cpu().numpy())
    for got, live, stored in zip((out, dq, dk, dv), (ref[0], *ref_grads),
                                 (gold["out"], gold["dq"], gold["dk"], gold["dv"])):
        np.testing.assert_allclose(got.cpu().numpy(), live, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(got.cpu().numpy(), stored, rtol=1e-5, atol=1e-5)


def test_reference_packed_fixture_fp32(device):
    """tests/kernels/test_attention.py:306-345 operands (D=8, seed 2)."""
    dims = FIX["attention_dims"]
    say("reference packed fixture D=8")
    rng = np.random.default_rng(dims["packed_seed"])
    shapes = [(2, 6, 4, 8), (2, 6, 2, 8), (2, 6, 2, 8)]
    q, k, v = (rng.normal(size=s).astype(np.float32) for s in shapes)
    mask = np.array(FIX["layouts"]["attention_packed"]["mask"], np.int32)
    seg = np.array(FIX["layouts"]["attention_packed"]["segment_ids"], np.int32)
    t = lambda x: torch.tensor(x, device=device)  # noqa: E731
    out = attention.dense_packed_causal_attention(t(q), t(k), t(v), t(mask), t(seg))
    ref = oatt.packed_causal_fp64(q, k, v, mask, seg)[0]
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    assert out.shape == (2, 6, 4, 8)


@pytest.mark.parametrize("mask_dtype", [torch.int32, torch.bool])
def test_bidirectional_uniform_fixture(mask_dtype, device):
    f = FIX["bidirectional"]["uniform"]
    say("bidirectional uniform fixture", mask_dtype)
    q = torch.zeros(f["query_shape"], device=device)
    k = torch.zeros(f["key_shape"], device=device)
    values = torch.tensor(f["values"], device=device)
    mask = torch.tensor(f["mask"], device=device).to(mask_dtype)
    out = bidirectional.attention(q, k, values, mask)
    np.testing.assert_allclose(out.cpu().numpy(), np.broadcast_to(f["output_row"], (1, 3, 2, 2)),
                               rtol=1e-6)
    vv = values.clone().requires_grad_(True)
    bidirectional.attention(q, k, vv, mask).sum().backward()
    np.testing.assert_allclose(vv.grad.cpu().numpy(), f["value_grad_of_sum"], rtol=1e-6)
    empty = bidirectional.attention(q, k, values, torch.zeros_like(mask))
    assert (empty == 0).all()


def test_bidirectional_packed_fixture(device):
    f = FIX["bidirectional"]["packed"]
    say("bidirectional packed fixture")
    q = torch.zeros(f["query_shape"], device=device)
    k = torch.zeros(f["key_shape"], device=device)
    values = torch.tensor(f["values"], device=device).reshape(1, 6, 1, 2)
    seg = torch.tensor(f["segment_ids"], device=device)
    out = bidirectional.attention(q, k, values, seg != 0, seg)
    expected = np.broadcast_to(np.array(f["output_rows"], float)[None, :, None], (1, 6, 2, 2))
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=1e-6)
    vv = values.clone().requires_grad_(True)
    bidirectional.attention(q, k, vv, seg != 0, seg).sum().backward()
    np.testing.assert_allclose(vv.grad.reshape(6, 2).cpu().numpy(), f["value_grad_of_sum"], rtol=1e-6)


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("t", [333, 517])
def test_random_layouts_against_oracle(mode, dtype, t, device):
    """Ragged T, non-contiguous ids, masked holes, GQA 2; FP64 oracle."""
    rng = np.random.default_rng(40 + mode + t)
    b, hq, hkv = 2, 4, 2
    s = (200 if t == 333 else 611) if mode == 2 else t
    say("random layout", mode, dtype, (b, t, s))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, DT[dtype], 0.5, s=s)
    if mode == 2:
        mask = (rng.random((b, s)) > 0.3).astype(np.int32)
        mask[1] = 0
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        seg = np.repeat(rng.integers(0, 5, size=(b, t // 37 + 1)), 37, axis=1)[:, :t].astype(np.int32)
        mask = (rng.random((b, t)) > 0.1).astype(np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), mask, seg,
                            d_out=do.float().cpu().numpy())
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        if dtype == "float32":
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            check_bf16(f"random layout mode {mode} T {t} {name}", a, r)


@pytest.mark.parametrize("t", [1, 2, 63, 64, 65, 127, 128, 129, 191])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_stage_and_tile_edge_lengths(t, mode, dtype, device):
    """Lengths on and beside the 64-row stage and 128-token tile edges (the work lists' units),
    two segments per row meeting at the middle, 16 query heads on one KV head (G = 16) for odd
    lengths and 4 on 2 otherwise; forward and backward against the FP64 oracle."""
    rng = np.random.default_rng(1000 + 10 * t + mode)
    b = 2
    hq, hkv = (16, 1) if t % 2 else (4, 2)
    say("edge length", t, mode, dtype, (hq, hkv))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, DT[dtype], 0.7)
    if mode == 2:
        mask = np.ones((b, t), np.int32)
        mask[1, : (t + 1) // 2] = 0
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        seg = np.ones((b, t), np.int32)
        seg[:, t // 2:] = 2
        seg[1, -1] = 0  # a padding token at the end of row 1
        mask = (seg != 0).astype(np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), mask, seg,
                            d_out=do.float().cpu().numpy())
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        if dtype == "float32":
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            check_bf16(f"edge T {t} mode {mode} {name}", a, r)


@pytest.mark.parametrize("seed", range(16))
def test_randomized_shapes(seed, device):
    """Seeded random calls: batch 1-3, lengths 1-400 (key lengths of their own in the key-mask
    mode), GQA ratios 1-4, ids with holes, repeats and negative values, fp32 and bf16, forward
    and backward against the FP64 oracle."""
    rng = np.random.default_rng(5000 + seed)
    mode = int(rng.integers(0, 3))
    b, t = int(rng.integers(1, 4)), int(rng.integers(1, 401))
    s = int(rng.integers(1, 401)) if mode == 2 else t
    hkv = int(rng.integers(1, 4))
    hq = hkv * int(rng.integers(1, 5))
    dtype = "float32" if seed % 2 else "bfloat16"
    say("randomized", seed, mode, dtype, (b, t, s, hq, hkv))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, DT[dtype], 0.6, s=s)
    if mode == 2:
        mask = (rng.random((b, s)) > 0.25).astype(np.int32)
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        run = int(rng.integers(1, 90))
        seg = np.repeat(rng.integers(-3, 5, size=(b, t // run + 1)), run, axis=1)[:, :t].astype(np.int32)
        mask = (rng.random((b, t)) > 0.15).astype(np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), mask, seg,
                            d_out=do.float().cpu().numpy())
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        if dtype == "float32":
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            check_bf16(f"randomized {seed} {name}", a, r)


@pytest.mark.parametrize("seed", range(12))
def test_randomized_multi_tile(seed, device):
    """Seeded random calls at multi-tile lengths: 400-5000 tokens (key lengths of their own in
    the key-mask mode), segments of 1-2048 tokens with padding and ids from -4 upward, 1-8 KV
    heads with G up to 8, bf16 forward and backward against the fp32 reference at the
    element-wise bf16 bar."""
    rng = np.random.default_rng(90000 + seed)
    mode = int(rng.integers(0, 3))
    b, t = int(rng.integers(1, 4)), int(rng.integers(400, 5001))
    s = int(rng.integers(64, 5001)) if mode == 2 else t
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = min(hkv * int(rng.choice([1, 2, 3, 4, 8])), 32)
    say("randomized multi-tile", seed, mode, (b, t, s, hq, hkv))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, torch.bfloat16, 0.6, s=s)
    if mode == 2:
        mask = (rng.random((b, s)) > rng.uniform(0.05, 0.9)).astype(np.int32)
        mask[:, 0] = 1
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        seg = np.zeros((b, t), np.int32)
        for r in range(b):
            pos, sid = 0, int(rng.integers(-5, 3))
            while pos < t:
                n = int(rng.integers(1, 91)) if rng.random() < 0.6 else int(rng.integers(91, 2049))
                sid += 1
                sid += sid == 0
                seg[r, pos:pos + n] = 0 if rng.random() < 0.1 else sid
                pos += n
        mask = (rng.random((b, t)) > 0.05).astype(np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = torch_reference(mode, q, k, v, mask, seg, do)
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        diff = (a.float() - r).abs()
        raw, excess = diff.max().item(), (diff - BF16_HALF_ULP * r.abs()).max().item()
        say(f"randomized multi-tile {seed} {name}: max-abs {raw:.3e} beyond-rounding {excess:.3e}")
        assert excess < BF16_TOL, (name, raw, excess)


@pytest.mark.parametrize("seed", range(4))
def test_randomized_multi_tile_fp32(seed, device):
    """The fp32 kernels at multi-tile lengths (400-3000 tokens, three modes, segments of
    1-2048 tokens, G up to 4) against the per-group reference in float64: rtol 1e-5 with the
    absolute term scaled by the tensor's largest magnitude, since dK/dV sum up to ~10^4 terms
    whose fp32 accumulation moves a cancelled element by ~1e-5 absolute."""
    rng = np.random.default_rng(95000 + seed)
    mode = int(rng.integers(0, 3))
    b, t = int(rng.integers(1, 3)), int(rng.integers(400, 3001))
    s = int(rng.integers(64, 3001)) if mode == 2 else t
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 3, 4]))
    say("randomized multi-tile fp32", seed, mode, (b, t, s, hq, hkv))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, torch.float32, 0.6, s=s)
    if mode == 2:
        mask = (rng.random((b, s)) > rng.uniform(0.05, 0.9)).astype(np.int32)
        mask[:, 0] = 1
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        seg = np.zeros((b, t), np.int32)
        for r in range(b):
            pos, sid = 0, 1
            while pos < t:
                n = int(rng.integers(1, 91)) if rng.random() < 0.6 else int(rng.integers(91, 2049))
                seg[r, pos:pos + n] = 0 if rng.random() < 0.1 else sid
                sid += 1
                pos += n
        mask = (rng.random((b, t)) > 0.05).astype(np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = torch_reference(mode, q, k, v, mask, seg, do, dtype=torch.float64)
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        scale = max(1.0, r.abs().max().item())
        excess = ((a.double() - r).abs() - 1e-5 * r.abs()).max().item()
        say(f"randomized multi-tile fp32 {seed} {name}: beyond rtol {excess:.3e} (atol {1e-5 * scale:.2e})")
        assert excess <= 1e-5 * scale, (name, excess)


def _chunked_row(rng, t):
    """One row of ``t`` tokens cut into chunks of 128-token multiples (up to 4096 tokens), each
    filled with whole segments of 16-128 tokens (one in eight of 129-4096, cut at the chunk's
    end) and 5 % padding; ids increase along the row, so no segment crosses a chunk edge."""
    bounds = [0]
    while bounds[-1] < t:
        bounds.append(min(t, bounds[-1] + 128 * int(rng.integers(1, 33))))
    seg = np.zeros(t, np.int32)
    sid = 0
    for lo, hi in zip(bounds, bounds[1:]):
        pos = lo
        while pos < hi:
            n = int(rng.integers(16, 129)) if rng.random() < 0.875 else int(rng.integers(129, 4097))
            n = min(n, hi - pos)
            if rng.random() >= 0.05:
                sid += 1
                seg[pos:pos + n] = sid
            pos += n
    return seg[None], bounds


def _packed_fn(mode, mask, seg, device):
    tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
    if mode == 0:
        return lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
    return lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731


@pytest.mark.parametrize("mode", [0, 1])
def test_long_row_against_reference_and_its_windows(mode, device):
    """One row of 524,288 tokens (a 1 GiB bf16 query row, 4096 query tiles: the block map
    classifies each tile's 8192 stages in eight rounds): forward and backward within the bf16
    bar of the fp32 reference (evaluated on the device in float32), and bit-identical to the
    same calls on windows of whole chunks cut out of the row at its start, middle and end."""
    t, hq, hkv = 524288, 16, 8
    rng = np.random.default_rng(524288 + mode)
    seg, bounds = _chunked_row(rng, t)
    mask = (seg != 0).astype(np.int32)
    say("long row", t, "mode", mode, "chunks", len(bounds) - 1)
    gen = torch.Generator(device=device).manual_seed(524288 + mode)
    mk = lambda h, sc: (torch.randn((1, t, h, 64), generator=gen, device=device) * sc).to(torch.bfloat16)  # noqa: E731
    q, k, v, do = mk(hq, 0.5), mk(hkv, 0.5), mk(hkv, 0.5), mk(hq, 1.0)
    got = _grads(_packed_fn(mode, mask, seg, device), q, k, v, do)
    ref = torch_reference(mode, q, k, v, mask, seg, do)
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        diff = (a.float() - r).abs()
        raw, excess = diff.max().item(), (diff - BF16_HALF_ULP * r.abs()).max().item()
        say(f"long row mode {mode} {name}: max-abs {raw:.3e} beyond-rounding {excess:.3e}")
        assert excess < BF16_TOL, (name, raw, excess)
    del ref, diff
    n = len(bounds) - 1
    for i0, i1 in ((0, 3), (n // 2, n // 2 + 3), (n - 3, n)):
        lo, hi = bounds[i0], bounds[i1]
        say("window", lo, hi)
        sub = _grads(_packed_fn(mode, mask[:, lo:hi], seg[:, lo:hi], device),
                     *(x[:, lo:hi] for x in (q, k, v, do)))
        for name, a, w in zip(("out", "dq", "dk", "dv"), got, sub):
            assert torch.equal(a[:, lo:hi], w), (name, lo, hi)


def _rounding_magnitudes(mode, q, k, v, do, mask, seg):
    """FP64 magnitude sums that bound what bf16 rounding inside the kernels can do to each
    output: P is rounded before P V and dS before dS K and dS^T Q (relative 2**-9 each), and
    D = rowsum(dO * O) is formed from the bf16-rounded O; the outputs are rounded once.
    Returns, per output element, the sum of the magnitudes of the terms those roundings touch
    (plus the output's own magnitude)."""
    q, k, v, do = (np.asarray(x, np.float64) for x in (q, k, v, do))
    b, t, hq, d = q.shape
    g = hq // k.shape[2]
    scale = d ** -0.5
    qid, kid = masks._token_ids(mode, mask, seg, t)
    causal = mode == masks.MODE_PACKED_CAUSAL
    m_out, m_dq = np.zeros_like(q), np.zeros_like(q)
    m_dk, m_dv = np.zeros_like(k), np.zeros_like(v)
    for row in range(b):
        for ident in np.unique(qid[row][qid[row] != masks.Q_INACTIVE]):
            qi, kj = np.flatnonzero(qid[row] == ident), np.flatnonzero(kid[row] == ident)
            if kj.size == 0:
                continue
            allowed = (kj[None, :] <= qi[:, None]) if causal else np.ones((qi.size, kj.size), bool)
            for h in range(hq):
                kh = h // g
                sc = np.where(allowed, q[row, qi, h] @ k[row, kj, kh].T * scale, -np.inf)
                m = np.where(allowed.any(1), sc.max(1), 0.0)
                e = np.where(allowed, np.exp(sc - m[:, None]), 0.0)
                p = e / np.maximum(e.sum(1), 1e-300)[:, None]
                o = p @ v[row, kj, kh]
                go = do[row, qi, h]
                ds = p * (go @ v[row, kj, kh].T - (go * o).sum(1)[:, None])
                dd = (np.abs(go) * np.abs(o)).sum(1)[:, None]  # bound on D's rounding error / 2**-9
                m_out[row, qi, h] = p @ np.abs(v[row, kj, kh])
                m_dv[row, kj, kh] += p.T @ np.abs(go)
                m_dq[row, qi, h] = scale * ((np.abs(ds) + p * dd) @ np.abs(k[row, kj, kh]))
                m_dk[row, kj, kh] += scale * ((np.abs(ds) + p * dd).T @ np.abs(q[row, qi, h]))
    return m_out, m_dq, m_dk, m_dv


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_large_logits_and_rising_maxima(mode, dtype, device):
    """Logits with a spread of tens (q, k scaled by 4) and keys scaled up along the sequence, so
    each query's running maximum keeps rising: the online softmax rescales at every step (its
    shift moves once the maximum grows by more than 8 in log2 units).  FP64 oracle; fp32 at
    1e-5, bf16 beyond what rounding P, dS, O and the outputs can move them (these logits make
    dQ and dK sums of large, cancelling terms, which the absolute bf16 bar cannot hold)."""
    rng = np.random.default_rng(77 + mode)
    b, t, hq, hkv = 2, 517, 4, 2
    say("large logits", mode, dtype)
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, DT[dtype], 4.0)
    ramp = torch.linspace(0.25, 2.0, t, device=device)[None, :, None, None]
    k = (k.float() * ramp).to(k.dtype)
    if mode == 2:
        mask = (rng.random((b, t)) > 0.2).astype(np.int32)
        seg = None
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, torch.tensor(mask, device=device))  # noqa: E731
    else:
        seg = np.repeat(rng.integers(1, 4, size=(b, t // 150 + 1)), 150, axis=1)[:, :t].astype(np.int32)
        mask = np.ones((b, t), np.int32)
        tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
        if mode == 0:
            fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
        else:
            fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), mask, seg,
                            d_out=do.float().cpu().numpy())
    mags = None if dtype == "float32" else _rounding_magnitudes(
        mode, *(x.float().cpu().numpy() for x in (q, k, v, do)), mask, seg)
    for i, (name, a, r) in enumerate(zip(("out", "dq", "dk", "dv"), got, ref)):
        assert bool(torch.isfinite(a).all()), name
        if dtype == "float32":
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5 * max(1.0, np.abs(r).max()),
                                       err_msg=name)
        else:
            check_bf16_sum(f"large logits mode {mode} {name}", a, r, mags[i] + np.abs(r))


@pytest.mark.parametrize("b, t, s, hq, hkv, seed", [(1, 286, 3, 6, 2, 5030), (3, 315, 10, 3, 1, 5472)])
def test_few_keys_many_queries(b, t, s, hq, hkv, seed, device):
    """Key-mask mode with 3-10 keys for ~300 queries (shapes a randomized sweep found): every dV
    element sums ~900 products P dO with P near 1/2, so bf16 effects that are relative 2**-9
    per term add up beyond the element-wise bf16 bar against FP64 (0.13 at |dV| ~ 37).  They
    are pinned exactly: the forward's lse is the log of the sum of the bf16-rounded
    probabilities (`v_dot2` row sums), and dV is bf16(sum over queries and heads of
    bf16(exp(s - lse)) dO) bit for bit (at most one bf16 ulp where P sits on a rounding
    boundary); every output is within what those roundings can move it from FP64."""
    rng = np.random.default_rng(seed)
    say("few keys", (b, t, s, hq, hkv))
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, torch.bfloat16, 0.6, s=s)
    mask = (rng.random((b, s)) > 0.25).astype(np.int32)
    mask[:, 0] = 1
    plan = ops.block_map(None, torch.tensor(mask, device=device), 2, t, s)
    out, lse = ops.attn_fwd(q, k, v, plan, 2, 0.125)
    dq, dk, dv = ops.attn_bwd(q, k, v, out, do, lse, plan, 2, 0.125)
    q64, k64, do64 = (x.double().cpu() for x in (q, k, do))
    g = hq // hkv
    log2e = 1.4426950408889634
    x = torch.einsum("bthd,bshd->bhts", q64, k64.repeat_interleave(g, dim=2)) * (0.125 * log2e)
    x = x.masked_fill(~torch.tensor(mask, dtype=torch.bool)[:, None, None, :], float("-inf"))
    bf = lambda y: y.float().to(torch.bfloat16).double()  # noqa: E731
    shift = x.max(-1, keepdim=True).values
    lse2_rounded_sums = shift + torch.log2(bf(torch.exp2(x - shift)).sum(-1, keepdim=True))
    lse2 = lse.double().cpu()[..., None] * log2e
    assert (lse2 - lse2_rounded_sums).abs().max().item() < 1e-5
    pb = bf(torch.exp2(x - lse2))
    dv_model = torch.einsum("bhts,bthd->bshd", pb, do64).reshape(b, s, hkv, g, 64).sum(3)
    terms = torch.einsum("bhts,bthd->bshd", pb, do64.abs()).reshape(b, s, hkv, g, 64).sum(3)
    ulps = (dv.cpu().view(torch.int16).int() - dv_model.float().to(torch.bfloat16).view(torch.int16).int()).abs()
    # where the sum cancels, the kernel's fp32 accumulation of ~900 terms (at most 2**-14 of
    # their magnitude sum) can move the small result by more than one of its bf16 ulps
    acc_ok = (dv.cpu().double() - dv_model).abs() <= 2.0 ** -8 * dv_model.abs() + 2.0 ** -14 * terms
    odd = ulps > 1
    say(f"few keys dV against the bf16 model: {int((ulps == 0).sum())} of {ulps.numel()} identical, "
        f"{int(odd.sum())} beyond one ulp at |dV| <= {dv_model.abs()[odd].max().item() if odd.any() else 0:.3g} "
        f"(term sums {terms[odd].min().item() if odd.any() else 0:.3g}+)")
    assert bool((~odd | acc_ok).all()) and float((ulps == 0).float().mean()) > 0.99
    ref = oatt.grouped_fp64(2, *(x_.float().cpu().numpy() for x_ in (q, k, v)), mask, None,
                            d_out=do.float().cpu().numpy())
    mags = _rounding_magnitudes(2, *(x_.float().cpu().numpy() for x_ in (q, k, v, do)), mask, None)
    for i, (name, a_, r) in enumerate(zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), ref)):
        check_bf16_sum(f"few keys {name}", a_, r, mags[i] + np.abs(r))


@pytest.mark.parametrize("hq, hkv", [(4, 4), (8, 2), (6, 2), (3, 1), (16, 2), (2, 2)])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("mode", [0, 1])
def test_gqa_ratios(hq, hkv, dtype, mode, device):
    """Every query-head group size the launchers dispatch on (G = 1, 3, 4, 8 next to the
    G = 2 of the other tests): one head per wave, head pairs, odd groups."""
    rng = np.random.default_rng(hq * 10 + hkv)
    b, t = 1, 256
    say("gqa", hq, hkv, dtype, "mode", mode)
    q, k, v, do = operands(rng, b, t, hq, hkv, 64, DT[dtype], 0.5)
    seg = np.repeat([[1, 2, 3, 0]], [100, 90, 50, 16], axis=1).astype(np.int32)
    ts = torch.tensor(seg, device=device)
    if mode == 0:
        fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, ts != 0, ts)  # noqa: E731
    else:
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, ts != 0, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), seg != 0, seg,
                            d_out=do.float().cpu().numpy())
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        if dtype == "float32":
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            check_bf16(f"gqa {hq}/{hkv} mode {mode} {name}", a, r)


@pytest.mark.parametrize("hq, hkv", [(4, 2), (3, 1), (8, 8), (16, 2)])
@pytest.mark.parametrize("mode", [0, 1])
def test_short_segment_rows_backward(hq, hkv, mode, device):
    """bf16 rows of short segments (gaps, single tokens, 128-token runs on and across tile
    edges, a ragged end) and a row with a longer run, in one batch, against the FP64
    oracle; the fused call and the phase entry points agree, and a second call is
    bit-identical."""
    rng = np.random.default_rng(hq * 3 + hkv + mode)
    t = 517
    seg = short_segment_rows(rng, t)
    say("short-segment rows", hq, hkv, "mode", mode)
    q, k, v, do = operands(rng, seg.shape[0], t, hq, hkv, 64, torch.bfloat16, 0.5)
    ts = torch.tensor(seg, device=device)
    if mode == 0:
        fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, ts != 0, ts)  # noqa: E731
    else:
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, ts != 0, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = oatt.grouped_fp64(mode, *(x.float().cpu().numpy() for x in (q, k, v)), seg != 0, seg,
                            d_out=do.float().cpu().numpy())
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        check_bf16(f"short segments {hq}/{hkv} mode {mode} {name}", a, r)
    plan = ops.block_map(ts, ts != 0, mode, t, t)
    out, lse = ops.attn_fwd(q, k, v, plan, mode, 0.125)
    fused = ops.attn_bwd(q, k, v, out, do, lse, plan, mode, 0.125)
    ws = ops.bwd_workspace(q)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ops.attn_bwd_delta(out, do, lse, ws)
    ops.attn_bwd_dq(q, k, v, do, lse, plan, mode, 0.125, ws, dq)
    ops.attn_bwd_dkdv(q, k, v, do, lse, plan, mode, 0.125, ws, dk, dv)
    for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), fused):
        check_bf16(f"short segments phases vs fused {name}", a, r)
    again = ops.attn_bwd(q, k, v, out, do, lse, plan, mode, 0.125)
    for a, r in zip(again, fused):
        assert torch.equal(a, r)


@pytest.mark.parametrize("name", ["C2", "C3", "C5"])
def test_baseline_config_bf16_fwd_bwd(name, device):
    """Full BASELINE shapes against the fp32 per-segment torch reference."""
    w = packing.make_workload(name)
    mode = masks.MODE_PACKED_CAUSAL if w.causal else masks.MODE_PACKED_BIDIR
    say("baseline", name, "mode", mode)
    rng = np.random.default_rng(w.seed)
    q, k, v, do = operands(rng, w.batch, w.length, w.q_heads, w.kv_heads, w.head_dim,
                           torch.bfloat16, w.qkv_scale)
    tm = torch.tensor(w.attention_mask, device=device)
    ts = torch.tensor(w.segment_ids, device=device)
    if mode == 0:
        fn = lambda a, bb, c: attention.packed_causal_attention(a, bb, c, tm, ts, backend="dense")  # noqa: E731
    else:
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    got = _grads(fn, q, k, v, do)
    ref = torch_reference(mode, q, k, v, w.attention_mask, w.segment_ids, do)
    names = ("out", "dq", "dk", "dv")
    say(name, "ref max |x|", {n: round(r.abs().max().item(), 3) for n, r in zip(names, ref)})
    for n, a, r in zip(names, got, ref):
        check_bf16(f"{name} {n}", a, r, summary=True)


def test_bf16_against_reference_cast_points(device):
    """The reference's bf16 dense path (attention.py:23-33) emulated on the
    CPU at a reduced packed shape; SDPA cast points for bidirectional."""
    rng = np.random.default_rng(77)
    b, t, hq, hkv = 2, 384, 4, 2
    say("cast points", (b, t))
    q, k, v, _ = operands(rng, b, t, hq, hkv, 64, torch.bfloat16, 0.5)
    seg = np.repeat([[1, 2, 3, 4, 0]], [120, 64, 130, 60, 10], axis=1).repeat(b, 0).astype(np.int32)
    mask = (seg != 0).astype(np.int32)
    tm, ts = torch.tensor(mask, device=device), torch.tensor(seg, device=device)
    causal = attention.dense_packed_causal_attention(q, k, v, tm, ts).cpu()
    bidir = bidirectional.attention(q, k, v, tm, ts).cpu()
    valid, active = masks.packed_valid(mask, seg)
    emu = oatt.dense_bf16_einsum(q.cpu(), k.cpu(), v.cpu(), torch.tensor(valid[:, None]))
    emu = emu * torch.tensor(active[:, :, None, None]).to(emu.dtype)
    assert max_abs(causal, emu) < BF16_TOL
    bvalid, present = masks.bidirectional_valid(mask, seg)
    emu = oatt.sdpa_bf16(q.cpu(), k.cpu(), v.cpu(), torch.tensor(bvalid[:, None]))
    emu = torch.where(torch.tensor(present[:, :, None, None]), emu, torch.zeros((), dtype=emu.dtype))
    assert max_abs(bidir, emu) < BF16_TOL


def test_inactive_rows_are_exact_zero_even_with_nan_queries(device):
    """bidirectional.py:31,35: inactive queries return exact 0."""
    rng = np.random.default_rng(1)
    say("nan inactive rows")
    q, k, v, _ = operands(rng, 1, 200, 4, 2, 64, torch.bfloat16)
    seg = np.repeat([[1, 0, 2, 0]], [60, 20, 100, 20], axis=1).astype(np.int32)
    inactive = torch.tensor(seg == 0, device=device)
    q[inactive] = float("nan")
    ts = torch.tensor(seg, device=device)
    out = bidirectional.attention(q, k, v, ts != 0, ts)
    assert torch.isfinite(out).all()
    assert (out[inactive] == 0).all()


def test_all_padding_rows_and_single_token_segments(device):
    rng = np.random.default_rng(2)
    say("padding rows / single tokens")
    q, k, v, do = operands(rng, 3, 130, 4, 2, 64, torch.float32)
    seg = np.zeros((3, 130), np.int32)
    seg[1] = np.arange(1, 131)          # every token its own segment
    seg[2, :64] = 5
    seg[2, 64:] = np.arange(66)         # repeated / mixed ids
    ts = torch.tensor(seg, device=device)
    for mode in (0, 1):
        fn = (lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, ts != 0, ts)) \
            if mode == 0 else (lambda a, bb, c: bidirectional.attention(a, bb, c, ts != 0, ts))
        got = _grads(fn, q, k, v, do)
        ref = oatt.grouped_fp64(mode, *(x.cpu().numpy() for x in (q, k, v)), seg != 0, seg,
                                d_out=do.cpu().numpy())
        for a, r in zip(got, ref):
            np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5)
        assert (got[0][0] == 0).all() and (got[3][0] == 0).all()


@pytest.mark.parametrize("name", ["C2", "C5"])
def test_deterministic_bitwise(name, device):
    w = packing.make_workload(name)
    say("determinism", name)
    rng = np.random.default_rng(9)
    q, k, v, do = operands(rng, w.batch, w.length, w.q_heads, w.kv_heads, 64, torch.bfloat16, 0.5)
    tm = torch.tensor(w.attention_mask, device=device)
    ts = torch.tensor(w.segment_ids, device=device)
    if w.causal:
        fn = lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, tm, ts)  # noqa: E731
    else:
        fn = lambda a, bb, c: bidirectional.attention(a, bb, c, tm, ts)  # noqa: E731
    first = _grads(fn, q, k, v, do)
    second = _grads(fn, q, k, v, do)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_head_dim_padding_path(device):
    """D < 64 is served by zero-padding the head dim (exact)."""
    rng = np.random.default_rng(4)
    say("head dim 32")
    q, k, v, do = operands(rng, 2, 100, 4, 2, 32, torch.float32)
    seg = np.repeat([[1, 2, 0]], [40, 50, 10], axis=1).repeat(2, 0).astype(np.int32)
    ts = torch.tensor(seg, device=device)
    got = _grads(lambda a, bb, c: attention.dense_packed_causal_attention(a, bb, c, ts != 0, ts),
                 q, k, v, do)
    ref = oatt.grouped_fp64(0, *(x.cpu().numpy() for x in (q, k, v)), seg != 0, seg,
                            d_out=do.cpu().numpy())
    for a, r in zip(got, ref):
        np.testing.assert_allclose(a.cpu().numpy(), r, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match="head_dim"):
        attention.dense_packed_causal_attention(
            torch.zeros(1, 8, 2, 128, device=device), torch.zeros(1, 8, 2, 128, device=device),
            torch.zeros(1, 8, 2, 128, device=device), ts[:1, :8] * 0 + 1, ts[:1, :8] * 0 + 1)


@pytest.mark.parametrize("dtype, name", [(torch.bfloat16, "C2"), (torch.bfloat16, "C5"),
                                         (torch.float32, "C1")])
def test_phase_entry_points_match_the_fused_backward(dtype, name, device):
    """mf_attn_bwd_delta / _dq / _dkdv in sequence give the fused backward's gradients, and the
    delta phase leaves -rowsum(dO * O) and lse * log2(e) in the workspace."""
    w = packing.make_workload(name)
    say(f"phase entry points {w.name} {dtype}")
    rng = np.random.default_rng(13)
    q, k, v, do = operands(rng, w.batch, w.length, w.q_heads, w.kv_heads, 64, dtype, 0.5)
    mode = _lib.MODE_PACKED_CAUSAL if w.causal else _lib.MODE_PACKED_BIDIR
    tm = torch.tensor(w.attention_mask, device=device)
    ts = torch.tensor(w.segment_ids, device=device)
    plan = ops.block_map(ts, tm, mode, w.length, w.length)
    out, lse = ops.attn_fwd(q, k, v, plan, mode, 0.125)
    fused = ops.attn_bwd(q, k, v, out, do, lse, plan, mode, 0.125)
    ws = ops.bwd_workspace(q)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ops.attn_bwd_delta(out, do, lse, ws)
    ops.attn_bwd_dq(q, k, v, do, lse, plan, mode, 0.125, ws, dq)
    ops.attn_bwd_dkdv(q, k, v, do, lse, plan, mode, 0.125, ws, dk, dv)
    rows = w.batch * w.q_heads * w.length
    words = ws.view(torch.float32)
    ndelta = words[:rows].view(w.batch, w.q_heads, w.length)
    lse2 = words[rows:2 * rows].view(w.batch, w.q_heads, w.length)
    d_ref = (do.float() * out.float()).sum(-1).permute(0, 2, 1)
    torch.testing.assert_close(-ndelta, d_ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(lse2, lse * float(np.float32(np.log2(np.e))))
    # the fused dq computes D with a different summation order: bf16 gradients agree to
    # the bf16 bar, fp32 ones to the fp32 bar
    for a, r in zip((dq, dk, dv), fused):
        if dtype == torch.float32:
            torch.testing.assert_close(a, r, rtol=1e-5, atol=1e-5)
        else:
            check_bf16("phase entry points vs fused", a, r)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("hq, hkv", [(4, 2), (8, 1)])
def test_stage_aligned_segments_packed_equal_alone_bitwise(mode, hq, hkv, device):
    """A bf16 segment that starts on a 64-token stage boundary of a packed row gives, in
    the forward and the backward, the bits it gives alone in a row of its own length
    (the reference's packed-equals-separate property, tests/models/lfm2_5/test_encoder.py
    :65-103, held exactly): each query (key) visits the segment's keys (queries) in the
    same stages at the same positions, the other segments' pairs contribute exact zeros,
    and the shift decisions of the forward are per query.  Segments that start off a
    stage boundary sum in another order and meet the bf16 bar instead."""
    rng = np.random.default_rng(40 + mode)
    lengths = [100, 64, 1, 37, 200, 130, 65]
    starts, pos = [], 0
    for n in lengths:
        starts.append(pos)
        pos = -(-(pos + n) // 64) * 64 + 64 * int(rng.integers(0, 2))  # gaps of padding
    t = pos + 23
    seg = np.zeros((1, t), np.int32)
    for i, (s0, n) in enumerate(zip(starts, lengths)):
        seg[0, s0:s0 + n] = i + 1
    say("stage-aligned segments", mode, (hq, hkv), t)
    q, k, v, do = operands(rng, 1, t, hq, hkv, 64, torch.bfloat16, 0.5)
    scale = 0.125

    def run(qq, kk, vv, dd, ids):
        ids = torch.tensor(ids, device=device)
        plan = ops.block_map(ids, (ids != 0).to(torch.int32), mode, ids.shape[1], ids.shape[1])
        out, lse = ops.attn_fwd(qq, kk, vv, plan, mode, scale)
        return (out, lse, *ops.attn_bwd(qq, kk, vv, out, dd, lse, plan, mode, scale))

    packed = run(q, k, v, do, seg)
    for s0, n in zip(starts, lengths):
        sl = slice(s0, s0 + n)
        alone = run(*(x[:, sl].contiguous() for x in (q, k, v, do)), np.ones((1, n), np.int32))
        got = (packed[0][:, sl], packed[1][:, :, sl], packed[2][:, sl], packed[3][:, sl],
               packed[4][:, sl])
        for name, a, r in zip(("out", "lse", "dq", "dk", "dv"), got, alone):
            assert torch.equal(a, r), (n, s0, name, max_abs(a, r))
    # the same segments shifted off the stage grid: equal to the bar, not bit for bit
    shifted = np.zeros_like(seg)
    shifted[0, 19:] = seg[0, :-19]
    moved = run(*(torch.roll(x, 19, dims=1).contiguous() for x in (q, k, v, do)), shifted)
    same = 0
    for s0, n in zip(starts, lengths):
        sl, sh = slice(s0, s0 + n), slice(s0 + 19, s0 + 19 + n)
        got = (moved[0][:, sh], moved[2][:, sh], moved[3][:, sh], moved[4][:, sh])
        ref = (packed[0][:, sl], packed[2][:, sl], packed[3][:, sl], packed[4][:, sl])
        for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
            same += int(torch.equal(a, r))
            check_bf16(f"shifted segment of {n} {name}", a, r.float())
    say(f"segments 19 tokens off the stage grid: {same} of {4 * len(lengths)} tensors bit-identical")
