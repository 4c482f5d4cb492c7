"""The drop-in composed the way the reference's layers call it (row a11).

``tests/_blocks.py`` restates the reference's block callers in torch over the
mfattn functions (HIP prologue, packed attention, cached decode step, conv);
``oracle/blocks.py`` is their FP64 restatement.  Checked here, after
tests/layers/test_blocks.py and tests/models/lfm2_5/test_encoder.py:

* a packed row equals its segments run as independent rows, and the FP64
  block (test_blocks.py:342-382, test_encoder.py:65-103);
* prefill plus per-row decode steps equal the uninterrupted block
  (test_blocks.py:223-291);
* input and gain gradients through the HIP prologue, attention and conv
  backward equal central differences of the FP64 block (test_blocks.py:156-174);
* one plan serves every layer that shares ``(segment_ids, mask)``, also under
  rematerialisation (models/lfm2_5/encoder.py:186-198).

The composition checks run in float32 against the FP64 blocks, as the
reference's block tests do, and in bfloat16 as the reference's encoder test
also does (``bf16=True``): a bf16 packed row against the same bf16 block run
on each segment alone, and bf16 decode steps against the bf16 forward.  A
block's output is its residual stream, rounded to bf16 at each of its two
residual adds, so each bf16 evaluation may sit 2 * 2**-8 |r| from the exact
value for that reason alone, and two of them 4 * 2**-8 |r| apart; the bar is
the kernels' 2e-2 beyond those four roundings (``check_bf16(...,
roundings=4)``).  Segments that start on a 64-token stage boundary give the
attention kernels' bits exactly
(``test_stage_aligned_segments_packed_equal_alone_bitwise``); whether a whole
bf16 block is bit-identical also depends on torch's projections, and each
case logs it.
"""

import numpy as np
import pytest
import torch
import torch.utils.checkpoint

import _blocks
from _helpers import check_bf16, say
from mfattn import ops
from mfattn.kernels import prologue
from oracle import blocks as oblocks
from oracle import prologue as oprol

pytestmark = pytest.mark.gpu

HEAD_DIM, THETA, EPS = 64, 10000.0, 1e-5


def _weights(seed, hidden, hq, hkv, ffn_dim, channels=None):
    rng = np.random.default_rng(seed)
    out = oblocks.random_weights(rng, hidden, hq, hkv, HEAD_DIM, ffn_dim, channels)
    return rng, out


def _dev(weights, device, dtype=torch.float32):
    return {k: torch.tensor(v, device=device, dtype=dtype) for k, v in weights.items()}


def _layout(lengths, pad):
    seg = np.repeat(np.arange(1, len(lengths) + 2), list(lengths) + [pad])
    seg[-pad:] = 0 if pad else seg[-pad:]
    pos = oprol.segment_positions(seg[None])
    return seg[None].astype(np.int32), pos


def test_packed_causal_block_equals_independent_rows_and_the_fp64_block(device):
    lengths, pad = [100, 57, 130], 13
    rng, (attn, ffn) = _weights(1, 256, 4, 2, 512)
    seg, pos = _layout(lengths, pad)
    t = seg.shape[1]
    say("packed causal block", lengths)
    x = rng.standard_normal((1, t, 256))
    w, f = _dev(attn, device), _dev(ffn, device)
    ts = torch.tensor(seg, device=device)
    # positions from the device producer, as the packer would give them
    tpos = prologue.segment_positions(ts)
    np.testing.assert_array_equal(tpos.cpu().numpy(), pos)
    tx = torch.tensor(x, device=device, dtype=torch.float32)
    got = _blocks.attention_block_packed(tx, w, f, ts != 0, ts, tpos, head_dim=HEAD_DIM,
                                         rope_theta=THETA, eps=EPS, backend="splash")
    want = oblocks.attention_block_packed(x, attn, ffn, seg != 0, seg, pos, head_dim=HEAD_DIM,
                                          rope_theta=THETA, eps=EPS)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=5e-5, atol=5e-5)
    start = 0
    for n in lengths:
        ones = torch.ones(1, n, dtype=torch.int32, device=device)
        alone = _blocks.attention_block_packed(tx[:, start:start + n], w, f, ones, ones, None,
                                               head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS,
                                               backend="dense")
        np.testing.assert_allclose(got[:, start:start + n].cpu().numpy(), alone.cpu().numpy(),
                                   rtol=1e-5, atol=1e-5)
        start += n


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_and_per_row_decode_steps_equal_the_uninterrupted_block(dtype, device):
    """Row 0 is prefilled with 8 tokens, row 1 with 5; both then decode one token per
    step at their own cache slot (one slot per row, the ragged append)."""
    rng, (attn, ffn) = _weights(2, 128, 4, 2, 256)
    n, cap, prefill = 40, 48, [8, 5]
    say("prefill + decode steps", dtype)
    x = rng.standard_normal((2, n, 128))
    w, f = _dev(attn, device, dtype), _dev(ffn, device, dtype)
    tx = torch.tensor(x, device=device).to(dtype)
    ones = torch.ones(2, n, dtype=torch.int32, device=device)
    full = _blocks.attention_block_packed(tx, w, f, ones, ones, None, head_dim=HEAD_DIM,
                                          rope_theta=THETA, eps=EPS, backend="dense")
    mask = torch.zeros(2, prefill[0], dtype=torch.int32, device=device)
    for r, p in enumerate(prefill):
        mask[r, :p] = 1
    first, kc, vc = _blocks.attention_block_prefill(tx[:, :prefill[0]], w, f, mask, capacity=cap,
                                                    head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS,
                                                    backend="dense")
    outs = {0: [first[0, :prefill[0]]], 1: [first[1, :prefill[1]]]}
    steps = n - min(prefill)
    for i in range(steps):
        position = torch.tensor([prefill[0] + i, prefill[1] + i], dtype=torch.int32, device=device)
        tok = torch.stack([tx[r, min(int(position[r]), n - 1)] for r in range(2)])[:, None]
        out, kc, vc = _blocks.attention_block_step(tok, w, f, kc, vc, position, head_dim=HEAD_DIM,
                                                   rope_theta=THETA, eps=EPS, backend="cudnn")
        for r in range(2):
            if int(position[r]) < n:
                outs[r].append(out[r])
    for r in range(2):
        inc = torch.cat(outs[r], 0)
        assert inc.shape[0] == n
        if dtype == torch.float32:
            np.testing.assert_allclose(inc.cpu().numpy(), full[r].cpu().numpy(), rtol=1e-5,
                                       atol=1e-5)
        else:
            check_bf16(f"decode steps row {r}", inc, full[r].float(), roundings=4)


def _central(fn, x, probe, step=1e-6):
    g = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        up, lo = x.copy(), x.copy()
        up[idx] += step
        lo[idx] -= step
        g[idx] = ((fn(up) - fn(lo)) * probe).sum() / (2 * step)
    return g


def test_packed_block_gradients_match_central_differences(device):
    """Input and QK-gain gradients through the HIP prologue and attention backward."""
    lengths, pad = [10, 9], 5
    rng, (attn, ffn) = _weights(3, 32, 2, 1, 48)
    seg, pos = _layout(lengths, pad)
    t = seg.shape[1]
    say("packed block gradients")
    x = rng.standard_normal((1, t, 32))
    probe = np.linspace(-0.7, 1.0, x.size).reshape(x.shape)
    w, f = _dev(attn, device), _dev(ffn, device)
    w["query_norm"].requires_grad_(True)
    ts = torch.tensor(seg, device=device)
    tx = torch.tensor(x, device=device, dtype=torch.float32, requires_grad=True)
    out = _blocks.attention_block_packed(tx, w, f, ts != 0, ts, torch.tensor(pos), head_dim=HEAD_DIM,
                                         rope_theta=THETA, eps=EPS, backend="dense")
    (out * torch.tensor(probe, device=device, dtype=torch.float32)).sum().backward()

    def fwd(xx, gain=attn["query_norm"]):
        ww = dict(attn, query_norm=gain)
        return oblocks.attention_block_packed(xx, ww, ffn, seg != 0, seg, pos, head_dim=HEAD_DIM,
                                              rope_theta=THETA, eps=EPS)
    np.testing.assert_allclose(tx.grad.cpu().numpy(), _central(fwd, x, probe), rtol=1e-4, atol=2e-6)
    gq = _central(lambda g: fwd(x, g), attn["query_norm"].copy(),
                  np.broadcast_to(probe, probe.shape))
    np.testing.assert_allclose(w["query_norm"].grad.cpu().numpy(), gq, rtol=1e-4, atol=2e-6)


def _aligned_layout(lengths, pad):
    """Segments starting on 64-token stage boundaries, padding (id 0) between them."""
    starts, pos = [], 0
    for n in lengths:
        starts.append(pos)
        pos = -(-(pos + n) // 64) * 64
    seg = np.zeros(pos + pad, np.int64)
    for i, (s0, n) in enumerate(zip(starts, lengths)):
        seg[s0:s0 + n] = i + 1
    return seg[None].astype(np.int32), oprol.segment_positions(seg[None]), starts


@pytest.mark.parametrize("aligned", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["conv", "attention"])
def test_encoder_blocks_packed_equal_independent_rows(kind, dtype, aligned, device):
    lengths, pad = [70, 33, 128, 17], 8
    rng, (attn, ffn, conv) = _weights(4, 128, 4, 2, 256, channels=64)
    params = conv if kind == "conv" else attn
    if aligned:
        seg, pos, starts = _aligned_layout(lengths, pad)
    else:
        seg, pos = _layout(lengths, pad)
        starts = list(np.cumsum([0] + lengths[:-1]))
    t = seg.shape[1]
    say("encoder block", kind, dtype, "stage-aligned" if aligned else "contiguous")
    x = rng.standard_normal((1, t, 128))
    p, f = _dev(params, device, dtype), _dev(ffn, device, dtype)
    ts = torch.tensor(seg, device=device)
    tx = torch.tensor(x, device=device).to(dtype)
    got = _blocks.encoder_block(tx, p, f, ts != 0, ts, torch.tensor(pos), kind=kind,
                                head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS)
    if dtype == torch.float32:
        want = oblocks.encoder_block(x, params, ffn, seg != 0, seg, pos, kind=kind,
                                     head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS)
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=5e-5, atol=5e-5)
    identical = 0
    for start, n in zip(starts, lengths):
        ones = torch.ones(1, n, dtype=torch.int32, device=device)
        alone = _blocks.encoder_block(tx[:, start:start + n], p, f, ones, ones, None, kind=kind,
                                      head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS)
        seg_out = got[:, start:start + n]
        identical += int(torch.equal(seg_out, alone))
        if dtype == torch.float32:
            np.testing.assert_allclose(seg_out.cpu().numpy(), alone.cpu().numpy(), rtol=1e-5,
                                       atol=1e-5)
        else:
            check_bf16(f"encoder {kind} segment of {n}", seg_out, alone.float(), roundings=4)
    say(f"encoder {kind} {dtype} {'stage-aligned' if aligned else 'contiguous'}: "
        f"{identical} of {len(lengths)} segments bit-identical to their rows alone")


def test_encoder_conv_block_gradients_match_central_differences(device):
    """Input gradient through the HIP conv backward, the way the encoder trains it."""
    lengths, pad = [9, 6], 3
    rng, (_, ffn, conv) = _weights(5, 16, 2, 1, 24, channels=8)
    seg, pos = _layout(lengths, pad)
    say("encoder conv gradients")
    x = rng.standard_normal((1, seg.shape[1], 16))
    probe = np.linspace(-0.7, 1.0, x.size).reshape(x.shape)
    p, f = _dev(conv, device), _dev(ffn, device)
    ts = torch.tensor(seg, device=device)
    tx = torch.tensor(x, device=device, dtype=torch.float32, requires_grad=True)
    out = _blocks.encoder_block(tx, p, f, ts != 0, ts, None, kind="conv", head_dim=HEAD_DIM,
                                rope_theta=THETA, eps=EPS)
    (out * torch.tensor(probe, device=device, dtype=torch.float32)).sum().backward()
    fwd = lambda xx: oblocks.encoder_block(xx, conv, ffn, seg != 0, seg, pos, kind="conv",  # noqa: E731
                                           head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS)
    np.testing.assert_allclose(tx.grad.cpu().numpy(), _central(fwd, x, probe), rtol=1e-4, atol=2e-6)


def test_one_plan_serves_every_layer_sharing_ids_under_rematerialisation(device):
    """Six encoder attention layers over one (segment_ids, mask), each forward run twice
    by torch.utils.checkpoint (jax.checkpoint in encoder.py:193-198): one block map for
    the whole step, and the same outputs and gradients as fresh plans per call."""
    lengths, pad = [300, 129, 64], 19
    rng, (attn, ffn) = _weights(6, 128, 4, 2, 256)
    seg, pos = _layout(lengths, pad)
    say("plan reuse")
    x = rng.standard_normal((1, seg.shape[1], 128))
    w, f = _dev(attn, device, torch.bfloat16), _dev(ffn, device, torch.bfloat16)
    ts = torch.tensor(seg, device=device)
    mask = ts != 0
    tpos = torch.tensor(pos, device=device)

    def run():
        h = torch.tensor(x, device=device).to(torch.bfloat16).requires_grad_(True)
        out = h
        for _ in range(6):
            out = torch.utils.checkpoint.checkpoint(
                lambda hh: _blocks.encoder_block(hh, w, f, mask, ts, tpos, kind="attention",
                                                 head_dim=HEAD_DIM, rope_theta=THETA, eps=EPS),
                out, use_reentrant=False)
        out.float().sum().backward()
        return out.detach(), h.grad

    ops.PLANS.clear()
    before = ops._BLOCK_MAP_CALLS[0]
    shared = run()
    assert ops._BLOCK_MAP_CALLS[0] - before == 1
    ops.PLANS.enabled = False
    try:
        before = ops._BLOCK_MAP_CALLS[0]
        fresh = run()
        assert ops._BLOCK_MAP_CALLS[0] - before == 12
    finally:
        ops.PLANS.enabled = True
    for a, b in zip(shared, fresh):
        assert torch.equal(a, b)
