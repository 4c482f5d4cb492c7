"""GPU parity of the ragged split-K decode (kernels/attention.py:264-282)."""

import json
import pathlib

import numpy as np
import pytest
import torch

from _helpers import check_bf16, max_abs, say
from mfattn.kernels import attention
from oracle import attention as oatt
from oracle import packing

FIX = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())
pytestmark = pytest.mark.gpu


def test_reference_cached_fixture(device):
    """tests/kernels/test_attention.py:377-398: seed 3, valid_length 4, D=8."""
    dims = FIX["attention_dims"]
    say("cached fixture")
    rng = np.random.default_rng(dims["cached_seed"])
    q, k, v = (rng.normal(size=s).astype(np.float32)
               for s in [(2, 1, 4, 8), (2, 6, 2, 8), (2, 6, 2, 8)])
    t = lambda x: torch.tensor(x, device=device)  # noqa: E731
    out = attention.cached_attention(t(q), t(k), t(v), torch.tensor(4, dtype=torch.int32),
                                     backend="dense")
    ref = oatt.cached_fp64(q, k, v, np.array(4))[0]
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    assert out.shape == (2, 1, 4, 8)


@pytest.mark.parametrize("dtype,hq,hkv", [
    (torch.float32, 8, 2),
    (torch.bfloat16, 8, 2),   # 4 query heads per KV head
    (torch.bfloat16, 2, 2),   # 1
    (torch.bfloat16, 4, 2),   # 2
    (torch.bfloat16, 6, 2),   # 3: served by the LDS-staged kernel
    (torch.bfloat16, 16, 2),  # 8
    (torch.bfloat16, 32, 2),  # 16: the LDS-staged kernel in two passes of 8 heads
    (torch.float32, 24, 2),   # 12: one pass of 8 heads and one of 4
    (torch.bfloat16, 40, 1),  # 40: five passes, one KV head
])
def test_ragged_lengths_and_edges(dtype, hq, hkv, device):
    rng = np.random.default_rng(5)
    b, cap = 7, 1000
    say("decode ragged", dtype, "hq", hq, "hkv", hkv)
    # 1 token, chunk and 32-key boundaries (256, 257, 31, 33), full and
    # over-full rows, and a length of 0 (uniform average over the capacity)
    lengths = np.array([1, 999, 1000, 1500, 0, 257, 31, 33, 256, -3], np.int32)
    b = lengths.size
    q = rng.standard_normal((b, 1, hq, 64)).astype(np.float32)
    k = rng.standard_normal((b, cap, hkv, 64)).astype(np.float32)
    v = rng.standard_normal((b, cap, hkv, 64)).astype(np.float32)
    t = lambda x: torch.tensor(x, device=device).to(dtype)  # noqa: E731
    out = attention.dense_cached_attention(t(q), t(k), t(v), torch.tensor(lengths, device=device))
    qq, kk, vv = (t(x).float().cpu().numpy() for x in (q, k, v))
    ref = oatt.cached_fp64(qq, kk, vv, lengths)[0]
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    else:
        check_bf16(f"decode ragged {hq}/{hkv}", out, ref)


def test_c4_full_shape(device):
    d = packing.make_decode_workload("C4")
    say("C4 full")
    rng = np.random.default_rng(d.seed)
    g = torch.Generator(device="cpu").manual_seed(d.seed)
    q = torch.randn(d.batch, 1, d.q_heads, d.head_dim, generator=g).to(device, torch.bfloat16)
    k = torch.randn(d.batch, d.capacity, d.kv_heads, d.head_dim, generator=g).to(device, torch.bfloat16)
    v = torch.randn(d.batch, d.capacity, d.kv_heads, d.head_dim, generator=g).to(device, torch.bfloat16)
    lengths = torch.tensor(d.valid_length, device=device)
    out = attention.cached_attention(q, k, v, lengths, backend="cudnn")
    ref = torch.empty(d.batch, 1, d.q_heads, d.head_dim, device=device)
    group = d.q_heads // d.kv_heads
    for row in range(d.batch):
        n = int(d.valid_length[row])
        kk = k[row, :n].float().repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()
        vv = v[row, :n].float().repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()
        qq = q[row, 0].float()[:, None, :].contiguous()
        p = torch.softmax(torch.matmul(qq, kk.transpose(1, 2).contiguous()) * 0.125, dim=-1)
        ref[row, 0] = torch.matmul(p, vv)[:, 0]
    check_bf16("C4 out", out, ref, summary=True)
    del rng


def test_scalar_length_broadcasts_and_backends_agree(device):
    rng = np.random.default_rng(8)
    say("scalar length")
    q = torch.tensor(rng.standard_normal((3, 1, 4, 64)), dtype=torch.float32, device=device)
    k = torch.tensor(rng.standard_normal((3, 50, 2, 64)), dtype=torch.float32, device=device)
    a = attention.cached_attention(q, k, k, 17, backend="dense")
    b = attention.cached_attention(q, k, k, torch.full((3,), 17, dtype=torch.int32), backend="cudnn")
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,hq,hkv", [
    (torch.float32, 8, 2),
    (torch.bfloat16, 8, 2),   # the streaming kernel appends (G = 4)
    (torch.bfloat16, 2, 2),   # G = 1
    (torch.bfloat16, 16, 2),  # G = 8
    (torch.bfloat16, 6, 2),   # G = 3: the prep kernel appends, the LDS-staged kernel decodes
    (torch.bfloat16, 32, 2),  # G = 16: likewise, in two passes of 8 query heads
])
def test_decode_step_appends_per_row(dtype, hq, hkv, device):
    """Ragged KV-cache append + decode (layers/attention.py:309-317, one slot per row).

    Slots follow dynamic_update_slice's start clamping to [0, capacity - 1];
    the step attends over position + 1 slots (position >= capacity reads every
    slot, a negative position gives the uniform average, as mf_decode)."""
    rng = np.random.default_rng(9)
    cap = 300
    positions = np.array([0, 1, 150, 255, 256, 299, 300, 1000, -1], np.int32)
    b = positions.size
    say("decode append", dtype, "hq", hq, "hkv", hkv, positions.tolist())
    t = lambda x: torch.tensor(x, device=device).to(dtype)  # noqa: E731
    q, kn, vn = (t(rng.standard_normal(s).astype(np.float32))
                 for s in ((b, 1, hq, 64), (b, 1, hkv, 64), (b, 1, hkv, 64)))
    kc, vc = (t(rng.standard_normal((b, cap, hkv, 64)).astype(np.float32)) for _ in range(2))
    ekc, evc = kc.clone(), vc.clone()
    slots = np.clip(positions, 0, cap - 1)
    for i in range(b):
        ekc[i, slots[i]] = kn[i, 0]
        evc[i, slots[i]] = vn[i, 0]
    out, kc2, vc2 = attention.cached_attention_step(q, kn, vn, kc, vc,
                                                     torch.tensor(positions, device=device))
    assert kc2 is kc and vc2 is vc
    assert torch.equal(kc, ekc) and torch.equal(vc, evc)
    # same kernels as a plain decode over the written caches: bit-identical
    plain = attention.dense_cached_attention(q, ekc, evc, torch.tensor(positions + 1, device=device))
    assert torch.equal(out, plain)
    ref = oatt.cached_fp64(q.float().cpu().numpy(), ekc.float().cpu().numpy(),
                           evc.float().cpu().numpy(), positions + 1)[0]
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    else:
        check_bf16(f"decode append {hq}/{hkv}", out, ref)


def test_decode_step_scalar_position_and_small_head_dim(device):
    rng = np.random.default_rng(10)
    say("decode append scalar / D=8")
    b, cap, hq, hkv, d = 3, 12, 4, 2, 8
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=device)  # noqa: E731
    q, kn, vn = (t(rng.standard_normal(s)) for s in ((b, 1, hq, d), (b, 1, hkv, d), (b, 1, hkv, d)))
    kc, vc = (t(rng.standard_normal((b, cap, hkv, d))) for _ in range(2))
    k0, v0 = kc.clone(), vc.clone()
    out, kc2, vc2 = attention.cached_attention_step(q, kn, vn, kc, vc, 5)
    k0[:, 5], v0[:, 5] = kn[:, 0], vn[:, 0]
    assert torch.equal(kc2, k0) and torch.equal(vc2, v0)
    ref = oatt.cached_fp64(q.cpu().numpy(), k0.cpu().numpy(), v0.cpu().numpy(), np.full(b, 6))[0]
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match="Unsupported cached attention backend"):
        attention.cached_attention_step(q, kn, vn, kc, vc, 5, backend="splash")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_incremental_decode_equals_the_causal_forward(dtype, device):
    """Token-by-token decode with per-row appends equals the packed causal
    forward over the whole sequence, at every position (the invariant of
    tests/layers/test_blocks.py:223-291: incremental decoding reproduces the
    uninterrupted pass).  Ties the decode path to the forward path: two
    different kernel families computing the same rows."""
    rng = np.random.default_rng(12)
    b, n, cap, hq, hkv = 3, 80, 96, 8, 2
    say("incremental decode", dtype, (b, n, cap))
    t = lambda x: torch.tensor(x, device=device).to(dtype)  # noqa: E731
    q, k, v = (t(rng.standard_normal((b, n, h, 64)).astype(np.float32) * 0.5) for h in (hq, hkv, hkv))
    ones = torch.ones(b, n, dtype=torch.int32, device=device)
    full = attention.dense_packed_causal_attention(q, k, v, ones, ones)
    kc = torch.zeros(b, cap, hkv, 64, dtype=dtype, device=device)
    vc = torch.zeros_like(kc)
    steps = []
    for i in range(n):
        pos = torch.full((b,), i, dtype=torch.int32, device=device)
        out, kc, vc = attention.cached_attention_step(q[:, i:i + 1], k[:, i:i + 1], v[:, i:i + 1],
                                                      kc, vc, pos)
        steps.append(out)
    inc = torch.cat(steps, dim=1)
    assert torch.equal(kc[:, :n], k) and torch.equal(vc[:, :n], v)
    if dtype == torch.float32:
        np.testing.assert_allclose(inc.cpu().numpy(), full.cpu().numpy(), rtol=1e-5, atol=1e-5)
    else:
        # both round P to bf16 at different points (the decode's split-K
        # partials against the forward's 32-key blocks)
        assert max_abs(inc.float(), full.float()) < 2e-2
