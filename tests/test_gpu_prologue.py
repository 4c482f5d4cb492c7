"""GPU parity of the attention prologue (layers/attention.py:62-97) and of the
device-side packer positions (batching/packing.py:92-100)."""

import numpy as np
import pytest
import torch

from _helpers import say
from mfattn.kernels import prologue
from oracle import packing
from oracle import prologue as oprol

pytestmark = pytest.mark.gpu


def _scaled_error(a, r):
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return np.abs(a - r).max() / max(1.0, np.abs(r).max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("theta", [10000.0, 1000000.0])
def test_qk_norm_rope_matches_the_oracle(dtype, theta, device):
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
    cast = lambda x: torch.tensor(x).to(dtype).double().numpy()  # noqa: E731
    rq, rk = oprol.qk_norm_rope(cast(q), cast(k), cast(qg), cast(kg), pos, 1e-5, theta)
    for name, got, ref in (("q", gq, rq), ("k", gk, rk)):
        got = got.double().cpu().numpy()
        if dtype == torch.float32:
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            assert _scaled_error(got, ref) < 2e-2, name


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
