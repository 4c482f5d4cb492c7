"""The packed attention step under HIP graph capture.

Serving loops and training steps capture their launches once and replay them
(hipGraph through torch.cuda.CUDAGraph).  Every launch of the step -- the
block map's kernels, the forward, the backward -- goes to the caller's stream
with no allocation, memset or host synchronisation inside the library, so the
captured step replays with new inputs and gives what the eager calls give,
bit for bit (the kernels are deterministic).  Replays alternate with eager
work and synchronisations, and every replay is checked.
"""

import numpy as np
import pytest
import torch

from _helpers import say
from mfattn import ops
from oracle import packing

pytestmark = pytest.mark.gpu


def _step(q, k, v, do, seg, mask, mode):
    plan = ops.block_map(seg, mask, mode, q.shape[1], k.shape[1])
    out, lse = ops.attn_fwd(q, k, v, plan, mode, q.shape[-1] ** -0.5)
    dq, dk, dv = ops.attn_bwd(q, k, v, out, do, lse, plan, mode, q.shape[-1] ** -0.5)
    return out, lse, dq, dk, dv


@pytest.mark.parametrize("mode", [0, 1])
def test_captured_step_replays_equal_eager(mode, device):
    rng = np.random.default_rng(11 + mode)
    b, t, hq, hkv, d = 2, 1000, 8, 4, 64
    say("graph capture", mode)
    seg_np = np.zeros((b, t), np.int32)
    for row in range(b):
        pos, sid = 0, 1
        while pos < t:
            n = int(rng.integers(20, 400))
            seg_np[row, pos:pos + n] = sid
            pos, sid = pos + n, sid + 1
        seg_np[row, t - 37:] = 0  # trailing padding
    seg = torch.tensor(seg_np, device=device)
    mask = (seg != 0).to(torch.int32)
    mk = lambda h: torch.empty(b, t, h, d, device=device, dtype=torch.bfloat16)  # noqa: E731
    q, k, v, do = mk(hq), mk(hkv), mk(hkv), mk(hq)

    def fill(seed):
        g = torch.Generator(device=device).manual_seed(seed)
        for x in (q, k, v, do):
            x.copy_(torch.randn(x.shape, generator=g, device=device))

    fill(0)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        _step(q, k, v, do, seg, mask, mode)  # warm-up on a side stream, as capture requires
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(q, k, v, do, seg, mask, mode)
    for trial in range(3):
        fill(100 + trial)
        graph.replay()
        torch.cuda.synchronize(device)
        eager = _step(q, k, v, do, seg, mask, mode)
        torch.cuda.synchronize(device)
        for name, a, r in zip(("out", "lse", "dq", "dk", "dv"), captured, eager):
            same = torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a.view(torch.int16),
                               r.view(torch.int32) if r.dtype == torch.float32 else r.view(torch.int16))
            assert same, (trial, name)


def _problem(seed, mode, device):
    rng = np.random.default_rng(seed)
    b, t, hq, hkv, d = 2, 777, 8, 2, 64
    seg_np = np.zeros((b, t), np.int32)
    for row in range(b):
        pos, sid = 0, 1
        while pos < t:
            n = int(rng.integers(10, 300))
            seg_np[row, pos:pos + n] = sid
            pos, sid = pos + n, sid + 1
    seg = torch.tensor(seg_np, device=device)
    mask = (seg != 0).to(torch.int32)
    g = torch.Generator(device=device).manual_seed(seed)
    mk = lambda h: torch.randn(b, t, h, d, generator=g, device=device).to(torch.bfloat16)  # noqa: E731
    return mk(hq), mk(hkv), mk(hkv), mk(hq), seg, mask, mode


def test_two_streams_at_once_equal_serial_calls(device):
    """The library keeps no state between calls: two problems launched alternately on two
    streams (default priority) while both are in flight give what serial calls give, bit for
    bit."""
    say("two streams")
    probs = [_problem(21, 0, device), _problem(22, 1, device)]
    serial = [_step(*p) for p in probs]
    torch.cuda.synchronize(device)
    streams = [torch.cuda.Stream(device) for _ in probs]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(device))
    results = [[], []]
    for _ in range(3):
        for i, (p, s) in enumerate(zip(probs, streams)):
            with torch.cuda.stream(s):
                results[i].append(_step(*p))
    torch.cuda.synchronize(device)
    for i in range(2):
        for rep in results[i]:
            for name, a, r in zip(("out", "lse", "dq", "dk", "dv"), rep, serial[i]):
                assert torch.equal(a, r), (i, name)


def _layout(rng, b, t):
    seg = np.zeros((b, t), np.int32)
    for row in range(b):
        pos, sid = int(rng.integers(0, 40)), 1
        while pos < t:
            n = int(rng.integers(16, 500))
            seg[row, pos:pos + n] = sid
            pos, sid = pos + n, sid + 1
    return seg


@pytest.mark.parametrize("mode", [0, 1])
def test_default_plan_cache_under_capture(mode, device):
    """``packed_attention`` with ``plan=None`` (the default plan cache) captured into a
    graph: each replay runs with the segment ids and mask then in the static buffers
    (new layouts copied in between replays), so the captured step records its own
    block map instead of reusing the warm-up's plan; eager calls after the capture on
    the same tensors, and on a second stream, equal calls with a fresh plan."""
    rng = np.random.default_rng(31 + mode)
    b, t, hq, hkv, d = 2, 900, 4, 2, 64
    scale = d ** -0.5
    say("plan cache under capture", mode)
    seg = torch.tensor(_layout(rng, b, t), device=device)
    mask = (seg != 0).to(torch.int32)
    g = torch.Generator(device=device).manual_seed(5)
    mk = lambda h: torch.randn(b, t, h, d, generator=g, device=device).to(torch.bfloat16)  # noqa: E731
    q, k, v, do = mk(hq), mk(hkv), mk(hkv), mk(hq)
    for x in (q, k, v):
        x.requires_grad_(True)

    def step():
        out = ops.packed_attention(q, k, v, mask, seg, mode, scale)
        return (out, *torch.autograd.grad(out, (q, k, v), do))

    def fresh():
        with torch.no_grad():
            plan = ops.block_map(seg, mask, mode, t, t)
            out, lse = ops.attn_fwd(q.detach(), k.detach(), v.detach(), plan, mode, scale)
            return (out, *ops.attn_bwd(q.detach(), k.detach(), v.detach(), out, do, lse, plan,
                                       mode, scale))

    ops.PLANS.clear()
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        step()  # warm-up: caches an eager plan of the first layout
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for trial in range(3):
        new = torch.tensor(_layout(rng, b, t), device=device)
        with torch.no_grad():
            seg.copy_(new)
            mask.copy_((new != 0).to(torch.int32))
        graph.replay()
        torch.cuda.synchronize(device)
        want = fresh()
        eager = step()
        torch.cuda.synchronize(device)
        for name, a, e, r in zip(("out", "dq", "dk", "dv"), captured, eager, want):
            assert torch.equal(a, r), (trial, "replay", name)
            assert torch.equal(e, r), (trial, "eager after capture", name)
    other = torch.cuda.Stream(device)
    other.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(other):
        again = step()
    torch.cuda.current_stream(device).wait_stream(other)
    torch.cuda.synchronize(device)
    for name, a, r in zip(("out", "dq", "dk", "dv"), again, fresh()):
        assert torch.equal(a, r), ("second stream", name)
