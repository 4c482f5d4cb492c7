"""Benchmark of the packed-attention hot path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

* step = one pass of the hot path over the C2 batch (LFM2.5-350M encoder
  shape: 8 rows x 4096 tokens, packed bidirectional attention, 16/8 heads,
  D=64, bf16): block map + flash forward + the backward (dq with the row
  sums D fused in, then dk/dv), with q/k/v/dO resident in HBM.  ``value`` =
  useful fwd+bwd TFLOP/s (12 * D * Hq * useful pairs per step / time) over
  ``--steps`` steps after ``--warmup`` untimed ones (defaults 100 and 50; the
  GPU needs ~25 steps to reach its steady clocks).
* ``roofline`` = the dominant kernel of the step (largest average launch
  duration, timed with HIP events on the launch stream) against the bf16 MFMA
  peak; ``traffic`` comes from the committed rocprofv3 PMC summary when one
  exists for that kernel and workload, else null.
* ``decode`` = the C4 ragged KV-cached decode (64 x 1 token, cache lengths
  U[128, 8192]): algorithmic HBM GB/s and its roofline fraction.
* ``rows`` = the kernels either side of the attention path (QK-norm+RoPE
  prologue, segment positions, segmented conv, decode with the KV append,
  block map from placements) at the same shapes, each timed over
  back-to-back C-ABI calls: microseconds, and algorithmic GB/s against the
  HBM peak for the streaming ones.
* ``cpu_baseline`` = the reference's dense bidirectional path restated in
  torch on the host cores (XLA-SDPA cast points: fp32 logits, bf16
  probabilities; fwd + autograd bwd), timed per (row, KV-group) chunk of the
  same C2 batch for about ``--cpu-seconds`` and scaled to useful TFLOP/s.

* ``configs`` = the same step on the causal packed workloads C3 (4 x 8192,
  mean segment 512) and C5 (1 x 32768, segments of 16-128 tokens): ms per
  step, useful TFLOP/s and the fraction of the max(MFMA, HBM) roofline time.

The decode, the rows, C5 and then C3 are measured before the C2 step.  Each
packed leg first runs ``SETTLE_STEPS`` untimed steps of its own workload (the
GPU's clocks take ~30 launches to settle after a change of load), then its
per-kernel sample, then its ``--warmup`` and ``--steps``.
``--config C3`` or ``--config C5`` (or ``--config C2 --step-only``) prints one of
those step lines alone.

Only one GPU is used; ``--gpus`` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "minifield-training_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "packed GQA attn fwd+bwd useful TFLOP/s @350M shape; ragged decode HBM GB/s"
MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBPS = 8000.0
# untimed steps of a packed leg's workload before its measurements (clock settling)
SETTLE_STEPS = 40


def _events(n):
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _time_calls(fn, iters):
    """Average ms of ``fn`` (stream-ordered launches) with events around each call."""
    import torch

    starts, ends = _events(iters), _events(iters)
    for i in range(iters):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / iters


def _traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed PMC summary, or None."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(workload, {}).get(kernel)
    return None if entry is None else entry["bytes"]


def gpu_leg(steps: int, warmup: int, profile: bool = False, name: str = "C2", decode: bool = True):
    import torch

    from mfattn import _lib, ops, workloads

    dev = torch.device("cuda:0")
    w = workloads.packed(name)
    mode = _lib.MODE_PACKED_CAUSAL if w.causal else _lib.MODE_PACKED_BIDIR
    # operands drawn on the device (seeded): no host-side pause between the
    # previous measurement and this one's warm-up, so the clocks stay up
    gen = torch.Generator(device=dev).manual_seed(w.seed)

    def mk(shape, scale):
        return (torch.randn(shape, generator=gen, device=dev) * scale).to(torch.bfloat16)

    q = mk((w.batch, w.length, w.q_heads, w.head_dim), w.qkv_scale)
    k = mk((w.batch, w.length, w.kv_heads, w.head_dim), w.qkv_scale)
    v = mk((w.batch, w.length, w.kv_heads, w.head_dim), w.qkv_scale)
    do = mk((w.batch, w.length, w.q_heads, w.head_dim), 1.0)
    mask = torch.tensor(w.attention_mask, device=dev)
    seg = torch.tensor(w.segment_ids, device=dev)
    scale = w.head_dim ** -0.5
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = ops.bwd_workspace(q)

    def step():
        # the product path: block map, forward, one backward call (mf_attn_bwd:
        # dq with D fused in, then dk/dv)
        plan = ops.block_map(seg, mask, mode, w.length, w.length)
        out, lse = ops.attn_fwd(q, k, v, plan, mode, scale)
        ops.attn_bwd(q, k, v, out, do, lse, plan, mode, scale)

    if profile:  # one step and one decode for the PMC passes, untimed
        step()
        torch.cuda.synchronize()
        del q, k, v, do, dq, dk, dv, ws
        torch.cuda.empty_cache()
        decode_leg(0, 0, profile=True)
        return None

    # Clock settling: after a switch from another workload (or from idle) the
    # step runs ~13 % slower for its first ~30 launches while the GPU's clocks
    # settle on the new load (one box, per-step times: ~700 us at steps 4-9,
    # ~615 us from step 35 on), which a 5-step warm-up leaves inside a 20-step
    # timed window.  SETTLE_STEPS untimed steps of this workload (~25 ms at C2)
    # come before any of this leg's measurements.
    for _ in range(SETTLE_STEPS):
        step()
    torch.cuda.synchronize()

    # Per-kernel durations: HIP events on the launch stream between the
    # launches of a step, over a fixed sample of at least 50 steps of this
    # workload.  The backward is the product call (dq with D fused in, then
    # dk/dv); dk/dv is then launched once more on its own through its phase
    # entry point (same kernel, D from an untimed delta launch), and dq is the
    # difference.
    names = ("block_map", "attn_fwd", "attn_bwd", "attn_bwd_dkdv")
    out, lse = ops.attn_fwd(q, k, v, ops.block_map(seg, mask, mode, w.length, w.length), mode, scale)
    ops.attn_bwd_delta(out, do, lse, ws)
    samples = max(steps, 50)
    marks = [_events(len(names) + 1) for _ in range(samples)]
    for ev in marks:
        ev[0].record()
        plan = ops.block_map(seg, mask, mode, w.length, w.length)
        ev[1].record()
        out, lse = ops.attn_fwd(q, k, v, plan, mode, scale)
        ev[2].record()
        ops.attn_bwd(q, k, v, out, do, lse, plan, mode, scale)
        ev[3].record()
        ops.attn_bwd_dkdv(q, k, v, do, lse, plan, mode, scale, ws, dk, dv)
        ev[4].record()
    torch.cuda.synchronize()
    kern = {name: sum(ev[i].elapsed_time(ev[i + 1]) for ev in marks) / samples
            for i, name in enumerate(names)}
    kern["attn_bwd_dq"] = kern["attn_bwd"] - kern["attn_bwd_dkdv"]

    # the product step: `warmup` untimed steps, then exactly `steps` timed ones
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = _events(2)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(end) / steps
    flops = workloads.attention_flops(w)
    nbytes = workloads.attention_bytes(w)["fwd_bwd"]
    algo = {"attn_fwd": flops["fwd"], "attn_bwd_dq": flops["dq"], "attn_bwd_dkdv": flops["dkdv"]}
    dominant = max(algo, key=lambda name: kern[name])
    achieved = algo[dominant] / (kern[dominant] * 1e-3) / 1e12
    value = flops["fwd_bwd"] / (ms * 1e-3) / 1e12
    result = {
        "value": value,
        "ms_per_step": ms,
        "wall_ms_per_step": wall_ms,
        "config": {"workload": w.description, "global_batch": w.batch, "seq_len": w.length,
                   "q_heads": w.q_heads, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "useful_pairs_per_head": workloads.useful_pairs(w.segment_ids, w.causal),
                   "useful_gflop_per_step": flops["fwd_bwd"] / 1e9, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "kernel": dominant, "achieved": achieved,
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
                     "traffic": _traffic(dominant, name),
                     "algorithmic_gflop_per_launch": algo[dominant] / 1e9},
        "fa2_convention_tflops": flops["fwd_bwd_fa2"] / (ms * 1e-3) / 1e12,
        "step_roofline_frac": (flops["fwd_bwd"] / (MFMA_BF16_PEAK_TFLOPS * 1e12)) / (ms * 1e-3),
        # the step against max(MFMA, HBM) roofline time (BASELINE.md accounting)
        "step_roofline": {
            "mfma_us": flops["fwd_bwd"] / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e6,
            "hbm_us": nbytes / (HBM_PEAK_GBPS * 1e9) * 1e6,
            "bound": "mfma" if flops["fwd_bwd"] / (MFMA_BF16_PEAK_TFLOPS * 1e12)
            >= nbytes / (HBM_PEAK_GBPS * 1e9) else "hbm",
            "frac": max(flops["fwd_bwd"] / (MFMA_BF16_PEAK_TFLOPS * 1e12),
                        nbytes / (HBM_PEAK_GBPS * 1e9)) / (ms * 1e-3),
            "algorithmic_bytes": nbytes},
        "kernels_ms": kern,
    }
    del q, k, v, do, dq, dk, dv, out, lse, plan, ws
    torch.cuda.empty_cache()
    result["decode"] = decode_leg(steps, warmup) if decode else None
    return result


def decode_leg(steps: int, warmup: int, profile: bool = False):
    import torch

    from mfattn import ops, workloads

    dev = torch.device("cuda:0")
    d = workloads.decode("C4")
    g = torch.Generator(device=dev).manual_seed(d.seed)
    shape_q = (d.batch, 1, d.q_heads, d.head_dim)
    shape_c = (d.batch, d.capacity, d.kv_heads, d.head_dim)
    q = torch.randn(shape_q, generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn(shape_c, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(shape_c, generator=g, device=dev).to(torch.bfloat16)
    lengths = torch.tensor(d.valid_length, device=dev)
    scale = d.head_dim ** -0.5
    run = lambda: ops.decode(q, kc, vc, lengths, scale)  # noqa: E731
    if profile:
        run()
        torch.cuda.synchronize()
        return None
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    iters = max(steps, 10)
    ms = _time_calls(run, iters)
    nbytes = workloads.decode_bytes(d)
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"metric": "ragged decode HBM GB/s", "value": gbps, "unit": "GB/s", "us_per_step": ms * 1e3,
            "workload": d.description, "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": gbps / HBM_PEAK_GBPS, "traffic": _traffic("decode", "C4")}}


def _time_batch(fn, iters: int) -> float:
    """Average ms of ``iters`` back-to-back calls between two events on the launch stream.

    The calls go straight to the C ABI with pointers computed beforehand, so
    the host enqueues faster than the GPU drains and the average is the
    kernels' own time (the first call's launch latency is spread over all).
    """
    import torch

    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    start, end = _events(2)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def rows_leg(steps: int, profile: bool = False):
    """The kernels on either side of the attention path at the bench shapes.

    qk_norm_rope, segment_positions and segmented_conv (and the backward of
    the prologue and the conv) run on the C2 layout (8 x 4096 packed tokens,
    16/8 heads of 64, an encoder conv over 1024 channels), decode_append on C4 (each row appends at its cache length, then
    decodes), block_map_placements on the placements of C2's segments.
    ``bytes`` counts each input read and each output written once.
    """
    import numpy as np
    import torch

    from mfattn import _lib, ops, workloads

    L = _lib.LIB
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    w = workloads.packed("C2")
    b, t = w.batch, w.length
    g = torch.Generator(device=dev).manual_seed(w.seed)
    bf = torch.bfloat16
    seg = torch.tensor(w.segment_ids, device=dev, dtype=torch.int32)
    pos = torch.empty_like(seg)
    rows = {}

    def run(name, fn, nbytes, bound="hbm", workload="C2"):
        if profile:
            fn()
            torch.cuda.synchronize()
            return
        ms = _time_batch(fn, max(steps, 20))
        entry = {"workload": workload, "us": ms * 1e3, "bound": bound}
        if nbytes:
            gbps = nbytes / (ms * 1e-3) / 1e9
            entry.update(bytes=nbytes, GBps=gbps, frac=gbps / HBM_PEAK_GBPS,
                         traffic=_traffic(name, workload))
        rows[name] = entry

    run("segment_positions", lambda: _lib.check(L.mf_segment_positions(p(seg), b, t, p(pos), stream)),
        0, "latency")
    q = torch.randn(b, t, w.q_heads, w.head_dim, generator=g, device=dev).to(bf)
    k = torch.randn(b, t, w.kv_heads, w.head_dim, generator=g, device=dev).to(bf)
    qg = (1 + 0.1 * torch.randn(w.head_dim, generator=g, device=dev)).to(bf)
    kg = (1 + 0.1 * torch.randn(w.head_dim, generator=g, device=dev)).to(bf)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    run("qk_norm_rope", lambda: _lib.check(L.mf_qk_norm_rope(
        p(q), p(k), p(qg), p(kg), p(pos), _lib.DTYPE_BF16, b, t, w.q_heads, w.kv_heads, w.head_dim,
        1e-5, 1e6, p(qo), p(ko), stream)), 2 * (q.nbytes + k.nbytes) + pos.nbytes)
    # backward: reads q, k and the output gradients, writes dq, dk (the gain
    # gradients are reduced through a [blocks, 2, D] fp32 workspace)
    dqo, dko = torch.randn_like(q), torch.randn_like(k)
    dqi, dki = torch.empty_like(q), torch.empty_like(k)
    dgq = torch.empty(w.head_dim, device=dev, dtype=torch.float32)
    dgk = torch.empty_like(dgq)
    rws_bytes = L.mf_qk_norm_rope_bwd_workspace_bytes(b, t)
    rws = torch.empty(max(rws_bytes, 1), dtype=torch.uint8, device=dev)
    run("qk_norm_rope_bwd", lambda: _lib.check(L.mf_qk_norm_rope_bwd(
        p(q), p(k), p(qg), p(kg), p(pos), p(dqo), p(dko), _lib.DTYPE_BF16, b, t, w.q_heads,
        w.kv_heads, w.head_dim, 1e-5, 1e6, p(dqi), p(dki), p(dgq), p(dgk), p(rws), rws_bytes,
        stream)), 3 * (q.nbytes + k.nbytes) + pos.nbytes)
    del dqo, dko, dqi, dki, rws
    # the prologue feeding the attention forward (C2, bidirectional): q and k
    # normalised and rotated, then the forward; against the key half alone
    # plus the forward with the query half in its query loads (the cos/sin
    # table launch included)
    v = torch.randn_like(k)
    mode = _lib.MODE_PACKED_CAUSAL if w.causal else _lib.MODE_PACKED_BIDIR
    mask = torch.tensor(w.attention_mask, device=dev)
    aplan = ops.block_map(seg, mask, mode, t, t)
    out, lse = torch.empty_like(q), torch.empty(b, w.q_heads, t, device=dev, dtype=torch.float32)
    table_bytes = L.mf_rope_table_bytes(b, t)
    table = torch.empty(table_bytes, dtype=torch.uint8, device=dev)
    scale = w.head_dim ** -0.5

    def separate():
        _lib.check(L.mf_qk_norm_rope(p(q), p(k), p(qg), p(kg), p(pos), _lib.DTYPE_BF16, b, t,
                                     w.q_heads, w.kv_heads, w.head_dim, 1e-5, 1e6, p(qo), p(ko),
                                     stream))
        _lib.check(L.mf_attn_fwd(p(qo), p(ko), p(v), _lib.DTYPE_BF16, b, t, t, w.q_heads,
                                 w.kv_heads, w.head_dim, mode, scale, p(aplan.buf), aplan.nbytes,
                                 p(out), p(lse), stream))

    def fused():
        _lib.check(L.mf_qk_norm_rope(None, p(k), None, p(kg), p(pos), _lib.DTYPE_BF16, b, t, 0,
                                     w.kv_heads, w.head_dim, 1e-5, 1e6, None, p(ko), stream))
        _lib.check(L.mf_attn_fwd_rope_q(p(q), p(ko), p(v), p(qg), p(pos), _lib.DTYPE_BF16, b, t,
                                        t, w.q_heads, w.kv_heads, w.head_dim, mode, scale, 1e-5,
                                        1e6, p(aplan.buf), aplan.nbytes, p(table), table_bytes,
                                        p(out), p(lse), stream))

    run("prologue_then_fwd", separate, 0, "composite")
    run("fwd_with_query_prologue", fused, 0, "composite")
    del q, k, qo, ko, v, out, lse, table, aplan
    ch, taps = 1024, 3
    x = [torch.randn(b, t, ch, generator=g, device=dev).to(bf) for _ in range(3)]
    wt = (0.5 * torch.randn(ch, taps, generator=g, device=dev)).to(bf)
    y = torch.empty_like(x[0])
    run("segmented_conv", lambda: _lib.check(L.mf_segmented_conv(
        p(x[0]), p(x[1]), p(x[2]), p(wt), p(seg), _lib.CONV_CENTERED, _lib.DTYPE_BF16, b, t, ch, taps,
        p(y), stream)), 4 * y.nbytes + seg.nbytes + wt.nbytes)
    # backward: reads the gates, the values and dy, writes their three
    # gradients; the tap gradients go through a per-tile fp32 workspace
    dx = [torch.empty_like(y) for _ in range(3)]
    dw = torch.empty(ch, taps, device=dev, dtype=torch.float32)
    cws_bytes = L.mf_segmented_conv_bwd_workspace_bytes(b, t, ch, taps)
    cws = torch.empty(max(cws_bytes, 1), dtype=torch.uint8, device=dev)
    dy = torch.randn_like(y)
    run("segmented_conv_bwd", lambda: _lib.check(L.mf_segmented_conv_bwd(
        p(x[0]), p(x[1]), p(x[2]), p(wt), p(seg), p(dy), _lib.CONV_CENTERED, _lib.DTYPE_BF16, b, t,
        ch, taps, p(dx[0]), p(dx[1]), p(dx[2]), p(dw), p(cws), cws_bytes, stream)),
        7 * y.nbytes + seg.nbytes + wt.nbytes)
    del x, y, dx, dy, cws
    runs = []
    for r in range(b):
        ids = w.segment_ids[r]
        edges = np.flatnonzero(np.diff(np.concatenate(([0], ids, [0]))) != 0)
        runs += [(r, int(s), int(e - s)) for s, e in zip(edges[:-1], edges[1:]) if ids[s] != 0]
    pl = torch.tensor(runs, device=dev, dtype=torch.int32)
    plan_bytes = L.mf_plan_bytes(b, t, t)
    plan = torch.empty(plan_bytes, dtype=torch.uint8, device=dev)
    seg2, pos2 = torch.empty_like(seg), torch.empty_like(seg)
    run("block_map_placements", lambda: _lib.check(L.mf_block_map_placements(
        p(pl), pl.shape[0], _lib.MODE_PACKED_BIDIR, b, t, p(plan), plan_bytes, p(seg2), p(pos2),
        stream)), 0, "latency")
    del plan
    d = workloads.decode("C4")
    gq, gc = (d.batch, 1, d.q_heads, d.head_dim), (d.batch, d.capacity, d.kv_heads, d.head_dim)
    dq = torch.randn(gq, generator=g, device=dev).to(bf)
    kn = torch.randn(d.batch, 1, d.kv_heads, d.head_dim, generator=g, device=dev).to(bf)
    vn = torch.randn_like(kn)
    kc = torch.randn(gc, generator=g, device=dev).to(bf)
    vc = torch.randn(gc, generator=g, device=dev).to(bf)
    at = np.minimum(np.asarray(d.valid_length, np.int64), d.capacity - 1)
    positions = torch.tensor(at, device=dev, dtype=torch.int32)
    out = torch.empty_like(dq)
    ws_bytes = L.mf_decode_workspace_bytes(d.batch, d.capacity, d.q_heads, d.head_dim)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    kv_row = d.kv_heads * d.head_dim * 2
    nbytes = (int((at + 1).sum()) * 2 * kv_row + 2 * dq.nbytes + positions.nbytes
              + 2 * (kn.nbytes + vn.nbytes))
    run("decode_append", lambda: _lib.check(L.mf_decode_append(
        p(dq), p(kn), p(vn), p(positions), _lib.DTYPE_BF16, d.batch, d.capacity, d.q_heads,
        d.kv_heads, d.head_dim, d.head_dim ** -0.5, p(kc), p(vc), p(out), p(ws), ws_bytes, stream)),
        nbytes, workload="C4")
    del dq, kn, vn, kc, vc, out, ws
    torch.cuda.empty_cache()
    return None if profile else rows


def cpu_leg(seconds: float):
    """Dense reference path on the host, per (row, KV-group) chunk of C2."""
    import numpy as np
    import torch

    from mfattn import workloads
    from oracle import attention as oatt
    from oracle import masks as omasks

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = workloads.packed("C2")
    g = w.q_heads // w.kv_heads
    rng = np.random.default_rng(w.seed)
    done_flops, elapsed, chunks = 0, 0.0, 0
    total_chunks = w.batch * w.kv_heads
    for row in range(w.batch):
        valid, present = omasks.bidirectional_valid(w.attention_mask[row : row + 1],
                                                    w.segment_ids[row : row + 1])
        valid_t = torch.tensor(valid[:, None])
        present_t = torch.tensor(present[:, :, None, None])
        pairs = workloads.useful_pairs(w.segment_ids[row : row + 1], w.causal)
        for _ in range(w.kv_heads):
            mk = lambda h: torch.tensor(  # noqa: E731
                rng.standard_normal((1, w.length, h, w.head_dim)).astype(np.float32) * w.qkv_scale
            ).to(torch.bfloat16).requires_grad_(True)
            q, k, v = mk(g), mk(1), mk(1)
            do = torch.randn(1, w.length, g, w.head_dim).to(torch.bfloat16)
            t0 = time.perf_counter()
            out = oatt.sdpa_bf16(q, k, v, valid_t)
            out = torch.where(present_t, out, torch.zeros((), dtype=out.dtype))
            out.backward(do)
            elapsed += time.perf_counter() - t0
            done_flops += 12 * w.head_dim * g * pairs
            chunks += 1
            if elapsed >= seconds:
                break
        if elapsed >= seconds:
            break
    return {"value": done_flops / elapsed / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{chunks} of {total_chunks} (row, KV-group) chunks of C2 in {elapsed:.1f} s; "
                      "dense bidirectional attention with XLA-SDPA cast points (fp32 logits, bf16 "
                      "probabilities) restated in torch-CPU, forward + autograd backward; useful "
                      "FLOPs of the chunks / time"}


# --------------------------------------------------------------------------
# HBM traffic of the measured kernels (rocprofv3 PMC passes)
#
#   cd /tmp && export TMPDIR=/tmp
#   rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/pmc_fetch -o run \
#       -- python3 <root>/bench.py --profile-step
#   rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/pmc_write -o run \
#       -- python3 <root>/bench.py --profile-step
#   python3 bench.py --traffic <out>/pmc_fetch <out>/pmc_write
#
# --profile-step runs one device-to-device copy of CALIB_BYTES (the
# calibration: it reads and writes exactly that many bytes), one C2 step,
# one C4 decode and one call of each ``rows`` kernel.  --traffic scales each kernel's FETCH_SIZE / WRITE_SIZE
# (KiB per dispatch) by what the counters read for the copy and writes
# profiles/traffic.json, which the timed run reports as roofline.traffic.
# --------------------------------------------------------------------------
CALIB_BYTES = 512 << 20
TRAFFIC_KERNELS = {
    # bench name -> (device kernels as name prefixes, workload, which dispatch of each kernel:
    # None = the mean over the run's dispatches; 0 / 1 = the first / second, for kernels that
    # --profile-step launches for two different calls)
    "block_map": (("mf::token_ids_kernel", "mf::tile_runs_kernel", "mf::tile_lists_kernel",
                   "mf::order_kernel"), "C2", None),
    # the plain forward only (the instances with the query prologue are <., true>)
    "attn_fwd": (("mf::attn_fwd_bf16_kernel<2, false>", "mf::attn_fwd_bf16_kernel<1, false>"),
                 "C2", None),
    "attn_bwd_dq": (("mf::bwd_dq_bf16_kernel<",), "C2", None),  # computes D itself in the product call
    "attn_bwd_dkdv": (("mf::bwd_dkdv_bf16_kernel",), "C2", None),
    "decode": (("mf::decode_prep_kernel", "mf::decode_rows_kernel<", "mf::decode_bf16_kernel<",
                "mf::decode_combine_kernel<"), "C4", 0),
    "decode_append": (("mf::decode_rows_kernel<", "mf::decode_bf16_kernel<",
                       "mf::decode_combine_kernel<"), "C4", 1),
    # the first dispatch: the qk_norm_rope row (the composite rows after it launch it again,
    # the last one for the keys alone)
    "qk_norm_rope": (("mf::qk_norm_rope_kernel<",), "C2", 0),
    "qk_norm_rope_bwd": (("mf::qk_norm_rope_bwd_kernel<", "mf::rope_gain_reduce_kernel"), "C2",
                         None),
    "segmented_conv": (("mf::segmented_conv_kernel<",), "C2", None),
    "segmented_conv_bwd": (("mf::segmented_conv_bwd_kernel<", "mf::conv_taps_reduce_kernel"),
                           "C2", None),
}


def profile_step() -> None:
    import torch

    src = torch.empty(CALIB_BYTES // 2, dtype=torch.bfloat16, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    gpu_leg(1, 0, profile=True)
    rows_leg(0, profile=True)


def _counter_values(path: pathlib.Path) -> dict:
    """Counter value per dispatch, grouped by kernel name in dispatch order."""
    import csv
    import re

    sums = {}
    for row in csv.DictReader(open(path)):
        name = re.sub(r"\(.*", "", row["Kernel_Name"]).replace("void ", "").strip()
        mangled = re.match(r"_ZN2mf(\d+)", name)  # left mangled when a template argument is __bf16
        if mangled:
            name = "mf::" + name[mangled.end():mangled.end() + int(mangled.group(1))] + "<"
        key = (int(row.get("Dispatch_Id", 0) or 0), name)
        sums[key] = sums.get(key, 0.0) + float(row["Counter_Value"])
    per_kernel = {}
    for (_, name), value in sorted(sums.items()):
        per_kernel.setdefault(name, []).append(value)
    return per_kernel


def traffic_from(fetch_dir: str, write_dir: str) -> dict:
    fetch = _counter_values(next(pathlib.Path(fetch_dir).rglob("*counter_collection.csv")))
    write = _counter_values(next(pathlib.Path(write_dir).rglob("*counter_collection.csv")))
    copy = "__amd_rocclr_copyBuffer"
    f_scale = CALIB_BYTES / (sum(fetch[copy]) * 1024)
    w_scale = CALIB_BYTES / (sum(write[copy]) * 1024)
    out = {"calibration": {"copy_bytes": CALIB_BYTES, "fetch_kib_per_copy": sum(fetch[copy]),
                           "write_kib_per_copy": sum(write[copy]),
                           "fetch_scale": f_scale, "write_scale": w_scale}}

    def per_launch(values: dict, kernels, occurrence):
        total = 0.0
        for name, v in values.items():
            if name.startswith(kernels):
                total += v[occurrence] if occurrence is not None else sum(v) / len(v)
        return total

    for name, (kernels, workload, occurrence) in TRAFFIC_KERNELS.items():
        fb = per_launch(fetch, kernels, occurrence) * 1024 * f_scale
        wb = per_launch(write, kernels, occurrence) * 1024 * w_scale
        out.setdefault(workload, {})[name] = {"fetch_bytes": fb, "write_bytes": wb,
                                              "bytes": fb + wb}
    (ROOT / "profiles").mkdir(exist_ok=True)
    (ROOT / "profiles" / "traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The first ~25 steps after launch run ~13% slower while the GPU's clocks
    # ramp up (measured: 790 us/step for steps 4-23, 690-705 for any later
    # window of 20-500 steps); 50 warm-up steps (~40 ms) reach steady state.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", default="C2", choices=("C2", "C3", "C5"),
                    help="packed workload of the step (C2, the default, is the headline line with "
                         "the decode, the rows and the CPU baseline; C3 and C5 print the step alone)")
    ap.add_argument("--step-only", action="store_true",
                    help="time only the --config step and print its line (no decode, rows, other "
                         "configs or CPU baseline): the command the per-config kernel traces use")
    ap.add_argument("--profile-step", action="store_true",
                    help="run the calibration copy, one C2 step, one C4 decode and the rows once "
                         "(for rocprofv3 --pmc)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two PMC runs of --profile-step into profiles/traffic.json")
    args = ap.parse_args()
    if args.traffic:
        print(json.dumps(traffic_from(*args.traffic), indent=1))
        return 0
    if args.profile_step:
        profile_step()
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
              "(the packed-attention path has no cross-GPU work in this build)", file=sys.stderr)
        return 2
    if args.config != "C2" or args.step_only:
        gpu = gpu_leg(args.steps, args.warmup, name=args.config, decode=False)
        print(json.dumps({"metric": METRIC.split(";")[0], "value": gpu["value"], "unit": "TFLOP/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": gpu["ms_per_step"], "higher_is_better": True,
                          "dtype": "bf16", "config": gpu["config"], "roofline": gpu["roofline"],
                          "kernels_ms": gpu["kernels_ms"],
                          "step_roofline_frac": gpu["step_roofline_frac"],
                          "step_roofline": gpu["step_roofline"]}))
        return 0
    # The other measurements run first, the headline C2 leg last; each packed
    # leg measures its per-kernel sample before its own warm-up and timed steps
    # (gpu_leg), so every timed window starts with the clocks settled on its
    # workload.
    decode = decode_leg(args.steps, args.warmup)
    rows = rows_leg(args.steps)
    configs = {}
    # The C5 and C3 lines are side figures: they take fixed samples (at least
    # 100 timed steps after 50 warm-up steps, whatever --steps says) so that
    # their per-step and per-kernel figures are stable.
    for name in ("C5", "C3"):
        other = gpu_leg(max(args.steps, 100), max(args.warmup, 50), name=name, decode=False)
        configs[name] = {"workload": other["config"]["workload"],
                         "ms_per_step": other["ms_per_step"],
                         "useful_tflops": other["value"],
                         "useful_gflop_per_step": other["config"]["useful_gflop_per_step"],
                         "step_roofline": other["step_roofline"],
                         "kernels_ms": other["kernels_ms"]}
    gpu = gpu_leg(args.steps, args.warmup, decode=False)
    line = {
        "metric": METRIC,
        "value": gpu["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": gpu["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded packed C2 layout, q/k/v ~ 0.5 N(0,1), dO ~ N(0,1))",
        "config": gpu["config"],
        "roofline": gpu["roofline"],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_leg(args.cpu_seconds),
        "decode": decode,
        "configs": configs,
        "kernels_ms": gpu["kernels_ms"],
        "rows": rows,
        "fa2_convention_tflops": gpu["fa2_convention_tflops"],
        "step_roofline_frac": gpu["step_roofline_frac"],
        "step_roofline": gpu["step_roofline"],
        "wall_ms_per_step": gpu["wall_ms_per_step"],
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
