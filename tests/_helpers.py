"""Shared helpers of the GPU tests: seeded operands and a torch fp32 reference.

The torch reference evaluates the attention of every canonical id group on
its own (the grouping the oracle's ``grouped_fp64`` uses and checks against
the dense grid), in float32 on the GPU, so the BASELINE shapes fit.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import masks as omasks

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16}


def say(*parts) -> None:
    print("[gpu-case]", *parts, flush=True)


def operands(rng: np.random.Generator, b, t, hq, hkv, d, dtype, scale=1.0, s=None, device="cuda"):
    s = t if s is None else s
    def mk(shape):
        x = rng.standard_normal(shape).astype(np.float32) * scale
        return torch.tensor(x, device=device).to(dtype)
    q, k, v = mk((b, t, hq, d)), mk((b, s, hkv, d)), mk((b, s, hkv, d))
    do = torch.tensor(rng.standard_normal((b, t, hq, d)).astype(np.float32), device=device).to(dtype)
    return q, k, v, do


def torch_reference(mode, q, k, v, mask, seg, do, dtype=torch.float32):
    """Forward and gradients in ``dtype`` (fp32 by default), one id group at a time (GPU)."""
    qf, kf, vf, dof = (x.to(dtype) for x in (q, k, v, do))
    b, t, hq, d = qf.shape
    hkv = kf.shape[2]
    g = hq // hkv
    scale = d ** -0.5
    qid, kid = omasks._token_ids(mode, mask, seg, t)
    causal = mode == omasks.MODE_PACKED_CAUSAL
    out = torch.zeros_like(qf)
    dq, dk, dv = torch.zeros_like(qf), torch.zeros_like(kf), torch.zeros_like(vf)
    for row in range(b):
        for ident in np.unique(qid[row][qid[row] != omasks.Q_INACTIVE]):
            qi = torch.tensor(np.flatnonzero(qid[row] == ident), device=q.device)
            kj = torch.tensor(np.flatnonzero(kid[row] == ident), device=q.device)
            if kj.numel() == 0:
                continue
            qq = qf[row, qi].permute(1, 0, 2).contiguous()          # [H, Lq, D]
            kk = kf[row, kj].repeat_interleave(g, dim=1).permute(1, 0, 2).contiguous()
            vv = vf[row, kj].repeat_interleave(g, dim=1).permute(1, 0, 2).contiguous()
            go = dof[row, qi].permute(1, 0, 2).contiguous()
            sc = torch.matmul(qq, kk.transpose(1, 2).contiguous()) * scale
            if causal:
                allowed = kj[None, :] <= qi[:, None]
                sc = sc.masked_fill(~allowed[None], float("-inf"))
            p = torch.softmax(sc, dim=-1)
            o = torch.matmul(p, vv)
            out[row, qi] = o.permute(1, 0, 2)
            dvh = torch.matmul(p.transpose(1, 2).contiguous(), go)
            dp = torch.matmul(go, vv.transpose(1, 2).contiguous())
            delta = (go * o).sum(-1, keepdim=True)
            ds = p * (dp - delta)
            dqh = torch.matmul(ds, kk) * scale
            dkh = torch.matmul(ds.transpose(1, 2).contiguous(), qq) * scale
            dq[row, qi] += dqh.permute(1, 0, 2)
            dk[row, kj] += dkh.reshape(hkv, g, -1, d).sum(1).permute(1, 0, 2)
            dv[row, kj] += dvh.reshape(hkv, g, -1, d).sum(1).permute(1, 0, 2)
    return out, dq, dk, dv


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float() - b.float()).abs().max().item() if a.numel() else 0.0


BF16_TOL = 2e-2
# (label, raw max-abs, beyond-rounding excess) of the full-shape cases, printed by
# tests/conftest.py at the end of the run so the record of a GPU run carries them
PARITY_SUMMARY: list[tuple[str, float, float]] = []
BF16_HALF_ULP = 2.0 ** -8  # bound on |bf16(x) - x| / |x| (8 significant bits, round to nearest)


def bf16_errors(a, r) -> tuple[float, float]:
    """``(max|a - r|, max(|a - r| - 2**-8 |r|))`` element-wise.

    The second figure is the error beyond the one rounding a bf16 result of
    the exact value ``r`` must carry (|bf16(x) - x| <= 2**-8 |x|): entries of
    magnitude 10 cannot be held within 2e-2 of their true values in bf16,
    while the excess stays a plain absolute error for every entry.
    """
    a = torch.as_tensor(a).double().cpu()
    r = torch.as_tensor(r).double().cpu()
    if not a.numel():
        return 0.0, 0.0
    diff = (a - r).abs()
    return diff.max().item(), (diff - BF16_HALF_ULP * r.abs()).max().item()


def check_bf16(label: str, a, r, tol: float = BF16_TOL, summary: bool = False,
               roundings: int = 1) -> tuple[float, float]:
    """Assert the bf16 bar ``max(|a - r| - 2**-8 |r|) < tol`` and log both figures
    (``summary``: also list them in the end-of-run parity summary).

    ``roundings`` > 1 is for results that pass through several bf16 roundings at
    their own magnitude (a block's residual adds, each of which rounds the running
    sum), compared with another bf16 evaluation: each rounding may move the result
    by 2**-8 |r|, so the bar becomes ``max(|a - r| - roundings * 2**-8 |r|) < tol``.
    """
    a_ = torch.as_tensor(a).double().cpu()
    r_ = torch.as_tensor(r).double().cpu()
    if not a_.numel():
        raw, excess = 0.0, 0.0
    else:
        diff = (a_ - r_).abs()
        raw = diff.max().item()
        excess = (diff - roundings * BF16_HALF_ULP * r_.abs()).max().item()
    say(f"{label}: max-abs {raw:.3e} beyond-rounding {excess:.3e}"
        + (f" ({roundings} roundings)" if roundings != 1 else ""))
    if summary:
        PARITY_SUMMARY.append((label, raw, excess))
    assert excess < tol, (label, raw, excess)
    return raw, excess


def check_bf16_sum(label: str, a, r, abs_sum, tol: float = BF16_TOL) -> float:
    """The bf16 bar for a reduction over many rounded terms (a gain or tap gradient).

    Each term carries at most one bf16 rounding of an operand (relative
    2**-8), so the sum may differ from the exact one by up to 2**-8 times the
    sum of the terms' magnitudes ``abs_sum``; the bar is the error beyond that:
    ``max(|a - r| - 2**-8 abs_sum) < tol``.
    """
    a = torch.as_tensor(a).double().cpu()
    r = torch.as_tensor(r).double().cpu()
    s = torch.as_tensor(abs_sum).double().cpu()
    diff = (a - r).abs()
    excess = (diff - BF16_HALF_ULP * s).max().item()
    say(f"{label}: max-abs {diff.max().item():.3e} beyond-rounding {excess:.3e}")
    assert excess < tol, (label, diff.max().item(), excess)
    return excess


def short_segment_rows(rng, t: int) -> np.ndarray:
    """Rows of short segments: increasing ids, runs of 1-128 tokens with and without gaps,
    128-token runs on and across tile edges next to a single token, and a 200-token run."""
    rows = []
    for gaps in (True, False):
        seg = np.zeros(t, np.int32)
        pos, sid = 0, int(rng.integers(-6, 0))
        while pos < t:
            if gaps and rng.random() < 0.25:
                pos += int(rng.integers(1, 12))
                continue
            n = int(rng.integers(1, 129))
            sid += int(rng.integers(1, 4))
            sid += sid == 0
            seg[pos:pos + n] = sid
            pos += n
        rows.append(seg)
    edge = np.zeros(t, np.int32)
    edge[:128], edge[128:256], edge[300:428], edge[428:429] = 1, 2, 3, 4
    rows.append(edge)
    bad = np.zeros(t, np.int32)
    bad[10:210], bad[210:260] = 7, 8
    rows.append(bad)
    return np.stack(rows)[:, :t]
