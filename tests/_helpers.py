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


def torch_reference(mode, q, k, v, mask, seg, do):
    """fp32 forward and gradients, one id group at a time (GPU)."""
    qf, kf, vf, dof = (x.float() for x in (q, k, v, do))
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
