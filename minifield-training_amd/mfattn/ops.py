"""Device-tensor wrappers over the C ABI, plus the autograd binding.

Tensors are torch tensors on a ROCm device; torch only supplies device
memory and the current HIP stream.  All arithmetic runs in ``libmfattn.so``.
The autograd ``Function`` plays the role of the reference's ``jax.custom_vjp``
boundary: the forward saves ``(q, k, v, out, lse, plan)`` and the backward
calls the HIP backward once.
"""

from __future__ import annotations

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor) -> torch.device:
    """Every operand must already live on one ROCm device (no host fallback)."""
    device = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                "mfattn runs on the GPU only; got a tensor on " + str(t.device)
            )
        if t.device != device:
            raise ValueError("all operands must be on the same device")
    return device


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"Unsupported dtype {t.dtype}; mfattn serves float32 and bfloat16") from None


def as_mask(mask: torch.Tensor, mode: int) -> tuple[torch.Tensor, int]:
    """Mask in a dtype the C ABI reads (int32 or uint8), values preserved.

    Other dtypes are reduced to their activity first: ``> 0`` for the packed
    causal mode (``attention.py:97``), ``!= 0`` for the bidirectional modes
    (``bidirectional.py:22,25``).
    """
    if mask.dtype == torch.int32:
        return mask.contiguous(), _lib.MASK_I32
    if mask.dtype in (torch.bool, torch.uint8):
        return mask.contiguous().view(torch.uint8), _lib.MASK_U8
    active = mask > 0 if mode == _lib.MODE_PACKED_CAUSAL else mask != 0
    return active.to(torch.uint8).contiguous(), _lib.MASK_U8


class Plan:
    """Device block map (canonical ids, tile map, work lists) of one call."""

    def __init__(self, buf: torch.Tensor, batch: int, q_len: int, kv_len: int, mode: int):
        self.buf, self.batch, self.q_len, self.kv_len, self.mode = buf, batch, q_len, kv_len, mode

    @property
    def nbytes(self) -> int:
        return self.buf.numel()

    def section(self, index: int, dtype: torch.dtype, shape: tuple[int, ...]) -> torch.Tensor:
        offs = _lib.plan_layout(self.batch, self.q_len, self.kv_len)
        count = 1
        for s in shape:
            count *= s
        width = torch.empty((), dtype=dtype).element_size()
        raw = self.buf[offs[index] : offs[index] + count * width]
        return raw.view(dtype).view(shape)

    def tile_map(self) -> torch.Tensor:
        nq, nk = -(-self.q_len // _lib.TILE), -(-self.kv_len // _lib.TILE)
        return self.section(2, torch.uint8, (self.batch, nq, nk))


def block_map(segment_ids: torch.Tensor | None, mask: torch.Tensor, mode: int,
              q_len: int, kv_len: int) -> Plan:
    batch = mask.shape[0]
    device = require_device(mask) if segment_ids is None else require_device(mask, segment_ids)
    m, mcode = as_mask(mask, mode)
    seg = None if segment_ids is None else segment_ids.to(torch.int32).contiguous()
    nbytes = _lib.LIB.mf_plan_bytes(batch, q_len, kv_len)
    if nbytes == 0:
        raise ValueError("Sizes must be positive")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _lib.check(_lib.LIB.mf_block_map(_ptr(seg), _ptr(m), mcode, mode, batch, q_len, kv_len,
                                     _ptr(buf), nbytes, _stream(device)))
    return Plan(buf, batch, q_len, kv_len, mode)


def block_map_from_placements(placements: torch.Tensor, mode: int, batch: int,
                              length: int) -> tuple[Plan, torch.Tensor, torch.Tensor]:
    """Plan, segment ids and positions from packer placements ``[N, 3]`` (row, start, len)."""
    device = require_device(placements)
    pl = placements.to(torch.int32).contiguous()
    if pl.dim() != 2 or pl.shape[1] != 3:
        raise ValueError("placements must be [count, 3] (row, start, length)")
    nbytes = _lib.LIB.mf_plan_bytes(batch, length, length)
    if nbytes == 0:
        raise ValueError("Sizes must be positive")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    seg = torch.empty((batch, length), dtype=torch.int32, device=device)
    pos = torch.empty_like(seg)
    _lib.check(_lib.LIB.mf_block_map_placements(_ptr(pl), pl.shape[0], mode, batch, length,
                                                _ptr(buf), nbytes, _ptr(seg), _ptr(pos),
                                                _stream(device)))
    return Plan(buf, batch, length, length, mode), seg, pos


def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: Plan, mode: int,
             scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    device = require_device(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("query, key and value must share one dtype")
    code = dtype_code(q)
    b, t, hq, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, t), dtype=torch.float32, device=device)
    _lib.check(_lib.LIB.mf_attn_fwd(_ptr(q), _ptr(k), _ptr(v), code, b, t, s, hq, hkv, d, mode,
                                    float(scale), _ptr(plan.buf), plan.nbytes, _ptr(out),
                                    _ptr(lse), _stream(device)))
    return out, lse


def attn_bwd(q, k, v, out, dout, lse, plan: Plan, mode: int, scale: float):
    device = require_device(q, k, v, out, dout, lse)
    code = dtype_code(q)
    b, t, hq, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    ws_bytes = _lib.LIB.mf_attn_bwd_workspace_bytes(b, t, hq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    _lib.check(_lib.LIB.mf_attn_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse),
                                    code, b, t, s, hq, hkv, d, mode, float(scale), _ptr(plan.buf),
                                    plan.nbytes, _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ws_bytes,
                                    _stream(device)))
    return dq, dk, dv


def bwd_workspace(q: torch.Tensor) -> torch.Tensor:
    b, t, hq, _ = q.shape
    return torch.empty(_lib.LIB.mf_attn_bwd_workspace_bytes(b, t, hq), dtype=torch.uint8,
                       device=q.device)


def attn_bwd_delta(out, dout, lse, ws) -> None:
    """Phase 1 of the backward: -rowsum(dO * O) and lse * log2(e) into ``ws``."""
    b, t, hq, d = out.shape
    _lib.check(_lib.LIB.mf_attn_bwd_delta(_ptr(out), _ptr(dout), _ptr(lse), dtype_code(out), b, t,
                                          hq, d, _ptr(ws), ws.numel(), _stream(out.device)))


def attn_bwd_dq(q, k, v, dout, lse, plan: Plan, mode: int, scale: float, ws, dq) -> None:
    """Phase 2 of the backward: dq (reads the delta phase's ``ws``)."""
    b, t, hq, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    _lib.check(_lib.LIB.mf_attn_bwd_dq(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(lse),
                                       dtype_code(q), b, t, s, hq, hkv, d, mode, float(scale),
                                       _ptr(plan.buf), plan.nbytes, _ptr(dq), _ptr(ws), ws.numel(),
                                       _stream(q.device)))


def attn_bwd_dkdv(q, k, v, dout, lse, plan: Plan, mode: int, scale: float, ws, dk, dv) -> None:
    """Phase 3 of the backward: dk and dv (reads the delta phase's ``ws``)."""
    b, t, hq, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    _lib.check(_lib.LIB.mf_attn_bwd_dkdv(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(lse),
                                         dtype_code(q), b, t, s, hq, hkv, d, mode, float(scale),
                                         _ptr(plan.buf), plan.nbytes, _ptr(dk), _ptr(dv), _ptr(ws),
                                         ws.numel(), _stream(q.device)))


def decode_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                  k_cache: torch.Tensor, v_cache: torch.Tensor, positions: torch.Tensor,
                  scale: float) -> torch.Tensor:
    """Write each row's new key/value into its cache slot (in place), then decode."""
    device = require_device(q, k_new, v_new, k_cache, v_cache, positions)
    code = dtype_code(q)
    b, _, hq, d = q.shape
    cap, hkv = k_cache.shape[1], k_cache.shape[2]
    out = torch.empty_like(q)
    ws_bytes = _lib.LIB.mf_decode_workspace_bytes(b, cap, hq, d)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    _lib.check(_lib.LIB.mf_decode_append(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(positions), code,
                                         b, cap, hq, hkv, d, float(scale), _ptr(k_cache),
                                         _ptr(v_cache), _ptr(out), _ptr(ws), ws_bytes,
                                         _stream(device)))
    return out


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
           lengths: torch.Tensor, scale: float) -> torch.Tensor:
    device = require_device(q, k_cache, v_cache, lengths)
    code = dtype_code(q)
    b, _, hq, d = q.shape
    cap, hkv = k_cache.shape[1], k_cache.shape[2]
    out = torch.empty_like(q)
    ws_bytes = _lib.LIB.mf_decode_workspace_bytes(b, cap, hq, d)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    _lib.check(_lib.LIB.mf_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(lengths), code, b,
                                  cap, hq, hkv, d, float(scale), _ptr(out), _ptr(ws), ws_bytes,
                                  _stream(device)))
    return out


class PackedAttention(torch.autograd.Function):
    """Masked attention with a HIP forward and a HIP backward.

    ``forward(q, k, v, mask, segment_ids, mode, scale)``: integer inputs get
    no gradient (the reference's float0 cotangents).
    """

    @staticmethod
    def forward(ctx, q, k, v, mask, segment_ids, mode, scale):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        plan = block_map(segment_ids, mask, mode, q.shape[1], k.shape[1])
        out, lse = attn_fwd(q, k, v, plan, mode, scale)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan, ctx.mode, ctx.scale = plan, mode, scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = attn_bwd(q, k, v, out, dout.contiguous(), lse, ctx.plan, ctx.mode, ctx.scale)
        return dq, dk, dv, None, None, None, None


def packed_attention(q, k, v, mask, segment_ids, mode: int, scale: float) -> torch.Tensor:
    return PackedAttention.apply(q, k, v, mask, segment_ids, mode, scale)
