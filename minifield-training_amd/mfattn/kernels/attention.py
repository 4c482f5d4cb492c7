"""Packed causal and KV-cached attention with the reference's signatures.

Mirrors ``src/minifield_training/kernels/attention.py`` of the reference:

* ``dense_packed_causal_attention`` -- ``attention.py:245-261``
* ``packed_causal_attention``       -- ``attention.py:571-588`` (dispatcher)
* ``dense_cached_attention``        -- ``attention.py:264-282``
* ``cached_attention``              -- ``attention.py:591-610`` (dispatcher)

Operands are torch tensors on a ROCm device in the reference's BTHD layout;
every call runs the HIP kernels of ``libmfattn.so`` (block map + flash
forward, HIP backward through autograd; split-K decode).  The reference's
backend names (``dense``, ``cudnn``, ``splash``) all name the same
mathematical function; on MI355X each of them, and ``hip``, runs the HIP
implementation.  Unknown names raise the reference's ``ValueError``.
"""

from __future__ import annotations

import torch

from .. import _lib, ops
from ._common import fit_head_dim, promote


def dense_packed_causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor,
    segment_ids: torch.Tensor,
    *,
    plan=None,
) -> torch.Tensor:
    """Causal attention confined to same-segment active tokens.

    A query sees key ``j`` iff ``j <= i``, both share one nonzero segment id
    and both are mask-active (``attention_mask > 0``); inactive query rows are
    zero.  Output has the query's shape and dtype.  ``plan`` (keyword only, not
    in the reference) is an ``ops.Plan`` built for these ids and this mask in
    the causal mode; by default one is taken from ``ops.PLANS``.
    """
    # the reference's own (weak) shape check, attention.py:92-93
    if query.shape != key.shape and key.shape != value.shape:
        raise ValueError("Packed attention query/KV shapes are incompatible")
    (q, k, v), d = fit_head_dim(*promote(query, key, value))
    out = ops.packed_attention(q, k, v, attention_mask, segment_ids,
                               _lib.MODE_PACKED_CAUSAL, d ** -0.5, plan)
    return out[..., :d] if out.shape[-1] != d else out


_PACKED_BACKENDS = {
    "dense": dense_packed_causal_attention,
    "cudnn": dense_packed_causal_attention,
    "splash": dense_packed_causal_attention,
    "hip": dense_packed_causal_attention,
}


def packed_causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor,
    segment_ids: torch.Tensor,
    *,
    backend: str,
    plan=None,
) -> torch.Tensor:
    """Apply causal attention confined to same-segment active tokens."""
    try:
        fn = _PACKED_BACKENDS[backend]
    except KeyError:
        raise ValueError(f"Unsupported packed attention backend: {backend}") from None
    return fn(query, key, value, attention_mask, segment_ids, plan=plan)


def _lengths(valid_length, batch: int, device: torch.device) -> torch.Tensor:
    if isinstance(valid_length, torch.Tensor):
        lengths = valid_length.to(device=device, dtype=torch.int32).reshape(-1)
    else:
        lengths = torch.tensor(valid_length, dtype=torch.int32, device=device).reshape(-1)
    if lengths.numel() == 1:
        lengths = lengths.expand(batch)
    if lengths.numel() != batch:
        raise ValueError("valid_length must be a scalar or hold one length per row")
    return lengths.contiguous()


def dense_cached_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_length,
) -> torch.Tensor:
    """Attend one query per row to the valid prefix of a fixed-size KV cache.

    Non-causal by design: slot ``j`` of row ``b`` is visible iff
    ``j < valid_length[b]`` (``valid_length`` a scalar or ``[B]``).
    """
    if query.shape[-1] != key.shape[-1] or key.shape != value.shape:
        raise ValueError("Cached attention query/KV shapes are incompatible")
    if query.shape[2] % key.shape[2]:
        raise ValueError("Query heads must be divisible by KV heads")
    if query.shape[1] != 1:
        # the reference broadcasts the same key set to every query row
        outs = [dense_cached_attention(query[:, i : i + 1], key, value, valid_length)
                for i in range(query.shape[1])]
        return torch.cat(outs, dim=1)
    (q, k, v), d = fit_head_dim(*promote(query.contiguous(), key.contiguous(),
                                         value.contiguous()))
    lengths = _lengths(valid_length, query.shape[0], query.device)
    out = ops.decode(q, k, v, lengths, d ** -0.5)
    return out[..., :d] if out.shape[-1] != d else out


_CACHED_BACKENDS = {
    "dense": dense_cached_attention,
    "cudnn": dense_cached_attention,
    "hip": dense_cached_attention,
}


def cached_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_length,
    *,
    backend: str = "cudnn",
) -> torch.Tensor:
    """Attend one query to the valid prefix of a fixed-size KV cache.

    Accepts ``dense``, ``cudnn`` and ``hip`` (the reference has no Splash
    decode, ``attention.py:599-604``).
    """
    try:
        fn = _CACHED_BACKENDS[backend]
    except KeyError:
        raise ValueError(f"Unsupported cached attention backend: {backend}") from None
    return fn(query, key, value, valid_length)


def cached_attention_step(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cache_key: torch.Tensor,
    cache_value: torch.Tensor,
    position,
    *,
    backend: str = "cudnn",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode step's cache write and attention, per row.

    The attention part of ``attention_block_step``
    (``layers/attention.py:309-317``): ``key``/``value`` ``[B, 1, Hkv, D]``
    are written at cache slot ``position`` -- a scalar, as in the reference,
    or one slot per row -- with ``dynamic_update_slice``'s clamping of the
    start index to ``[0, capacity - 1]``, and the query attends over
    ``position + 1`` slots.  The caches are updated in place and returned, so
    callers that rebind them (``cache_key = ...``) keep working.
    """
    if backend not in _CACHED_BACKENDS:
        raise ValueError(f"Unsupported cached attention backend: {backend}")
    if (query.shape[-1] != cache_key.shape[-1] or cache_key.shape != cache_value.shape
            or key.shape != value.shape or key.shape[1] != 1 or query.shape[1] != 1
            or key.shape[0] != cache_key.shape[0] or key.shape[2:] != cache_key.shape[2:]):
        raise ValueError("Cached attention query/KV shapes are incompatible")
    if query.shape[2] % cache_key.shape[2]:
        raise ValueError("Query heads must be divisible by KV heads")
    if query.shape[-1] != _lib.HEAD_DIM:
        # padded head dims: append through the padded copies, then write back
        (q, kn, vn, kc, vc), d = fit_head_dim(query.contiguous(), key.contiguous(),
                                              value.contiguous(), cache_key.contiguous(),
                                              cache_value.contiguous())
        out = ops.decode_append(q, kn, vn, kc, vc, _lengths(position, query.shape[0],
                                                              query.device), d ** -0.5)
        cache_key.copy_(kc[..., :d])
        cache_value.copy_(vc[..., :d])
        return out[..., :d], cache_key, cache_value
    for t in (cache_key, cache_value):
        if not t.is_contiguous():
            raise ValueError("the KV caches must be contiguous to be updated in place")
    positions = _lengths(position, query.shape[0], query.device)
    out = ops.decode_append(query.contiguous(), key.contiguous(), value.contiguous(), cache_key,
                            cache_value, positions, query.shape[-1] ** -0.5)
    return out, cache_key, cache_value
