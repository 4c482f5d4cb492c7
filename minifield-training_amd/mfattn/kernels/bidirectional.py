"""Pad-safe bidirectional attention with the reference's signature.

Mirrors ``bidirectional.attention`` (``src/minifield_training/kernels/bidirectional.py:7-35``)
on the HIP kernels of ``libmfattn.so``.
"""

from __future__ import annotations

import torch

from .. import _lib, ops
from ._common import fit_head_dim, promote


def attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    mask: torch.Tensor,
    segment_ids: torch.Tensor | None = None,
    *,
    plan=None,
) -> torch.Tensor:
    """Attend in both directions with GQA and zero fully masked rows.

    Inputs use BTHD layout; ``mask`` is ``[B, S]`` (int or bool).  With packed
    ``segment_ids`` (``[B, T]``, 0 for padding) a query sees only active keys
    of its own nonzero segment and inactive queries return exact zeros.
    Without them every query of an example sees that example's active keys,
    and examples with no active key return zeros.  ``T`` may differ from
    ``S`` in the unpacked mode (cross attention).  ``plan`` (keyword only,
    not in the reference) is an ``ops.Plan`` built for this mask and these ids;
    by default one is taken from ``ops.PLANS``.
    """
    mode = _lib.MODE_KEYMASK_BIDIR if segment_ids is None else _lib.MODE_PACKED_BIDIR
    (q, k, v), d = fit_head_dim(*promote(query, key, value))
    out = ops.packed_attention(q, k, v, mask, segment_ids, mode, d ** -0.5, plan)
    return out[..., :d] if out.shape[-1] != d else out
