"""Shared argument handling for the drop-in kernel modules."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib


def fit_head_dim(*xs: torch.Tensor) -> tuple[list[torch.Tensor], int]:
    """Zero-pad the head dimension to the 64 the kernels serve.

    Zero columns change no dot product and produce zero output columns, so
    padding then slicing is exact; the logit scale stays ``D ** -0.5`` of the
    caller's D.  Head dims above 64 are left for the C ABI to reject.
    """
    d = xs[0].shape[-1]
    if 0 < d < _lib.HEAD_DIM:
        return [F.pad(x, (0, _lib.HEAD_DIM - d)) for x in xs], d
    return list(xs), d


def promote(*xs: torch.Tensor) -> list[torch.Tensor]:
    """Cast operands of mixed float dtypes to their common dtype.

    The reference's einsums promote (a float32 query over a bfloat16 cache
    scores and returns float32, ``attention.py:23-33``); the kernels serve one
    dtype per call, so mixed operands are cast up front.
    """
    dtype = xs[0].dtype
    for x in xs[1:]:
        dtype = torch.promote_types(dtype, x.dtype)
    return [x if x.dtype == dtype else x.to(dtype) for x in xs]
