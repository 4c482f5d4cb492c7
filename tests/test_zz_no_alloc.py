"""mf_decode_static: the decode entry point that allocates nothing.

It runs mf_decode's kernels on the library's static device scratch array
instead of a caller workspace.  On the GPU its output must equal mf_decode's
bit for bit (same kernels, same order) on consecutive calls, the second
smaller than the first, so what the first call leaves in the shared array
cannot leak into the second.  On the host, sizes whose workspace exceeds the
array are rejected before any HIP call.
"""

import numpy as np
import pytest
import torch

from _helpers import say
from mfattn import _lib, ops


def test_oversized_calls_are_rejected_before_any_launch():
    cap = _lib.LIB.mf_static_scratch_bytes()
    assert cap == 32 << 20
    # 64 rows x 8192 slots x 16 heads need ~17.3 MB and fit; 256 rows do not
    rc = _lib.LIB.mf_decode_static(None, None, None, None, _lib.DTYPE_BF16, 256, 8192, 16, 8, 64,
                                   0.125, None, None)
    assert rc == _lib.ERR_WORKSPACE
    assert "static array holds" in _lib.LIB.mf_last_error().decode()
    rc = _lib.LIB.mf_decode_static(None, None, None, None, _lib.DTYPE_BF16, 64, 8192, 16, 8, 64,
                                   0.125, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT  # fits; then the null pointers are refused
    rc = _lib.LIB.mf_decode_static(None, None, None, None, _lib.DTYPE_BF16, 4, 64, 6, 4, 64,
                                   0.125, None, None)
    assert rc == _lib.ERR_HEADS


def _static_decode(q, kc, vc, lengths, scale):
    out = torch.empty_like(q)
    b, _, hq, d = q.shape
    cap, hkv = kc.shape[1], kc.shape[2]
    rc = _lib.LIB.mf_decode_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), lengths.data_ptr(),
                                   ops.dtype_code(q), b, cap, hq, hkv, d, scale, out.data_ptr(),
                                   torch.cuda.current_stream(q.device).cuda_stream)
    _lib.check(rc)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_static_decode_equals_mf_decode_on_two_calls(dtype, device):
    rng = np.random.default_rng(91)
    # first the larger call (C4 shape for bf16), then a smaller one on the same array
    shapes = [(64, 8192, 16, 8), (7, 300, 8, 2)] if dtype == torch.bfloat16 else \
        [(16, 2048, 8, 2), (3, 130, 4, 4)]
    for b, cap, hq, hkv in shapes:
        say("static decode", dtype, (b, cap, hq, hkv))
        lengths = rng.integers(1, cap + 1, size=b).astype(np.int32)
        lengths[0] = cap + 5      # over-full: every slot
        lengths[-1] = 0           # the reference's uniform average
        g = torch.Generator(device=device).manual_seed(b * 131 + cap)
        q = torch.randn(b, 1, hq, 64, generator=g, device=device).to(dtype)
        kc = torch.randn(b, cap, hkv, 64, generator=g, device=device).to(dtype)
        vc = torch.randn(b, cap, hkv, 64, generator=g, device=device).to(dtype)
        lt = torch.tensor(lengths, device=device)
        out = _static_decode(q, kc, vc, lt, 0.125)
        ref = ops.decode(q, kc, vc, lt, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (dtype, b, cap)
