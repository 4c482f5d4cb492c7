"""The C ABI without a GPU: exports, plan layout and host-side error paths.

Every check here runs before any HIP call, so the library is exercised on a
machine with no GPU.  Messages follow the reference's ValueErrors
(kernels/attention.py:92-93, :276-279, :585-588, :608-610).
"""

import ctypes
import pathlib
import re

import pytest
import torch

from mfattn import _lib
from mfattn.kernels import attention, bidirectional

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "mfattn.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(mf_\w+)\(", text, re.M)))


def test_header_declares_what_the_library_exports():
    names = _declared()
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(_lib.LIB, name), name


def test_plan_layout_is_aligned_and_increasing():
    for b, t, s in ((1, 1, 1), (8, 4096, 4096), (1, 32768, 32768), (2, 300, 77)):
        offs = _lib.plan_layout(b, t, s)
        assert offs == sorted(offs)
        assert all(o % 256 == 0 for o in offs)
        assert len(offs) == 11
        assert _lib.LIB.mf_plan_bytes(b, t, s) == offs[10]
    assert _lib.LIB.mf_plan_bytes(0, 4, 4) == 0


def _fwd(**kw):
    args = dict(q=None, k=None, v=None, dtype=_lib.DTYPE_BF16, b=1, t=8, s=8, hq=4, hkv=2, d=64,
                mode=0, scale=0.125, plan=None, plan_bytes=1 << 30, out=None, lse=None)
    args.update(kw)
    return _lib.LIB.mf_attn_fwd(args["q"], args["k"], args["v"], args["dtype"], args["b"],
                                args["t"], args["s"], args["hq"], args["hkv"], args["d"],
                                args["mode"], args["scale"], args["plan"], args["plan_bytes"],
                                args["out"], args["lse"], None)


def _msg():
    return _lib.LIB.mf_last_error().decode()


@pytest.mark.parametrize(
    "kw, code, text",
    [
        (dict(d=128), _lib.ERR_HEAD_DIM, "head_dim 128"),
        (dict(hq=3), _lib.ERR_HEADS, "Query heads must be divisible by KV heads"),
        (dict(s=9), _lib.ERR_SHAPE, "Packed attention query/KV shapes are incompatible"),
        (dict(dtype=7), _lib.ERR_DTYPE, "dtype"),
        (dict(mode=5), _lib.ERR_MODE, "mode"),
        (dict(b=0), _lib.ERR_INVALID_ARGUMENT, "positive"),
        (dict(plan_bytes=16), _lib.ERR_WORKSPACE, "plan holds 16 bytes"),
        # the kernels' 32-bit DMA offsets cover one batch row of q and of k/v
        (dict(t=1 << 20, s=1 << 20, hq=16, hkv=8), _lib.ERR_SHAPE, "exceeds 4 GiB"),
        (dict(), _lib.ERR_INVALID_ARGUMENT, "non-null"),
        # the reference scales by head_dim ** -0.5; the forward's running max relies on scale > 0
        (dict(scale=0.0), _lib.ERR_INVALID_ARGUMENT, "scale must be finite and positive"),
        (dict(scale=-0.125), _lib.ERR_INVALID_ARGUMENT, "scale must be finite and positive"),
        (dict(scale=float("nan")), _lib.ERR_INVALID_ARGUMENT, "scale must be finite and positive"),
        (dict(scale=float("inf")), _lib.ERR_INVALID_ARGUMENT, "scale must be finite and positive"),
    ],
)
def test_forward_rejects_bad_arguments_on_the_host(kw, code, text):
    assert _fwd(**kw) == code
    assert text in _msg()


def test_keymask_mode_allows_cross_attention_lengths():
    # T != S passes the shape checks in the key-mask mode (then stops at null pointers)
    assert _fwd(mode=2, s=9) == _lib.ERR_INVALID_ARGUMENT


def test_block_map_and_decode_reject_bad_arguments():
    L = _lib.LIB
    assert L.mf_block_map(None, None, 0, 0, 1, 8, 8, None, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert "segment_ids" in _msg()
    assert L.mf_block_map(None, None, 3, 0, 1, 8, 8, None, 0, None) == _lib.ERR_DTYPE
    assert L.mf_block_map(None, None, 0, 0, 1, 8, 9, None, 0, None) == _lib.ERR_SHAPE
    assert L.mf_decode(None, None, None, None, 1, 2, 6, 4, 2, 8, 1.0, None, None, 0, None) == \
        _lib.ERR_SHAPE
    assert "Cached attention query/KV shapes are incompatible" in _msg()
    assert L.mf_decode(None, None, None, None, 1, 2, 6, 3, 2, 64, 1.0, None, None, 0, None) == \
        _lib.ERR_HEADS
    # any whole number of query heads per KV head (32 / 2 = 16 passes the head check and
    # stops at the null pointers)
    assert L.mf_decode(None, None, None, None, 1, 2, 6, 32, 2, 64, 1.0, None, None, 0, None) == \
        _lib.ERR_INVALID_ARGUMENT
    assert L.mf_decode(None, None, None, None, 1, 2, 6, 4, 2, 64, 1.0, None, None, 0, None) == \
        _lib.ERR_INVALID_ARGUMENT
    assert L.mf_attn_bwd_workspace_bytes(2, 6, 4) == 2 * 2 * 6 * 4 * 4
    assert L.mf_decode_workspace_bytes(64, 8192, 16, 64) > 0


@pytest.mark.parametrize("scale", [0.0, -1.0, float("nan"), float("-inf")])
def test_every_attention_entry_point_refuses_a_bad_scale(scale):
    L = _lib.LIB
    buf = ctypes.create_string_buffer(64)  # non-null host addresses: checks fail before launch
    p = ctypes.cast(buf, ctypes.c_void_p)
    big = 1 << 40
    calls = {
        "mf_attn_bwd": lambda: L.mf_attn_bwd(p, p, p, p, p, p, _lib.DTYPE_BF16, 1, 8, 8, 4, 2, 64, 0,
                                             scale, p, big, p, p, p, p, big, None),
        "mf_attn_bwd_dq": lambda: L.mf_attn_bwd_dq(p, p, p, p, p, _lib.DTYPE_BF16, 1, 8, 8, 4, 2, 64,
                                                   0, scale, p, big, p, p, big, None),
        "mf_attn_bwd_dkdv": lambda: L.mf_attn_bwd_dkdv(p, p, p, p, p, _lib.DTYPE_BF16, 1, 8, 8, 4, 2,
                                                       64, 0, scale, p, big, p, p, p, big, None),
        "mf_decode": lambda: L.mf_decode(p, p, p, p, _lib.DTYPE_BF16, 2, 6, 4, 2, 64, scale, p, p,
                                         big, None),
        "mf_decode_append": lambda: L.mf_decode_append(p, p, p, p, _lib.DTYPE_BF16, 2, 6, 4, 2, 64,
                                                       scale, p, p, p, p, big, None),
        "mf_decode_static": lambda: L.mf_decode_static(p, p, p, p, _lib.DTYPE_BF16, 2, 6, 4, 2, 64,
                                                       scale, p, None),
        "mf_attn_fwd_rope_q": lambda: L.mf_attn_fwd_rope_q(p, p, p, p, None, _lib.DTYPE_BF16, 2, 8, 8,
                                                           4, 2, 64, 0, scale, 1e-6, 10000.0, p, big,
                                                           p, big, p, p, None),
    }
    for name, call in calls.items():
        assert call() == _lib.ERR_INVALID_ARGUMENT, name
        assert "scale must be finite and positive" in _msg(), name


def test_decode_append_rejects_bad_arguments():
    L = _lib.LIB
    args = [None] * 4 + [1, 2, 6, 4, 2, 64, 1.0] + [None] * 4 + [0, None]
    assert L.mf_decode_append(*args) == _lib.ERR_INVALID_ARGUMENT
    buf = ctypes.c_char_p(b"x")  # any non-null host address: validation fails before any launch
    p = ctypes.cast(buf, ctypes.c_void_p)
    full = [p] * 4 + [1, 2, 6, 4, 2, 64, 1.0] + [p] * 4 + [0, None]
    assert L.mf_decode_append(*full) == _lib.ERR_WORKSPACE
    full[9] = 8
    assert L.mf_decode_append(*full) == _lib.ERR_SHAPE
    full[9], full[7] = 64, 3
    assert L.mf_decode_append(*full) == _lib.ERR_HEADS


def test_fused_query_prologue_rejects_bad_arguments():
    L = _lib.LIB
    buf = ctypes.create_string_buffer(64)  # non-null host addresses: checks fail before launch
    p = ctypes.cast(buf, ctypes.c_void_p)
    mis = ctypes.c_void_p(p.value + 4)

    def call(dtype=_lib.DTYPE_BF16, theta=10000.0, ptr=p, table=p, table_bytes=1 << 20, d=64):
        return L.mf_attn_fwd_rope_q(ptr, p, p, p, None, dtype, 2, 8, 8, 4, 2, d, 0, 0.125,
                                    1e-6, theta, p, 1 << 30, table, table_bytes, p, p, None)

    assert L.mf_rope_table_bytes(2, 8) == 2 * 8 * 32 * 4
    assert L.mf_rope_table_bytes(0, 8) == 0
    assert call(dtype=_lib.DTYPE_F32) == _lib.ERR_DTYPE
    assert "bf16" in _msg()
    assert call(theta=0.0) == _lib.ERR_INVALID_ARGUMENT
    assert "rope_theta" in _msg()
    assert call(d=128) == _lib.ERR_HEAD_DIM
    assert call(ptr=None) == _lib.ERR_INVALID_ARGUMENT
    assert call(table_bytes=16) == _lib.ERR_WORKSPACE
    assert "table holds 16 bytes" in _msg()
    assert call(table=mis) == _lib.ERR_INVALID_ARGUMENT
    assert "16-byte aligned" in _msg()
    # the key-only prologue: q_heads = 0 needs q, q_gain and q_out null
    assert L.mf_qk_norm_rope(p, None, None, p, None, _lib.DTYPE_BF16, 2, 8, 0, 2, 64, 1e-6,
                             1e4, None, p, None) == _lib.ERR_INVALID_ARGUMENT
    assert L.mf_qk_norm_rope(None, None, None, p, None, _lib.DTYPE_BF16, 2, 8, 0, 2, 64, 1e-6,
                             1e4, None, p, None) == _lib.ERR_INVALID_ARGUMENT  # k null


def test_error_codes_map_to_value_errors():
    rc = _fwd(hq=3)
    with pytest.raises(ValueError, match="divisible"):
        _lib.check(rc)
    with pytest.raises(_lib.MfError):
        _lib.check(_lib.ERR_HIP)


def test_dispatchers_reject_unknown_backends():
    q = torch.zeros(2, 6, 4, 8)
    k = torch.zeros(2, 6, 2, 8)
    m = torch.ones(2, 6, dtype=torch.int32)
    with pytest.raises(ValueError, match="Unsupported packed attention backend: tpu"):
        attention.packed_causal_attention(q, k, k, m, m, backend="tpu")
    with pytest.raises(ValueError, match="Unsupported cached attention backend: tpu"):
        attention.cached_attention(q[:, :1], k, k, 4, backend="tpu")


def test_shape_errors_match_the_reference():
    q = torch.zeros(2, 6, 4, 8)
    with pytest.raises(ValueError, match="Packed attention query/KV shapes are incompatible"):
        attention.dense_packed_causal_attention(q, torch.zeros(2, 5, 2, 8), torch.zeros(2, 4, 2, 8),
                                                torch.ones(2, 6), torch.ones(2, 6))
    with pytest.raises(ValueError, match="Cached attention query/KV shapes are incompatible"):
        attention.dense_cached_attention(q[:, :1], torch.zeros(2, 6, 2, 4), torch.zeros(2, 6, 2, 4), 4)
    with pytest.raises(ValueError, match="Query heads must be divisible by KV heads"):
        attention.dense_cached_attention(torch.zeros(2, 1, 3, 8), torch.zeros(2, 6, 2, 8),
                                         torch.zeros(2, 6, 2, 8), 4)


def test_product_path_refuses_host_tensors():
    """No CPU fallback: host tensors are rejected before any work."""
    q = torch.zeros(1, 4, 2, 64)
    m = torch.ones(1, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU only"):
        bidirectional.attention(q, q, q, m, m)
    with pytest.raises(ValueError, match="GPU only"):
        attention.dense_cached_attention(q[:, :1], q, q, 2)


def test_last_error_is_per_thread():
    """mf_last_error reports the calling thread's own failure while other threads fail
    differently in between (ctypes drops the GIL around each call, so the C calls interleave)."""
    import threading

    cases = {0: (dict(d=128), "head_dim 128"), 1: (dict(hq=3), "divisible by KV heads")}
    start = threading.Barrier(2)
    wrong = []

    def worker(i):
        kw, text = cases[i]
        start.wait()
        for _ in range(2000):
            assert _fwd(**kw) != 0
            if text not in _msg():
                wrong.append((i, _msg()))

    threads = [threading.Thread(target=worker, args=(i,)) for i in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not wrong, wrong[:3]
