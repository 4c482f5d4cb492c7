"""ctypes binding of ``libmfattn.so`` (the C ABI declared in ``include/mfattn.h``).

The library is loaded at import.  There is no fallback: if it is missing or
does not load, importing this module raises ``ImportError`` naming the file
and the build command, so nothing can silently run another implementation.
``MFATTN_LIB`` may name another build of the same library (the tests' build
with the host code under AddressSanitizer and UBSan).
"""

from __future__ import annotations

import ctypes
import os
import pathlib

LIB_PATH = pathlib.Path(os.environ.get("MFATTN_LIB") or
                        pathlib.Path(__file__).resolve().parent / "libmfattn.so")

# status codes (include/mfattn.h)
OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_SHAPE = -2
ERR_HEADS = -3
ERR_HEAD_DIM = -4
ERR_DTYPE = -5
ERR_MODE = -6
ERR_WORKSPACE = -7
ERR_HIP = -9

DTYPE_F32 = 0
DTYPE_BF16 = 1
MASK_I32 = 0
MASK_U8 = 1

MODE_PACKED_CAUSAL = 0
MODE_PACKED_BIDIR = 1
MODE_KEYMASK_BIDIR = 2

CONV_CAUSAL = 0
CONV_CENTERED = 1

TILE = 128
HEAD_DIM = 64

EXPORTS = (
    "mf_plan_layout",
    "mf_plan_bytes",
    "mf_block_map",
    "mf_block_map_placements",
    "mf_attn_fwd",
    "mf_rope_table_bytes",
    "mf_attn_fwd_rope_q",
    "mf_attn_bwd_workspace_bytes",
    "mf_attn_bwd",
    "mf_attn_bwd_delta",
    "mf_attn_bwd_dq",
    "mf_attn_bwd_dkdv",
    "mf_decode_workspace_bytes",
    "mf_decode",
    "mf_decode_append",
    "mf_qk_norm_rope",
    "mf_qk_norm_rope_bwd_workspace_bytes",
    "mf_qk_norm_rope_bwd",
    "mf_segment_positions",
    "mf_segmented_conv",
    "mf_segmented_conv_bwd_workspace_bytes",
    "mf_segmented_conv_bwd",
    "mf_static_scratch_bytes",
    "mf_decode_static",
    "mf_last_error",
    "mf_version",
)


class MfError(RuntimeError):
    """A failed C-ABI call; ``code`` is the MF_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class MfValueError(MfError, ValueError):
    """Invalid shapes, dtypes or modes (the reference raises ValueError)."""


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"mfattn native library missing: {LIB_PATH} (build it with "
            "`python minifield-training_amd/mfattn/build.py`)"
        )
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the machine
        raise ImportError(f"mfattn native library failed to load: {exc}") from exc
    vp, i32, sz, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
    lib.mf_plan_layout.argtypes = [i32, i32, i32, ctypes.POINTER(sz)]
    lib.mf_plan_layout.restype = None
    lib.mf_plan_bytes.argtypes = [i32, i32, i32]
    lib.mf_plan_bytes.restype = sz
    lib.mf_block_map.argtypes = [vp, vp, i32, i32, i32, i32, i32, vp, sz, vp]
    lib.mf_block_map.restype = i32
    lib.mf_attn_fwd.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, f32, vp, sz,
                                vp, vp, vp]
    lib.mf_attn_fwd.restype = i32
    lib.mf_rope_table_bytes.argtypes = [i32, i32]
    lib.mf_rope_table_bytes.restype = sz
    lib.mf_attn_fwd_rope_q.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32,
                                       f32, f32, f32, vp, sz, vp, sz, vp, vp, vp]
    lib.mf_attn_fwd_rope_q.restype = i32
    lib.mf_attn_bwd_workspace_bytes.argtypes = [i32, i32, i32]
    lib.mf_attn_bwd_workspace_bytes.restype = sz
    lib.mf_attn_bwd.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32,
                                f32, vp, sz, vp, vp, vp, vp, sz, vp]
    lib.mf_attn_bwd.restype = i32
    lib.mf_attn_bwd_delta.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp, sz, vp]
    lib.mf_attn_bwd_delta.restype = i32
    lib.mf_attn_bwd_dq.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32,
                                   f32, vp, sz, vp, vp, sz, vp]
    lib.mf_attn_bwd_dq.restype = i32
    lib.mf_attn_bwd_dkdv.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32,
                                     f32, vp, sz, vp, vp, vp, sz, vp]
    lib.mf_attn_bwd_dkdv.restype = i32
    lib.mf_decode_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.mf_decode_workspace_bytes.restype = sz
    lib.mf_decode.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, vp, vp, sz, vp]
    lib.mf_decode.restype = i32
    lib.mf_decode_append.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, vp, vp, vp,
                                     vp, sz, vp]
    lib.mf_decode_append.restype = i32
    lib.mf_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, f32,
                                    vp, vp, vp]
    lib.mf_qk_norm_rope.restype = i32
    lib.mf_qk_norm_rope_bwd_workspace_bytes.argtypes = [i32, i32]
    lib.mf_qk_norm_rope_bwd_workspace_bytes.restype = sz
    lib.mf_qk_norm_rope_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                        f32, f32, vp, vp, vp, vp, vp, sz, vp]
    lib.mf_qk_norm_rope_bwd.restype = i32
    lib.mf_segmented_conv_bwd_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.mf_segmented_conv_bwd_workspace_bytes.restype = sz
    lib.mf_segmented_conv_bwd.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                          vp, vp, vp, vp, vp, sz, vp]
    lib.mf_segmented_conv_bwd.restype = i32
    lib.mf_segment_positions.argtypes = [vp, i32, i32, vp, vp]
    lib.mf_segment_positions.restype = i32
    lib.mf_block_map_placements.argtypes = [vp, i32, i32, i32, i32, vp, sz, vp, vp, vp]
    lib.mf_block_map_placements.restype = i32
    lib.mf_segmented_conv.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, vp]
    lib.mf_segmented_conv.restype = i32
    lib.mf_static_scratch_bytes.argtypes = []
    lib.mf_static_scratch_bytes.restype = sz
    lib.mf_decode_static.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, vp, vp]
    lib.mf_decode_static.restype = i32
    lib.mf_last_error.argtypes = []
    lib.mf_last_error.restype = ctypes.c_char_p
    lib.mf_version.argtypes = []
    lib.mf_version.restype = ctypes.c_char_p
    return lib


LIB = _load()

_VALUE_CODES = {ERR_SHAPE, ERR_HEADS, ERR_HEAD_DIM, ERR_DTYPE, ERR_MODE, ERR_INVALID_ARGUMENT,
                ERR_WORKSPACE}


def check(rc: int) -> None:
    """Raise for a nonzero status with the library's own message."""
    if rc == OK:
        return
    message = LIB.mf_last_error().decode()
    if rc in _VALUE_CODES:
        raise MfValueError(rc, message)
    raise MfError(rc, message)


def plan_layout(batch: int, q_len: int, kv_len: int) -> list[int]:
    out = (ctypes.c_size_t * 11)()
    LIB.mf_plan_layout(batch, q_len, kv_len, out)
    return list(out)


def version() -> str:
    return LIB.mf_version().decode()
