"""Write the committed golden fixtures of this directory.

* ``reference_fixtures.json`` -- the hand-derived inputs and expected outputs
  that the reference's own tests hold for this path, restated as data:
  ``tests/batching/test_packing.py:11-29, :44-48, :74-88, :52-63``,
  ``tests/kernels/test_attention.py:16, :26-37, :306-320, :377-398``,
  ``tests/kernels/test_bidirectional.py:12-26, :41-65``,
  ``tests/batching/test_pointer.py:155-157``, ``tests/layers/test_blocks.py:346``.
* ``c1_fp64.npz`` -- configuration C1 (2 rows x 256 tokens, 4/2 heads, D=64,
  fp32, causal within segment): the seeded inputs' layout, the FP64 oracle
  output and gradients (stored as float32) for a fixed upstream gradient.
  The q/k/v/dO tensors themselves are regenerated from the seed by
  ``c1_inputs`` and checked against the stored checksums.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention as oatt  # noqa: E402
from oracle import packing  # noqa: E402

FIXTURES = {
    "packing": {
        "ffd_two_rows": {
            "sequences": [[11, 12, 13], [21, 22, 23, 24, 25], [31, 32], [41, 42, 43, 44]],
            "rows": 2, "length": 8, "pad_token_id": 0,
            "placements": [[0, 5, 3], [0, 0, 5], [1, 4, 2], [1, 0, 4]],
            "input_ids": [[21, 22, 23, 24, 25, 11, 12, 13], [41, 42, 43, 44, 31, 32, 0, 0]],
            "segment_ids": [[2, 2, 2, 2, 2, 1, 1, 1], [4, 4, 4, 4, 3, 3, 0, 0]],
            "positions": [[0, 1, 2, 3, 4, 0, 1, 2], [0, 1, 2, 3, 0, 1, 0, 0]],
            "rows_required": 2,
        },
        "ties_keep_input_order": {
            "sequences": [[1, 1], [2, 2], [3, 3]], "rows": 2, "length": 4, "pad_token_id": 0,
            "placement_rows": [0, 0, 1], "placement_starts": [0, 2, 0],
        },
        "exact_fill": {
            "sequences": [[1, 2, 3], [4], [5, 6], [7, 8]], "rows": 2, "length": 4, "pad_token_id": 0,
            "input_ids": [[1, 2, 3, 4], [5, 6, 7, 8]],
            "segment_ids": [[1, 1, 1, 2], [3, 3, 4, 4]],
            "positions": [[0, 1, 2, 0], [0, 1, 0, 1]],
            "rows_required": 2,
        },
        "admission_errors": [
            {"sequences": [[1] * 9], "rows": 4, "length": 8, "message": "1 to 8 tokens"},
            {"sequences": [[]], "rows": 4, "length": 8, "message": "1 to 8 tokens"},
            {"sequences": [[1] * 5, [2] * 5, [3] * 5], "rows": 2, "length": 8,
             "message": "more than 2 packed rows"},
        ],
    },
    "layouts": {
        "attention_packed": {
            "mask": [[1, 1, 1, 1, 1, 0], [1, 1, 1, 0, 0, 0]],
            "segment_ids": [[1, 1, 1, 2, 2, 0], [1, 1, 2, 0, 0, 0]],
        },
        "attention_suffix_mask": [[1, 1, 1, 1, 0, 0], [1, 1, 1, 0, 0, 0]],
        "packing_rows": [[2, 2, 2, 2, 2, 1, 1, 1], [4, 4, 4, 4, 3, 3, 0, 0]],
        "packing_exact_fill": [[1, 1, 1, 2], [3, 3, 4, 4]],
        "pointer_row": [[1] * 21 + [2] * 21 + [0] * 6],
        "bidirectional_packed": [[1, 1, 2, 2, 2, 0]],
        "blocks_packed": [[1, 1, 2, 2]],
    },
    "attention_dims": {"batch": 2, "length": 6, "prefix": 3, "heads": 4, "kv_heads": 2, "dim": 8,
                        "packed_seed": 2, "cached_seed": 3, "cached_valid_length": 4},
    "bidirectional": {
        "uniform": {
            "query_shape": [1, 3, 2, 2], "key_shape": [1, 3, 1, 2],
            "values": [[[[2.0, 4.0]], [[6.0, 8.0]], [[99.0, 99.0]]]],
            "mask": [[1, 1, 0]],
            "output_row": [4.0, 6.0],
            "value_grad_of_sum": [[[[3.0, 3.0]], [[3.0, 3.0]], [[0.0, 0.0]]]],
        },
        "packed": {
            "query_shape": [1, 6, 2, 2], "key_shape": [1, 6, 1, 2],
            "values": [[2.0, 4.0], [6.0, 8.0], [1.0, 1.0], [2.0, 2.0], [6.0, 3.0], [99.0, 99.0]],
            "segment_ids": [[1, 1, 2, 2, 2, 0]],
            "output_rows": [[4, 6], [4, 6], [3, 2], [3, 2], [3, 2], [0, 0]],
            "value_grad_of_sum": [[2, 2], [2, 2], [2, 2], [2, 2], [2, 2], [0, 0]],
        },
    },
}


def c1_inputs():
    """Seeded C1 operands (float32) and upstream gradient."""
    w = packing.make_workload("C1")
    rng = np.random.default_rng(w.seed)
    q = rng.standard_normal((w.batch, w.length, w.q_heads, w.head_dim)).astype(np.float32)
    k = rng.standard_normal((w.batch, w.length, w.kv_heads, w.head_dim)).astype(np.float32)
    v = rng.standard_normal((w.batch, w.length, w.kv_heads, w.head_dim)).astype(np.float32)
    do = rng.standard_normal((w.batch, w.length, w.q_heads, w.head_dim)).astype(np.float32)
    return w, q, k, v, do


def main() -> None:
    (HERE / "reference_fixtures.json").write_text(json.dumps(FIXTURES, indent=1) + "\n")
    w, q, k, v, do = c1_inputs()
    out, probs, active = oatt.packed_causal_fp64(q, k, v, w.attention_mask, w.segment_ids)
    dq, dk, dv = oatt.vjp_fp64(q, k, v, probs, active, do)
    np.savez_compressed(
        HERE / "c1_fp64.npz",
        segment_ids=w.segment_ids, attention_mask=w.attention_mask,
        checksums=np.array([q.sum(dtype=np.float64), k.sum(dtype=np.float64),
                            v.sum(dtype=np.float64), do.sum(dtype=np.float64)]),
        out=out.astype(np.float32), dq=dq.astype(np.float32),
        dk=dk.astype(np.float32), dv=dv.astype(np.float32),
    )
    print("wrote", HERE / "reference_fixtures.json", HERE / "c1_fp64.npz")


if __name__ == "__main__":
    main()
