"""The package's benchmark generators equal the oracle's, bit for bit, and
their closed-form work counts equal the oracle's grid counts."""

import numpy as np
import pytest

from mfattn import workloads
from oracle import masks, packing, workload


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_packed_layouts_match_oracle(name):
    a, b = workloads.packed(name), packing.make_workload(name)
    np.testing.assert_array_equal(a.segment_ids, b.segment_ids)
    np.testing.assert_array_equal(a.attention_mask, b.attention_mask)
    assert (a.batch, a.length, a.q_heads, a.kv_heads, a.head_dim, a.dtype, a.causal, a.qkv_scale,
            a.seed) == (b.batch, b.length, b.q_heads, b.kv_heads, b.head_dim, b.dtype, b.causal,
                        b.qkv_scale, b.seed)
    mode = masks.MODE_PACKED_CAUSAL if a.causal else masks.MODE_PACKED_BIDIR
    pairs = workload.useful_pairs(mode, b.attention_mask, b.segment_ids)
    assert workloads.useful_pairs(a.segment_ids, a.causal) == pairs
    assert workloads.attention_flops(a)["fwd_bwd"] == workload.attention_flops(pairs, 64, a.q_heads)["fwd_bwd"]
    assert workloads.attention_bytes(a)["fwd_bwd"] == workload.attention_bytes(
        a.batch, a.length, a.q_heads, a.kv_heads, 64)["fwd_bwd"]


def test_decode_layout_matches_oracle():
    a, b = workloads.decode(), packing.make_decode_workload()
    np.testing.assert_array_equal(a.valid_length, b.valid_length)
    assert workloads.decode_bytes(a) == workload.decode_bytes(b.valid_length, 64, 16, 8, 64)
