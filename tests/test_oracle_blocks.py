"""The FP64 block oracle (the callers of the hot path) pinned on the CPU.

* the composed causal block equals an independent token/head-loop evaluation
  with 2x2 rotation matrices (the method of tests/layers/test_blocks.py:98-134);
* a packed row equals its segments evaluated as independent rows, for the
  causal block, the encoder's bidirectional attention block and its centered
  conv block (tests/layers/test_blocks.py:342-382, test_encoder.py:65-103).
"""

import numpy as np

from oracle import blocks


def _setup(seed=0, hidden=32, hq=2, hkv=1, d=8, ffn_dim=24, channels=16):
    rng = np.random.default_rng(seed)
    attn, ffn, conv = blocks.random_weights(rng, hidden, hq, hkv, d, ffn_dim, channels)
    return rng, attn, ffn, conv


def test_composed_block_equals_the_loop_evaluation():
    rng, attn, ffn, _ = _setup()
    x = rng.standard_normal((1, 6, 32))
    got = blocks.attention_block(x, attn, ffn, np.ones((1, 6), np.int32), head_dim=8,
                                 rope_theta=10000.0, eps=0.01)
    want = blocks.loop_attention_block(x, attn, ffn, head_dim=8, rope_theta=10000.0, eps=0.01)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_packed_rows_equal_independent_rows():
    rng, attn, ffn, conv = _setup(1)
    lengths = [3, 5, 2]
    x = rng.standard_normal((1, 12, 32))
    seg = np.repeat([1, 2, 3, 0], lengths + [2])[None].astype(np.int32)
    pos = np.concatenate([np.arange(n) for n in lengths] + [np.zeros(2, int)])[None]
    mask = (seg != 0).astype(np.int32)
    causal = blocks.attention_block_packed(x, attn, ffn, mask, seg, pos, head_dim=8,
                                           rope_theta=1e4, eps=1e-5)
    enc_attn = blocks.encoder_block(x, attn, ffn, mask, seg, pos, kind="attention", head_dim=8,
                                    rope_theta=1e4, eps=1e-5)
    enc_conv = blocks.encoder_block(x, conv, ffn, mask, seg, pos, kind="conv", head_dim=8,
                                    rope_theta=1e4, eps=1e-5)
    start = 0
    for n in lengths:
        xs = x[:, start:start + n]
        ones = np.ones((1, n), np.int32)
        np.testing.assert_allclose(causal[:, start:start + n],
                                   blocks.attention_block(xs, attn, ffn, ones, head_dim=8,
                                                          rope_theta=1e4, eps=1e-5), atol=1e-12)
        np.testing.assert_allclose(enc_attn[:, start:start + n],
                                   blocks.encoder_block(xs, attn, ffn, ones, ones, None,
                                                        kind="attention", head_dim=8,
                                                        rope_theta=1e4, eps=1e-5), atol=1e-12)
        np.testing.assert_allclose(enc_conv[:, start:start + n],
                                   blocks.encoder_block(xs, conv, ffn, ones, ones, None,
                                                        kind="conv", head_dim=8,
                                                        rope_theta=1e4, eps=1e-5), atol=1e-12)
        start += n
