"""The oracle against the golden vectors of config 1 (tests/golden/config1.npz, produced by the
reference's own src/ref/ops.cpp): q fp16 bits, the appended int8 codes and fp16 scales, and the
gated attention output in bf16 must all be bit-identical. These fixtures pin the oracle where
/root/reference (and the oracle/_ref build) is absent."""
import numpy as np

from golden_util import BLOCK_TABLE, CTX, NKV, NQ, expected_pool, load, prior_pool

LD = 2 * (NQ + NKV) * 256


def test_oracle_append_matches_golden(orc):
    g = load()
    pool = prior_pool(g)
    q = orc.qk_norm_rope_append(g["proj"][None, :], LD, [CTX], [0], [0], g["q_norm"], g["k_norm"], NQ, NKV, pool, 0,
                                BLOCK_TABLE)
    assert np.array_equal(q[0], g["q16"])
    assert np.array_equal(pool, expected_pool(g))


def test_oracle_attention_matches_golden(orc):
    g = load()
    pool = expected_pool(g)
    gate = np.ascontiguousarray(g["proj"][None, NQ * 256:2 * NQ * 256])
    out = orc.attention_ragged(NQ, NKV, np.array([0, 1], np.int32), np.array([0], np.int32),
                               np.array([CTX], np.int32), g["q16"][None], gate, NQ * 256, pool, 0, BLOCK_TABLE)
    assert np.array_equal(out[0], g["out_bf16"])
