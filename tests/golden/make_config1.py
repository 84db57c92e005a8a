"""Writes tests/golden/config1.npz: golden vectors of BASELINE configs[0] (one full-attention layer,
one sequence, one decode token at context 130, 24 q / 4 kv heads, head_dim 256, seed 0) computed
by the reference's own CPU ops (reference src/ref/ops.cpp:79-171, built from the reference sources
into oracle/_ref by `make -C oracle ref`; run this in a container that has /root/reference).

Inputs: bf16 N(0,1) K/V rows of positions 0..129 passed through the reference int8 round trip
(ops.cpp:79-90, stored here as int8 codes + fp16 scales: the reference keeps the dequantized
floats, from which scale = max|x| / 127 and code = x / scale follow exactly), the new token's bf16
projection row [q | gate | k | v] and the RMSNorm weights N(1, 0.1).
Expected: q as fp16 bits and the new K/V codes + scales from ref::qk_norm_rope_append
(ops.cpp:125-142), and the gated attention output as bf16 bits from ref::attention_token
(ops.cpp:144-171) over keys 0..130.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(os.path.dirname(HERE))]
from oracle.oracle import Reference  # noqa: E402

NQ, NKV, HD, CTX = 24, 4, 256, 130


def bf16_round(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return u


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def codes_scales(x):
    """Dequantized reference values [..., 256] -> (int8 codes, fp16 scale bits [..., 4])."""
    g = x.reshape(*x.shape[:-1], 4, 64)
    scale = (np.abs(g).max(axis=-1) / np.float32(127)).astype(np.float32)
    codes = np.where(scale[..., None] > 0, g / np.where(scale > 0, scale, 1)[..., None], 0)
    assert np.all(codes == np.round(codes)) and np.all(np.abs(codes) <= 127)
    return codes.astype(np.int8).reshape(x.shape), scale.astype(np.float16).view(np.uint16)


def main():
    ref = Reference()
    rng = np.random.default_rng(0)
    prior_k = ref.int8_group_roundtrip(bf16_to_f32(bf16_round(rng.standard_normal((CTX, NKV, HD)))))
    prior_v = ref.int8_group_roundtrip(bf16_to_f32(bf16_round(rng.standard_normal((CTX, NKV, HD)))))
    proj = bf16_round(rng.standard_normal(2 * (NQ + NKV) * HD))
    q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    rq, rk, rv = ref.qk_norm_rope_append_token(NQ, NKV, bf16_to_f32(proj), CTX, q_norm, k_norm, 0)
    st = ref.store(NKV, CTX + 1)
    st.k[:, :CTX] = prior_k.transpose(1, 0, 2)
    st.v[:, :CTX] = prior_v.transpose(1, 0, 2)
    st.k[:, CTX] = rk
    st.v[:, CTX] = rv
    gate = bf16_to_f32(proj[NQ * HD:2 * NQ * HD])
    out = st.attention_token(NQ, rq.ravel(), gate, CTX)
    st.close()
    assert np.array_equal(bf16_to_f32(bf16_round(out)), out)  # the reference rounds its output to bf16
    pk, pks = codes_scales(prior_k)
    pv, pvs = codes_scales(prior_v)
    nk, nks = codes_scales(rk)
    nv, nvs = codes_scales(rv)
    np.savez_compressed(os.path.join(HERE, "config1.npz"), proj=proj, q_norm=q_norm, k_norm=k_norm,
                        prior_k_codes=pk, prior_k_scales=pks, prior_v_codes=pv, prior_v_scales=pvs,
                        q16=rq.astype(np.float16).view(np.uint16), k_codes=nk, k_scales=nks, v_codes=nv,
                        v_scales=nvs, out_bf16=bf16_round(out))
    print("wrote", os.path.join(HERE, "config1.npz"))


if __name__ == "__main__":
    main()
