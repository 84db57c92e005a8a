"""GPU parity of q38a_attention_decode (split-KV flash-decoding + gated merge) against the oracle's
exact double-precision attention (reference src/ref/ops.cpp:144-171), within the north star's
tolerance: max-abs 2e-3 and max-rel 1e-2 on bf16 outputs. The step is run as the engine runs it:
append the new token (bit-checked against the oracle), then attend over [0, pos]."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev, stream
from util import assert_bits_equal, bf16_bits_to_f32, check_close, f32_to_bf16_bits, randn_bf16

pytestmark = pytest.mark.gpu


def build_context(orc, rng, ctxs, kv_dtype, bt, pages, nkv=NKV, k_scale=1.0, v_scale=1.0, dominant=None):
    """Prior K/V for positions [0, ctx) of every sequence: bf16 N(0, scale^2) rows through the
    reference quantizer (or bf16 store), written into a host pool. dominant = (position, factor):
    that key row of every sequence is multiplied by factor (one key then dominates the softmax of
    about half of the heads)."""
    pool = np.zeros(q38a.page_bytes(kv_dtype, nkv) * pages, np.uint8)
    for b, ctx in enumerate(ctxs):
        if ctx == 0:
            continue
        k = bf16_bits_to_f32(randn_bf16(rng, (ctx, nkv, HD), k_scale))
        v = bf16_bits_to_f32(randn_bf16(rng, (ctx, nkv, HD), v_scale))
        if dominant is not None and dominant[0] < ctx:
            k[dominant[0]] = bf16_bits_to_f32(f32_to_bf16_bits(k[dominant[0]] * np.float32(dominant[1])))
        orc.fill_rows(k, v, 0, b, nkv, pool, kv_dtype, bt)
    return pool


def scale_proj_kv(rng, proj, k_scale, v_scale, nq=NQ, nkv=NKV):
    """The new tokens' k and v columns of proj redrawn at the given scales (k is RMS-normalised by
    the append, so only v's scale reaches the cache)."""
    M = proj.shape[0]
    k0, v0 = 2 * nq * HD, 2 * nq * HD + nkv * HD
    proj[:, k0:v0] = randn_bf16(rng, (M, nkv * HD), k_scale)
    proj[:, v0:v0 + nkv * HD] = randn_bf16(rng, (M, nkv * HD), v_scale)
    return proj


def decode_step(orc, ctxs, kv_dtype, seed, max_splits=64, check_pool=True, bt_override=None, return_out=False,
                k_scale=1.0, v_scale=1.0, dominant=None):
    rng = np.random.default_rng(seed)
    B = len(ctxs)
    bt, pages = paged_layout(rng, [c + 1 for c in ctxs])
    if bt_override is not None:
        bt = bt_override
    pool_host = build_context(orc, rng, ctxs, kv_dtype, bt, pages, k_scale=k_scale, v_scale=v_scale,
                              dominant=dominant)
    pool = Pool(kv_dtype, pages, bt, fill=pool_host)
    b = Batch([(i, c, 1) for i, c in enumerate(ctxs)])
    proj = randn_bf16(rng, (B, LD))
    if k_scale != 1.0 or v_scale != 1.0:
        proj = scale_proj_kv(rng, proj, k_scale, v_scale)
    q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    proj_t, qn_t, kn_t = dev(proj), dev(q_norm), dev(k_norm)
    q_t = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
    out_t = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
    scratch_t = torch.zeros(q38a.split_scratch_floats(B, NQ, max_splits), dtype=torch.float32, device="cuda")
    rope_t = rope_dev(max(ctxs) + 1)
    print(f"decode: B={B} ctxs={ctxs[:8]} dtype={kv_dtype} splits={max_splits}", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_t), b.desc, pool.desc, stream())
    q38a.attention_decode(attention_params(q_t, proj_t, out_t, scratch_t, max_splits), b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    got = bf16_bits_to_f32(host(out_t, np.uint16)).reshape(B, NQ * HD)
    q16 = host(q_t, np.uint16).reshape(B, NQ, HD)
    q_ref = orc.qk_norm_rope_append(proj, LD, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, NQ, NKV, pool_host,
                                    kv_dtype, bt)
    if check_pool:
        assert_bits_equal(q16, q_ref, "q fp16")
        assert_bits_equal(pool.download(), pool_host, "pool bytes")
    gate = np.ascontiguousarray(proj[:, NQ * HD:2 * NQ * HD])
    want = orc.attention_ragged(NQ, NKV, b.seq_start, b.seq_slot, b.tok_pos, q16, gate, NQ * HD, pool_host,
                                kv_dtype, bt)
    want = bf16_bits_to_f32(want).reshape(B, NQ * HD)
    if return_out:
        return got, want
    return check_close(got, want, what=f"decode ctxs={ctxs} dtype={kv_dtype}")


@pytest.mark.parametrize("kv_dtype", [q38a.KV_INT8, q38a.KV_BF16, q38a.KV_INT8_VT])
def test_decode_page_edges(orc, kv_dtype):
    # contexts around page boundaries, plus the config-1 shape (context 130)
    decode_step(orc, [0, 1, 62, 63, 64, 65, 127, 128, 130, 300, 2100], kv_dtype, seed=1)


def test_decode_config1_plumbing(orc):
    """Config 1: one sequence, one decode token at context 130 (3 pages)."""
    decode_step(orc, [130], q38a.KV_INT8, seed=0)


@pytest.mark.parametrize("kv_dtype", [q38a.KV_INT8, q38a.KV_BF16, q38a.KV_INT8_VT])
def test_decode_ragged_batch8(orc, kv_dtype):
    rng = np.random.default_rng(2)
    ctxs = [int(x) for x in rng.integers(1024, 8192, 8)]
    decode_step(orc, ctxs, kv_dtype, seed=3)


def test_decode_split_count_independent(orc):
    """Result independent of how keys are split (log-sum-exp merge is associative)."""
    ctxs = [5000, 70, 1234]
    a, want = decode_step(orc, ctxs, q38a.KV_INT8, seed=4, max_splits=1, return_out=True)
    b, _ = decode_step(orc, ctxs, q38a.KV_INT8, seed=4, max_splits=64, return_out=True)
    check_close(a, want, what="1 split")
    check_close(b, want, what="64 splits")
    check_close(a, b, atol=2e-3, rtol=1e-2, what="1 vs 64 splits")


def test_decode_paging_permutation_bitwise():
    """Permuting which pool pages hold a sequence leaves the output bit-identical."""
    pytest.importorskip("oracle.oracle")
    from oracle.oracle import Oracle
    orc = Oracle()
    ctxs = [700, 1500]
    rng = np.random.default_rng(5)
    bt1, pages = paged_layout(rng, [c + 1 for c in ctxs])
    perm = rng.permutation(pages).astype(np.int32)
    bt2 = perm[bt1]
    g1, _ = decode_step(orc, ctxs, q38a.KV_INT8, seed=6, bt_override=bt1, return_out=True)
    g2, _ = decode_step(orc, ctxs, q38a.KV_INT8, seed=6, bt_override=bt2, return_out=True)
    assert np.array_equal(g1, g2)


def test_decode_config1_golden():
    """Config 1 on the GPU against the reference's own golden vectors (tests/golden/config1.npz):
    q and the appended K/V bit-exact, the output within the tolerance of the reference's bf16."""
    from golden_util import BLOCK_TABLE, CTX, expected_pool, load, prior_pool
    g = load()
    pool = Pool(q38a.KV_INT8, 3, BLOCK_TABLE, fill=prior_pool(g))
    b = Batch([(0, CTX, 1)])
    proj_t = dev(g["proj"][None, :])
    qn_t, kn_t = dev(g["q_norm"]), dev(g["k_norm"])
    q_t = torch.zeros(NQ * HD, dtype=torch.int16, device="cuda")
    out_t = torch.zeros(NQ * HD, dtype=torch.int16, device="cuda")
    scratch_t = torch.zeros(q38a.split_scratch_floats(1, NQ, 64), dtype=torch.float32, device="cuda")
    print("decode: config 1 golden", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_dev(CTX + 1)), b.desc, pool.desc, stream())
    q38a.attention_decode(attention_params(q_t, proj_t, out_t, scratch_t, 64), b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    assert_bits_equal(host(q_t, np.uint16).reshape(NQ, HD), g["q16"], "q fp16")
    assert_bits_equal(pool.download(), expected_pool(g), "pool bytes")
    check_close(bf16_bits_to_f32(host(out_t, np.uint16))[None], bf16_bits_to_f32(g["out_bf16"])[None],
                what="config 1 output vs reference")


@pytest.mark.parametrize("B", [65, 200])
def test_decode_more_than_64_rows(orc, B):
    """More decode rows than a wave has lanes: the plan's per-64-row passes (page sums, the item
    scan and its running base across passes) and items of rows past 64; some rows are empty-prefix
    (context 0) and some long."""
    rng = np.random.default_rng(40 + B)
    ctxs = [int(x) for x in rng.integers(0, 400, B)]
    ctxs[3] = 0
    ctxs[B - 1] = 3000
    ctxs[70 % B] = 1500
    decode_step(orc, ctxs, q38a.KV_INT8, seed=41 + B, max_splits=32)
