"""GPU parity of q38a_attention_prefill (causal chunked prefill over paged int8 KV, fp16 MFMA)
against the oracle's exact attention (reference src/ref/ops.cpp:144-171 per token), within the
north star's tolerance (|d| <= 2e-3 + 1e-2 |ref|, bf16 out). As in the reference kernel test
(tests/gpu/test_kernels.cu:395-495) a sequence is built from chunks that start at prefixes
{0, 1, 63, 64, 300, 2100}, so chunks start mid-page and cross pages; the appended K/V bytes are
checked bit for bit before the attention output is compared."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev, stream
from util import assert_bits_equal, bf16_bits_to_f32, check_close, randn_bf16
from test_gpu_decode import build_context, scale_proj_kv

pytestmark = pytest.mark.gpu


def prefill_step(orc, seqs, seed, kv_dtype=q38a.KV_INT8, check_tokens=None, k_scale=1.0, v_scale=1.0, dominant=None,
                 return_out=False):
    """seqs: [(prefix, n)] one chunk per sequence, appended then attended in one prefill launch.
    check_tokens: per sequence, the chunk-token indices compared with the oracle (default all).
    k_scale, v_scale, dominant: K/V magnitudes of the context and the chunk (see build_context)."""
    rng = np.random.default_rng(seed)
    B = len(seqs)
    bt, pages = paged_layout(rng, [p + n for p, n in seqs])
    pool_host = build_context(orc, rng, [p for p, _ in seqs], kv_dtype, bt, pages, k_scale=k_scale, v_scale=v_scale,
                              dominant=dominant)
    pool = Pool(kv_dtype, pages, bt, fill=pool_host)
    b = Batch([(i, p, n) for i, (p, n) in enumerate(seqs)])
    proj = randn_bf16(rng, (b.M, LD))
    if k_scale != 1.0 or v_scale != 1.0:
        proj = scale_proj_kv(rng, proj, k_scale, v_scale)
    q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    proj_t, qn_t, kn_t = dev(proj), dev(q_norm), dev(k_norm)
    q_t = torch.zeros(b.M * NQ * HD, dtype=torch.int16, device="cuda")
    out_t = torch.zeros(b.M * NQ * HD, dtype=torch.int16, device="cuda")
    rope_t = rope_dev(max(p + n for p, n in seqs) + 1)
    print(f"prefill: seqs={seqs} dtype={kv_dtype}", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_t), b.desc, pool.desc, stream())
    q38a.attention_prefill(attention_params(q_t, proj_t, out_t, None, 0), b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    q16 = host(q_t, np.uint16).reshape(b.M, NQ, HD)
    q_ref = orc.qk_norm_rope_append(proj, LD, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, NQ, NKV, pool_host,
                                    kv_dtype, bt)
    assert_bits_equal(q16, q_ref, "q fp16")
    assert_bits_equal(pool.download(), pool_host, "pool bytes")
    got = bf16_bits_to_f32(host(out_t, np.uint16)).reshape(b.M, NQ * HD)
    # oracle on the selected tokens: a ragged batch of single-token rows at their positions
    sel = []
    for i, (p, n) in enumerate(seqs):
        idx = range(n) if check_tokens is None else check_tokens[i]
        sel += [int(b.seq_start[i]) + t for t in idx]
    sel = np.array(sel, np.int64)
    gate = np.ascontiguousarray(proj[sel, NQ * HD:2 * NQ * HD])
    seq_of = b.tok_seq[sel]
    starts = np.searchsorted(seq_of, np.arange(B + 1)).astype(np.int32)
    want = orc.attention_ragged(NQ, NKV, starts, b.seq_slot, b.tok_pos[sel], q16[sel], gate, NQ * HD, pool_host,
                                kv_dtype, bt)
    want = bf16_bits_to_f32(want).reshape(len(sel), NQ * HD)
    if return_out:
        return got[sel], want
    return check_close(got[sel], want, what=f"prefill seqs={seqs}")


@pytest.mark.parametrize("prefix", [0, 1, 63, 64, 300, 2100])
def test_prefill_chunks_from_prefixes(orc, prefix):
    # the reference test's chunk sizes, each as its own launch after the previous chunk's K/V
    prefill_step(orc, [(prefix, 37), (prefix, 64), (prefix, 90), (prefix, 211)], seed=prefix)


@pytest.mark.parametrize("kv_dtype", [q38a.KV_INT8, q38a.KV_BF16, q38a.KV_INT8_VT])
def test_prefill_ragged_batch(orc, kv_dtype):
    """Several sequences of different lengths and prefixes in one launch, incl. a 1-token row."""
    prefill_step(orc, [(0, 130), (500, 1), (777, 300), (64, 64), (2000, 17)], seed=21, kv_dtype=kv_dtype)


def test_prefill_bf16_chunks_from_prefixes(orc):
    """bf16 pages (staged to fp16 in LDS): chunks at the reference test's prefixes."""
    for prefix in (0, 63, 300):
        prefill_step(orc, [(prefix, 37), (prefix, 90), (prefix, 211)], seed=40 + prefix, kv_dtype=q38a.KV_BF16)


def test_prefill_config3_shape(orc):
    """Config 3: a 2048-token chunk on a 6000-token prefix (starts at page 93, row 48); the oracle
    checks 40 tokens spread over the chunk, first and last included."""
    toks = sorted(set([0, 1, 2, 47, 48, 63, 64, 1000, 2046, 2047] + list(range(5, 2048, 70))))
    prefill_step(orc, [(6000, 2048)], seed=3, check_tokens=[toks])


@pytest.mark.parametrize("kv_dtype", [q38a.KV_INT8, q38a.KV_BF16, q38a.KV_INT8_VT])
def test_prefill_ragged_batch_256_row_tiles(orc, kv_dtype):
    """Enough rows that the launch takes 256-row workgroups (1,556 tokens x 6 heads x 4 kv heads
    / 128 > 256 CUs): ragged lengths, a 1-token row and tiles that end mid-sequence; the oracle
    checks a spread of tokens of every sequence, first and last included."""
    seqs = [(0, 700), (130, 555), (4000, 300), (64, 1)]
    checks = [sorted(set([0, 1, 42, 43, 85, 86, 699] + list(range(3, n, 37)))) if n > 1 else [0] for _, n in seqs]
    checks = [[t for t in c if t < n] for c, (_, n) in zip(checks, seqs)]
    prefill_step(orc, seqs, seed=77, kv_dtype=kv_dtype, check_tokens=checks)
