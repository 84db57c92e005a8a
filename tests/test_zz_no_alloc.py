"""q38a_attention_decode_noalloc (split partials in the library's static device array) against
q38a_attention_decode (caller scratch) on the same inputs, through the C ABI: two calls in a row,
the second with a smaller batch, each output bit-identical to the existing entry point's (the two
share their kernels and the decode plan, so the fp32 summation order is the same) and within the
north star's tolerance of the oracle. Also: a batch too large for the static array is refused."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev, stream
from test_gpu_decode import build_context
from util import assert_bits_equal, bf16_bits_to_f32, check_close, randn_bf16

pytestmark = pytest.mark.gpu


def prepare(orc, ctxs, seed, kv_dtype=q38a.KV_INT8):
    rng = np.random.default_rng(seed)
    B = len(ctxs)
    bt, pages = paged_layout(rng, [c + 1 for c in ctxs])
    pool_host = build_context(orc, rng, ctxs, kv_dtype, bt, pages)
    pool = Pool(kv_dtype, pages, bt, fill=pool_host)
    b = Batch([(i, c, 1) for i, c in enumerate(ctxs)])
    proj = randn_bf16(rng, (B, LD))
    q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    proj_t, qn_t, kn_t = dev(proj), dev(q_norm), dev(k_norm)
    q_t = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_dev(max(ctxs) + 1)), b.desc, pool.desc,
                             stream())
    torch.cuda.synchronize()
    q16 = host(q_t, np.uint16).reshape(B, NQ, HD)
    orc.qk_norm_rope_append(proj, LD, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, NQ, NKV, pool_host, kv_dtype,
                            bt)
    gate = np.ascontiguousarray(proj[:, NQ * HD:2 * NQ * HD])
    want = orc.attention_ragged(NQ, NKV, b.seq_start, b.seq_slot, b.tok_pos, q16, gate, NQ * HD, pool_host, kv_dtype,
                                bt)
    return dict(b=b, pool=pool, proj_t=proj_t, q_t=q_t, B=B, want=bf16_bits_to_f32(want).reshape(B, NQ * HD))


def run_both(c, max_splits):
    B = c["B"]
    out_ref = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
    out_na = torch.full((B * NQ * HD,), -1, dtype=torch.int16, device="cuda")
    scratch = torch.zeros(q38a.split_scratch_floats(B, NQ, max_splits), dtype=torch.float32, device="cuda")
    q38a.attention_decode(attention_params(c["q_t"], c["proj_t"], out_ref, scratch, max_splits), c["b"].desc,
                          c["pool"].desc, stream())
    q38a.attention_decode_noalloc(attention_params(c["q_t"], c["proj_t"], out_na, None, max_splits), c["b"].desc,
                                  c["pool"].desc, stream())
    torch.cuda.synchronize()
    return host(out_ref, np.uint16), host(out_na, np.uint16)


def test_noalloc_matches_decode_two_calls(orc):
    first = prepare(orc, [9000, 20000, 300, 4100, 12000, 64, 7000, 15000], seed=91)
    second = prepare(orc, [5000, 1, 777], seed=92)
    for i, (c, splits) in enumerate([(first, 64), (second, 16)]):
        print(f"noalloc call {i}: B={c['B']} splits={splits}", flush=True)
        ref, na = run_both(c, splits)
        assert_bits_equal(na, ref, f"noalloc vs decode, call {i}")
        max_abs, max_rel = check_close(bf16_bits_to_f32(na).reshape(c["B"], NQ * HD), c["want"],
                                       what=f"noalloc vs oracle, call {i}")
        print(f"  bitwise equal to q38a_attention_decode; vs oracle max_abs {max_abs:.3g} max_rel {max_rel:.3g}",
              flush=True)


def test_noalloc_refuses_oversized_batch(orc):
    c = prepare(orc, [100, 200], seed=93)
    cap = q38a.noalloc_scratch_floats()
    splits = 512
    assert 2 * NQ * splits * (HD + 2) <= cap  # fits
    too_many = cap // (NQ * splits * (HD + 2)) + 1
    b = Batch([(i % 2, 100, 1) for i in range(too_many)])
    out = torch.zeros(too_many * NQ * HD, dtype=torch.int16, device="cuda")
    q = torch.zeros(too_many * NQ * HD, dtype=torch.int16, device="cuda")
    proj = torch.zeros(too_many * LD, dtype=torch.int16, device="cuda")
    with pytest.raises(q38a.Q38AError, match="static scratch"):
        q38a.attention_decode_noalloc(attention_params(q, proj, out, None, splits), b.desc, c["pool"].desc, stream())
