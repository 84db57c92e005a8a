"""GPU parity for other head geometries than Qwen3.8's 24 q / 4 kv heads: GQA groups 1, 3, 4 and 8
(the kernels accept any group up to 8, reference attention_decode.cu instantiates the group as a
template parameter) and a single kv head. Each case appends a mixed batch (decode rows and prefill
chunks, bit-checked against the oracle), then runs the ragged launch, and the decode and prefill
launches on the same inputs; all outputs are checked against the oracle's exact attention
(reference src/ref/ops.cpp:144-171) within the north star's tolerance."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev, stream
from util import assert_bits_equal, bf16_bits_to_f32, check_close, randn_bf16
from test_gpu_decode import build_context

pytestmark = pytest.mark.gpu

GEOMETRIES = [(8, 1), (16, 2), (8, 8), (12, 4), (16, 4)]


def run_case(orc, nq, nkv, kv_dtype, seed):
    rng = np.random.default_rng(seed)
    ld = 2 * (nq + nkv) * HD
    dec = [(700, 1), (63, 1), (4100, 1)]
    pre = [(0, 70), (1000, 150)]
    seqs = dec + pre
    B = len(seqs)
    bt, pages = paged_layout(rng, [p + n for p, n in seqs])
    pool_host = build_context(orc, rng, [p for p, _ in seqs], kv_dtype, bt, pages, nkv=nkv)
    pool = Pool(kv_dtype, pages, bt, nkv=nkv, fill=pool_host)
    b = Batch([(i, p, n) for i, (p, n) in enumerate(seqs)])
    proj = randn_bf16(rng, (b.M, ld))
    q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
    proj_t, qn_t, kn_t = dev(proj), dev(q_norm), dev(k_norm)
    q_t = torch.zeros(b.M * nq * HD, dtype=torch.int16, device="cuda")
    rope_t = rope_dev(max(p + n for p, n in seqs) + 1)
    print(f"geometry: nq={nq} nkv={nkv} dtype={kv_dtype}", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_t, nq=nq, nkv=nkv, ld=ld), b.desc, pool.desc,
                             stream())
    torch.cuda.synchronize()
    q16 = host(q_t, np.uint16).reshape(b.M, nq, HD)
    q_ref = orc.qk_norm_rope_append(proj, ld, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, nq, nkv, pool_host,
                                    kv_dtype, bt)
    assert_bits_equal(q16, q_ref, "q fp16")
    assert_bits_equal(pool.download(), pool_host, "pool bytes")
    gate = np.ascontiguousarray(proj[:, nq * HD:2 * nq * HD])
    want = orc.attention_ragged(nq, nkv, b.seq_start, b.seq_slot, b.tok_pos, q16, gate, nq * HD, pool_host, kv_dtype,
                                bt)
    want = bf16_bits_to_f32(want).reshape(b.M, nq * HD)
    max_splits = 32
    # ragged launch over the whole batch
    out_t = torch.zeros(b.M * nq * HD, dtype=torch.int16, device="cuda")
    scratch = torch.zeros(q38a.ragged_scratch_floats(B, b.M, b.desc.max_tokens_per_seq, nq, nkv, max_splits),
                          dtype=torch.float32, device="cuda")
    params = attention_params(q_t, proj_t, out_t, scratch, max_splits, nq=nq, nkv=nkv, ld=ld)
    q38a.attention_ragged(params, b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    got = bf16_bits_to_f32(host(out_t, np.uint16)).reshape(b.M, nq * HD)
    check_close(got, want, what=f"ragged nq={nq} nkv={nkv}")
    # the prefill launch over the same batch (decode rows are 1-token chunks for it)
    out2 = torch.zeros_like(out_t)
    q38a.attention_prefill(attention_params(q_t, proj_t, out2, None, 0, nq=nq, nkv=nkv, ld=ld), b.desc, pool.desc,
                           stream())
    torch.cuda.synchronize()
    check_close(bf16_bits_to_f32(host(out2, np.uint16)).reshape(b.M, nq * HD), want, what=f"prefill nq={nq} nkv={nkv}")
    # the decode launch over the decode rows alone (their q rows are the batch's first three)
    bd = Batch([(i, p, 1) for i, (p, _) in enumerate(dec)])
    out3 = torch.zeros(len(dec) * nq * HD, dtype=torch.int16, device="cuda")
    scr = torch.zeros(q38a.split_scratch_floats(len(dec), nq, max_splits), dtype=torch.float32, device="cuda")
    q38a.attention_decode(attention_params(q_t, proj_t, out3, scr, max_splits, nq=nq, nkv=nkv, ld=ld), bd.desc,
                          pool.desc, stream())
    torch.cuda.synchronize()
    check_close(bf16_bits_to_f32(host(out3, np.uint16)).reshape(len(dec), nq * HD), want[:len(dec)],
                what=f"decode nq={nq} nkv={nkv}")


@pytest.mark.parametrize("nq,nkv", GEOMETRIES)
def test_geometry_int8(orc, nq, nkv):
    run_case(orc, nq, nkv, q38a.KV_INT8, seed=50 + nq + nkv)


@pytest.mark.parametrize("nq,nkv", [(8, 1), (12, 4)])
def test_geometry_bf16(orc, nq, nkv):
    run_case(orc, nq, nkv, q38a.KV_BF16, seed=70 + nq + nkv)
