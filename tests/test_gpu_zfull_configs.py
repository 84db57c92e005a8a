"""The benchmark's own workloads at full size, checked against the oracle. These are the exact inputs
bench.py times (q38a.workloads, seed 0): config 2 (B = 8, contexts U[1024, 32768]), 5a (B = 8,
Dirichlet split of 204,800 tokens), 5b (one sequence at 262,143 + the new token) and 5c (5a on bf16
pages); also config 2 and 5a through the ragged launch (dynamic item queue and block claims).

For each: the append's q (fp16) and the whole pool (every page, so the new K/V bytes and scales)
are compared bit for bit with the oracle's append on a host copy of the pool, then every q head of
every row is compared with the oracle's exact double-precision attention within the north star's
tolerance (|d| <= 2e-3 + 1e-2 |ref|). Reference test shape: tests/gpu/test_kernels.cu:395-495.
Named to run after the smaller parity tests (each case moves ~0.5-1 GB through the host)."""
import numpy as np
import pytest
import torch

import q38a
from q38a.workloads import NKV, NQ, LD, DecodeBatch, decode_contexts
from util import assert_bits_equal, bf16_bits_to_f32, check_close

pytestmark = pytest.mark.gpu

HD = 256


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run_config(orc, ctxs, kv_dtype, max_splits, launch):
    db = DecodeBatch(ctxs, dtype=kv_dtype, seed=0, pools=1)
    if max_splits != db.max_splits:
        db.max_splits = max_splits
        db.scratch = torch.zeros(q38a.split_scratch_floats(db.B, NQ, max_splits), dtype=torch.float32, device="cuda")
    if launch == "ragged":
        db.scratch = torch.zeros(q38a.ragged_scratch_floats(db.B, db.B, 1, NQ, NKV, db.max_splits),
                                 dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    pool_host = db.pools[0].cpu().numpy()  # prior KV, before the append
    s = torch.cuda.current_stream().cuda_stream
    print(f"full config: B={db.B} sum_ctx={sum(ctxs)} max={max(ctxs)} dtype={kv_dtype} splits={max_splits} "
          f"launch={launch}", flush=True)
    q38a.qk_norm_rope_append(db.append_params(), db.batch, db.kv_desc(0), s)
    if launch == "ragged":
        q38a.attention_ragged(db.attention_params(), db.batch, db.kv_desc(0), s)
    else:
        q38a.attention_decode(db.attention_params(), db.batch, db.kv_desc(0), s)
    torch.cuda.synchronize()
    got = bf16_bits_to_f32(bits16(db.out)).reshape(db.B, NQ * HD)
    q16 = bits16(db.q16).reshape(db.B, NQ, HD)
    proj = bits16(db.proj)
    seq = np.arange(db.B, dtype=np.int32)
    pos = np.array(ctxs, np.int32)
    q_ref = orc.qk_norm_rope_append(proj, LD, pos, seq, seq, db.q_norm.cpu().numpy(), db.k_norm.cpu().numpy(), NQ,
                                    NKV, pool_host, kv_dtype, db.block_table)
    assert_bits_equal(q16, q_ref, "q fp16")
    dev_pool = db.pools[0].cpu().numpy()
    if not np.array_equal(dev_pool, pool_host):
        assert_bits_equal(dev_pool, pool_host, "pool bytes")
    gate = np.ascontiguousarray(proj[:, NQ * HD:2 * NQ * HD])
    want = orc.attention_ragged(NQ, NKV, np.arange(db.B + 1, dtype=np.int32), seq, pos, q16, gate, NQ * HD,
                                pool_host, kv_dtype, db.block_table)
    want = bf16_bits_to_f32(want).reshape(db.B, NQ * HD)
    max_abs, max_rel = check_close(got, want, what=f"full config ctxs={ctxs[:8]} dtype={kv_dtype}")
    print(f"  rows {db.B} x {NQ} heads: max_abs {max_abs:.3g} max_rel {max_rel:.3g}", flush=True)


def test_config2_decode_b8(orc):
    run_config(orc, decode_contexts("decode_b8"), q38a.KV_INT8, 256, "decode")


def test_config2_decode_b8_ragged_launch(orc):
    run_config(orc, decode_contexts("decode_b8"), q38a.KV_INT8, 256, "ragged")


def test_config5a_long_b8(orc):
    run_config(orc, decode_contexts("long_b8"), q38a.KV_INT8, 256, "decode")


def test_config5a_long_b8_ragged_launch(orc):
    run_config(orc, decode_contexts("long_b8"), q38a.KV_INT8, 256, "ragged")


@pytest.mark.parametrize("max_splits", [256, 64])
def test_config5b_long_b1(orc, max_splits):
    """One sequence of 262,144 keys (4,096 pages): with 64 splits the plan is limited by
    max_splits (64 pages per item) instead of by the item target."""
    run_config(orc, decode_contexts("long_b1"), q38a.KV_INT8, max_splits, "decode")


def test_config2_decode_b8_int8_vt(orc):
    run_config(orc, decode_contexts("decode_b8"), q38a.KV_INT8_VT, 256, "decode")


def test_config5a_long_b8_int8_vt(orc):
    run_config(orc, decode_contexts("long_b8"), q38a.KV_INT8_VT, 256, "decode")


def test_config5c_long_b8_bf16(orc):
    run_config(orc, decode_contexts("long_b8_bf16"), q38a.KV_BF16, 256, "decode")
