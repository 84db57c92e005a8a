"""GPU parity of q38a_attention_ragged: decode rows (one new token) and prefill chunks (several) of
one continuous-batching step in a single attention launch plus the merge, against the oracle's
exact attention per token (reference src/ref/ops.cpp:144-171), within the north star's tolerance
(|d| <= 2e-3 + 1e-2 |ref|, bf16 out). The appended K/V bytes are checked bit for bit first. The
split prefill tiles and their merge are also compared with q38a_attention_prefill (one unit per
tile, no merge) on the same inputs."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev, stream
from util import assert_bits_equal, bf16_bits_to_f32, check_close, randn_bf16
from test_gpu_decode import build_context, scale_proj_kv

pytestmark = pytest.mark.gpu


def ragged_step(orc, seqs, seed, kv_dtype=q38a.KV_INT8, check_tokens=None, max_splits=64, compare_split_launches=False,
                k_scale=1.0, v_scale=1.0, dominant=None, return_out=False):
    """seqs: [(prefix, n)]; n == 1 is a decode row. check_tokens: per sequence, the chunk-token
    indices compared with the oracle (default all)."""
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
    nfl = q38a.ragged_scratch_floats(B, b.M, max(n for _, n in seqs), NQ, NKV, max_splits)
    scratch_t = torch.full((nfl,), float("nan"), dtype=torch.float32, device="cuda")
    q38a.ragged_scratch_init(scratch_t.data_ptr(), stream())  # counters zero, partials stay NaN
    rope_t = rope_dev(max(p + n for p, n in seqs) + 1)
    print(f"ragged: seqs={seqs[:10]} dtype={kv_dtype} scratch={nfl * 4 / 2**20:.1f} MiB", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_t), b.desc, pool.desc, stream())
    params = attention_params(q_t, proj_t, out_t, scratch_t, max_splits)
    q38a.attention_ragged(params, b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    q16 = host(q_t, np.uint16).reshape(b.M, NQ, HD)
    q_ref = orc.qk_norm_rope_append(proj, LD, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, NQ, NKV, pool_host,
                                    kv_dtype, bt)
    assert_bits_equal(q16, q_ref, "q fp16")
    assert_bits_equal(pool.download(), pool_host, "pool bytes")
    got = bf16_bits_to_f32(host(out_t, np.uint16)).reshape(b.M, NQ * HD)
    if compare_split_launches:
        # the same rows through the separate prefill launch (whole tiles, final output in-kernel)
        out2 = torch.zeros_like(out_t)
        q38a.attention_prefill(attention_params(q_t, proj_t, out2, None, 0), b.desc, pool.desc, stream())
        torch.cuda.synchronize()
        alt = bf16_bits_to_f32(host(out2, np.uint16)).reshape(b.M, NQ * HD)
        rows = np.concatenate([np.arange(b.seq_start[i], b.seq_start[i + 1]) for i, (_, n) in enumerate(seqs) if n > 1])
        check_close(got[rows], alt[rows], what="ragged vs prefill launch")
    sel = []
    for i, (p, n) in enumerate(seqs):
        idx = range(n) if check_tokens is None or check_tokens[i] is None else check_tokens[i]
        sel += [int(b.seq_start[i]) + t for t in idx]
    sel = np.array(sel, np.int64)
    gate = np.ascontiguousarray(proj[sel, NQ * HD:2 * NQ * HD])
    seq_of = b.tok_seq[sel]
    starts = np.searchsorted(seq_of, np.arange(B + 1)).astype(np.int32)
    want = orc.attention_ragged(NQ, NKV, starts, b.seq_slot, b.tok_pos[sel], q16[sel], gate, NQ * HD, pool_host,
                                kv_dtype, bt)
    want = bf16_bits_to_f32(want).reshape(len(sel), NQ * HD)
    assert np.isfinite(got[sel]).all()
    if return_out:
        return got[sel], want
    return check_close(got[sel], want, what=f"ragged seqs={seqs[:10]}")


def test_ragged_mixed_small(orc):
    """Chunks starting mid-page and on page edges, decode rows at 0, 63 and 5000, one 2-token chunk."""
    ragged_step(orc, [(0, 130), (500, 1), (777, 300), (64, 64), (2000, 17), (5000, 1), (63, 1), (0, 1), (129, 2)],
                seed=31, compare_split_launches=True)


def test_ragged_only_decode(orc):
    ragged_step(orc, [(c, 1) for c in (1, 64, 1000, 4097, 9000, 300, 77, 2048)], seed=32)


@pytest.mark.parametrize("kv_dtype", [q38a.KV_BF16])
def test_ragged_only_decode_bf16(orc, kv_dtype):
    ragged_step(orc, [(c, 1) for c in (5, 640, 3000, 129)], seed=33, kv_dtype=kv_dtype)


def test_ragged_mixed_int8_vt(orc):
    """int8 VT pages (V transposed per page): chunks (split and unsplit tiles) and decode rows in one
    launch, and the same rows through the prefill launch."""
    ragged_step(orc, [(0, 130), (5000, 1), (777, 300), (20000, 3), (63, 1), (129, 2), (64, 1)], seed=36,
                kv_dtype=q38a.KV_INT8_VT, compare_split_launches=True)


def test_ragged_mixed_bf16(orc):
    """bf16 pages: chunks (split and unsplit tiles) and decode rows in one launch."""
    ragged_step(orc, [(0, 130), (5000, 1), (777, 300), (20000, 3), (63, 1)], seed=35, kv_dtype=q38a.KV_BF16,
                compare_split_launches=True)


def test_ragged_long_prefix_short_chunks(orc):
    """Few rows over long prefixes: every tile is cut into many key parts (merge of up to ~100)."""
    ragged_step(orc, [(20000, 2), (33000, 7), (12345, 1)], seed=34, compare_split_launches=True)


def test_ragged_config4_shape(orc):
    """Config 4: a 512-token chunk plus 7 decode rows, contexts lognormal (median 8192, sigma 1)
    clipped to [64, 65536]; 40 chunk tokens and every decode row are checked."""
    rng = np.random.default_rng(0)
    ctx = np.clip(np.round(np.exp(np.log(8192) + rng.normal(0, 1, 8))), 64, 65536).astype(int)
    seqs = [(int(ctx[0]), 512)] + [(int(c), 1) for c in ctx[1:]]
    toks = sorted(set([0, 1, 2, 63, 64, 255, 256, 510, 511] + list(range(5, 512, 17))))
    ragged_step(orc, seqs, seed=4, check_tokens=[toks] + [None] * 7, compare_split_launches=True)


def test_ragged_config3_through_ragged(orc):
    """Config 3 (2048-token chunk on a 6000-token prefix) through the ragged launch: tiles split."""
    toks = sorted(set([0, 1, 47, 48, 1000, 2046, 2047] + list(range(5, 2048, 97))))
    ragged_step(orc, [(6000, 2048)], seed=3, check_tokens=[toks], compare_split_launches=True)


def test_ragged_back_to_back_launches(orc):
    """Launches of different shapes in a row (with and without prefill chunks, so with and without
    decode workgroups placed before the prefill units): the launch-wide decode item queue and the
    block-claim counters must start every launch at zero, which the previous launch's last draw
    restores."""
    mixed = [(3000, 40), (9000, 1), (700, 1), (15000, 1), (64, 1)]
    decode = [(c, 1) for c in (4000, 129, 20000, 640)]
    for i, seqs in enumerate([mixed, decode, mixed, decode, [(6000, 300)], mixed]):
        ragged_step(orc, seqs, seed=40 + i)


def test_ragged_more_than_64_decode_rows(orc):
    """A chunk beside 100 decode rows: the decode items of rows past 64 in the ragged launch."""
    rng = np.random.default_rng(50)
    seqs = [(int(x), 1) for x in rng.integers(0, 600, 100)]
    seqs[10] = (700, 40)
    ragged_step(orc, seqs, seed=51)
