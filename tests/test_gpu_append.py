"""GPU parity of q38a_qk_norm_rope_append against the oracle: q fp16 bits and every byte of the
page pool (int8 codes + fp16 scales, or bf16) must be identical. Mirrors the reference kernel test
tests/gpu/test_kernels.cu:395-495 (prefixes {0, 1, 63, 64, 300, 2100}, chunks crossing page
boundaries) but demands bit equality where the reference allowed one int8 step."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, dev, host, paged_layout, rope_dev, stream
from util import assert_bits_equal, f32_to_bf16_bits, randn_bf16

pytestmark = pytest.mark.gpu


def run_append(orc, seqs, kv_dtype, rng, layers=1, layer=0, proj=None, max_pos=None, pool_fill=None):
    """Appends the batch on the GPU and with the oracle; returns (q_gpu, q_orc, pool_gpu, pool_orc)."""
    b = Batch(seqs)
    lengths = [p0 + n for _, p0, n in seqs]
    bt, pages = paged_layout(rng, lengths, extra_pages=3)
    # slots are the sequence index here
    pool = Pool(kv_dtype, pages, bt, layers=layers, fill=pool_fill)
    if proj is None:
        proj = randn_bf16(rng, (b.M, LD))
    q_norm = rng.normal(1.0, 0.2, HD).astype(np.float32)
    k_norm = rng.normal(1.0, 0.2, HD).astype(np.float32)
    proj_t, qn_t, kn_t = dev(proj), dev(q_norm), dev(k_norm)
    q_t = torch.zeros(b.M * NQ * HD, dtype=torch.int16, device="cuda")
    rope_t = rope_dev((max_pos or max(lengths)) + 1)
    print(f"append: seqs={seqs} dtype={kv_dtype} layer={layer}", flush=True)
    q38a.qk_norm_rope_append(append_params(proj_t, qn_t, kn_t, q_t, rope_t, layer=layer), b.desc, pool.desc, stream())
    torch.cuda.synchronize()
    ref_pool = pool.layer_host(layer).copy()
    q_ref = orc.qk_norm_rope_append(proj, LD, b.tok_pos, b.tok_seq, b.seq_slot, q_norm, k_norm, NQ, NKV, ref_pool,
                                    kv_dtype, bt)
    return host(q_t, np.uint16).reshape(b.M, NQ, HD), q_ref, pool.download(layer), ref_pool, pool


@pytest.mark.parametrize("kv_dtype", [q38a.KV_INT8, q38a.KV_BF16, q38a.KV_INT8_VT])
def test_append_ragged_bitwise(orc, kv_dtype):
    rng = np.random.default_rng(100 + kv_dtype)
    # prefill chunks that start mid-page and cross pages, decode rows at page edges
    seqs = [(0, 0, 37), (1, 37, 64), (2, 63, 2), (3, 64, 1), (4, 130, 1), (5, 2100, 211), (6, 6000, 90)]
    q, q_ref, pool, pool_ref = run_append(orc, seqs, kv_dtype, rng)[:4]
    assert_bits_equal(q, q_ref, "q fp16")
    assert_bits_equal(pool, pool_ref, "pool bytes")


def test_append_edge_values_bitwise(orc):
    """Rows that force the ordered double sum (huge dynamic range), all-zero heads (scale 0),
    subnormal-scale groups, and the last RoPE position of the model (262,143)."""
    rng = np.random.default_rng(7)
    seqs = [(0, 262_143, 1), (1, 5, 3)]
    M = 4
    proj = randn_bf16(rng, (M, LD))
    kcol = 2 * NQ * HD
    proj[0, :HD] = f32_to_bf16_bits(np.concatenate([np.full(128, 3e4), np.full(128, 1e-20)]).astype(np.float32))
    proj[1, kcol:kcol + HD] = 0                                   # zero k head
    proj[2, kcol + NKV * HD:kcol + NKV * HD + 64] = f32_to_bf16_bits(np.full(64, 1e-7, np.float32))  # tiny v group
    proj[3, kcol:kcol + HD] = f32_to_bf16_bits(rng.standard_normal(HD).astype(np.float32) * 1e3)
    proj[3, HD:2 * HD] = f32_to_bf16_bits(np.geomspace(1e-30, 1e30, HD).astype(np.float32))
    q, q_ref, pool, pool_ref = run_append(orc, seqs, q38a.KV_INT8, rng, proj=proj)[:4]
    assert_bits_equal(q, q_ref, "q fp16")
    assert_bits_equal(pool, pool_ref, "pool bytes")


def test_append_layer_offset(orc):
    """attn_layer selects the layer block of the pool; other layers stay untouched."""
    rng = np.random.default_rng(8)
    seqs = [(0, 10, 20), (1, 300, 1)]
    q, q_ref, pool, pool_ref, p = run_append(orc, seqs, q38a.KV_INT8, rng, layers=3, layer=2)
    assert_bits_equal(pool, pool_ref, "pool bytes")
    assert not p.download(0).any() and not p.download(1).any()


def test_append_large_prefill_chunk(orc):
    """Config 3's append: a 2048-token chunk starting at position 6000 (mid-page)."""
    rng = np.random.default_rng(9)
    q, q_ref, pool, pool_ref = run_append(orc, [(0, 6000, 2048)], q38a.KV_INT8, rng)[:4]
    assert_bits_equal(q, q_ref, "q fp16")
    assert_bits_equal(pool, pool_ref, "pool bytes")
