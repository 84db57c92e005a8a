"""CPU checks of the C ABI: the library loads, exports every function include/q38a.h declares,
the page layout matches the reference format (reference src/kernels/kernels.h:41-70,
docs/FORMAT.md 3.1), and invalid arguments fail with a status and a message (no GPU needed:
validation happens before any HIP call)."""
import ctypes
import os
import re

import pytest

import q38a

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header="q38a.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q38a_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 19
    lib = ctypes.CDLL(q38a.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(q38a.EXPORTED) <= set(names)
    from q38a import runtime
    rt = declared_functions("q38a_runtime.h")
    assert len(rt) >= 20
    missing = [n for n in rt if not hasattr(lib, n)]
    assert not missing, missing
    assert set(runtime.EXPORTED) == set(rt)
    from q38a import probe
    pr = declared_functions("q38a_probe.h")
    missing = [n for n in pr if not hasattr(lib, n)]
    assert not missing, missing
    assert set(probe.EXPORTED) == set(pr)
    from q38a import gemm
    gm = declared_functions("q38a_gemm.h")
    missing = [n for n in gm if not hasattr(lib, n)]
    assert not missing, missing
    assert set(gemm.EXPORTED) == set(gm)


def test_page_layout_matches_reference_format():
    # int8: K [4][64][256] i8 | V same | K scales [4][64][4] f16 | V scales same -> 2112 B per token
    assert q38a.page_bytes(q38a.KV_INT8, 4) == 135_168 == 64 * 2112
    assert q38a.page_bytes(q38a.KV_BF16, 4) == 2 * 4 * 64 * 256 * 2
    k, v, ks, vs = q38a.kv_offsets(q38a.KV_INT8, 4, 2, 5)
    assert k == (2 * 64 + 5) * 256
    assert v == 4 * 64 * 256 + k
    assert ks == 2 * 4 * 64 * 256 + (2 * 64 + 5) * 8
    assert vs == ks + 4 * 64 * 8
    k, v, _, _ = q38a.kv_offsets(q38a.KV_BF16, 4, 3, 63)
    assert k == (3 * 64 + 63) * 512 and v == 4 * 64 * 512 + k


def test_invalid_arguments_report_errors():
    with pytest.raises(q38a.Q38AError, match="must be set"):
        q38a.qk_norm_rope_append(q38a.QkNormRopeParams(), q38a.BatchDesc(), q38a.KvCacheDesc())
    kv = q38a.KvCacheDesc(1, 0, 4, 10, q38a.page_bytes(0, 4), q38a.page_bytes(0, 4) * 10, 1, 4)
    b = q38a.BatchDesc(1, 1, 1, 8, 8, 8, 8, 8)
    p = q38a.AttentionParams(8, 8, 14336, 8, 24, 5, 0, 8, 64)
    with pytest.raises(q38a.Q38AError, match="multiple") as e:
        q38a.attention_decode(p, b, kv)
    assert e.value.code == 2  # Q38A_ERR_UNSUPPORTED
    p = q38a.AttentionParams(8, 8, 14336, 8, 48, 4, 0, 8, 64)  # group 12 > 8
    with pytest.raises(q38a.Q38AError, match="group"):
        q38a.attention_decode(p, b, kv)
    p = q38a.AttentionParams(8, 8, 14336, 8, 24, 4, 0, None, 0)
    with pytest.raises(q38a.Q38AError, match="scratch"):
        q38a.attention_decode(p, b, kv)
    bad_kv = q38a.KvCacheDesc(1, 0, 4, 10, 1234, 12340, 1, 4)
    p = q38a.AttentionParams(8, 8, 14336, 8, 24, 4, 0, 8, 64)
    with pytest.raises(q38a.Q38AError, match="page_bytes"):
        q38a.attention_decode(p, b, bad_kv)
    b2 = q38a.BatchDesc(2, 3, 2, 8, 8, 8, 8, 8)
    with pytest.raises(q38a.Q38AError, match="one token per sequence"):
        q38a.attention_decode(p, b2, kv)
    # append without a RoPE table is refused (the table carries the bit-exact libm values)
    ap = q38a.QkNormRopeParams(8, 14336, 8, 8, 1e-6, 1e7, 24, 4, 8, 0, None, 0)
    with pytest.raises(q38a.Q38AError, match="rope"):
        q38a.qk_norm_rope_append(ap, b, kv)
    assert "rope" in q38a.last_error()


def test_rope_table_rejects_other_rotary_dims():
    with pytest.raises(q38a.Q38AError):
        q38a.rope_table(0, 4, rotary_dim=128)


def test_ragged_scratch_size_and_refusals():
    # header (4096 ints) + claim counters (4096 x 32 ints) + decode partials [B][nq][splits][258] fp32
    # + prefill units (tiles bound + 256) x 256 rows x 132 floats (fp16 O / l [256], m, l, pad)
    B, M, nq, nkv, splits = 8, 519, 24, 4, 64
    tiles = nkv * (M * (nq // nkv) // 256 + B)
    want = 4096 + 4096 * 32 + B * nq * splits * 258 + (tiles + 256) * 256 * 132
    assert q38a.ragged_scratch_floats(B, M, 512, nq, nkv, splits) == want
    # all-decode batches need no prefill partials
    assert q38a.ragged_scratch_floats(B, B, 1, nq, nkv, splits) == 4096 + 4096 * 32 + B * nq * splits * 258
    assert q38a.ragged_scratch_floats(0, 1, 1, nq, nkv, splits) == 0
    assert q38a.ragged_scratch_floats(1, 1, 1, 24, 5, splits) == 0
    # refused before any device call
    kv = q38a.KvCacheDesc(1, 1, 4, 10, q38a.page_bytes(1, 4), q38a.page_bytes(1, 4) * 10, 1, 4)
    with pytest.raises(q38a.Q38AError, match="sequences"):
        q38a.attention_ragged(q38a.AttentionParams(8, 8, 14336, 8, 24, 4, 0, 8, 64),
                              q38a.BatchDesc(1024, 1024, 1, 8, 8, 8, 8, 8), kv)
    with pytest.raises(q38a.Q38AError, match="max_splits"):
        q38a.attention_ragged(q38a.AttentionParams(8, 8, 14336, 8, 24, 4, 0, 8, 600),
                              q38a.BatchDesc(2, 2, 1, 8, 8, 8, 8, 8), kv)


def test_runtime_buckets_and_refusals():
    from q38a import runtime
    # reference src/model_runner.cpp:28-33: {1, 2, 4, 8, 12, 16, 24, 32, 48, 64} capped by max_batch
    assert [runtime.bucket_for(n, 8) for n in range(1, 9)] == [1, 2, 4, 4, 8, 8, 8, 8]
    assert [runtime.bucket_for(n, 64) for n in (9, 13, 17, 25, 33, 49, 64)] == [12, 16, 24, 32, 48, 64, 64]
    assert runtime.bucket_for(10, 10) == 10
    # bad options are refused before any device call
    with pytest.raises(q38a.Q38AError, match="bad options"):
        runtime.Runner(0, 0)
    with pytest.raises(q38a.Q38AError, match="bad options"):
        runtime.Runner(8, 8, num_q_heads=24, num_kv_heads=5)
    with pytest.raises(q38a.Q38AError, match="bad options"):
        runtime.Runner(8, 8, max_splits=513)
