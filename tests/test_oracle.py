"""Pins the CPU oracle (oracle/oracle.cpp) before it is trusted as the parity reference.

Each oracle function is checked against something that does not share its code:
  * the reference's own CPU ops (oracle/_ref, built from /root/reference/src/ref/ops.cpp), bit for
    bit, on many seeded tokens and positions up to the model's 262,144-position limit;
  * independent implementations (numpy's IEEE float16 conversion, a numpy bf16 rounding);
  * closed forms and invariants of the mathematics (quantizer bounds, RoPE identity at position 0
    and norm preservation, single-key and identical-key attention, GQA head mapping).
"""
import numpy as np
import pytest

from util import bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits, randn_bf16

NQ, NKV = 24, 4
LD = 2 * (NQ + NKV) * 256


def boundary_patterns():
    """Every sign/exponent/top-mantissa pattern combined with rounding-boundary low bits."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x7FFF, 0x8000, 0x8001, 0xA5A5, 0xFFFF,
                     0x6000, 0x5FFF, 0x9000], dtype=np.uint32)
    return (hi[:, None] | lows[None, :]).ravel()


def test_f16_conversion_matches_ieee(orc):
    u = boundary_patterns()
    x = u.view(np.float32)
    got = orc.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(x)
    assert np.array_equal(got[finite], want[finite])
    assert np.all((got[~finite] & 0x7E00) == 0x7E00)  # NaN stays a quiet NaN


def test_bf16_conversion_matches_numpy_rne(orc):
    u = boundary_patterns()
    x = u.view(np.float32)
    assert np.array_equal(orc.f32_to_bf16(x), f32_to_bf16_bits(x))


def test_quantizer_invariants(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((512, 256)).astype(np.float32) * rng.uniform(1e-3, 50, (512, 1)).astype(np.float32)
    x[0, :64] = 0.0  # an all-zero group
    codes, scales = orc.quantize_int8(x)
    s = f16_bits_to_f32(scales)  # [512][4]
    g = x.reshape(512, 4, 64)
    c = codes.reshape(512, 4, 64).astype(np.float32)
    assert np.all(np.abs(codes.astype(np.int32)) <= 127)
    assert scales[0, 0] == 0 and np.all(codes[0, :64] == 0)
    amax = np.abs(g).max(axis=2)
    # scale = fp16(amax / 127)
    assert np.array_equal(scales, (amax / np.float32(127)).astype(np.float32).astype(np.float16).view(np.uint16))
    nz = s > 0
    # the amax element maps to +-127, every element within half a step
    arg = np.abs(g).argmax(axis=2)
    top = np.take_along_axis(c, arg[..., None], axis=2)[..., 0]
    assert np.all(np.abs(top[nz]) == 127)
    err = np.abs(c * s[..., None] - g)
    assert np.all(err[nz] <= s[nz][..., None] * 0.5 * (1 + 1e-6) + 1e-30)


def test_quantizer_matches_reference_roundtrip(orc, ref):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(64 * 400).astype(np.float32) * rng.uniform(1e-4, 100, 64 * 400).astype(np.float32))
    codes, scales = orc.quantize_int8(x)
    deq = codes.astype(np.float32) * np.repeat(f16_bits_to_f32(scales), 64)
    # equal as values: the reference dequantizes a code of 0 from a negative input to -0.0, the
    # int8 byte (and thus every kernel) sees +0; nonzero values must match bit for bit
    assert np.array_equal(deq, ref.int8_group_roundtrip(x))


def test_rms_offset_norm_textbook(orc):
    rng = np.random.default_rng(7)
    x = bf16_bits_to_f32(randn_bf16(rng, 256))
    w = rng.normal(1.0, 0.1, 256).astype(np.float32)
    y = orc.rms_offset_norm(x, w)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(y, want, rtol=2e-6, atol=0)


def test_rope_table_identity_and_norm(orc):
    t = orc.rope_table(0, 4096)
    assert np.all(t[0, :32] == 1.0) and np.all(t[0, 32:] == 0.0)  # position 0 is the identity
    norm = t[:, :32].astype(np.float64) ** 2 + t[:, 32:].astype(np.float64) ** 2
    assert np.allclose(norm, 1.0, atol=1e-6)
    # frequency i: angle = pos * theta^(-i/32)
    pos = np.arange(4096, dtype=np.float64)[:, None]
    inv = 1e7 ** (-np.arange(32) / 32.0)
    assert np.allclose(t[:, :32], np.cos(pos * inv), atol=2e-4)


def test_rope_table_matches_product_table(orc):
    """The library's host table (same libm calls) must equal the oracle's, bit for bit."""
    import q38a
    for start, n in [(0, 5000), (130, 1), (200_000, 4000), (262_000, 144)]:
        assert np.array_equal(orc.rope_table(start, n).view(np.uint32), q38a.rope_table(start, n).view(np.uint32))


def _random_proj(rng, m):
    return randn_bf16(rng, (m, LD))


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_append_matches_reference_bitwise(orc, ref, kv_dtype):
    """q (fp16) and the appended K/V (bytes -> values) equal ops.cpp:125-142 exactly."""
    rng = np.random.default_rng(11 + kv_dtype)
    q_norm = rng.normal(1.0, 0.2, 256).astype(np.float32)
    k_norm = rng.normal(1.0, 0.2, 256).astype(np.float32)
    positions = np.concatenate([np.arange(0, 70), rng.integers(70, 262_144, 90)]).astype(np.int32)
    M = len(positions)
    proj = _random_proj(rng, M)
    proj[3, :256] = f32_to_bf16_bits(np.full(256, 1e-30, np.float32))  # tiny row
    proj[4, 2 * NQ * 256: 2 * NQ * 256 + 256] = 0  # zero k head: scale 0
    # one slot, each token on its own page so rows never collide
    pages = M
    bt = np.arange(pages, dtype=np.int32)[None, :].repeat(1, 0)
    bt_full = np.zeros((1, max(pages, positions.max() // 64 + 1)), dtype=np.int32)
    pb = orc_page_bytes(kv_dtype)
    pool = np.zeros(pb * pages, dtype=np.uint8)
    import q38a
    for i, pos in enumerate(positions):
        bt_full[0, pos // 64] = i
        q = orc.qk_norm_rope_append(proj[i:i + 1], LD, [pos], [0], [0], q_norm, k_norm, NQ, NKV, pool, kv_dtype, bt_full)
        page = pool[i * pb:(i + 1) * pb]
        rq, rk, rv = ref.qk_norm_rope_append_token(NQ, NKV, bf16_bits_to_f32(proj[i]), int(pos), q_norm, k_norm,
                                                   kv_dtype)
        assert np.array_equal(f16_bits_to_f32(q[0]).view(np.uint32), rq.view(np.uint32)), f"q pos {pos}"
        for h in range(NKV):
            off = q38a.kv_offsets(kv_dtype, NKV, h, int(pos) % 64)
            k, v = (dequant_row(page, kv_dtype, off[j], off[j + 2]) for j in (0, 1))
            assert np.array_equal(k, rk[h]), f"k pos {pos}"  # values: +-0 may differ, see above
            assert np.array_equal(v, rv[h]), f"v pos {pos}"
    del bt


def dequant_row(page, kv_dtype, off, soff):
    if kv_dtype == 1:
        return bf16_bits_to_f32(page[off:off + 512].view(np.uint16))
    sc = f16_bits_to_f32(page[soff:soff + 8].view(np.uint16))
    return page[off:off + 256].view(np.int8).astype(np.float32) * np.repeat(sc, 64)


def orc_page_bytes(kv_dtype, nkv=NKV):
    return 2 * nkv * 64 * (256 + 8) if kv_dtype in (0, 2) else 2 * nkv * 64 * 256 * 2


def test_int8_bytes_recoverable_from_reference_values(orc, ref):
    """The reference keeps dequantized floats; codes and scales follow from them exactly
    (scale = max|x'| / 127, code = x' / scale), and must equal the oracle's bytes."""
    rng = np.random.default_rng(12)
    q_norm = rng.normal(1.0, 0.1, 256).astype(np.float32)
    k_norm = rng.normal(1.0, 0.1, 256).astype(np.float32)
    bt = np.zeros((1, 4), dtype=np.int32)
    bt[0] = [0, 1, 2, 3]
    pool = np.zeros(orc_page_bytes(0) * 4, dtype=np.uint8)
    proj = _random_proj(rng, 1)
    orc.qk_norm_rope_append(proj, LD, [200], [0], [0], q_norm, k_norm, NQ, NKV, pool, 0, bt)
    _, rk, rv = ref.qk_norm_rope_append_token(NQ, NKV, bf16_bits_to_f32(proj[0]), 200, q_norm, k_norm, 0)
    page = pool[3 * orc_page_bytes(0): 4 * orc_page_bytes(0)]
    import q38a
    for h in range(NKV):
        offs = q38a.kv_offsets(0, NKV, h, 200 % 64)
        for vals, off, soff in ((rk[h], offs[0], offs[2]), (rv[h], offs[1], offs[3])):
            g = vals.reshape(4, 64)
            scale = (np.abs(g).max(axis=1) / np.float32(127)).astype(np.float32)
            codes = np.where(scale[:, None] > 0, g / np.where(scale > 0, scale, 1)[:, None], 0).astype(np.float32)
            assert np.all(codes == np.round(codes))
            assert np.array_equal(page[off:off + 256].view(np.int8), codes.ravel().astype(np.int8))
            assert np.array_equal(page[soff:soff + 8].view(np.uint16), scale.astype(np.float16).view(np.uint16))


def test_attention_matches_reference_bitwise(orc, ref):
    rng = np.random.default_rng(13)
    L = 300
    st = ref.store(NKV, L)
    k = rng.standard_normal((NKV, L, 256)).astype(np.float32)
    v = rng.standard_normal((NKV, L, 256)).astype(np.float32)
    st.k[...] = k
    st.v[...] = v
    for pos in (0, 1, 63, 64, 299):
        q = f16_bits_to_f32(rng.standard_normal(NQ * 256).astype(np.float16).view(np.uint16))
        gate = bf16_bits_to_f32(randn_bf16(rng, NQ * 256))
        a = orc.attention_token(q, gate, pos, k, v, NQ, NKV)
        b = st.attention_token(NQ, q, gate, pos)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), pos
    st.close()


def _sigmoid(g):
    return 1.0 / (1.0 + np.exp(-g.astype(np.float64)))


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(14)
    nq, nkv = 6, 2
    q = rng.standard_normal(nq * 256).astype(np.float32)
    gate = rng.standard_normal(nq * 256).astype(np.float32)
    k = rng.standard_normal((nkv, 5, 256)).astype(np.float32)
    v = rng.standard_normal((nkv, 5, 256)).astype(np.float32)
    # a single key: out = v * sigmoid(gate), head h reads kv head h // 3
    out = orc.attention_token(q, gate, 0, k, v, nq, nkv).reshape(nq, 256)
    for h in range(nq):
        want = v[h // 3, 0] * _sigmoid(gate[h * 256:(h + 1) * 256])
        assert np.allclose(out[h], want, rtol=8e-3, atol=1e-6)
    # identical keys: uniform weights -> mean of V
    k2 = np.repeat(k[:, :1], 5, axis=1)
    out = orc.attention_token(q, gate, 4, k2, v, nq, nkv).reshape(nq, 256)
    for h in range(nq):
        want = v[h // 3].mean(axis=0) * _sigmoid(gate[h * 256:(h + 1) * 256])
        assert np.allclose(out[h], want, rtol=8e-3, atol=1e-6)
    # brute force softmax in float64 on a tiny case
    out = orc.attention_token(q, gate, 4, k, v, nq, nkv).reshape(nq, 256)
    for h in range(nq):
        s = k[h // 3] @ q[h * 256:(h + 1) * 256].astype(np.float64) / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        want = (p @ v[h // 3]) * _sigmoid(gate[h * 256:(h + 1) * 256])
        assert np.allclose(out[h], want, rtol=8e-3, atol=1e-6)


def test_paging_is_invisible(orc):
    """Permuting page ids leaves the attention output bitwise unchanged."""
    rng = np.random.default_rng(15)
    nq, nkv, L = 6, 1, 200
    pages = 4
    kr = rng.standard_normal((L, nkv, 256)).astype(np.float32)
    vr = rng.standard_normal((L, nkv, 256)).astype(np.float32)
    q16 = rng.standard_normal((1, nq, 256)).astype(np.float16).view(np.uint16)
    gate = randn_bf16(rng, (1, nq * 256))
    outs = []
    for perm in (np.arange(pages), rng.permutation(pages)):
        bt = perm.astype(np.int32)[None, :]
        pool = np.zeros(orc_page_bytes(0, nkv) * pages, dtype=np.uint8)
        orc.fill_rows(kr, vr, 0, 0, nkv, pool, 0, bt)
        outs.append(orc.attention_ragged(nq, nkv, [0, 1], [0], [L - 1], q16, gate, nq * 256, pool, 0, bt))
    assert np.array_equal(outs[0], outs[1])


def int8_page_to_vt(page, nkv=NKV):
    """The int8 VT layout stated independently of the oracle: the same page with the V code block
    [kvh][64 tok][256] rearranged to [kvh][4 quarters][256][16 tok] and the V scale block
    [kvh][64][4] transposed to [kvh][4][64]."""
    page = page.copy()
    cb = nkv * 64 * 256
    v = page[cb:2 * cb].reshape(nkv, 4, 16, 256)
    page[cb:2 * cb] = np.ascontiguousarray(v.transpose(0, 1, 3, 2)).reshape(-1)
    s0 = 2 * cb + nkv * 64 * 8
    vs = page[s0:s0 + nkv * 64 * 8].view(np.uint16).reshape(nkv, 64, 4)
    page[s0:s0 + nkv * 64 * 8] = np.ascontiguousarray(vs.transpose(0, 2, 1)).reshape(-1).view(np.uint8)
    return page


def test_int8_vt_layout_is_the_transposed_int8_page(orc):
    """int8 VT pages hold exactly the int8 page's codes and scales, with the V block transposed:
    fill and append into both formats and compare byte for byte through the transposition; the
    attention over either pool is bitwise the same."""
    rng = np.random.default_rng(21)
    L, pages = 150, 3
    kr = bf16_bits_to_f32(randn_bf16(rng, (L, NKV, 256)))
    vr = bf16_bits_to_f32(randn_bf16(rng, (L, NKV, 256)))
    vr[7, 2, 64:128] = 0.0  # a zero group: scale 0
    bt = np.array([[2, 0, 1]], np.int32)
    pb = orc_page_bytes(0)
    pools = {}
    for dt in (0, 2):
        pool = np.zeros(pb * pages, np.uint8)
        orc.fill_rows(kr, vr, 0, 0, NKV, pool, dt, bt)
        pools[dt] = pool
    proj = randn_bf16(np.random.default_rng(5), (2, LD))
    qn = np.random.default_rng(6).normal(1.0, 0.2, 256).astype(np.float32)
    kn = np.random.default_rng(7).normal(1.0, 0.2, 256).astype(np.float32)
    qs = {dt: orc.qk_norm_rope_append(proj, LD, [L, L + 1], [0, 0], [0], qn, kn, NQ, NKV, pools[dt], dt, bt)
          for dt in (0, 2)}
    assert np.array_equal(qs[0], qs[2])
    for p in range(pages):
        a = pools[0][p * pb:(p + 1) * pb]
        b = pools[2][p * pb:(p + 1) * pb]
        assert np.array_equal(int8_page_to_vt(a), b), f"page {p}"
    gate = randn_bf16(rng, (2, NQ * 256))
    outs = [orc.attention_ragged(NQ, NKV, [0, 2], [0], [L, L + 1], qs[dt], gate, NQ * 256, pools[dt], dt, bt)
            for dt in (0, 2)]
    assert np.array_equal(outs[0], outs[1])
    k0, v0 = orc.read_back(pools[0], 0, NKV, bt, 0, L + 2)
    k2, v2 = orc.read_back(pools[2], 2, NKV, bt, 0, L + 2)
    assert np.array_equal(k0, k2) and np.array_equal(v0, v2)
