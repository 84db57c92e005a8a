"""CPU checks of the BQ weight handling (no GPU): the oracle's writer and reader of the reference's
file layout (docs/FORMAT.md section 2) against hand-derived positions from the format text and
against numpy's bf16(code * scale); and the library's repack into the q38a MFMA layout, decoded
back by a numpy restatement of the layout in include/q38a_gemm.h."""
import numpy as np
import pytest

from util import bf16_bits_to_f32, f32_to_bf16_bits

BITS = [4, 5, 6]


def random_weight(rng, bits, n, k):
    codes = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), (n, k)).astype(np.int8)
    scales = f32_to_bf16_bits(rng.uniform(0.002, 0.05, (n, k // 64)).astype(np.float32))
    return codes, scales


@pytest.mark.parametrize("bits", BITS)
def test_file_layout_roundtrip_is_bf16_code_times_scale(orc, bits):
    rng = np.random.default_rng(bits)
    n, k = 128, 256
    codes, scales = random_weight(rng, bits, n, k)
    lo, hi, sc = orc.bq_pack_file(bits, codes, scales)
    w = orc.bq_file_weight(bits, n, k, lo, hi, sc)
    want = bf16_bits_to_f32(f32_to_bf16_bits(codes.astype(np.float32) * np.repeat(bf16_bits_to_f32(scales), 64, 1)))
    assert np.array_equal(w, want)


@pytest.mark.parametrize("bits", BITS)
def test_file_layout_positions_from_the_format_text(orc, bits):
    """One nonzero code at (n = 9, k = 19): by FORMAT.md 2.2-2.4, slab (kb = 1, nb = 0) = slab 1,
    lane 4 g + t with g = 9 % 8 = 1, t = (19 % 8) / 2 = 1 -> lane 5, pair q = 2 j + h with
    j = 9 / 8 = 1, h = (19 % 16) / 8 = 0 -> q = 2, second element of the pair (19 is odd): lo word
    q / 4 = 0, bits 16 + 4 (q % 4) = 24..27, i.e. the low nibble of byte 512 + 16 * 5 + 3 = 595; bq5
    hi bit 16 + q = 18 of lane 5's word at 128 + 4 * 5; bq6 hi bits 16 + 2q = 20..21 of word 0 at
    256 + 8 * 5; scale of (row 9, group 0) at block 0, entry 8 g + j = 9."""
    n, k = 64, 64
    codes = np.full((n, k), -(1 << (bits - 1)), np.int8)  # stored code 0 everywhere ...
    u = (1 << bits) - 1  # ... except u = all ones at (9, 19)
    codes[9, 19] = u - (1 << (bits - 1))
    scales = np.zeros((n, 1), np.uint16)
    scales[9, 0] = 0x3F80  # 1.0
    lo, hi, sc = orc.bq_pack_file(bits, codes, scales)
    expect_lo = np.zeros_like(lo)
    expect_lo[595] = 0x0F
    assert np.array_equal(lo, expect_lo)
    if bits == 5:
        expect_hi = np.zeros_like(hi)
        expect_hi[128 + 20 + 2] = 0x04  # bit 18 of the little-endian word
        assert np.array_equal(hi, expect_hi)
    if bits == 6:
        expect_hi = np.zeros_like(hi)
        expect_hi[256 + 40 + 2] = 0x30  # bits 20..21
        assert np.array_equal(hi, expect_hi)
    expect_sc = np.zeros_like(sc)
    expect_sc[9] = 0x3F80
    assert np.array_equal(sc, expect_sc)


def decode_q38a_layout(bits, n, k, lo, hi, sc):
    """Codes and scales from the q38a layout, as include/q38a_gemm.h states it."""
    G = k // 64
    codes = np.zeros((n, k), np.int32)
    scales = np.zeros((n, G), np.uint16)
    lo = np.frombuffer(lo.tobytes(), np.uint32).reshape(n // 32, G, 64, 4)
    hw = {4: 0, 5: 1, 6: 2}[bits]
    if hw:
        hi = np.frombuffer(hi.tobytes(), np.uint32).reshape(n // 32, G, 64, hw)
    sc = sc.reshape(n // 32, G, 32)
    for nb in range(n // 32):
        for g in range(G):
            for l in range(64):
                col, kg = 32 * nb + l % 32, l // 32
                for s in range(4):
                    for i in range(8):
                        p, e, q = i // 2, i % 2, 4 * s + i // 2
                        u = (int(lo[nb, g, l, s]) >> (16 * e + 4 * p)) & 15
                        if bits == 5:
                            u |= ((int(hi[nb, g, l, 0]) >> (16 * e + q)) & 1) << 4
                        if bits == 6:
                            u |= ((int(hi[nb, g, l, q // 8]) >> (16 * e + 2 * (q % 8))) & 3) << 4
                        codes[col, 64 * g + 16 * s + 8 * kg + i] = u - (1 << (bits - 1))
            scales[32 * nb:32 * nb + 32, g] = sc[nb, g]
    return codes, scales


@pytest.mark.parametrize("bits", BITS)
def test_repack_into_mfma_layout(orc, bits):
    from q38a import gemm
    rng = np.random.default_rng(10 + bits)
    n, k = 128, 192
    codes, scales = random_weight(rng, bits, n, k)
    lo, hi, sc = orc.bq_pack_file(bits, codes, scales)
    rlo, rhi, rsc = gemm.repack(bits, n, k, lo, hi, sc)
    c2, s2 = decode_q38a_layout(bits, n, k, rlo, rhi, rsc)
    assert np.array_equal(c2, codes.astype(np.int32))
    assert np.array_equal(s2, scales)


def test_repack_refuses_8_bit_and_bad_shapes():
    import q38a
    from q38a import gemm
    z = np.zeros(64 * 64, np.uint8)
    with pytest.raises(q38a.Q38AError):
        gemm.repack(8, 64, 64, z, z, np.zeros(64, np.uint16))
    with pytest.raises(q38a.Q38AError):
        gemm.repacked_bytes(5, 48, 64)
