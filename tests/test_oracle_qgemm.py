"""CPU pins of the oracle's GEMM (`orc_qgemm`, the checker of the projection GEMMs) against numpy
float64 and closed forms, following the reference epilogues (src/kernels/qgemm.cu:285-384):

  * StoreBF16: out = bf16(float(A W^T) * rs), rs = 1 / sqrt(sum(partials_in[row]) / hidden + eps);
  * StoreF32:  out = float(A W^T) * rs, only the first n_store columns written;
  * Residual:  residual += float(A W^T); xbf = bf16(residual); partials_out[row][b] = sum of squares
    of the new residual over columns [128 b, 128 b + 128).

The cases are chosen so that a transposed W (n != k, asymmetric), a wrong `hidden`, a dropped
`eps`, a missing row scale, a wrong 128-column block or an n_store overrun each fail."""
import numpy as np
import pytest

from util import bf16_bits_to_f32, f32_to_bf16_bits, randn_bf16


def numpy_c(a_bits, w):
    """A W^T in float64 from bf16 bits A [m][k] and fp32 W [n][k]."""
    return bf16_bits_to_f32(a_bits).astype(np.float64) @ np.asarray(w, np.float64).T


def rowscale(partials, hidden, eps):
    """The reference's row scale in float32, partials summed in order (qgemm.cu:291-296)."""
    out = np.empty(partials.shape[0], np.float32)
    for r, row in enumerate(partials.astype(np.float32)):
        s = np.float32(0.0)
        for x in row:
            s = np.float32(s + x)
        out[r] = np.float32(1.0) / np.sqrt(np.float32(s / np.float32(hidden) + np.float32(eps)))
    return out


def assert_within_one_bf16_step(got_bits, want_bits, what, max_frac_off=1e-3):
    """bf16 bit patterns equal except for rare one-step flips (float64 sums in a different order can
    land on the other side of a rounding tie); sign-magnitude order makes adjacent values 1 apart."""
    g = got_bits.astype(np.int64)
    w = want_bits.astype(np.int64)
    key = lambda x: np.where(x & 0x8000, -(x & 0x7FFF), x)  # noqa: E731
    step = np.abs(key(g) - key(w))
    assert step.max() <= 1, f"{what}: {int((step > 1).sum())} values more than one bf16 step off"
    assert (step != 0).mean() <= max_frac_off, f"{what}: {int((step != 0).sum())} of {step.size} off by one step"


@pytest.mark.parametrize("m,n,k", [(3, 256, 192), (17, 384, 128)])
def test_store_bf16_row_scale_against_numpy(orc, m, n, k):
    rng = np.random.default_rng(m * 7 + n)
    a = randn_bf16(rng, (m, k))
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    hidden = 256
    partials = rng.uniform(50.0, 300.0, (m, hidden // 128)).astype(np.float32)
    eps = 0.5  # large enough that dropping it changes every row scale by far more than a bf16 step
    got = orc.qgemm(a, w, 0, partials_in=partials, hidden=hidden, eps=eps)
    rs = rowscale(partials, hidden, eps)
    want = f32_to_bf16_bits(numpy_c(a, w).astype(np.float32) * rs[:, None])
    assert_within_one_bf16_step(got, want, "StoreBF16")
    # the plausible mistakes land far outside one step
    y = bf16_bits_to_f32(got)
    no_eps = numpy_c(a, w).astype(np.float32) * rowscale(partials, hidden, 0.0)[:, None]
    wrong_hidden = numpy_c(a, w).astype(np.float32) * rowscale(partials, 2 * hidden, eps)[:, None]
    for bad in (no_eps, wrong_hidden, numpy_c(a, w).astype(np.float32)):
        assert np.median(np.abs(y - bad) / np.maximum(np.abs(bad), 1e-3)) > 0.05


def test_store_bf16_one_hot_rows_pick_weight_columns(orc):
    """A = rows of the identity (bf16 1.0): C = W^T's rows, i.e. out[r][c] = W[c][r] (a transposed W
    would give W[r][c]); with no partials the row scale is 1."""
    k, n = 64, 96
    rng = np.random.default_rng(5)
    w = f32_to_bf16_bits(rng.standard_normal((n, k)).astype(np.float32))
    w = bf16_bits_to_f32(w)  # bf16-exact weights: the product is exact
    a = f32_to_bf16_bits(np.eye(k, dtype=np.float32)[:10])
    got = bf16_bits_to_f32(orc.qgemm(a, w, 0))
    assert np.array_equal(got, w[:, :10].T)


def test_store_f32_partial_columns(orc):
    rng = np.random.default_rng(9)
    m, n, k = 5, 320, 128
    a = randn_bf16(rng, (m, k))
    w = rng.standard_normal((n, k)).astype(np.float32)
    n_store = 200
    got = orc.qgemm(a, w, 3, n_store=n_store)
    want = numpy_c(a, w).astype(np.float32)
    ulp = np.spacing(np.abs(want[:, :n_store]))
    assert np.all(np.abs(got[:, :n_store] - want[:, :n_store]) <= ulp)
    assert not got[:, n_store:].any(), "columns past n_store written"


def test_store_f32_row_scale_closed_form(orc):
    """partials = hidden * (x - eps) per row puts the row scale at 1/sqrt(x) exactly for x = 4, 16."""
    k, n, hidden, eps = 64, 64, 256, 1e-6
    a = f32_to_bf16_bits(np.eye(k, dtype=np.float32)[:2])
    w = np.eye(n, k, dtype=np.float32)
    partials = np.zeros((2, hidden // 128), np.float32)
    partials[0, 0], partials[1, 1] = np.float32(hidden * (4.0 - eps)), np.float32(hidden * (16.0 - eps))
    got = orc.qgemm(a, w, 3, partials_in=partials, hidden=hidden, eps=eps)
    assert abs(got[0, 0] - 0.5) < 1e-6 and abs(got[1, 1] - 0.25) < 1e-6
    assert not np.delete(got[0], 0).any() and not np.delete(got[1], 1).any()


def test_residual_update_and_block_sums_of_squares(orc):
    rng = np.random.default_rng(12)
    m, n, k = 4, 384, 128
    a = randn_bf16(rng, (m, k))
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.1
    res0 = rng.standard_normal((m, n)).astype(np.float32) * 3
    res, xbf, pout = orc.qgemm(a, w, 2, residual=res0)
    want = res0 + numpy_c(a, w).astype(np.float32)
    assert np.all(np.abs(res - want) <= np.spacing(np.abs(want)))
    assert np.array_equal(xbf, f32_to_bf16_bits(res))
    blocks = (res.astype(np.float64) ** 2).reshape(m, n // 128, 128).sum(-1)
    assert np.allclose(pout, blocks, rtol=1e-6, atol=0)
    # each partial covers its own 128 columns: a spike in column 300 only moves block 2
    res1 = res0.copy()
    res1[1, 300] += 100.0
    _, _, pout1 = orc.qgemm(a, w, 2, residual=res1)
    moved = np.abs(pout1 - pout) > 1.0
    assert moved.sum() == 1 and moved[1, 2]


def test_residual_zero_weight_keeps_residual(orc):
    rng = np.random.default_rng(2)
    m, n, k = 2, 256, 64
    res0 = rng.standard_normal((m, n)).astype(np.float32)
    res, xbf, pout = orc.qgemm(randn_bf16(rng, (m, k)), np.zeros((n, k), np.float32), 2, residual=res0)
    assert np.array_equal(res, res0)
    assert np.allclose(pout, (res0.astype(np.float64) ** 2).reshape(m, 2, 128).sum(-1), rtol=1e-6)
