"""Shared helpers of the test suite: bf16/fp16 bit views and tolerance checks."""
import numpy as np


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even float32 -> bf16 bits (numpy, independent of the oracle)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def f16_bits_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def randn_bf16(rng, shape, scale=1.0):
    """bf16 bit patterns of RNE(N(0, scale^2))."""
    return f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


# Attention output tolerance of the north star (bf16 out, fp32 accumulate): max-abs 2e-3 and
# max-rel 1e-2, combined per element the way numpy.allclose combines them:
#     |got - want| <= ATOL + RTOL * |want|
# (a bf16 output has a 1-ulp step of 3.9e-3 at |y| in [0.5, 1), so a pure 2e-3 absolute bound would
# reject correctly rounded results; the relative term covers that range).
ATOL = 2e-3
RTOL = 1e-2


def check_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output ({int((~np.isfinite(got)).sum())} elements)"
    d = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = d > bound
    max_abs = float(d.max()) if d.size else 0.0
    max_rel = float((d / np.maximum(np.abs(want), atol)).max()) if d.size else 0.0
    if bad.any():
        i = np.unravel_index(np.argmax(d - bound), d.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {d.size} outside {atol} + {rtol}*|ref|; worst at {i}: "
                             f"got {got[i]:.6g} want {want[i]:.6g}; max_abs {max_abs:.3g}")
    return max_abs, max_rel


def assert_bits_equal(got, want, what=""):
    """Bitwise equality with a readable report of the first mismatches (index, got, want)."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = np.argwhere(got != want)
    if len(bad):
        show = [(tuple(int(i) for i in ix), int(got[tuple(ix)]), int(want[tuple(ix)])) for ix in bad[:12]]
        raise AssertionError(f"{what}: {len(bad)} of {got.size} differ; first (index, got, want): {show}")
