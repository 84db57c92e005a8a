"""CPU check of the append kernel's exactness test for the sum of squares (csrc/append.hip).

The reference sums x_i^2 (x bf16, 256 values) in double, left to right (src/ref/ops.cpp:79-90);
the kernel sums them as a 64-lane butterfly of 4-element lane sums and uses that result whenever
(a) the nonzero exponents span at most 14 binades or (b) exponent(tree) + 2 - 2 * lowest set bit
<= 53. This test draws bf16 vectors with wide exponent spans and checks that whenever either test
admits a vector, the butterfly sum equals the left-to-right sum bit for bit, and that (b) admits
vectors (a) rejects (the point of it)."""
import math

import numpy as np


def bf16_round(x):
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def lowest_bit(v):
    m, e = math.frexp(v)  # v = m 2^e, 0.5 <= |m| < 1, exact for floats
    m = abs(m)
    k = 0
    while m != int(m):
        m *= 2
        k += 1
    return e - k


def butterfly(x):
    part = [sum(float(x[4 * l + e]) ** 2 for e in range(4)) for l in range(64)]  # lane order e = 0..3
    off = 32
    while off:
        part = [part[l] + part[l ^ off] for l in range(64)]
        off >>= 1
    return part[0]


def test_exact_sum_criteria():
    rng = np.random.default_rng(7)
    admitted_b_only = 0
    for trial in range(3000):
        x = rng.normal(0, 1, 256) * np.exp2(rng.integers(-30, 4, 256) * (rng.random(256) < 0.05))
        x = bf16_round(x).astype(np.float64)
        seq = 0.0
        for v in x:
            seq = seq + v * v
        nz = [v for v in x if v != 0]
        ex = [math.frexp(v)[1] - 1 for v in nz]
        a = max(ex) - min(ex) <= 14
        tree = butterfly(x)
        lmin = min(lowest_bit(v) for v in nz)
        b = tree > 0 and (math.frexp(tree)[1] - 1) + 2 - 2 * lmin <= 53
        if a or b:
            assert tree == seq, (trial, a, b)
        if b and not a:
            admitted_b_only += 1
    assert admitted_b_only > 0
