"""CPU check of the append kernel's exactness test for the sum of squares (csrc/append.hpp).

The reference sums x_i^2 (x bf16, 256 values) in double, left to right (src/ref/ops.cpp:79-90);
the kernel sums 4-element lane sums across the wave in the order of its cross-lane steps (lane ^ 1,
lane ^ 2, the mirror within 8 lanes, the mirror within 16, lane ^ 16, lane ^ 32) and uses that
result whenever exponent(tree) + 2 - 2 * (lowest set bit of any x_i^2 / 2) <= 53, i.e. when every
partial sum of any order fits in 53 bits. This test draws bf16 vectors with wide exponent spans and
checks that whenever the test admits a vector, the tree sum equals the left-to-right sum bit for
bit, and that it admits vectors whose exponents span more than 14 binades (where a plain span test
would have fallen back to the sequential sum)."""
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


def tree_sum(x):
    part = [sum(float(x[4 * l + e]) ** 2 for e in range(4)) for l in range(64)]  # lane order e = 0..3
    partners = [lambda l: l ^ 1, lambda l: l ^ 2, lambda l: (l & ~7) | (7 - (l & 7)),
                lambda l: (l & ~15) | (15 - (l & 15)), lambda l: l ^ 16, lambda l: l ^ 32]
    for p in partners:
        part = [part[l] + part[p(l)] for l in range(64)]
    assert len(set(part)) == 1
    return part[0]


def test_exact_sum_criteria():
    rng = np.random.default_rng(7)
    admitted_wide = 0
    for trial in range(3000):
        x = rng.normal(0, 1, 256) * np.exp2(rng.integers(-30, 4, 256) * (rng.random(256) < 0.05))
        x = bf16_round(x).astype(np.float64)
        seq = 0.0
        for v in x:
            seq = seq + v * v
        nz = [v for v in x if v != 0]
        ex = [math.frexp(v)[1] - 1 for v in nz]
        wide = max(ex) - min(ex) > 14
        tree = tree_sum(x)
        lmin = min(lowest_bit(v) for v in nz)
        ok = tree > 0 and (math.frexp(tree)[1] - 1) + 2 - 2 * lmin <= 53
        if ok:
            assert tree == seq, trial
            admitted_wide += wide
    assert admitted_wide > 0
