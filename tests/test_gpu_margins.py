"""Precision margins of the attention kernels away from N(0,1) data: K/V drawn at 2^-10 and 2^10
times the usual scale (int8 and bf16 pages), and a single dominant key. Outputs scale with V, so
they are compared after multiplying both sides by 1 / v_scale (a power of two: the comparison is
exact), i.e. with the north star's tolerance (max-abs 2e-3, max-rel 1e-2) applied relative to the
data's own scale; otherwise a 2^-10 output would pass any absolute bound. Both literal figures are
printed for every case.

What these probe: decode rounds P' = p * v_scale to fp16, which is subnormal for small V groups;
prefill feeds the exact K codes to the MFMA and applies the K scale to the fp32 group partials (V is
staged dequantised as fp16; bf16 pages: exact only within fp16's normal range);
large K makes the softmax nearly one-hot, so the running-max rescaling is exercised at every block.
"""
import numpy as np
import pytest

import q38a
from test_gpu_decode import decode_step
from test_gpu_ragged import ragged_step
from util import check_close

pytestmark = pytest.mark.gpu

SCALES = [
    pytest.param((2.0 ** -10, 2.0 ** -10, None), id="small_kv"),
    pytest.param((2.0 ** 10, 2.0 ** 10, None), id="large_kv"),
    pytest.param((2.0 ** 10, 2.0 ** -10, None), id="large_k_small_v"),
    pytest.param((1.0, 1.0, (37, 64.0)), id="dominant_key"),
]
DTYPES = [pytest.param(q38a.KV_INT8, id="int8"), pytest.param(q38a.KV_BF16, id="bf16"),
          pytest.param(q38a.KV_INT8_VT, id="int8_vt")]


def report(what, got, want, v_scale):
    f = 1.0 / v_scale
    lit_abs = float(np.abs(got - want).max())
    max_abs, max_rel = check_close(got * f, want * f, what=what)
    print(f"{what}: scaled max_abs {max_abs:.3g} max_rel {max_rel:.3g}; literal max_abs {lit_abs:.3g}", flush=True)


@pytest.mark.parametrize("kv_dtype", DTYPES)
@pytest.mark.parametrize("case", SCALES)
def test_decode_margins(orc, kv_dtype, case):
    k_scale, v_scale, dominant = case
    got, want = decode_step(orc, [1, 63, 700, 3000, 9000], kv_dtype, seed=71, k_scale=k_scale, v_scale=v_scale,
                            dominant=dominant, return_out=True)
    report(f"decode k{k_scale:g} v{v_scale:g} dom={dominant} dtype={kv_dtype}", got, want, v_scale)


@pytest.mark.parametrize("kv_dtype", DTYPES)
@pytest.mark.parametrize("case", SCALES)
def test_ragged_margins(orc, kv_dtype, case):
    """A split prefill chunk, an unsplit one and decode rows in one ragged launch."""
    k_scale, v_scale, dominant = case
    seqs = [(4000, 40), (9000, 1), (0, 100), (700, 1), (63, 1)]
    got, want = ragged_step(orc, seqs, seed=72, kv_dtype=kv_dtype, k_scale=k_scale, v_scale=v_scale,
                            dominant=dominant, return_out=True)
    report(f"ragged k{k_scale:g} v{v_scale:g} dom={dominant} dtype={kv_dtype}", got, want, v_scale)


@pytest.mark.parametrize("kv_dtype", DTYPES)
@pytest.mark.parametrize("case", SCALES)
@pytest.mark.parametrize("shape", ["four_wave", "eight_wave"])
def test_prefill_margins(orc, kv_dtype, case, shape):
    """The prefill launch in both workgroup shapes: 140 tokens (128-row workgroups, one per CU) and
    a 1,400-token chunk (256-row workgroups; 14 tokens spread over it are checked)."""
    from test_gpu_prefill import prefill_step
    k_scale, v_scale, dominant = case
    if shape == "four_wave":
        seqs, checks = [(4000, 40), (0, 100)], None
    else:
        seqs, checks = [(3000, 1400)], [[0, 1, 63, 64, 200, 511, 512, 700, 901, 1100, 1300, 1397, 1398, 1399]]
    got, want = prefill_step(orc, seqs, seed=73, kv_dtype=kv_dtype, check_tokens=checks, k_scale=k_scale,
                             v_scale=v_scale, dominant=dominant, return_out=True)
    report(f"prefill {shape} k{k_scale:g} v{v_scale:g} dom={dominant} dtype={kv_dtype}", got, want, v_scale)
