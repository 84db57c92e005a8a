"""GPU parity of the projection GEMMs (include/q38a_gemm.h) against the oracle: q38a_qgemm with its
StoreBF16 (folded-norm row scale), StoreF32 and Residual epilogues on BQ4/5/6 weights written in the
reference's file layout and repacked by the library (reference src/kernels/qgemm.cu:285-384), and
the in-projection with the fused norm / RoPE / append, which must equal q38a_qgemm followed by
q38a_qk_norm_rope_append bit for bit (q, K/V bytes and scales, the gate columns of proj).

The oracle's double-precision product is taken over the weights the kernel path multiplies by:
  * the 256 x 256-tile kernel (large M) dequantises each weight to bf16(code x scale), the
    reference's own weight rounding, so it is checked against those weights;
  * the other kernels apply each group's scale in fp32 to the exact code sum, so they are checked
    against the exact weights code x scale (exact in fp32).
The bound is one output rounding step plus the fp32 accumulation: |d| <= ulp(ref) + 2^-18 (|A| |W'|^T)
x rs, where ulp is the bf16 (or fp32) spacing at |ref| and W' bounds the magnitude the kernel sums
(|W| for bf16 weights; 256 x scale for the offset codes 128 + u of the exact path)."""
import numpy as np
import pytest
import torch

import q38a
from q38a import gemm
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, dev, host, paged_layout, rope_dev, stream
from test_gpu_decode import build_context
from util import assert_bits_equal, bf16_bits_to_f32, f32_to_bf16_bits, randn_bf16

pytestmark = pytest.mark.gpu


def bf16_ulp(x):
    """Spacing of bf16 at |x| (2^(e - 7) for |x| in [2^e, 2^(e + 1)); the smallest normal's below)."""
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def close(got, want, what, a=None, wmag=None, rs=None, out="bf16"):
    """|got - want| <= ulp(want) + 2^-18 (|A| wmag^T) rs (see the module docstring); `out` names the
    stored type whose rounding step is allowed ("bf16" or "f32")."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = np.abs(got - want)
    ulp = bf16_ulp(want) if out == "bf16" else np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    acc = 0.0
    if a is not None:
        acc = 2.0 ** -18 * (np.abs(bf16_bits_to_f32(a).astype(np.float64)) @ np.asarray(wmag, np.float64).T)
        if rs is not None:
            acc = acc * np.asarray(rs, np.float64)[:, None]
    bound = ulp + acc
    assert np.isfinite(got).all(), f"{what}: non-finite"
    bad = d > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {d.size} outside one rounding step + accumulation; "
                           f"worst excess {float((d - bound).max()):.3g}")
    print(f"{what}: max |d| / bound {float((d / bound).max()):.3f}, max |d| / ulp {float((d / ulp).max()):.3f}",
          flush=True)


def row_scales(partials, hidden, eps=1e-6):
    p = np.asarray(partials, np.float32)
    return 1.0 / np.sqrt(p.sum(1, dtype=np.float64) / hidden + eps)


def big_path(m, n):
    """Whether q38a_qgemm takes the 256 x 256-tile kernel (bf16 weights) for m rows of n columns: its
    planner picks it when there are more than 32 rows and the tiles fill the CUs."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return m > 32 and ((m + 255) // 256) * (n // 256) >= cus


class Weight:
    """A random BQ weight [n][k]: codes and bf16 scales, the reference file planes (oracle writer),
    the library's repack on the device, and the oracle's dequantised fp32 weights."""

    def __init__(self, orc, bits, n, k, seed, scale_lo=0.002, scale_hi=0.05):
        rng = np.random.default_rng(seed)
        self.bits, self.n, self.k = bits, n, k
        codes = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), (n, k)).astype(np.int8)
        scales = f32_to_bf16_bits(rng.uniform(scale_lo, scale_hi, (n, k // 64)).astype(np.float32))
        lo, hi, sc = orc.bq_pack_file(bits, codes, scales)
        self.w_ref = orc.bq_file_weight(bits, n, k, lo, hi, sc)  # bf16(code x scale), the reference's
        scale_f32 = np.repeat(bf16_bits_to_f32(scales), 64, 1)
        self.w_exact = codes.astype(np.float32) * scale_f32  # exact in fp32 (<= 6 + 8 significant bits)
        self.w_offset_mag = 256.0 * scale_f32
        rlo, rhi, rsc = gemm.repack(bits, n, k, lo, hi, sc)
        self.t = [dev(rlo), dev(rhi) if rhi is not None else None, dev(rsc)]
        self.desc = gemm.BQWeight(self.t[0].data_ptr(), self.t[1].data_ptr() if self.t[1] is not None else None,
                                  self.t[2].data_ptr(), bits, n, k, n)


def oracle_weight(w, m):
    """(weights the kernel path for m rows multiplies by, the magnitude bound its fp32 sums carry)"""
    return (w.w_ref, np.abs(w.w_ref)) if big_path(m, w.n) else (w.w_exact, w.w_offset_mag)


def check_residual(orc, w, a, res0, res, xbf, pout, m=None):
    """The Residual epilogue against the oracle: residual within one fp32 step + accumulation, its
    bf16 copy within one bf16 step + accumulation, each 128-column sum of squares within the bound
    those residual errors imply (2 sum |r| e + one fp32 step)."""
    n = w.n
    wo, wmag = oracle_weight(w, m if m is not None else a.shape[0])
    r_want, x_want, p_want = orc.qgemm(a, wo, 2, residual=res0)
    close(res, r_want, "residual", a, wmag, out="f32")
    close(bf16_bits_to_f32(xbf), bf16_bits_to_f32(x_want), "xbf", a, wmag)
    acc = 2.0 ** -18 * (np.abs(bf16_bits_to_f32(a).astype(np.float64)) @ wmag.T.astype(np.float64))
    e = acc + np.spacing(np.abs(r_want)).astype(np.float64)
    pb = (2 * np.abs(r_want.astype(np.float64)) * e).reshape(len(r_want), n // 128, 128).sum(-1)
    pb += np.spacing(np.abs(p_want)).astype(np.float64) * 4
    d = np.abs(pout.astype(np.float64) - p_want)
    assert (d <= pb).all(), f"partials_out: {int((d > pb).sum())} outside; worst excess {float((d - pb).max()):.3g}"


def workspace(m, n, k):
    pf, nc = gemm.workspace_size(m, n, k)
    p = torch.zeros(max(pf, 1), dtype=torch.float32, device="cuda")
    c = torch.zeros(max(nc, 1), dtype=torch.int32, device="cuda")
    return gemm.GemmWorkspace(p.data_ptr(), pf, c.data_ptr(), nc), (p, c)


@pytest.mark.parametrize("bits", [4, 5, 6])
@pytest.mark.parametrize("m", [1, 8, 33, 100])
def test_qgemm_store_bf16_folded_norm(orc, bits, m):
    n, k = 512, 1024
    w = Weight(orc, bits, n, k, seed=100 + bits)
    rng = np.random.default_rng(m)
    a = randn_bf16(rng, (m, k))
    partials = rng.uniform(50.0, 200.0, (m, k // 128)).astype(np.float32)
    a_t, p_t = dev(a), dev(partials)
    out = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    ws, keep = workspace(m, n, k)
    ep = gemm.GemmEpilogue(gemm.EPI_STORE_BF16, out.data_ptr(), n, 0, None, None, None, p_t.data_ptr(), k, 1e-6)
    print(f"qgemm bf16: bits={bits} m={m} n={n} k={k}", flush=True)
    for rep in range(2):  # twice: the split-K counters must be back at zero
        gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
        torch.cuda.synchronize()
        got = bf16_bits_to_f32(host(out, np.uint16)).reshape(m, n)
        wo, wmag = oracle_weight(w, m)
        want = bf16_bits_to_f32(orc.qgemm(a, wo, 0, partials_in=partials, hidden=k))
        close(got, want, f"bits {bits} m {m} rep {rep}", a, wmag, row_scales(partials, k))


def test_qgemm_store_f32_and_partial_columns(orc):
    m, n, k = 20, 768, 512
    w = Weight(orc, 5, n, k, seed=7)
    a = randn_bf16(np.random.default_rng(3), (m, k))
    a_t = dev(a)
    out = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
    ws, keep = workspace(m, n, k)
    n_store = 700
    ep = gemm.GemmEpilogue(gemm.EPI_STORE_F32, out.data_ptr(), n, n_store, None, None, None, None, 0, 1e-6)
    gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
    torch.cuda.synchronize()
    got = host(out).reshape(m, n)
    wo, wmag = oracle_weight(w, m)
    want = orc.qgemm(a, wo, 3, n_store=n_store)
    close(got[:, :n_store], want[:, :n_store], "store f32", a, wmag[:n_store], out="f32")
    assert np.isnan(got[:, n_store:]).all()  # columns past n_store untouched


@pytest.mark.parametrize("m", [8, 70])
def test_qgemm_residual(orc, m):
    """The o-projection's epilogue: residual += C, xbf = bf16(residual), per-128-column sums of squares."""
    n, k = 1024, 6144
    w = Weight(orc, 5, n, k, seed=11)
    rng = np.random.default_rng(5)
    a = randn_bf16(rng, (m, k))
    res0 = rng.standard_normal((m, n)).astype(np.float32) * 4
    a_t, res_t = dev(a), dev(res0)
    xbf = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    pout = torch.zeros(m * n // 128, dtype=torch.float32, device="cuda")
    ws, keep = workspace(m, n, k)
    ep = gemm.GemmEpilogue(gemm.EPI_RESIDUAL, None, 0, 0, res_t.data_ptr(), xbf.data_ptr(), pout.data_ptr(), None, 0,
                           1e-6)
    gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
    torch.cuda.synchronize()
    check_residual(orc, w, a, res0, host(res_t).reshape(m, n), host(xbf, np.uint16).reshape(m, n),
                   host(pout).reshape(m, n // 128))


@pytest.mark.parametrize("bits", [4, 5, 6])
@pytest.mark.parametrize("m,kind", [(1, "bf16"), (5, "f32"), (8, "bf16"), (8, "f32")])
def test_qgemm_decode_rows_wide_tiles(orc, bits, m, kind):
    """Up to 8 rows on a weight wide enough for the 64-column-tile kernel (no split-K; the in-projection
    shape, 14,336 x 5,120): against the oracle, and bit for bit across repeated launches (its waves'
    sums are added in a fixed order)."""
    n, k = 14336, 5120
    w = Weight(orc, bits, n, k, seed=60 + bits, scale_lo=0.0005, scale_hi=0.004)
    rng = np.random.default_rng(61 + m)
    a = randn_bf16(rng, (m, k), 3.0)
    a_t = dev(a)
    ws, keep = workspace(m, n, k)
    wo, wmag = oracle_weight(w, m)
    print(f"qgemm wide tiles: bits={bits} m={m} kind={kind}", flush=True)
    outs = []
    for rep in range(3):
        if kind == "f32":
            n_store = n - 100
            out = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
            ep = gemm.GemmEpilogue(gemm.EPI_STORE_F32, out.data_ptr(), n, n_store, None, None, None, None, 0, 1e-6)
        else:
            partials = rng.uniform(2000.0, 9000.0, (m, k // 128)).astype(np.float32) if rep == 0 else partials
            p_t = dev(partials)
            out = torch.zeros(m * n, dtype=torch.int16, device="cuda")
            ep = gemm.GemmEpilogue(gemm.EPI_STORE_BF16, out.data_ptr(), n, 0, None, None, None, p_t.data_ptr(), k, 1e-6)
        gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
        torch.cuda.synchronize()
        outs.append(host(out) if kind == "f32" else host(out, np.uint16))
    for o in outs[1:]:
        assert_bits_equal(o.view(np.uint32) if kind == "f32" else o, outs[0].view(np.uint32) if kind == "f32" else outs[0],
                          "repeated launch")
    if kind == "f32":
        got = outs[0].reshape(m, n)
        want = orc.qgemm(a, wo, 3, n_store=n_store)
        close(got[:, :n_store], want[:, :n_store], "wide f32", a, wmag[:n_store], out="f32")
        assert np.isnan(got[:, n_store:]).all()
    else:
        got = bf16_bits_to_f32(outs[0]).reshape(m, n)
        want = bf16_bits_to_f32(orc.qgemm(a, wo, 0, partials_in=partials, hidden=k))
        close(got, want, "wide bf16", a, wmag, row_scales(partials, k))


@pytest.mark.parametrize("bits", [4, 5, 6])
@pytest.mark.parametrize("kind", ["bf16", "f32", "residual"])
def test_qgemm_large_m_tiles(orc, bits, kind):
    """Large M with enough 256 x 256 tiles to fill the CUs: the kernel that dequantises each weight
    group once per workgroup into bf16(code x scale). m = 1,000 leaves a partial last row tile; 24
    rows spread over all tiles are checked against the oracle."""
    m, n, k = 1000, 16384, 256
    w = Weight(orc, bits, n, k, seed=40 + bits)
    rng = np.random.default_rng(41)
    a = randn_bf16(rng, (m, k))
    a_t = dev(a)
    rows = np.linspace(0, m - 1, 24).astype(int)
    ws, keep = workspace(m, n, k)
    print(f"qgemm large m: bits={bits} kind={kind} m={m} n={n} k={k}", flush=True)
    if kind == "residual":
        res0 = rng.standard_normal((m, n)).astype(np.float32) * 4
        res_t = dev(res0)
        xbf = torch.zeros(m * n, dtype=torch.int16, device="cuda")
        pout = torch.zeros(m * n // 128, dtype=torch.float32, device="cuda")
        ep = gemm.GemmEpilogue(gemm.EPI_RESIDUAL, None, 0, 0, res_t.data_ptr(), xbf.data_ptr(), pout.data_ptr(), None,
                               0, 1e-6)
        gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
        torch.cuda.synchronize()
        check_residual(orc, w, a[rows], res0[rows], host(res_t).reshape(m, n)[rows],
                       host(xbf, np.uint16).reshape(m, n)[rows], host(pout).reshape(m, n // 128)[rows], m=m)
    elif kind == "f32":
        n_store = n - 100
        out = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
        ep = gemm.GemmEpilogue(gemm.EPI_STORE_F32, out.data_ptr(), n, n_store, None, None, None, None, 0, 1e-6)
        gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
        torch.cuda.synchronize()
        got = host(out).reshape(m, n)
        wo, wmag = oracle_weight(w, m)
        want = orc.qgemm(a[rows], wo, 3, n_store=n_store)
        close(got[rows][:, :n_store], want[:, :n_store], "store f32", a[rows], wmag[:n_store], out="f32")
        assert np.isnan(got[:, n_store:]).all()
    else:
        partials = rng.uniform(50.0, 200.0, (m, k // 128)).astype(np.float32)
        p_t = dev(partials)
        out = torch.zeros(m * n, dtype=torch.int16, device="cuda")
        ep = gemm.GemmEpilogue(gemm.EPI_STORE_BF16, out.data_ptr(), n, 0, None, None, None, p_t.data_ptr(), k, 1e-6)
        for rep in range(2):
            gemm.qgemm(a_t.data_ptr(), m, w.desc, ep, ws, stream())
            torch.cuda.synchronize()
            got = bf16_bits_to_f32(host(out, np.uint16)).reshape(m, n)
            wo, wmag = oracle_weight(w, m)
            want = bf16_bits_to_f32(orc.qgemm(a[rows], wo, 0, partials_in=partials[rows], hidden=k))
            close(got[rows], want, f"bf16 rep {rep}", a[rows], wmag, row_scales(partials[rows], k))


class InProj:
    """The attention in-projection of one layer at the model's shape: W [q | gate | k | v] (14,336 x
    5,120, bq5), hidden rows a, and a paged cache with prior context for every sequence."""

    def __init__(self, orc, seqs, seed, kv_dtype=q38a.KV_INT8, bits=5):
        self.orc = orc
        self.k = 5120
        self.n = LD
        self.w = Weight(orc, bits, self.n, self.k, seed=seed, scale_lo=0.0005, scale_hi=0.004)
        rng = np.random.default_rng(seed + 1)
        self.seqs, self.kv_dtype = seqs, kv_dtype
        self.bt, self.pages = paged_layout(rng, [p + n for p, n in seqs])
        self.pool_host = build_context(orc, rng, [p for p, _ in seqs], kv_dtype, self.bt, self.pages)
        self.b = Batch([(i, p, n) for i, (p, n) in enumerate(seqs)])
        self.m = self.b.M
        self.a = randn_bf16(rng, (self.m, self.k), 3.0)
        self.partials = rng.uniform(2000.0, 9000.0, (self.m, self.k // 128)).astype(np.float32)
        self.q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
        self.k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
        self.a_t, self.p_t = dev(self.a), dev(self.partials)
        self.qn_t, self.kn_t = dev(self.q_norm), dev(self.k_norm)
        self.rope_t = rope_dev(max(p + n for p, n in seqs) + 1)

    def run(self, fused):
        pool = Pool(self.kv_dtype, self.pages, self.bt, fill=self.pool_host)
        proj = torch.zeros(self.m * LD, dtype=torch.int16, device="cuda")
        q = torch.zeros(self.m * NQ * HD, dtype=torch.int16, device="cuda")
        ws, keep = workspace(self.m, self.n, self.k)
        ep = gemm.GemmEpilogue(gemm.EPI_STORE_BF16, proj.data_ptr(), LD, 0, None, None, None, self.p_t.data_ptr(),
                               self.k, 1e-6)
        ap = append_params(proj, self.qn_t, self.kn_t, q, self.rope_t)
        print(f"in-projection: m={self.m} fused={fused} seqs={self.seqs[:4]}", flush=True)
        if fused:
            gemm.qgemm_qkv_append(self.a_t.data_ptr(), self.m, self.w.desc, ep, ws, ap, self.b.desc, pool.desc, stream())
        else:
            gemm.qgemm(self.a_t.data_ptr(), self.m, self.w.desc, ep, ws, stream())
            q38a.qk_norm_rope_append(ap, self.b.desc, pool.desc, stream())
        torch.cuda.synchronize()
        return host(proj, np.uint16).reshape(self.m, LD), host(q, np.uint16), pool.download()


@pytest.mark.parametrize("seqs", [
    pytest.param([(130, 1), (5000, 1), (63, 1), (2000, 1), (64, 1), (700, 1), (1, 1), (9000, 1)], id="decode_b8"),
    pytest.param([(300, 200), (40, 1), (0, 64), (1000, 35)], id="mixed_300"),
    # large M: the fused call runs the 256 x 256-tile GEMM and then the append launch
    pytest.param([(3000, 2048)], id="chunk_2048"),
])
def test_in_projection_fused_append_matches_unfused(orc, seqs):
    ip = InProj(orc, seqs, seed=21)
    proj_u, q_u, pool_u = ip.run(fused=False)
    proj_f, q_f, pool_f = ip.run(fused=True)
    assert_bits_equal(q_f, q_u, "q fp16")
    assert_bits_equal(pool_f, pool_u, "pool bytes")
    gate = slice(NQ * HD, 2 * NQ * HD)
    assert_bits_equal(proj_f[:, gate], proj_u[:, gate], "gate columns of proj")
    # the unfused projection against the oracle (every row for small m, 24 rows otherwise)
    rows = np.arange(ip.m) if ip.m <= 16 else np.linspace(0, ip.m - 1, 24).astype(int)
    wo, wmag = oracle_weight(ip.w, ip.m)
    want = orc.qgemm(ip.a[rows], wo, 0, partials_in=ip.partials[rows], hidden=ip.k)
    close(bf16_bits_to_f32(proj_u[rows]), bf16_bits_to_f32(want), "in-projection vs oracle", ip.a[rows], wmag,
          row_scales(ip.partials[rows], ip.k))


@pytest.mark.parametrize("ctxs,n", [
    pytest.param([130, 5000, 63, 2000, 64, 700, 1, 9000], 5120, id="b8"),
    pytest.param([20000, 513], 5120, id="b2_long"),
    pytest.param([40 + 37 * i for i in range(40)], 1024, id="b40_merge_kernel"),
])
@pytest.mark.parametrize("in_loader", [False, True])
def test_merge_oproj_matches_decode_then_gemm(orc, ctxs, n, in_loader):
    """q38a_qgemm_merge_oproj (the merge kernel then the GEMM) equals q38a_attention_decode followed
    by q38a_qgemm on its out, bit for bit in out, residual, xbf and partials_out, and that GEMM matches
    the oracle's. q38a_qgemm_merge_oproj_in_loader (the merge inside the split-K kernel's A staging,
    or for more than 32 rows as the former) matches the oracle at the GEMM tolerance (at <= 8 rows
    the two-call path's GEMM is the wide-tile kernel, whose sums run in another order)."""
    from gpu_util import attention_params
    from util import randn_bf16
    rng = np.random.default_rng(77)
    B, max_splits = len(ctxs), 64
    bt, pages = paged_layout(rng, [c + 1 for c in ctxs])
    pool_host = build_context(orc, rng, ctxs, q38a.KV_INT8, bt, pages)
    pool = Pool(q38a.KV_INT8, pages, bt, fill=pool_host)
    b = Batch([(i, c, 1) for i, c in enumerate(ctxs)])
    proj = randn_bf16(rng, (B, LD))
    qn = dev(rng.normal(1.0, 0.1, HD).astype(np.float32))
    kn = dev(rng.normal(1.0, 0.1, HD).astype(np.float32))
    proj_t = dev(proj)
    q_t = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
    rope_t = rope_dev(max(ctxs) + 1)
    q38a.qk_norm_rope_append(append_params(proj_t, qn, kn, q_t, rope_t), b.desc, pool.desc, stream())
    w = Weight(orc, 5, n, NQ * HD, seed=31, scale_lo=0.0005, scale_hi=0.004)
    res0 = (rng.standard_normal((B, n)) * 4).astype(np.float32)
    print(f"merge_oproj: B={B} n={n} ctxs={ctxs[:8]}", flush=True)

    def run(fused):
        out_t = torch.zeros(B * NQ * HD, dtype=torch.int16, device="cuda")
        scratch_t = torch.full((q38a.split_scratch_floats(B, NQ, max_splits),), float("nan"), dtype=torch.float32,
                               device="cuda")
        attn = attention_params(q_t, proj_t, out_t, scratch_t, max_splits)
        res_t = dev(res0)
        xbf = torch.zeros(B * n, dtype=torch.int16, device="cuda")
        pout = torch.zeros(B * n // 128, dtype=torch.float32, device="cuda")
        ws, keep = workspace(B, n, NQ * HD)
        ep = gemm.GemmEpilogue(gemm.EPI_RESIDUAL, None, 0, 0, res_t.data_ptr(), xbf.data_ptr(), pout.data_ptr(), None,
                               0, 1e-6)
        if fused:
            q38a.attention_decode_partials(attn, b.desc, pool.desc, stream())
            gemm.merge_oproj(attn, b.desc, w.desc, ep, ws, stream(), in_loader=in_loader)
        else:
            q38a.attention_decode(attn, b.desc, pool.desc, stream())
            gemm.qgemm(out_t.data_ptr(), B, w.desc, ep, ws, stream())
        torch.cuda.synchronize()
        return host(res_t), host(xbf, np.uint16), host(pout), host(out_t, np.uint16)

    r_u, x_u, p_u, a_u = run(False)
    r_f, x_f, p_f, a_f = run(True)
    a = a_u.reshape(B, NQ * HD)
    if in_loader and B <= 32:
        # the merged A rows are the merge kernel's bits, but the GEMM is the split-K kernel (the
        # two-call path takes the wide-tile kernel at <= 8 rows, which sums in another order): both
        # against the oracle
        check_residual(orc, w, a, res0, r_f.reshape(B, n), x_f.reshape(B, n), p_f.reshape(B, n // 128))
    else:
        assert_bits_equal(r_f, r_u, "residual")
        assert_bits_equal(x_f, x_u, "xbf")
        assert_bits_equal(p_f, p_u, "partials_out")
        assert_bits_equal(a_f, a_u, "out")  # the merge kernel wrote out
    check_residual(orc, w, a, res0, r_u.reshape(B, n), x_u.reshape(B, n), p_u.reshape(B, n // 128))
