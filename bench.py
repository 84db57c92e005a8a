"""Benchmark of the ragged paged-KV attention step on one MI355X.

A "step" is one pass of the hot path over one batch: q/k RMSNorm + RoPE + int8 KV append of the new
tokens, then attention (split-KV decode + gated merge). The headline workload is BASELINE.json's
batch-8 ragged decode, contexts U[1024, 32768], int8 KV, one Qwen3.8 full-attention
layer (24 q heads, 4 kv heads, head_dim 256), synthetic N(0,1) data. `value` is KV GB/s: algorithmic
KV bytes of the step (every key and value of [0, ctx] read once, 2112 B per token) divided by the
step time, with all inputs resident in HBM. The KV pool is rotated among three copies so that the
256 MB Infinity Cache cannot serve a step from the previous one.

Also reported (in "extra"): the long-context decode configs 5a/5b/5c, the chunked prefill of
config 3 (separate prefill launch and through the ragged launch) and the mixed continuous-batching
step of config 4 (one 512-token chunk + 7 decode rows in one ragged launch; tokens/s = 519 / step),
and config 2 across all 16 attention layers through the native runner, as one replayed hipGraph
per step and as eager launches.

The CPU baseline is the reference's own ops.cpp attention (built from the reference sources into
oracle/_ref, single-threaded, one token at a time in double precision) on the same contexts.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "qwen3.8-27b-cuda-kernel_amd")]

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16


def time_steps(run_step, steps, warmup, rotate):
    import torch
    for i in range(warmup):
        run_step(i % rotate)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        run_step(i % rotate)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms


def time_attention_only(batch, steps, rotate):
    """Average duration of the attention launch (decode + merge kernels) alone, HIP events on the
    launch stream, over the same rotation of pools."""
    import torch
    import q38a
    s = torch.cuda.current_stream().cuda_stream
    ap = batch.attention_params()
    descs = [batch.kv_desc(i) for i in range(rotate)]
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record()
        q38a.attention_decode(ap, batch.batch, descs[i % rotate], s)
        evs[i][1].record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / steps


def measured_peaks(reps=10):
    """The ceilings this GPU reaches (include/q38a_probe.h): HBM read rate of a 4 GiB buffer with
    16-byte loads, and the fp16 MFMA issue rate of register-only MFMA chains. HIP events on the
    launch stream; the best of `reps` launches."""
    import torch
    from q38a import probe
    s = torch.cuda.current_stream().cuda_stream
    nbytes = 4 << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(4096, dtype=torch.float32, device="cuda")
    best_read = best_mfma = 0.0
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        probe.read(buf.data_ptr(), nbytes, sink.data_ptr(), 1024, s)
        b.record()
        torch.cuda.synchronize()
        best_read = max(best_read, nbytes / (a.elapsed_time(b) * 1e-3) / 1e9)
    del buf
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fl = probe.mfma(sink.data_ptr(), 2000, s)
        b.record()
        torch.cuda.synchronize()
        best_mfma = max(best_mfma, fl / (a.elapsed_time(b) * 1e-3) / 1e12)
    return {"hbm_read_gbs": round(best_read, 1), "mfma_fp16_tflops": round(best_mfma, 1)}


def read_ceiling(nbytes, launches=30):
    """The rate one launch reaches when it reads `nbytes` of contiguous device memory once (the read
    probe over three rotating buffers, so the 256 MB MALL cannot serve a launch from the previous
    one; HIP events over `launches` back-to-back launches, as the attention launches are timed). A
    decode launch reads its KV bytes once: this is its ceiling at the same size, fixed costs of a
    launch included."""
    import torch
    from q38a import probe
    s = torch.cuda.current_stream().cuda_stream
    n = (int(nbytes) + 32767) // 32768 * 32768
    bufs = [torch.ones(n, dtype=torch.uint8, device="cuda") for _ in range(3)]
    sink = torch.zeros(4096, dtype=torch.float32, device="cuda")
    for i in range(3):
        probe.read(bufs[i].data_ptr(), n, sink.data_ptr(), 1024, s)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(launches):
        probe.read(bufs[i % 3].data_ptr(), n, sink.data_ptr(), 1024, s)
    b.record()
    torch.cuda.synchronize()
    del bufs
    return n / (a.elapsed_time(b) * 1e-3 / launches) / 1e9


def decode_config(name, dtype, steps, warmup, pools=3, ctx_name=None):
    import torch
    import q38a
    from q38a.workloads import DecodeBatch, decode_contexts
    ctxs = decode_contexts(ctx_name or name)
    batch = DecodeBatch(ctxs, dtype=dtype, seed=0, pools=pools)
    s = torch.cuda.current_stream().cuda_stream
    appp, ap = batch.append_params(), batch.attention_params()
    descs = [batch.kv_desc(i) for i in range(pools)]

    def step(i):
        q38a.qk_norm_rope_append(appp, batch.batch, descs[i], s)
        q38a.attention_decode(ap, batch.batch, descs[i], s)

    ms = time_steps(step, steps, warmup, pools)
    attn_ms = time_attention_only(batch, steps, pools)
    kv = batch.kv_bytes()
    return {
        "config": name, "ctxs": ctxs, "kv_dtype": {0: "int8", 1: "bf16", 2: "int8_vt"}[dtype],
        "ms_per_step": ms, "tokens_per_s": batch.B / (ms * 1e-3),
        "kv_bytes": kv, "kv_gbs": kv / (ms * 1e-3) / 1e9,
        "attn_ms": attn_ms, "attn_gbs": (kv + batch.io_bytes()) / (attn_ms * 1e-3) / 1e9,
        "_batch": batch,
    }


def prefill_config(steps, warmup, dtype=0):
    """Config 3: one sequence appends a 2048-token chunk onto a 6000-token int8 prefix."""
    import torch
    import q38a
    from q38a.workloads import RaggedBatch
    rb = RaggedBatch([(6000, 2048)], dtype=dtype, seed=0)
    s = torch.cuda.current_stream().cuda_stream
    appp, ap, kvd = rb.append_params(), rb.attention_params(), rb.kv_desc(0)

    def step(i):
        q38a.qk_norm_rope_append(appp, rb.batch, kvd, s)
        q38a.attention_prefill(ap, rb.batch, kvd, s)

    ms = time_steps(step, steps, warmup, 1)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record()
        q38a.attention_prefill(ap, rb.batch, kvd, s)
        evs[i][1].record()
    torch.cuda.synchronize()
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / steps
    fl = rb.flops()
    return {"config": "prefill_2048_on_6000", "ms_per_step": round(ms, 5), "tokens_per_s": round(2048 / (ms * 1e-3), 1),
            "attn_ms": round(attn_ms, 5), "flops": fl, "attn_tflops": round(fl / (attn_ms * 1e-3) / 1e12, 2),
            "mfma_frac": round(fl / (attn_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)}


def ragged_config(name, seqs, steps, warmup, pools=3, dtype=0):
    """One continuous-batching step through the single ragged launch (q38a_attention_ragged):
    append of every new token, then decode rows and prefill chunks together. Config 4 is one
    512-token chunk + 7 decode rows; t_roof = decode KV bytes / HBM peak + prefill flops / MFMA peak."""
    import torch
    import q38a
    from q38a.workloads import RaggedBatch
    rb = RaggedBatch(seqs, dtype=dtype, seed=0, pools=pools)
    s = torch.cuda.current_stream().cuda_stream
    appp, ap = rb.append_params(), rb.attention_params()
    descs = [rb.kv_desc(i) for i in range(pools)]

    def step(i):
        q38a.qk_norm_rope_append(appp, rb.batch, descs[i], s)
        q38a.attention_ragged(ap, rb.batch, descs[i], s)

    ms = time_steps(step, steps, warmup, pools)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record()
        q38a.attention_ragged(ap, rb.batch, descs[i % pools], s)
        evs[i][1].record()
    torch.cuda.synchronize()
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / steps
    fl, kvb = rb.flops(), rb.decode_kv_bytes()
    t_roof = kvb / (HBM_PEAK_GBS * 1e9) + fl / (MFMA_PEAK_TFLOPS * 1e12)
    return {"config": name, "seqs": seqs, "tokens": rb.M, "ms_per_step": round(ms, 5),
            "tokens_per_s": round(rb.M / (ms * 1e-3), 1), "attn_ms": round(attn_ms, 5),
            "prefill_flops": fl, "decode_kv_bytes": kvb, "t_roof_ms": round(t_roof * 1e3, 5),
            "roof_frac": round(t_roof / (attn_ms * 1e-3), 4)}


def random_bq_weight(n, k, bits, gen):
    """Random weights of the in-projection's shape in the q38a BQ layout, on the device (every byte
    pattern is a valid code; scales ~ U[0.0005, 0.004] in bf16)."""
    import torch
    from q38a import gemm
    nl, nh, ns = gemm.repacked_bytes(bits, n, k)
    lo = torch.randint(0, 256, (nl,), dtype=torch.uint8, device="cuda", generator=gen)
    hi = torch.randint(0, 256, (nh,), dtype=torch.uint8, device="cuda", generator=gen) if nh else None
    sc = (torch.rand(ns // 2, device="cuda", generator=gen) * 0.0035 + 0.0005).to(torch.bfloat16)
    keep = (lo, hi, sc)
    w = gemm.BQWeight(lo.data_ptr(), hi.data_ptr() if hi is not None else None, sc.data_ptr(), bits, n, k, n)
    return w, keep, nl + nh + ns


INPROJ_COPIES = 8  # 8 x 48 MB of weights: more than the 256 MB MALL, as 16 layers' weights are


def inproj_setup(name):
    """The attention layer's in-projection (W [q | gate | k | v] = 14,336 x 5,120, bq5 as the reference
    model stores it, reference docs/FORMAT.md 1.3) on the decode batch of config 2 (M = 8) or the
    prefill chunk of config 3 (M = 2,048). Launch i uses weight copy i % INPROJ_COPIES, so weights
    stream from HBM as a step's different layers do. Returns (gemm(i), gemm + append(i), fused(i),
    facts)."""
    import torch
    import q38a
    from q38a import gemm
    from q38a.workloads import LD, DecodeBatch, RaggedBatch, decode_contexts
    s = torch.cuda.current_stream().cuda_stream
    gen = torch.Generator(device="cuda").manual_seed(0)
    b = DecodeBatch(decode_contexts("decode_b8"), seed=0) if name.endswith("b8") else RaggedBatch([(6000, 2048)], seed=0)
    m = b.batch.num_tokens
    K, bits = 5120, 5
    ws_ = [random_bq_weight(LD, K, bits, gen) for _ in range(INPROJ_COPIES)]
    wbytes = ws_[0][2]
    a = torch.randn((m, K), generator=gen, device="cuda").to(torch.bfloat16)
    partials = torch.rand((m, K // 128), generator=gen, device="cuda") * 100 + 50
    pf, nc = gemm.workspace_size(m, LD, K)
    wsp = torch.zeros(max(pf, 1), dtype=torch.float32, device="cuda")
    wsc = torch.zeros(max(nc, 1), dtype=torch.int32, device="cuda")
    ws = gemm.GemmWorkspace(wsp.data_ptr(), pf, wsc.data_ptr(), nc)
    ep = gemm.GemmEpilogue(gemm.EPI_STORE_BF16, b.proj.data_ptr(), LD, 0, None, None, None, partials.data_ptr(), K,
                           1e-6)
    ap, kvd = b.append_params(), b.kv_desc(0)
    keep = (b, ws_, a, partials, wsp, wsc)
    W = lambda i: ws_[i % INPROJ_COPIES][0]  # noqa: E731
    run_gemm = lambda i: gemm.qgemm(a.data_ptr(), m, W(i), ep, ws, s)  # noqa: E731
    run_unfused = lambda i: (gemm.qgemm(a.data_ptr(), m, W(i), ep, ws, s),  # noqa: E731
                             q38a.qk_norm_rope_append(ap, b.batch, kvd, s))
    run_fused = lambda i: gemm.qgemm_qkv_append(a.data_ptr(), m, W(i), ep, ws, ap, b.batch, kvd, s)  # noqa: E731
    return run_gemm, run_unfused, run_fused, {"m": m, "n": LD, "k": K, "bits": bits, "weight_bytes": wbytes,
                                              "keep": keep}


def inproj_config(name, steps, warmup):
    """The in-projection (inproj_setup) timed three ways: the GEMM alone, GEMM + append (two
    launches, proj written and re-read), and the fused launch (q38a_qgemm_qkv_append)."""
    import torch
    run_gemm, run_unfused, run_fused, f = inproj_setup(name)

    def timed(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    t_gemm, t_unfused, t_fused = timed(run_gemm), timed(run_unfused), timed(run_fused)
    m, n, k, wbytes = f["m"], f["n"], f["k"], f["weight_bytes"]
    flops = 2.0 * m * n * k
    return {"config": name, "m": m, "n": n, "k": k, "bits": f["bits"], "weight_bytes": wbytes,
            "weight_copies": INPROJ_COPIES,
            "gemm_ms": round(t_gemm, 5), "gemm_plus_append_ms": round(t_unfused, 5), "fused_ms": round(t_fused, 5),
            "gemm_weight_gbs": round(wbytes / (t_gemm * 1e-3) / 1e9, 1),
            "gemm_tflops": round(flops / (t_gemm * 1e-3) / 1e12, 2),
            "fused_tflops": round(flops / (t_fused * 1e-3) / 1e12, 2)}


OPROJ_COPIES = 14  # 14 x 20 MB of o-projection weights: more than the 256 MB MALL


def oproj_setup(name):
    """The attention layer's tail on a decode step (config 2 contexts for "o_proj_b8", 5a for
    "o_proj_long_b8"): split attention, then the o-projection (W_o 5,120 x 6,144, bq5) with the
    residual epilogue. Returns (unfused(i), in_loader(i), gemm_only(i), facts). Unfused:
    q38a_attention_decode (split kernel + merge kernel writing out), then q38a_qgemm on out (what the
    default q38a_qgemm_merge_oproj runs). In-loader: q38a_attention_decode_partials, then
    q38a_qgemm_merge_oproj_in_loader (the merge inside the GEMM's A staging). Launch i uses KV pool
    i % 3 and weight copy i % OPROJ_COPIES."""
    import torch
    import q38a
    from q38a import gemm
    from q38a.workloads import DecodeBatch, decode_contexts
    s = torch.cuda.current_stream().cuda_stream
    ctx_name = "long_b8" if "long" in name else "decode_b8"
    b = DecodeBatch(decode_contexts(ctx_name), seed=0, pools=3)
    gen = torch.Generator(device="cuda").manual_seed(1)
    n, K, B = 5120, 6144, b.B
    ws_ = [random_bq_weight(n, K, 5, gen) for _ in range(OPROJ_COPIES)]
    res = torch.randn((B, n), generator=gen, device="cuda")
    xbf = torch.empty((B, n), dtype=torch.bfloat16, device="cuda")
    pout = torch.empty((B, n // 128), dtype=torch.float32, device="cuda")
    pf, nc = gemm.workspace_size(B, n, K)
    wsp = torch.zeros(max(pf, 1), dtype=torch.float32, device="cuda")
    wsc = torch.zeros(max(nc, 1), dtype=torch.int32, device="cuda")
    ws = gemm.GemmWorkspace(wsp.data_ptr(), pf, wsc.data_ptr(), nc)
    ep = gemm.GemmEpilogue(gemm.EPI_RESIDUAL, None, 0, 0, res.data_ptr(), xbf.data_ptr(), pout.data_ptr(), None, 0,
                           1e-6)
    ap, descs = b.attention_params(), [b.kv_desc(i) for i in range(3)]
    q38a.qk_norm_rope_append(b.append_params(), b.batch, descs[0], s)

    def unfused(i):
        q38a.attention_decode(ap, b.batch, descs[i % 3], s)
        gemm.qgemm(b.out.data_ptr(), B, ws_[i % OPROJ_COPIES][0], ep, ws, s)

    def fused(i):
        q38a.attention_decode_partials(ap, b.batch, descs[i % 3], s)
        gemm.merge_oproj(ap, b.batch, ws_[i % OPROJ_COPIES][0], ep, ws, s, in_loader=True)

    def gemm_only(i):
        gemm.qgemm(b.out.data_ptr(), B, ws_[i % OPROJ_COPIES][0], ep, ws, s)

    return unfused, fused, gemm_only, {"B": B, "n": n, "k": K, "keep": (b, ws_, res, xbf, pout, wsp, wsc)}


def oproj_config(name, steps, warmup):
    """oproj_setup's three ways, timed with HIP events."""
    import torch
    unfused, fused, gemm_only, f = oproj_setup(name)
    B, n, K = f["B"], f["n"], f["k"]

    def timed(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    t_u, t_f, t_g = timed(unfused), timed(fused), timed(gemm_only)
    return {"config": name, "B": B, "n": n, "k": K, "bits": 5, "weight_copies": OPROJ_COPIES,
            "attention_plus_oproj_ms": round(t_u, 5), "in_loader_merge_oproj_ms": round(t_f, 5),
            "oproj_gemm_only_ms": round(t_g, 5), "in_loader_saved_ms": round(t_u - t_f, 5),
            "default": "merge kernel then GEMM (q38a_qgemm_merge_oproj)"}


def runner_decode_config(steps, warmup, layers=16, ctxs=None, name="decode_b8_16_layers_runner"):
    """A decode step across all 16 full-attention layers through the native runner
    (include/q38a_runtime.h): one hipGraph per batch bucket (metadata upload + append + decode +
    merge for every layer, 48 kernels), replayed, against the same step launched eagerly. Default:
    config 2's batch, whose KV over 16 layers (3.2 GB) is far larger than the 256 MB MALL; `ctxs`
    gives another batch (one short row shows what the graph saves when kernels are short)."""
    import torch
    import q38a
    from q38a.runtime import Runner
    from q38a.workloads import INT8_TOKEN_BYTES, LD, decode_contexts
    ctxs = list(ctxs) if ctxs is not None else decode_contexts("decode_b8")
    pages = sum((c + 1 + 63) // 64 for c in ctxs)
    gen = torch.Generator(device="cuda").manual_seed(0)
    qn = (1.0 + 0.1 * torch.randn(layers * 256, generator=gen, device="cuda")).float()
    kn = (1.0 + 0.1 * torch.randn(layers * 256, generator=gen, device="cuda")).float()
    r = Runner(qn.data_ptr(), kn.data_ptr(), kv_dtype=q38a.KV_INT8, attn_layers=layers, num_pages=pages + 8,
               max_batch=8, max_chunk=64, max_context=32832, max_splits=256, use_graphs=True)
    for slot, c in enumerate(ctxs):
        assert r.ensure(slot, c + 1)
    # random pool bytes and projection rows (synthetic): the pool through its device address
    d = r.kv_desc()
    pool = torch.empty(d.layer_stride * layers, dtype=torch.uint8, device="cuda")
    pool.random_(0, 256, generator=gen)
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    # int8 codes are any byte; scales must be finite fp16: write N(0,1)/127-sized scales
    view = pool.view(layers * d.num_pages, d.page_bytes)
    sc = (torch.rand((layers * d.num_pages, 2 * 4 * 64 * 4), generator=gen, device="cuda") * 0.02 + 0.005)
    view[:, 2 * 4 * 64 * 256:] = sc.to(torch.float16).view(torch.uint8).reshape(layers * d.num_pages, -1)
    torch.cuda.synchronize()
    assert hip.hipMemcpy(d.pool, pool.data_ptr(), pool.numel(), 4) == 0
    b = r.buffers
    proj = torch.randn((layers, b.rows, LD), generator=gen, device="cuda").to(torch.bfloat16)
    assert hip.hipMemcpy(b.proj, proj.data_ptr(), proj.numel() * 2, 4) == 0
    del pool, proj
    s = torch.cuda.current_stream().cuda_stream
    rows = [(slot, c) for slot, c in enumerate(ctxs)]
    out = {}
    for mode in ("graph", "eager"):
        r.set_graphs(mode == "graph")
        for _ in range(warmup):
            r.decode(rows, s)
        torch.cuda.synchronize()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            r.decode(rows, s)
        e.record()
        torch.cuda.synchronize()
        out[mode] = a.elapsed_time(e) / steps
        # host time to issue one step (the previous step has finished, so nothing waits): what the
        # calling thread spends per step, free for scheduling while the GPU runs the step
        t_issue = 0.0
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            r.decode(rows, s)
            t_issue += time.perf_counter() - t0
        torch.cuda.synchronize()
        out[mode + "_issue"] = t_issue / steps * 1e6
    kv = layers * sum(c + 1 for c in ctxs) * INT8_TOKEN_BYTES
    r.close()
    return {"config": name, "ctxs": ctxs, "layers": layers, "graph_ms": round(out["graph"], 5),
            "eager_ms": round(out["eager"], 5), "graph_host_issue_us": round(out["graph_issue"], 1),
            "eager_host_issue_us": round(out["eager_issue"], 1), "kv_bytes": kv,
            "graph_kv_gbs": round(kv / (out["graph"] * 1e-3) / 1e9, 1),
            "graph_tokens_per_s": round(len(ctxs) / (out["graph"] * 1e-3), 1)}


def profile_workload(name, reps=20):
    """The launches the rocprofv3 summaries under profiles/ are made from: 3 warm-up and `reps`
    timed attention launches of one workload, then 4 passes of a plain copy kernel over known bytes
    (y = -x on 1 GiB of fp32: 1 GiB read, 1 GiB written; no workload uses neg) that calibrate FETCH_SIZE and
    WRITE_SIZE. Prints one line per phase."""
    import torch
    import q38a
    from q38a.workloads import DecodeBatch, RaggedBatch, decode_contexts, mixed_seqs
    s = torch.cuda.current_stream().cuda_stream
    vt = name.endswith("_int8_vt")  # the same workload on int8 VT pages
    base = name[:-len("_int8_vt")] if vt else name
    if base in ("decode_b8", "long_b8", "long_b1", "long_b8_bf16"):
        dt = q38a.KV_INT8_VT if vt else (q38a.KV_BF16 if base.endswith("bf16") else q38a.KV_INT8)
        b = DecodeBatch(decode_contexts(base), dtype=dt, seed=0, pools=3)
        ap, descs = b.attention_params(), [b.kv_desc(i) for i in range(3)]
        q38a.qk_norm_rope_append(b.append_params(), b.batch, descs[0], s)
        run = lambda i: q38a.attention_decode(ap, b.batch, descs[i % 3], s)  # noqa: E731
    elif base == "prefill":
        rb = RaggedBatch([(6000, 2048)], dtype=q38a.KV_INT8_VT if vt else q38a.KV_INT8, seed=0)
        ap, kvd = rb.attention_params(), rb.kv_desc(0)
        q38a.qk_norm_rope_append(rb.append_params(), rb.batch, kvd, s)
        run = lambda i: q38a.attention_prefill(ap, rb.batch, kvd, s)  # noqa: E731
    elif base == "prefill_ragged":
        rb = RaggedBatch([(6000, 2048)], dtype=q38a.KV_INT8_VT if vt else q38a.KV_INT8, seed=0)
        ap, kvd = rb.attention_params(), rb.kv_desc(0)
        q38a.qk_norm_rope_append(rb.append_params(), rb.batch, kvd, s)
        run = lambda i: q38a.attention_ragged(ap, rb.batch, kvd, s)  # noqa: E731
    elif base in ("in_proj_b8", "in_proj_2048"):
        run, _, _, keep = inproj_setup(base)
    elif base in ("o_proj_b8", "o_proj_b8_fused"):
        unfused, fused, _, keep = oproj_setup("o_proj_b8")
        run = fused if base.endswith("fused") else unfused
    elif base == "mixed":
        rb = RaggedBatch(mixed_seqs(0), dtype=q38a.KV_INT8_VT if vt else q38a.KV_INT8, seed=0, pools=3)
        ap, descs = rb.attention_params(), [rb.kv_desc(i) for i in range(3)]
        q38a.qk_norm_rope_append(rb.append_params(), rb.batch, descs[0], s)
        run = lambda i: q38a.attention_ragged(ap, rb.batch, descs[i % 3], s)  # noqa: E731
    else:
        raise SystemExit(f"unknown profile workload {name}")
    for i in range(3):
        run(i)
    torch.cuda.synchronize()
    for i in range(reps):
        run(i)
    torch.cuda.synchronize()
    print(f"profile {name}: {reps} attention launches", flush=True)
    x = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(4):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print("profile copy: 4 x (1 GiB read + 1 GiB written)", flush=True)
    del x, y
    from q38a import probe
    sink = torch.zeros(4096, dtype=torch.float32, device="cuda")
    for _ in range(2):
        probe.mfma(sink.data_ptr(), 2000, s)
    torch.cuda.synchronize()
    print("profile mfma probe: 2 launches (MFMA-busy calibration)", flush=True)


def _csv_rows(d, suffix):
    import csv
    import glob
    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        rows += list(csv.DictReader(open(f)))
    if not rows:
        raise SystemExit(f"no *{suffix} under {d}")
    return rows


def pmc_summary(fetch_dir, write_dir, out=None):
    """Per-kernel mean FETCH_SIZE / WRITE_SIZE (KiB per dispatch) from two rocprofv3 --pmc runs of
    `bench.py --profile`, scaled by what the same counters read for the 1 GiB copy kernel."""
    import collections
    vals = collections.defaultdict(list)
    for d, counter in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        for r in _csv_rows(d, "counter_collection.csv"):
            if r["Counter_Name"] == counter:
                vals[(r["Kernel_Name"], counter)].append(float(r["Counter_Value"]))
    names = sorted({k for k, _ in vals})
    copy = [n for n in names if "neg_kernel" in n]
    if not copy:
        raise SystemExit("copy kernel not found")
    gib_kib = float(1 << 20)
    cf = gib_kib / (sum(vals[(copy[0], "FETCH_SIZE")]) / len(vals[(copy[0], "FETCH_SIZE")]))
    cw = gib_kib / (sum(vals[(copy[0], "WRITE_SIZE")]) / len(vals[(copy[0], "WRITE_SIZE")]))
    lines = [f"copy kernel: {copy[0][:80]}", f"scale FETCH_SIZE x {cf:.4f}, WRITE_SIZE x {cw:.4f} (1 GiB each way)",
             "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | scaled read MB | scaled write MB |",
             "|---|---|---|---|---|---|"]
    total = 0.0  # the attention launch: q38a attention and merge kernels
    for n in names:
        if n in copy or not short_name(n).startswith("q38a::"):
            continue
        f, w = vals.get((n, "FETCH_SIZE"), [0.0]), vals.get((n, "WRITE_SIZE"), [0.0])
        fm, wm = sum(f) / len(f), sum(w) / len(w)
        rb, wb = fm * 1024 * cf, wm * 1024 * cw
        if short_name(n).startswith("q38a::attn_"):
            total += rb + wb
        lines.append(f"| {short_name(n)} | {len(f)} | {fm:.0f} | {wm:.0f} | {rb / 1e6:.2f} | {wb / 1e6:.2f} |")
    lines.append(f"traffic_bytes_per_launch: {total:.0f}")
    text = "\n".join(lines)
    print(text)
    if out:
        open(out, "w").write(text + "\n")


def mfma_summary(d, out=None, simds=1024):
    """MFMA utilisation per kernel from a rocprofv3 --pmc run of SQ_VALU_MFMA_BUSY_CYCLES,
    GRBM_GUI_ACTIVE and SQ_INSTS_VALU_MFMA_MOPS_F16 over `bench.py --profile`: busy fraction =
    sum of MFMA-busy cycles over all SIMDs / (GPU-active cycles x SIMDs) (rocprofv3's own MFMA_UTIL
    expression), and the fp16 flops the MFMAs did (MOPS x 512). The MFMA probe kernel, which does
    nothing but MFMAs, gives the fraction that counts as fully busy."""
    import collections
    per = collections.defaultdict(lambda: collections.defaultdict(lambda: collections.defaultdict(float)))
    for r in _csv_rows(d, "counter_collection.csv"):
        k = r["Kernel_Name"]
        disp = r.get("Dispatch_Id") or r.get("Correlation_Id") or "0"
        name = r["Counter_Name"]
        v = float(r["Counter_Value"])
        if name == "GRBM_GUI_ACTIVE":
            per[k][disp][name] = max(per[k][disp][name], v)
        else:
            per[k][disp][name] += v
    rows = []
    for k, disps in per.items():
        util = [x["SQ_VALU_MFMA_BUSY_CYCLES"] / (x["GRBM_GUI_ACTIVE"] * simds) for x in disps.values()
                if x["GRBM_GUI_ACTIVE"] > 0]
        fl = [x["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512 for x in disps.values()]
        if util:
            rows.append((short_name(k), len(util), sum(util) / len(util), sum(fl) / len(fl)))
    probe = [r for r in rows if "mfma_probe" in r[0]]
    ref = probe[0][2] if probe else None
    lines = [f"mfma probe busy fraction (calibration, counts as 1.0): {ref:.4f}" if ref else "no probe",
             "| kernel | dispatches | MFMA busy (raw) | MFMA busy / probe | fp16 MFMA flops per dispatch |",
             "|---|---|---|---|---|"]
    for name, n, u, f in sorted(rows):
        if not name.startswith("q38a::"):
            continue
        lines.append(f"| {name} | {n} | {u:.4f} | {u / ref if ref else float('nan'):.4f} | {f:.4g} |")
    text = "\n".join(lines)
    print(text)
    if out:
        open(out, "w").write(text + "\n")


def short_name(n):
    n = n.replace("(anonymous namespace)::", "").replace("void ", "")
    return n.split("(")[0][:80]


def stats_summary(d):
    """Kernel table of a rocprofv3 --kernel-trace --stats run (average durations in microseconds)."""
    rows = _csv_rows(d, "kernel_stats.csv")
    print("| kernel | calls | average us | min us | max us | share % |")
    print("|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {short_name(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")


def read_traffic(workload):
    """Scaled HBM bytes per attention launch from profiles/<workload>_traffic.txt, or None."""
    path = os.path.join(ROOT, "profiles", f"attention_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":")[1])
    return None


def read_mfma_busy():
    """MFMA busy fraction (relative to the probe) of the attention kernel of the prefill and mixed
    workloads, from profiles/attention_<workload>_mfma.txt, or {}."""
    out = {}
    for w, kern in (("prefill", "attn_prefill"), ("mixed", "attn_ragged_kernel")):
        path = os.path.join(ROOT, "profiles", f"attention_{w}_mfma.txt")
        if not os.path.exists(path):
            continue
        for line in open(path):
            cells = [c.strip() for c in line.split("|")]
            if len(cells) > 4 and kern in cells[1]:
                out[w] = float(cells[4])
    return out


def cpu_sample(batch, picks, budget_s, cores):
    """The oracle's C port of the reference's CPU attention (src/ref/ops.cpp:144-171, one query
    token over its whole causal context, all 24 q heads) on picked query rows of a workload batch
    whose append has run on the GPU, reading the batch's own pages. picks: [(row m, sequence b,
    position)]. Each row is cut into its 4 kv heads (independent jobs); rows are timed one after
    another on one thread until budget_s is spent, then the same rows are timed again spread over
    `cores` threads (ctypes releases the GIL). Returns the sample's figures."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle.oracle import Oracle
    orc = Oracle()
    pool = batch.pools[0].cpu().numpy()
    q = batch.q16.cpu().float().numpy().reshape(-1, 24 * 256)
    gate = batch.proj.cpu().float().numpy()[:, 24 * 256:48 * 256]
    kv = {}
    for _, b, pos in picks:
        kv[b] = max(kv.get(b, 0), pos + 1)
    kv = {b: orc.read_back(pool, batch.dtype, 4, batch.block_table, b, L) for b, L in kv.items()}

    def jobs_of(m, b, pos):
        k, v = kv[b]
        return [lambda h=h: orc.attention_token(q[m, 1536 * h:1536 * (h + 1)], gate[m, 1536 * h:1536 * (h + 1)], pos,
                                                 k[h:h + 1, :pos + 1], v[h:h + 1, :pos + 1], 6, 1)
                for h in range(4)]

    done, spent, keys = [], 0.0, 0
    for m, b, pos in picks:
        jobs = jobs_of(m, b, pos)
        t0 = time.perf_counter()
        for f in jobs:
            f()
        spent += time.perf_counter() - t0
        done.append(jobs)
        keys += pos + 1
        if spent > budget_s:
            break
    flat = [f for jobs in done for f in jobs]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(cores) as ex:
        list(ex.map(lambda f: f(), flat))
    wall = time.perf_counter() - t0
    per = 4096 if batch.dtype == 1 else 2112
    n = len(done)
    return {"rows": n, "of_picks": len(picks), "kv_tokens": keys, "s_1core": round(spent, 3),
            "tokens_per_s_1core": round(n / spent, 3), "kv_gbs_1core": round(keys * per / spent / 1e9, 4),
            "s_all_cores": round(wall, 3), "cores": cores, "tokens_per_s_all_cores": round(n / wall, 3),
            "kv_gbs_all_cores": round(keys * per / wall / 1e9, 4),
            "tflops_all_cores": round(keys * 4 * 256 * 24 / wall / 1e12, 6)}


def cpu_baselines(head_batch):
    """The reference CPU path timed on the host for every BASELINE config, on bounded samples (about
    15 s of single-thread work in all); the headline cpu_baseline is config 2 (the bench workload),
    all host cores."""
    import numpy as np
    import torch
    import q38a
    from q38a.workloads import DecodeBatch, RaggedBatch, decode_contexts, mixed_seqs
    cores = len(os.sched_getaffinity(0))
    s = torch.cuda.current_stream().cuda_stream
    out = {}

    def appended(b):
        q38a.qk_norm_rope_append(b.append_params(), b.batch, b.kv_desc(0), s)
        torch.cuda.synchronize()
        return b

    c1 = appended(DecodeBatch([130], seed=0))
    r = cpu_sample(c1, [(0, 0, 130)] * 200, 2.0, cores)
    r["sample"] = "config 1: one decode token at context 130, repeated 200 times"
    out["config1_decode_ctx130"] = r
    r = cpu_sample(head_batch, [(b, b, c) for b, c in sorted(enumerate(head_batch.ctxs), key=lambda x: x[1])],
                   8.0, cores)
    r["sample"] = "config 2: the bench's 8 decode rows, shortest first"
    out["config2_decode_b8"] = r
    c3 = appended(RaggedBatch([(6000, 2048)], seed=0))
    toks = np.linspace(0, 2047, 48).astype(int)
    r = cpu_sample(c3, [(int(t), 0, 6000 + int(t)) for t in toks], 4.0, cores)
    pick_keys = [6001 + int(t) for t in toks[:r["rows"]]]
    scale = sum(6001 + t for t in range(2048)) / sum(pick_keys)
    r["est_full_chunk_s_1core"] = round(r["s_1core"] * scale, 2)
    r["est_full_chunk_s_all_cores"] = round(r["s_all_cores"] * scale, 2)
    r["sample"] = f"config 3: {r['rows']} of the chunk's 2,048 tokens, evenly spaced; full chunk scaled by keys"
    out["config3_prefill_2048_on_6000"] = r
    seqs = mixed_seqs(0)
    c4 = appended(RaggedBatch(seqs, seed=0))
    starts = np.cumsum([0] + [n for _, n in seqs])
    pb = [b for b, (_, n) in enumerate(seqs) if n > 1][0]
    p0, n0 = seqs[pb]
    dec = [(int(starts[b]), b, p) for b, (p, n) in enumerate(seqs) if n == 1]
    pre = [(int(starts[pb]) + int(t), pb, p0 + int(t)) for t in np.linspace(0, n0 - 1, 32).astype(int)]
    r = cpu_sample(c4, dec + pre, 6.0, cores)
    full_keys = sum(p + 1 for p, n in seqs if n == 1) + sum(p0 + t + 1 for t in range(n0))
    sampled_keys = r["kv_tokens"]
    r["est_full_step_s_1core"] = round(r["s_1core"] * full_keys / sampled_keys, 2)
    r["est_full_step_s_all_cores"] = round(r["s_all_cores"] * full_keys / sampled_keys, 2)
    r["sample"] = (f"config 4: the 7 decode rows and {max(0, r['rows'] - len(dec))} of the chunk's {n0} tokens; "
                   "full step scaled by keys")
    out["config4_mixed_512_plus_7"] = r
    c5 = appended(DecodeBatch(decode_contexts("long_b8"), seed=0))
    r = cpu_sample(c5, [(b, b, c) for b, c in sorted(enumerate(c5.ctxs), key=lambda x: x[1])], 6.0, cores)
    r["sample"] = "config 5a: the 8 decode rows (contexts sum 204,800), shortest first"
    out["config5a_long_b8"] = r
    h = out["config2_decode_b8"]
    return {"value": h["kv_gbs_all_cores"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"config 2 decode rows: {h['rows']} of 8, {h['kv_tokens']} KV tokens, one attention layer, "
                      f"{h['s_all_cores']} s on {cores} threads (one job per row and kv head)",
            "tokens_per_s": h["tokens_per_s_all_cores"],
            "single_core": {"value": h["kv_gbs_1core"], "tokens_per_s": h["tokens_per_s_1core"], "s": h["s_1core"]},
            "host": {"nproc": cores, "cpu": cpu_model()},
            "configs": out}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of extra configs to run (default: all; "
                                                "'headline' runs none)")
    ap.add_argument("--profile", default="", help="run one workload's launches for rocprofv3 and exit")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--pmc-out", default=None)
    ap.add_argument("--stats-summary", metavar="DIR")
    ap.add_argument("--mfma-summary", metavar="DIR")
    args = ap.parse_args()
    if args.mfma_summary:
        return mfma_summary(args.mfma_summary, out=args.pmc_out)
    if args.pmc_summary:
        return pmc_summary(*args.pmc_summary, out=args.pmc_out)
    if args.stats_summary:
        return stats_summary(args.stats_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the single-GPU number is the reported value.", file=sys.stderr)
        sys.exit(2)

    import torch
    import q38a
    torch.cuda.init()
    if args.profile:
        return profile_workload(args.profile)
    only = set(filter(None, args.only.split(",")))
    extra = {}
    head = decode_config("decode_b8", q38a.KV_INT8, args.steps, args.warmup)
    for name, dt, cn in (("long_b8", q38a.KV_INT8, None), ("long_b1", q38a.KV_INT8, None),
                         ("long_b8_bf16", q38a.KV_BF16, None), ("decode_b8_int8_vt", q38a.KV_INT8_VT, "decode_b8"),
                         ("long_b8_int8_vt", q38a.KV_INT8_VT, "long_b8")):
        if only and name not in only:
            continue
        r = decode_config(name, dt, args.steps, args.warmup, ctx_name=cn)
        r.pop("_batch")
        r["hbm_frac"] = r["attn_gbs"] / HBM_PEAK_GBS
        extra[name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items() if k != "ctxs"}
        extra[name]["sum_ctx"] = sum(r["ctxs"])
    if not only or "prefill" in only:
        extra["prefill_2048_on_6000"] = prefill_config(max(10, args.steps // 5), 3)
    if not only or "prefill_int8_vt" in only:
        extra["prefill_2048_on_6000_int8_vt"] = prefill_config(max(10, args.steps // 5), 3, dtype=q38a.KV_INT8_VT)
    if not only or "mixed" in only:
        from q38a.workloads import mixed_seqs
        extra["mixed_512_plus_7"] = ragged_config("mixed_512_plus_7", mixed_seqs(0), max(10, args.steps // 2), 3)
    if not only or "mixed_int8_vt" in only:
        from q38a.workloads import mixed_seqs
        extra["mixed_512_plus_7_int8_vt"] = ragged_config("mixed_512_plus_7_int8_vt", mixed_seqs(0),
                                                          max(10, args.steps // 2), 3, dtype=q38a.KV_INT8_VT)
    if not only or "runner" in only:
        extra["decode_b8_16_layers_runner"] = runner_decode_config(max(10, args.steps // 5), 3)
        extra["decode_b1_short_16_layers_runner"] = runner_decode_config(max(10, args.steps // 5), 3, ctxs=[500],
                                                                         name="decode_b1_short_16_layers_runner")
    for name in ("in_proj_b8", "in_proj_2048"):
        if not only or name in only:
            extra[name] = inproj_config(name, max(10, args.steps // 5), 3)
    for name in ("o_proj_b8", "o_proj_long_b8"):
        if not only or name in only:
            extra[name] = oproj_config(name, max(10, args.steps // 5), 3)
    if not only or "prefill_ragged" in only:
        extra["prefill_2048_on_6000_ragged"] = ragged_config("prefill_2048_on_6000_ragged", [(6000, 2048)],
                                                             max(10, args.steps // 5), 3, pools=1)
    peaks = measured_peaks()
    for r in extra.values():
        if "attn_gbs" in r:
            r["hbm_frac_of_measured"] = round(r["attn_gbs"] / peaks["hbm_read_gbs"], 4)
            if "kv_bytes" in r and str(r.get("config", "")).startswith("long"):
                ceil = read_ceiling(r["kv_bytes"])
                r["same_bytes_read_ceiling_gbs"] = round(ceil, 1)
                r["frac_of_same_bytes_ceiling"] = round(r["attn_gbs"] / ceil, 4)
        if "attn_tflops" in r:
            r["mfma_frac_of_measured"] = round(r["attn_tflops"] / peaks["mfma_fp16_tflops"], 4)
    # MFMA-pipe busy fractions need hardware counters (rocprofv3 --pmc around this script), so they
    # are read from the committed profile summaries and labelled as such
    busy = read_mfma_busy()
    for w, key in (("prefill", "prefill_2048_on_6000"), ("mixed", "mixed_512_plus_7")):
        if busy.get(w) is not None and key in extra:
            extra[key]["mfma_busy_frac_from_profile"] = busy[w]
            extra[key]["mfma_busy_source"] = f"profiles/attention_{w}_mfma.txt (rocprofv3 --pmc, not this run)"
    head_ceiling = read_ceiling(head["kv_bytes"])
    batch = head.pop("_batch")
    cpu = None if args.no_cpu else cpu_baselines(batch)
    line = {
        "metric": "decode-attn KV GB/s (% HBM peak) + mixed-batch step tokens/s, batch 8",
        "value": round(head["kv_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: N(0,1) bf16 q/k/v/gate, prior KV quantized with the reference int8 quantizer, "
                "random page permutation",
        "config": {"workload": "configs[1] batched decode: 8 seqs x 1 token, ctx U[1024,32768] seed 0, "
                               "24q/4kv heads, head_dim 256, int8 64-token pages",
                   "sum_ctx": sum(head["ctxs"]), "tokens_per_step": 8},
        "roofline": {"bound": "hbm", "achieved": round(head["attn_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["attn_gbs"] / HBM_PEAK_GBS, 4), "traffic": read_traffic("decode_b8"),
                     "traffic_source": "profiles/attention_decode_b8_traffic.txt (rocprofv3 --pmc FETCH_SIZE / "
                                       "WRITE_SIZE, not this run)",
                     "kernel": "attention_decode (attn_decode_kernel + attn_merge_kernel)",
                     "kernel_ms": round(head["attn_ms"], 5),
                     "measured_peak": peaks["hbm_read_gbs"],
                     "frac_of_measured": round(head["attn_gbs"] / peaks["hbm_read_gbs"], 4),
                     "same_bytes_read_ceiling": round(head_ceiling, 1),
                     "frac_of_same_bytes_ceiling": round(head["attn_gbs"] / head_ceiling, 4)},
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "tokens_per_s": round(head["tokens_per_s"], 1),
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
