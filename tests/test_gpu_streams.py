"""Launch independence: the decode and ragged launches keep no state between launches outside the
caller's scratch, so two batches with their own scratch may run concurrently on two streams, and one
scratch buffer serves any sequence of launches of different shapes. Every output is checked against
the oracle's exact attention (reference src/ref/ops.cpp:144-171) within the north star's tolerance."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import HD, LD, NKV, NQ, Batch, Pool, append_params, attention_params, dev, host, paged_layout, rope_dev
from test_gpu_decode import build_context
from util import bf16_bits_to_f32, check_close, randn_bf16

pytestmark = pytest.mark.gpu


class Case:
    """One batch [(prefix, n)] with its pool, proj rows, q/out buffers and (optionally) scratch; the
    append runs once at construction, on the current stream."""

    def __init__(self, orc, seqs, seed, kv_dtype=q38a.KV_INT8, max_splits=64, scratch=True, ragged=False):
        rng = np.random.default_rng(seed)
        self.seqs, self.kv_dtype, self.max_splits = seqs, kv_dtype, max_splits
        self.bt, pages = paged_layout(rng, [p + n for p, n in seqs])
        self.pool_host = build_context(orc, rng, [p for p, _ in seqs], kv_dtype, self.bt, pages)
        self.pool = Pool(kv_dtype, pages, self.bt, fill=self.pool_host)
        self.b = Batch([(i, p, n) for i, (p, n) in enumerate(seqs)])
        M = self.b.M
        self.proj = randn_bf16(rng, (M, LD))
        q_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
        k_norm = rng.normal(1.0, 0.1, HD).astype(np.float32)
        self.proj_t, qn_t, kn_t = dev(self.proj), dev(q_norm), dev(k_norm)
        self.q_t = torch.zeros(M * NQ * HD, dtype=torch.int16, device="cuda")
        self.out_t = torch.zeros(M * NQ * HD, dtype=torch.int16, device="cuda")
        self.scratch_t = None
        if scratch:
            n = (q38a.ragged_scratch_floats(len(seqs), M, max(n for _, n in seqs), NQ, NKV, max_splits) if ragged
                 else q38a.split_scratch_floats(len(seqs), NQ, max_splits))
            self.scratch_t = torch.zeros(n, dtype=torch.float32, device="cuda")
        rope_t = rope_dev(max(p + n for p, n in seqs) + 1)
        s = torch.cuda.current_stream().cuda_stream
        q38a.qk_norm_rope_append(append_params(self.proj_t, qn_t, kn_t, self.q_t, rope_t), self.b.desc,
                                 self.pool.desc, s)
        torch.cuda.synchronize()
        q16 = host(self.q_t, np.uint16).reshape(M, NQ, HD)
        orc.qk_norm_rope_append(self.proj, LD, self.b.tok_pos, self.b.tok_seq, self.b.seq_slot, q_norm, k_norm, NQ,
                                NKV, self.pool_host, kv_dtype, self.bt)
        gate = np.ascontiguousarray(self.proj[:, NQ * HD:2 * NQ * HD])
        want = orc.attention_ragged(NQ, NKV, self.b.seq_start, self.b.seq_slot, self.b.tok_pos, q16, gate, NQ * HD,
                                    self.pool_host, kv_dtype, self.bt)
        self.want = bf16_bits_to_f32(want).reshape(M, NQ * HD)

    def params(self, scratch_t=None):
        sc = scratch_t if scratch_t is not None else self.scratch_t
        return attention_params(self.q_t, self.proj_t, self.out_t, sc, self.max_splits)

    def check(self, what):
        torch.cuda.synchronize()
        got = bf16_bits_to_f32(host(self.out_t, np.uint16)).reshape(self.b.M, NQ * HD)
        max_abs, max_rel = check_close(got, self.want, what=what)
        print(f"{what}: max_abs {max_abs:.3g} max_rel {max_rel:.3g}", flush=True)
        self.out_t.zero_()


def test_decode_two_streams(orc):
    """Two decode batches with separate scratch, launched alternately on two streams, several times
    each; the launches overlap in time on the device."""
    a = Case(orc, [(c, 1) for c in (9000, 20000, 300, 4100, 12000, 64, 7000, 15000)], seed=81)
    b = Case(orc, [(c, 1) for c in (30000, 1, 2500, 18000)], seed=82)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("streams: 2 decode batches x 6 launches, alternating", flush=True)
    for _ in range(6):
        with torch.cuda.stream(s1):
            q38a.attention_decode(a.params(), a.b.desc, a.pool.desc, s1.cuda_stream)
        with torch.cuda.stream(s2):
            q38a.attention_decode(b.params(), b.b.desc, b.pool.desc, s2.cuda_stream)
    a.check("decode stream 1")
    b.check("decode stream 2")


def test_ragged_two_streams(orc):
    """Two mixed batches (prefill chunks + decode rows: dynamic item queue and block claims) with
    separate scratch on two streams."""
    a = Case(orc, [(3000, 40), (9000, 1), (700, 1), (15000, 1), (64, 1)], seed=83, ragged=True)
    b = Case(orc, [(c, 1) for c in (4000, 129, 20000, 640)] + [(6000, 300)], seed=84, ragged=True)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("streams: 2 ragged batches x 6 launches, alternating", flush=True)
    for _ in range(6):
        with torch.cuda.stream(s1):
            q38a.attention_ragged(a.params(), a.b.desc, a.pool.desc, s1.cuda_stream)
        with torch.cuda.stream(s2):
            q38a.attention_ragged(b.params(), b.b.desc, b.pool.desc, s2.cuda_stream)
    a.check("ragged stream 1")
    b.check("ragged stream 2")


def test_ragged_scratch_reused_across_shapes(orc):
    """One scratch buffer (sized for the largest batch, zeroed once) for a sequence of launches of
    different shapes: each launch must find the counters the previous one left at zero."""
    cases = [Case(orc, s, seed=85 + i, scratch=False) for i, s in enumerate([
        [(3000, 40), (9000, 1), (700, 1), (15000, 1), (64, 1)],
        [(c, 1) for c in (4000, 129, 20000, 640)],
        [(6000, 300)],
        [(c, 1) for c in (40000, 2, 33000)],
    ])]
    n = max(q38a.ragged_scratch_floats(len(c.seqs), c.b.M, max(k for _, k in c.seqs), NQ, NKV, 64) for c in cases)
    scratch = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    q38a.ragged_scratch_init(scratch.data_ptr(), torch.cuda.current_stream().cuda_stream)
    s = torch.cuda.current_stream().cuda_stream
    for rep in range(2):
        for i, c in enumerate(cases):
            print(f"scratch reuse: round {rep} case {i} seqs={c.seqs[:5]}", flush=True)
            q38a.attention_ragged(c.params(scratch), c.b.desc, c.pool.desc, s)
            c.check(f"reuse round {rep} case {i}")
