"""Synthetic workloads of the benchmark configurations, built on the
device with torch as plain buffers: page pools of random int8 (or bf16) KV quantized from N(0,1)
bf16 with the reference quantizer (fp16 scale = amax/127 per 64-dim group, round-half-even codes),
ragged contexts, randomly permuted page tables, and bf16 projection rows for the new tokens.

Nothing here computes attention; the kernels are called through the C ABI by the caller.
"""
import numpy as np
import torch

import q38a

NQ, NKV, HD = 24, 4, 256
LD = 2 * (NQ + NKV) * HD
INT8_TOKEN_BYTES = 2 * NKV * (HD + 8)   # 2112 B: K + V codes + fp16 scales, all kv heads
BF16_TOKEN_BYTES = 2 * NKV * HD * 2     # 4096 B


def decode_contexts(config, seed=0):
    """Per-sequence prior context lengths of a decode batch."""
    rng = np.random.default_rng(seed)
    if config == "decode_b8":          # config 2: U[1024, 32768], not page-aligned
        return [int(x) for x in rng.integers(1024, 32769, 8)]
    if config in ("long_b8", "long_b8_bf16"):  # config 5a/5c: Dirichlet(1) split of 204,800 tokens
        w = rng.dirichlet(np.ones(8))
        c = np.floor(w * 204_800).astype(np.int64)
        c[np.argmax(c)] += 204_800 - int(c.sum())
        return [int(max(1, x)) for x in c]
    if config == "long_b1":            # config 5b: one sequence at 262,144 tokens
        return [262_143]
    raise ValueError(config)


def quantize_rows_int8(x):
    """x float32 [..., 256] -> (codes int8 [..., 256], scales fp16 [..., 4]) as the reference does."""
    g = x.reshape(*x.shape[:-1], 4, 64)
    amax = g.abs().amax(dim=-1)
    scale = (amax / 127.0).to(torch.float16)
    sf = scale.to(torch.float32)
    q = torch.where(sf[..., None] > 0, torch.round(g / torch.where(sf > 0, sf, 1.0)[..., None]), torch.zeros_like(g))
    return q.clamp(-127, 127).to(torch.int8).reshape(x.shape), scale


def random_pool(num_pages, dtype, gen, layers=1, chunk=512):
    """Page pool [layers][num_pages][page_bytes] of N(0,1) bf16 K/V rows, quantized to int8 pages
    (or stored as bf16), generated in chunks of pages on the device."""
    pb = q38a.page_bytes(dtype, NKV)
    pool = torch.empty(layers * num_pages * pb, dtype=torch.uint8, device="cuda")
    view = pool.view(layers * num_pages, pb)
    for p0 in range(0, layers * num_pages, chunk):
        n = min(chunk, layers * num_pages - p0)
        kv = torch.randn((n, 2, NKV, 64, HD), generator=gen, device="cuda").to(torch.bfloat16).to(torch.float32)
        if dtype in (q38a.KV_INT8, q38a.KV_INT8_VT):
            codes, scales = quantize_rows_int8(kv)  # [n][K|V][kvh][64 tok][256], [n][K|V][kvh][64][4]
            if dtype == q38a.KV_INT8_VT:  # V codes [kvh][4][256][16], V scales [kvh][4][64]
                vq = codes[:, 1].reshape(n, NKV, 4, 16, HD).transpose(-1, -2).contiguous()
                codes = torch.stack([codes[:, 0], vq.view(n, NKV, 64, HD)], 1)
                scales = torch.stack([scales[:, 0], scales[:, 1].transpose(-1, -2).contiguous().view(n, NKV, 64, 4)], 1)
            view[p0:p0 + n, :2 * NKV * 64 * HD] = codes.contiguous().view(torch.uint8).reshape(n, -1)
            view[p0:p0 + n, 2 * NKV * 64 * HD:] = scales.contiguous().view(torch.uint8).reshape(n, -1)
        else:
            view[p0:p0 + n] = kv.to(torch.bfloat16).view(torch.uint8).reshape(n, -1)
    return pool


class DecodeBatch:
    """A decode step: B sequences with prior contexts `ctxs`, one new token each at position ctx."""

    def __init__(self, ctxs, dtype=q38a.KV_INT8, seed=0, pools=1):
        self.ctxs = list(ctxs)
        self.B = len(ctxs)
        self.dtype = dtype
        rng = np.random.default_rng(seed + 1)
        gen = torch.Generator(device="cuda").manual_seed(seed)
        pages = [(c + 1 + 63) // 64 for c in self.ctxs]
        self.num_pages = sum(pages)
        perm = rng.permutation(self.num_pages).astype(np.int32)
        self.max_pages = max(pages)
        bt = np.zeros((self.B, self.max_pages), np.int32)
        o = 0
        for b, p in enumerate(pages):
            bt[b, :p] = perm[o:o + p]
            o += p
        self.block_table = bt
        self.bt_t = torch.from_numpy(bt).cuda()
        self.pools = [random_pool(self.num_pages, dtype, gen) for _ in range(pools)]
        self.page_bytes = q38a.page_bytes(dtype, NKV)
        self.meta = [torch.from_numpy(a).cuda() for a in (
            np.arange(self.B + 1, dtype=np.int32), np.arange(self.B, dtype=np.int32),
            np.array(self.ctxs, np.int32), np.array(self.ctxs, np.int32), np.arange(self.B, dtype=np.int32))]
        self.batch = q38a.BatchDesc(self.B, self.B, 1, *[t.data_ptr() for t in self.meta])
        self.proj = torch.randn((self.B, LD), generator=gen, device="cuda").to(torch.bfloat16)
        self.q_norm = (1.0 + 0.1 * torch.randn(HD, generator=gen, device="cuda")).float()
        self.k_norm = (1.0 + 0.1 * torch.randn(HD, generator=gen, device="cuda")).float()
        self.rope = torch.from_numpy(q38a.rope_table(0, max(self.ctxs) + 1)).cuda()
        self.q16 = torch.empty((self.B, NQ * HD), dtype=torch.float16, device="cuda")
        self.out = torch.empty((self.B, NQ * HD), dtype=torch.bfloat16, device="cuda")
        self.max_splits = 256
        self.scratch = torch.empty(q38a.split_scratch_floats(self.B, NQ, self.max_splits), dtype=torch.float32,
                                   device="cuda")

    def kv_desc(self, i=0):
        return q38a.KvCacheDesc(self.pools[i].data_ptr(), self.dtype, NKV, self.num_pages, self.page_bytes,
                                self.page_bytes * self.num_pages, self.bt_t.data_ptr(), self.max_pages)

    def append_params(self):
        return q38a.QkNormRopeParams(self.proj.data_ptr(), LD, self.q_norm.data_ptr(), self.k_norm.data_ptr(), 1e-6,
                                     1e7, NQ, NKV, self.q16.data_ptr(), 0, self.rope.data_ptr(), self.rope.shape[0])

    def attention_params(self):
        return q38a.AttentionParams(self.q16.data_ptr(), self.proj.data_ptr() + NQ * HD * 2, LD, self.out.data_ptr(),
                                    NQ, NKV, 0, self.scratch.data_ptr(), self.max_splits)

    def kv_bytes(self):
        """Algorithmic KV bytes one decode step reads: every key/value of [0, ctx] once."""
        per = BF16_TOKEN_BYTES if self.dtype == q38a.KV_BF16 else INT8_TOKEN_BYTES
        return sum(c + 1 for c in self.ctxs) * per

    def io_bytes(self):
        """q (fp16) + gate (bf16) reads and the bf16 output write per step."""
        return self.B * NQ * HD * 2 * 3


def prefill_flops(seqs):
    """Unmasked causal (query, key) pairs x 4 * head_dim * nq: 2 flops per multiply-add of QK^T
    and of PV. seqs: [(prefix, n)]."""
    pairs = sum(n * prefix + n * (n + 1) // 2 for prefix, n in seqs)
    return 4 * HD * NQ * pairs


def mixed_seqs(seed=0):
    """Config 4: one 512-token prefill chunk + 7 decode rows; all 8 contexts (the chunk's prefix
    first) lognormal with median 8192 and sigma 1, rounded and clipped to [64, 65536]."""
    rng = np.random.default_rng(seed)
    ctx = np.clip(np.round(np.exp(np.log(8192) + rng.normal(0, 1, 8))), 64, 65536).astype(int)
    return [(int(ctx[0]), 512)] + [(int(c), 1) for c in ctx[1:]]


class RaggedBatch:
    """A continuous-batching step: sequences [(prefix, n)] (n == 1: decode row, n > 1: prefill
    chunk), pages of all sequences interleaved by one random permutation of the pool."""

    def __init__(self, seqs, dtype=q38a.KV_INT8, seed=0, pools=1):
        self.seqs = list(seqs)
        self.B = len(seqs)
        self.dtype = dtype
        rng = np.random.default_rng(seed + 1)
        gen = torch.Generator(device="cuda").manual_seed(seed)
        pages = [(p + n + 63) // 64 for p, n in self.seqs]
        self.num_pages = sum(pages)
        perm = rng.permutation(self.num_pages).astype(np.int32)
        self.max_pages = max(pages)
        bt = np.zeros((self.B, self.max_pages), np.int32)
        o = 0
        for b, pg in enumerate(pages):
            bt[b, :pg] = perm[o:o + pg]
            o += pg
        self.block_table = bt
        self.bt_t = torch.from_numpy(bt).cuda()
        self.pools = [random_pool(self.num_pages, dtype, gen) for _ in range(pools)]
        self.page_bytes = q38a.page_bytes(dtype, NKV)
        seq_start = np.zeros(self.B + 1, np.int32)
        tok_pos, tok_seq = [], []
        for b, (p, n) in enumerate(self.seqs):
            seq_start[b + 1] = seq_start[b] + n
            tok_pos += list(range(p, p + n))
            tok_seq += [b] * n
        self.M = int(seq_start[-1])
        self.meta = [torch.from_numpy(np.asarray(a, np.int32)).cuda() for a in (
            seq_start, np.arange(self.B), [p for p, _ in self.seqs], tok_pos, tok_seq)]
        self.batch = q38a.BatchDesc(self.B, self.M, max(n for _, n in self.seqs), *[t.data_ptr() for t in self.meta])
        self.proj = torch.randn((self.M, LD), generator=gen, device="cuda").to(torch.bfloat16)
        self.q_norm = (1.0 + 0.1 * torch.randn(HD, generator=gen, device="cuda")).float()
        self.k_norm = (1.0 + 0.1 * torch.randn(HD, generator=gen, device="cuda")).float()
        self.rope = torch.from_numpy(q38a.rope_table(0, max(p + n for p, n in self.seqs))).cuda()
        self.q16 = torch.empty((self.M, NQ * HD), dtype=torch.float16, device="cuda")
        self.out = torch.empty((self.M, NQ * HD), dtype=torch.bfloat16, device="cuda")
        self.max_splits = 256
        self.scratch = torch.zeros(q38a.ragged_scratch_floats(self.B, self.M, max(n for _, n in self.seqs), NQ, NKV,
                                                              self.max_splits), dtype=torch.float32, device="cuda")

    kv_desc = DecodeBatch.kv_desc
    append_params = DecodeBatch.append_params
    attention_params = DecodeBatch.attention_params

    def flops(self):
        return prefill_flops([(p, n) for p, n in self.seqs if n > 1])

    def decode_kv_bytes(self):
        per = BF16_TOKEN_BYTES if self.dtype == q38a.KV_BF16 else INT8_TOKEN_BYTES
        return sum(p + 1 for p, n in self.seqs if n == 1) * per
