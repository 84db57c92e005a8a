"""GPU tests of the native runner and engine (include/q38a_runtime.h).

Runner (reference src/model_runner.cpp:488-560): a decode step replayed from its bucket's hipGraph
gives the same bytes as the eager launches, on every replay, with other eager steps (and other
buckets) in between; the output of the last layer matches the oracle's exact attention over the
pages the runner wrote. A mixed ragged step gives the same appended K/V bytes as a prefill step
plus a decode step and outputs within the north star's tolerance.

Engine (reference src/engine.cpp:62-184): requests run to completion under both policies with the
reference's accounting (every prompt token prefilled once, max_new - 1 decode rows per request,
all pages and slots returned, an impossible request failed)."""
import numpy as np
import pytest
import torch

import q38a
from q38a import runtime
from gpu_util import HD, LD, NKV, NQ, from_device_ptr, stream, to_device_ptr
from util import assert_bits_equal, bf16_bits_to_f32, check_close, randn_bf16

pytestmark = pytest.mark.gpu


class Rig:
    def __init__(self, layers=2, seed=0, **kw):
        self.rng = np.random.default_rng(seed)
        self.layers = layers
        qn = self.rng.normal(1.0, 0.1, (layers, HD)).astype(np.float32)
        kn = self.rng.normal(1.0, 0.1, (layers, HD)).astype(np.float32)
        self.qn_host, self.kn_host = qn, kn
        self.qn, self.kn = torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda()
        self.r = runtime.Runner(self.qn.data_ptr(), self.kn.data_ptr(), attn_layers=layers, **kw)
        self.b = self.r.buffers
        self.s = stream()

    def proj_ptr(self, layer, row):
        return self.b.proj + 2 * (layer * self.b.proj_layer_stride + row * self.b.ld_proj)

    def fill(self, row0, n, data=None):
        """Random bf16 proj rows [row0, row0 + n) of every layer; returns them [layers][n][LD]."""
        if data is None:
            data = randn_bf16(self.rng, (self.layers, n, LD))
        for l in range(self.layers):
            to_device_ptr(self.proj_ptr(l, row0), data[l])
        return data

    def out(self, layer, row0, n):
        ptr = self.b.out + 2 * (layer * self.b.out_layer_stride + row0 * NQ * HD)
        return from_device_ptr(ptr, (n, NQ * HD), np.uint16)

    def q16(self, row0, n):
        return from_device_ptr(self.b.q16 + 2 * row0 * NQ * HD, (n, NQ, HD), np.uint16)

    def pool(self, layer):
        d = self.r.kv_desc()
        return from_device_ptr(d.pool + layer * d.layer_stride, (d.layer_stride,), np.uint8)

    def block_table(self):
        d = self.r.kv_desc()
        return from_device_ptr(d.block_table, (self.r.opt.max_batch + 1, d.max_pages_per_seq), np.int32)

    def build_context(self, slot, ctx, chunk):
        """Prefill positions [0, ctx) of `slot` through the runner, chunk by chunk."""
        assert self.r.ensure(slot, ctx + 256)
        for p0 in range(0, ctx, chunk):
            n = min(chunk, ctx - p0)
            self.fill(self.b.prefill_row, n)
            self.r.prefill(slot, p0, n, self.s)
        torch.cuda.synchronize()


def oracle_rows(orc, rig, layer, seqs, q16, gate):
    """Oracle attention of tokens given as seqs [(slot, pos0, n)] with q16 [M][NQ][HD] and gate rows."""
    bt = rig.block_table()
    starts = np.zeros(len(seqs) + 1, np.int32)
    pos, slots = [], []
    for i, (slot, p0, n) in enumerate(seqs):
        starts[i + 1] = starts[i] + n
        pos += list(range(p0, p0 + n))
        slots.append(slot)
    want = orc.attention_ragged(NQ, NKV, starts, np.array(slots, np.int32), np.array(pos, np.int32), q16,
                                np.ascontiguousarray(gate), NQ * HD, rig.pool(layer), q38a.KV_INT8, bt)
    return bf16_bits_to_f32(want).reshape(len(pos), NQ * HD)


def test_runner_decode_graph_replays_match_eager(orc):
    rig = Rig(layers=2, seed=1, num_pages=64, max_batch=8, max_chunk=256, max_context=4096, use_graphs=False)
    ctxs = [5, 64, 130, 300]
    for slot, c in enumerate(ctxs):
        rig.build_context(slot, c, 256)
    rows = [(0, ctxs[0]), (2, ctxs[2]), (3, ctxs[3])]  # 3 rows -> bucket 4 (one dummy row)
    data = rig.fill(0, len(rows))
    print("runner: eager decode", rows, flush=True)
    rig.r.decode(rows, rig.s)
    torch.cuda.synchronize()
    eager = [rig.out(l, 0, len(rows)) for l in range(2)]
    q16 = rig.q16(0, len(rows))
    want = oracle_rows(orc, rig, 1, [(s, p, 1) for s, p in rows], q16, data[1][:, NQ * HD:2 * NQ * HD])
    check_close(bf16_bits_to_f32(eager[1]), want, what="runner eager decode vs oracle")
    rig.r.set_graphs(True)
    for rep in range(3):
        print("runner: graph replay", rep, flush=True)
        rig.fill(0, len(rows), data)
        rig.r.decode(rows, rig.s)
        torch.cuda.synchronize()
        for l in range(2):
            assert_bits_equal(rig.out(l, 0, len(rows)), eager[l], f"graph replay {rep} layer {l}")
        # other work between replays: an eager-launched bucket and a second graph bucket
        rig.r.set_graphs(False)
        rig.fill(0, 1)
        rig.r.decode([(1, ctxs[1])], rig.s)
        rig.r.set_graphs(True)
        rig.fill(0, 1)
        rig.r.decode([(1, ctxs[1])], rig.s)
        torch.cuda.synchronize()
    assert rig.r.graph_buckets() == [1, 4]


def test_runner_mixed_step_matches_separate_launches(orc):
    rig = Rig(layers=2, seed=2, num_pages=64, max_batch=8, max_chunk=256, max_context=4096, use_graphs=True)
    ctxs = [100, 640, 77, 300]
    for slot, c in enumerate(ctxs):
        rig.build_context(slot, c, 256)
    dec = [(0, ctxs[0]), (1, ctxs[1]), (2, ctxs[2])]
    chunk = (3, ctxs[3], 200)
    ddata = randn_bf16(rig.rng, (2, 3, LD))
    cdata = randn_bf16(rig.rng, (2, 200, LD))
    # reference policy: a prefill step, then a decode step
    rig.fill(rig.b.prefill_row, 200, cdata)
    rig.fill(0, 3, ddata)
    rig.r.prefill(*chunk, rig.s)
    rig.r.decode(dec, rig.s)
    torch.cuda.synchronize()
    sep = [(rig.out(l, 0, 3), rig.out(l, rig.b.prefill_row, 200)) for l in range(2)]
    pools = [rig.pool(l) for l in range(2)]
    # mixed: one ragged batch, decode rows first, then the chunk
    rig.fill(0, 3, ddata)
    rig.fill(3, 200, cdata)
    print("runner: mixed step", flush=True)
    rig.r.step([(s, p, 1) for s, p in dec] + [chunk], rig.s)
    torch.cuda.synchronize()
    for l in range(2):
        assert_bits_equal(rig.pool(l), pools[l], f"pool layer {l}")
        got = bf16_bits_to_f32(rig.out(l, 0, 203))
        want = bf16_bits_to_f32(np.concatenate(sep[l]))
        check_close(got, want, what=f"mixed vs separate layer {l}")
    # and the last layer against the oracle
    q16 = rig.q16(0, 203)
    gate = np.concatenate([ddata[1], cdata[1]])[:, NQ * HD:2 * NQ * HD]
    want = oracle_rows(orc, rig, 1, [(s, p, 1) for s, p in dec] + [chunk], q16, gate)
    check_close(bf16_bits_to_f32(rig.out(1, 0, 203)), want, what="mixed step vs oracle")


@pytest.mark.parametrize("mixed", [False, True])
def test_engine_runs_requests_to_completion(mixed):
    rig = Rig(layers=1, seed=3, num_pages=41, max_batch=4, max_chunk=128, max_context=2048, use_graphs=True)
    e = runtime.Engine(rig.r, prefill_chunk=128, mixed=mixed)
    free0 = rig.r.free_pages()
    reqs = [(300, 5), (50, 1), (130, 20), (700, 3), (10, 40), (1000, 2), (5000, 4), (1, 1)]
    ids = [e.submit(p, m) for p, m in reqs]
    last_pos = {}
    it = 0
    while not e.idle():
        plan = e.plan()
        if not plan:
            break
        assert len([x for x in plan if x[3] > 1]) <= 1  # at most one prefill chunk
        tokens = sum(x[3] for x in plan)
        rows_end = max(x[4] + x[3] for x in plan)
        rig.fill(0, rows_end)
        for rid, slot, p0, n, row in sorted(plan, key=lambda x: -x[3]):  # a chunk precedes its decode row
            if rid in last_pos and n == 1:
                assert p0 == last_pos[rid], (rid, p0, last_pos[rid])  # decode continues where it stopped
            last_pos[rid] = p0 + n
        e.execute(rig.s)
        it += 1
        assert it < 500
    torch.cuda.synchronize()
    done = sorted(e.take_finished())
    ok = [i for i, (p, m) in zip(ids, reqs) if p < 2048]
    assert done == sorted([-1 - ids[6]] + ok)
    st = e.stats()
    assert st["prefill_tokens"] == sum(p for p, _ in reqs if p < 2048)
    assert st["decode_tokens"] == sum(m - 1 for p, m in reqs if p < 2048)
    assert st["requests_done"] == len(ok) and st["requests_failed"] == 1
    assert rig.r.free_pages() == free0
    if mixed:
        assert st["launches"] == st["iterations"]
    else:
        assert st["launches"] >= st["iterations"]
    print("engine:", "mixed" if mixed else "reference", st, flush=True)
