"""Empty batches through every launch of the C ABI: a batch with no sequences (or no tokens) is a
valid call that returns Q38A_OK and touches nothing. The reference launchers size their grids from
the batch (src/kernels/attention_decode.cu:280-300, attention_prefill.cu:316-340,
qk_norm_rope.cu:92-100) and an empty batch launches no work there either. The same scratch then
serves a normal launch, whose outputs are checked against the oracle."""
import numpy as np
import pytest
import torch

import q38a
from gpu_util import append_params, host, rope_dev
from test_gpu_streams import Case

pytestmark = pytest.mark.gpu


def _canary(t, value):
    t.fill_(value)
    return host(t).copy()


def test_empty_batches_launch_nothing(orc):
    """num_seqs = num_tokens = 0 (null metadata pointers) on append, decode, decode partials,
    prefill, the ragged launch and the no-allocation decode: rc 0, and the q buffer, the output, the
    page pool and the ragged scratch keep their bytes; a normal ragged launch on the same scratch is
    then exact."""
    c = Case(orc, [(3000, 20), (900, 1), (64, 1)], seed=91, ragged=True)
    empty = q38a.BatchDesc(0, 0, 0, None, None, None, None, None)
    s = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    q_before = _canary(c.q_t, 0x1357)
    out_before = _canary(c.out_t, 0x2468)
    pool_before = host(c.pool.t).copy()
    scratch_before = host(c.scratch_t).copy()
    qn = torch.ones(256, dtype=torch.float32, device="cuda")
    rope = rope_dev(4096)
    print("edges: empty batch on every launch", flush=True)
    q38a.qk_norm_rope_append(append_params(c.proj_t, qn, qn, c.q_t, rope), empty, c.pool.desc, s)
    q38a.attention_decode(c.params(), empty, c.pool.desc, s)
    q38a.attention_decode_partials(c.params(), empty, c.pool.desc, s)
    q38a.attention_prefill(c.params(), empty, c.pool.desc, s)
    q38a.attention_ragged(c.params(), empty, c.pool.desc, s)
    q38a.attention_decode_noalloc(c.params(), empty, c.pool.desc, s)
    torch.cuda.synchronize()
    assert np.array_equal(host(c.q_t), q_before)
    assert np.array_equal(host(c.out_t), out_before)
    assert np.array_equal(host(c.pool.t), pool_before)
    assert np.array_equal(host(c.scratch_t), scratch_before)

    # the q buffer holds the canary now: run the append again, then the ragged launch on the same scratch
    print("edges: normal ragged launch after the empty ones", flush=True)
    c2 = Case(orc, [(3000, 20), (900, 1), (64, 1)], seed=91, ragged=True, scratch=False)
    q38a.attention_ragged(c2.params(c.scratch_t), c2.b.desc, c2.pool.desc, s)
    c2.check("ragged after empty launches")
