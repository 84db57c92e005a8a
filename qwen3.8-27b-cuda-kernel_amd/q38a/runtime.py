"""ctypes mirror of include/q38a_runtime.h: the step runner (reference ModelRunner's launch
interface for the full-attention layers, src/model_runner.cpp) and the continuous-batching engine
(reference src/engine.cpp). Every call goes to libq38a.so; errors raise Q38AError."""
import ctypes

import numpy as np

from . import Q38AError, lib, last_error

_p = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t


class RunnerOptions(ctypes.Structure):
    _fields_ = [("kv_dtype", _i), ("num_q_heads", _i), ("num_kv_heads", _i), ("attn_layers", _i),
                ("num_pages", _i), ("max_batch", _i), ("max_chunk", _i), ("max_context", _i), ("max_splits", _i),
                ("eps", ctypes.c_float), ("rope_theta", ctypes.c_double), ("q_norm", _p), ("k_norm", _p),
                ("use_graphs", _i)]


class RunnerBuffers(ctypes.Structure):
    _fields_ = [("proj", _p), ("ld_proj", _i), ("proj_layer_stride", _sz), ("out", _p), ("out_layer_stride", _sz),
                ("q16", _p), ("rows", _i), ("prefill_row", _i)]


class StepSeq(ctypes.Structure):
    _fields_ = [("slot", _i), ("pos0", _i), ("n", _i)]


class EngineOptions(ctypes.Structure):
    _fields_ = [("prefill_chunk", _i), ("mixed", _i)]


class PlanEntry(ctypes.Structure):
    _fields_ = [("request_id", _i), ("slot", _i), ("pos0", _i), ("n", _i), ("row", _i)]


class EngineStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_longlong) for n in
                ("iterations", "launches", "prefill_tokens", "decode_tokens", "requests_done", "requests_failed")]


_SIGS = {
    "q38a_runner_create": (_i, [ctypes.POINTER(RunnerOptions), ctypes.POINTER(_p)]),
    "q38a_runner_destroy": (None, [_p]),
    "q38a_runner_get_buffers": (_i, [_p, ctypes.POINTER(RunnerBuffers)]),
    "q38a_runner_kv": (_p, [_p]),
    "q38a_runner_num_slots": (_i, [_p]),
    "q38a_runner_bucket_for": (_i, [_i, _i]),
    "q38a_runner_decode": (_i, [_p, ctypes.POINTER(StepSeq), _i, _p]),
    "q38a_runner_prefill": (_i, [_p, _i, _i, _i, _p]),
    "q38a_runner_step": (_i, [_p, ctypes.POINTER(StepSeq), _i, _p]),
    "q38a_runner_set_graphs": (_i, [_p, _i]),
    "q38a_runner_graph_buckets": (_i, [_p, ctypes.POINTER(_i), _i]),
    "q38a_engine_create": (_i, [_p, ctypes.POINTER(EngineOptions), ctypes.POINTER(_p)]),
    "q38a_engine_destroy": (None, [_p]),
    "q38a_engine_submit": (_i, [_p, _i, _i]),
    "q38a_engine_plan": (_i, [_p, ctypes.POINTER(PlanEntry), _i, ctypes.POINTER(_i)]),
    "q38a_engine_execute": (_i, [_p, _p]),
    "q38a_engine_idle": (_i, [_p]),
    "q38a_engine_get_stats": (_i, [_p, ctypes.POINTER(EngineStats)]),
    "q38a_engine_take_finished": (_i, [_p, ctypes.POINTER(_i), _i, ctypes.POINTER(_i)]),
    "q38a_engine_position": (_i, [_p, _i]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args

EXPORTED = sorted(_SIGS)


def _check(rc):
    if rc != 0:
        raise Q38AError(rc, last_error())


def bucket_for(n, max_batch):
    return lib.q38a_runner_bucket_for(n, max_batch)


def _seqs(seqs):
    arr = (StepSeq * len(seqs))(*[StepSeq(*s) for s in seqs])
    return arr, len(seqs)


class Runner:
    """Owner of the KV cache, the step buffers and the decode graphs of `attn_layers` layers."""

    def __init__(self, q_norm_ptr, k_norm_ptr, kv_dtype=0, num_q_heads=24, num_kv_heads=4, attn_layers=16,
                 num_pages=1024, max_batch=8, max_chunk=512, max_context=65536, max_splits=256, eps=1e-6,
                 rope_theta=1e7, use_graphs=True):
        self.opt = RunnerOptions(kv_dtype, num_q_heads, num_kv_heads, attn_layers, num_pages, max_batch, max_chunk,
                                 max_context, max_splits, eps, rope_theta, q_norm_ptr, k_norm_ptr, int(use_graphs))
        h = _p()
        _check(lib.q38a_runner_create(ctypes.byref(self.opt), ctypes.byref(h)))
        self._h = h
        b = RunnerBuffers()
        _check(lib.q38a_runner_get_buffers(h, ctypes.byref(b)))
        self.buffers = b

    def close(self):
        if self._h:
            lib.q38a_runner_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def kv_handle(self):
        return lib.q38a_runner_kv(self._h)

    def ensure(self, slot, tokens):
        ok = _i()
        _check(lib.q38a_kv_cache_ensure(self.kv_handle(), slot, tokens, ctypes.byref(ok)))
        return bool(ok.value)

    def release(self, slot):
        _check(lib.q38a_kv_cache_release(self.kv_handle(), slot))

    def free_pages(self):
        return lib.q38a_kv_cache_free_pages(self.kv_handle())

    def kv_desc(self):
        from . import KvCacheDesc
        d = KvCacheDesc()
        _check(lib.q38a_kv_cache_desc_get(self.kv_handle(), ctypes.byref(d)))
        return d

    def page_list(self, slot):
        n = _i()
        _check(lib.q38a_kv_cache_page_list(self.kv_handle(), slot, None, 0, ctypes.byref(n)))
        out = np.zeros(max(n.value, 1), dtype=np.int32)
        _check(lib.q38a_kv_cache_page_list(self.kv_handle(), slot, out.ctypes.data, n.value, ctypes.byref(n)))
        return out[: n.value]

    def decode(self, rows, stream=0):
        arr, n = _seqs([(s, p, 1) for s, p in rows])
        _check(lib.q38a_runner_decode(self._h, arr, n, stream))

    def prefill(self, slot, pos0, n, stream=0):
        _check(lib.q38a_runner_prefill(self._h, slot, pos0, n, stream))

    def step(self, seqs, stream=0):
        arr, n = _seqs(seqs)
        _check(lib.q38a_runner_step(self._h, arr, n, stream))

    def set_graphs(self, on):
        _check(lib.q38a_runner_set_graphs(self._h, int(on)))

    def graph_buckets(self):
        buf = (_i * 16)()
        n = lib.q38a_runner_graph_buckets(self._h, buf, 16)
        return list(buf[:n])


class Engine:
    """Continuous-batching scheduler over a Runner (reference src/engine.cpp)."""

    def __init__(self, runner, prefill_chunk=512, mixed=True):
        self.runner = runner
        h = _p()
        _check(lib.q38a_engine_create(runner.handle, ctypes.byref(EngineOptions(prefill_chunk, int(mixed))),
                                      ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib.q38a_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def submit(self, prompt_tokens, max_new_tokens):
        rid = lib.q38a_engine_submit(self._h, prompt_tokens, max_new_tokens)
        if rid < 0:
            raise Q38AError(-rid, last_error())
        return rid

    def plan(self, cap=1024):
        buf = (PlanEntry * cap)()
        n = _i()
        _check(lib.q38a_engine_plan(self._h, buf, cap, ctypes.byref(n)))
        return [(e.request_id, e.slot, e.pos0, e.n, e.row) for e in buf[:n.value]]

    def execute(self, stream=0):
        _check(lib.q38a_engine_execute(self._h, stream))

    def idle(self):
        return bool(lib.q38a_engine_idle(self._h))

    def stats(self):
        s = EngineStats()
        _check(lib.q38a_engine_get_stats(self._h, ctypes.byref(s)))
        return {k: getattr(s, k) for k, _ in EngineStats._fields_}

    def take_finished(self):
        buf = (_i * 4096)()
        n = _i()
        _check(lib.q38a_engine_take_finished(self._h, buf, 4096, ctypes.byref(n)))
        return list(buf[:min(n.value, 4096)])

    def position(self, rid):
        return lib.q38a_engine_position(self._h, rid)
