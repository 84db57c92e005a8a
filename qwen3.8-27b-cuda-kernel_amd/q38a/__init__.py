"""Python binding of libq38a.so, the MI355X ragged paged-KV attention step.

A thin ctypes mirror of include/q38a.h: the descriptor structs of the reference launch API
(reference src/kernels/kernels.h:22-70, 142-179), the kernel entry points, and the host KV cache
class (reference include/qwen38/kv_cache.h:19-51). Functions raise Q38AError when the library
returns a nonzero status, the way the reference raises qwen38::Error.

Device buffers are passed as integer addresses (e.g. torch tensor .data_ptr()), streams as the
raw hipStream_t handle (torch.cuda.current_stream().cuda_stream). Nothing here computes: every
call goes to the HIP library, and importing fails loudly if it has not been built.
"""
import ctypes
import os

import numpy as np

PAGE_TOKENS = 64
HEAD_DIM = 256
KV_INT8 = 0
KV_BF16 = 1
KV_INT8_VT = 2  # int8 with V transposed per page (V^T [kvh][256][64], V scales [kvh][4][64])

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("Q38A_LIB") or os.path.join(os.path.dirname(_HERE), "lib", "libq38a.so")


class Q38AError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"q38a error {code}: {message}")
        self.code = code


def _load():
    # One HIP runtime per process: when torch (which ships its own libamdhip64.so.7) is present it
    # must be loaded first, so that this library binds to the same runtime instance as the
    # device buffers and streams the caller passes in.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or build.py) first")
    return ctypes.CDLL(LIB_PATH)


lib = _load()

_p = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t


class BatchDesc(ctypes.Structure):
    _fields_ = [("num_seqs", _i), ("num_tokens", _i), ("max_tokens_per_seq", _i),
                ("seq_start", _p), ("seq_slot", _p), ("seq_pos0", _p), ("tok_pos", _p), ("tok_seq", _p)]


class KvCacheDesc(ctypes.Structure):
    _fields_ = [("pool", _p), ("dtype", _i), ("kv_heads", _i), ("num_pages", _i), ("page_bytes", _sz),
                ("layer_stride", _sz), ("block_table", _p), ("max_pages_per_seq", _i)]


class QkNormRopeParams(ctypes.Structure):
    _fields_ = [("proj", _p), ("ld_proj", _i), ("q_norm", _p), ("k_norm", _p), ("eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("num_q_heads", _i), ("num_kv_heads", _i), ("q_out", _p),
                ("attn_layer", _i), ("rope_cos_sin", _p), ("rope_rows", _i)]


class AttentionParams(ctypes.Structure):
    _fields_ = [("q", _p), ("gate", _p), ("ld_gate", _i), ("out", _p), ("num_q_heads", _i),
                ("num_kv_heads", _i), ("attn_layer", _i), ("split_scratch", _p), ("max_splits", _i)]


_PBatch = ctypes.POINTER(BatchDesc)
_PKv = ctypes.POINTER(KvCacheDesc)

_SIGS = {
    "q38a_last_error": (ctypes.c_char_p, []),
    "q38a_kv_page_bytes": (_sz, [_i, _i]),
    "q38a_kv_offsets": (_i, [_i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "q38a_rope_table_fill": (_i, [_p, _i, _i, ctypes.c_double, _i]),
    "q38a_qk_norm_rope_append": (_i, [ctypes.POINTER(QkNormRopeParams), _PBatch, _PKv, _p]),
    "q38a_attention_decode_splits": (_i, [_i, _i, _i, _i]),
    "q38a_split_scratch_floats": (_sz, [_i, _i, _i]),
    "q38a_ragged_scratch_floats": (_sz, [_i, _i, _i, _i, _i, _i]),
    "q38a_attention_decode": (_i, [ctypes.POINTER(AttentionParams), _PBatch, _PKv, _p]),
    "q38a_attention_decode_partials": (_i, [ctypes.POINTER(AttentionParams), _PBatch, _PKv, _p]),
    "q38a_attention_prefill": (_i, [ctypes.POINTER(AttentionParams), _PBatch, _PKv, _p]),
    "q38a_attention_ragged": (_i, [ctypes.POINTER(AttentionParams), _PBatch, _PKv, _p]),
    "q38a_ragged_scratch_init": (_i, [_p, _p]),
    "q38a_attention_decode_noalloc": (_i, [ctypes.POINTER(AttentionParams), _PBatch, _PKv, _p]),
    "q38a_noalloc_scratch_floats": (_sz, []),
    "q38a_kv_cache_create": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_p)]),
    "q38a_kv_cache_destroy": (None, [_p]),
    "q38a_kv_cache_desc_get": (_i, [_p, _PKv]),
    "q38a_kv_cache_ensure": (_i, [_p, _i, _i, ctypes.POINTER(_i)]),
    "q38a_kv_cache_release": (_i, [_p, _i]),
    "q38a_kv_cache_sync": (_i, [_p, _p]),
    "q38a_kv_cache_free_pages": (_i, [_p]),
    "q38a_kv_cache_pages_of": (_i, [_p, _i]),
    "q38a_kv_cache_page_list": (_i, [_p, _i, _p, _i, ctypes.POINTER(_i)]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args

EXPORTED = sorted(_SIGS)


def last_error():
    return lib.q38a_last_error().decode()


def _check(rc):
    if rc != 0:
        raise Q38AError(rc, last_error())


def page_bytes(dtype, kv_heads):
    return lib.q38a_kv_page_bytes(dtype, kv_heads)


def kv_offsets(dtype, kv_heads, head, tok):
    out = (_sz * 4)()
    _check(lib.q38a_kv_offsets(dtype, kv_heads, head, tok, out))
    return tuple(out)


def rope_table(pos_begin, count, theta=1e7, rotary_dim=64):
    """Host RoPE table [count][64] float32: [cos | sin] per position, libm as the reference CPU path."""
    out = np.empty((count, rotary_dim), dtype=np.float32)
    _check(lib.q38a_rope_table_fill(out.ctypes.data, pos_begin, count, theta, rotary_dim))
    return out


def split_scratch_floats(rows, num_q_heads, max_splits):
    return lib.q38a_split_scratch_floats(rows, num_q_heads, max_splits)


def ragged_scratch_floats(num_seqs, num_tokens, max_tokens_per_seq, num_q_heads, num_kv_heads, max_splits):
    return lib.q38a_ragged_scratch_floats(num_seqs, num_tokens, max_tokens_per_seq, num_q_heads, num_kv_heads,
                                          max_splits)


def qk_norm_rope_append(params, batch, kv, stream=0):
    _check(lib.q38a_qk_norm_rope_append(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


def attention_decode(params, batch, kv, stream=0):
    _check(lib.q38a_attention_decode(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


def attention_decode_partials(params, batch, kv, stream=0):
    """The decode split kernel alone (partials for q38a_qgemm_merge_oproj; params.out not written)."""
    _check(lib.q38a_attention_decode_partials(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


def attention_prefill(params, batch, kv, stream=0):
    _check(lib.q38a_attention_prefill(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


def attention_decode_noalloc(params, batch, kv, stream=0):
    """q38a_attention_decode with the split partials in the library's static device array."""
    _check(lib.q38a_attention_decode_noalloc(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


def noalloc_scratch_floats():
    return lib.q38a_noalloc_scratch_floats()


def ragged_scratch_init(scratch_ptr, stream=0):
    """Zero the work counters at the front of a ragged scratch buffer (once per new buffer)."""
    _check(lib.q38a_ragged_scratch_init(scratch_ptr, stream))


def attention_ragged(params, batch, kv, stream=0):
    _check(lib.q38a_attention_ragged(ctypes.byref(params), ctypes.byref(batch), ctypes.byref(kv), stream))


class KvCache:
    """Owner of the device page pool and block table (reference src/kv_cache.cpp:14-88)."""

    def __init__(self, dtype, kv_heads, layers, num_pages, num_slots, max_pages_per_seq):
        h = _p()
        _check(lib.q38a_kv_cache_create(dtype, kv_heads, layers, num_pages, num_slots, max_pages_per_seq,
                                        ctypes.byref(h)))
        self._h = h
        self.dtype, self.kv_heads, self.layers = dtype, kv_heads, layers
        self.num_pages, self.num_slots, self.max_pages_per_seq = num_pages, num_slots, max_pages_per_seq

    def close(self):
        if self._h:
            lib.q38a_kv_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def desc(self):
        d = KvCacheDesc()
        _check(lib.q38a_kv_cache_desc_get(self._h, ctypes.byref(d)))
        return d

    def ensure(self, slot, tokens):
        ok = _i()
        _check(lib.q38a_kv_cache_ensure(self._h, slot, tokens, ctypes.byref(ok)))
        return bool(ok.value)

    def release(self, slot):
        _check(lib.q38a_kv_cache_release(self._h, slot))

    def sync(self, stream=0):
        _check(lib.q38a_kv_cache_sync(self._h, stream))

    def free_pages(self):
        return lib.q38a_kv_cache_free_pages(self._h)

    def pages_of(self, slot):
        return lib.q38a_kv_cache_pages_of(self._h, slot)

    def page_list(self, slot):
        n = _i()
        _check(lib.q38a_kv_cache_page_list(self._h, slot, None, 0, ctypes.byref(n)))
        out = np.zeros(max(n.value, 1), dtype=np.int32)
        _check(lib.q38a_kv_cache_page_list(self._h, slot, out.ctypes.data, n.value, ctypes.byref(n)))
        return out[: n.value]
