"""ctypes binding of the projection GEMMs (include/q38a_gemm.h): BQ weight repacking, q38a_qgemm
(reference kernels.h:120 qgemm) and the in-projection with the fused append."""
import ctypes

import numpy as np

from . import AttentionParams, BatchDesc, KvCacheDesc, QkNormRopeParams, _check, lib

_p, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

EPI_STORE_BF16, EPI_RESIDUAL, EPI_STORE_F32 = 0, 2, 3


class BQWeight(ctypes.Structure):
    _fields_ = [("lo", _p), ("hi", _p), ("scales", _p), ("bits", _i), ("n", _i), ("k", _i), ("rows", _i)]


class GemmEpilogue(ctypes.Structure):
    _fields_ = [("kind", _i), ("out", _p), ("ldo", _i), ("n_store", _i), ("residual", _p), ("xbf", _p),
                ("partials_out", _p), ("partials_in", _p), ("hidden", _i), ("eps", _f)]


class GemmWorkspace(ctypes.Structure):
    _fields_ = [("partials", _p), ("partial_floats", _sz), ("counters", _p), ("num_counters", _i)]


_SIGS = {
    "q38a_bq_repacked_bytes": (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    "q38a_bq_repack": (_i, [_i, _i, _i, _p, _p, _p, _p, _p, _p]),
    "q38a_qgemm": (_i, [_p, _i, ctypes.POINTER(BQWeight), ctypes.POINTER(GemmEpilogue), ctypes.POINTER(GemmWorkspace), _p]),
    "q38a_qgemm_qkv_append": (_i, [_p, _i, ctypes.POINTER(BQWeight), ctypes.POINTER(GemmEpilogue),
                                   ctypes.POINTER(GemmWorkspace), ctypes.POINTER(QkNormRopeParams),
                                   ctypes.POINTER(BatchDesc), ctypes.POINTER(KvCacheDesc), _p]),
    "q38a_qgemm_workspace_size": (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    "q38a_qgemm_merge_oproj": (_i, [ctypes.POINTER(AttentionParams), ctypes.POINTER(BatchDesc), ctypes.POINTER(BQWeight),
                                    ctypes.POINTER(GemmEpilogue), ctypes.POINTER(GemmWorkspace), _p]),
    "q38a_qgemm_merge_oproj_in_loader": (_i, [ctypes.POINTER(AttentionParams), ctypes.POINTER(BatchDesc),
                                              ctypes.POINTER(BQWeight), ctypes.POINTER(GemmEpilogue),
                                              ctypes.POINTER(GemmWorkspace), _p]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = sorted(_SIGS)


def repacked_bytes(bits, n, k):
    out = (_sz * 3)()
    _check(lib.q38a_bq_repacked_bytes(bits, n, k, out))
    return tuple(out)


def repack(bits, n, k, ref_lo, ref_hi, ref_scales):
    """Reference file planes (numpy, host) -> (lo, hi or None, scales) numpy arrays in the q38a layout."""
    nl, nh, ns = repacked_bytes(bits, n, k)
    lo = np.zeros(nl, np.uint8)
    hi = np.zeros(nh, np.uint8) if nh else None
    sc = np.zeros(ns // 2, np.uint16)
    ref_lo = np.ascontiguousarray(ref_lo, np.uint8)
    ref_sc = np.ascontiguousarray(ref_scales, np.uint16)
    ref_hi = None if ref_hi is None else np.ascontiguousarray(ref_hi, np.uint8)
    _check(lib.q38a_bq_repack(bits, n, k, ref_lo.ctypes.data, None if ref_hi is None else ref_hi.ctypes.data,
                              ref_sc.ctypes.data, lo.ctypes.data, None if hi is None else hi.ctypes.data,
                              sc.ctypes.data))
    return lo, hi, sc


def workspace_size(m, n, k):
    out = (_sz * 2)()
    _check(lib.q38a_qgemm_workspace_size(m, n, k, out))
    return tuple(out)


def qgemm(a_ptr, m, w, ep, ws, stream=0):
    _check(lib.q38a_qgemm(a_ptr, m, ctypes.byref(w), ctypes.byref(ep), ctypes.byref(ws), stream))


def merge_oproj(attn, batch, w, ep, ws, stream=0, in_loader=False):
    """The o-projection after attention_decode_partials: the merge kernel then the GEMM, or with
    in_loader the merge inside the small-M GEMM's A staging (same bits)."""
    fn = lib.q38a_qgemm_merge_oproj_in_loader if in_loader else lib.q38a_qgemm_merge_oproj
    _check(fn(ctypes.byref(attn), ctypes.byref(batch), ctypes.byref(w), ctypes.byref(ep), ctypes.byref(ws), stream))


def qgemm_qkv_append(a_ptr, m, w, ep, ws, append, batch, kv, stream=0):
    _check(lib.q38a_qgemm_qkv_append(a_ptr, m, ctypes.byref(w), ctypes.byref(ep), ctypes.byref(ws),
                                     ctypes.byref(append), ctypes.byref(batch), ctypes.byref(kv), stream))
