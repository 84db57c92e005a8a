"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so) and, when it was built, of the
reference's own CPU ops (oracle/_ref/libref_ops.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, always as the checker, never as the thing measured on the GPU path or shipped.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "_build", "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libref_ops.so")
REFERENCE_TREE = "/root/reference"

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_d = ctypes.c_double


def build(with_ref=True):
    """Compile liboracle.so, and libref_ops.so when the reference tree is present."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if with_ref and os.path.isdir(os.path.join(REFERENCE_TREE, "src", "ref")):
        subprocess.run(["make", "-s", "-C", HERE, "ref", f"REF={REFERENCE_TREE}"], check=True)


def _ptr(a):
    return a.ctypes.data if a is not None else None


class Oracle:
    def __init__(self, path=ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [_f]),
            "orc_f16_to_f32": (_f, [ctypes.c_uint16]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [_f]),
            "orc_bf16_to_f32": (_f, [ctypes.c_uint16]),
            "orc_f32_to_f16_n": (None, [_p, _p, ctypes.c_int64]),
            "orc_f32_to_bf16_n": (None, [_p, _p, ctypes.c_int64]),
            "orc_quantize_int8": (None, [_p, _i, _p, _p]),
            "orc_rope_table": (None, [_i, _i, _d, _i, _p]),
            "orc_rms_offset_norm": (None, [_p, _i, _p, _f, _p]),
            "orc_qk_norm_rope_append": (None, [_p, _i, _i, _p, _p, _p, _p, _p, _f, _d, _i, _i, _i, _p, _p, _i, _p, _i]),
            "orc_fill_rows": (None, [_p, _p, _i, _i, _i, _i, _p, _i, _p, _i]),
            "orc_read_back": (None, [_p, _i, _i, _p, _i, _i, _i, _p, _p]),
            "orc_attention_token": (None, [_i, _i, _p, _p, _i, _p, _p, _i, _p]),
            "orc_attention_ragged": (None, [_i, _i, _i, _p, _p, _p, _p, _p, _i, _p, _i, _p, _i, _p]),
            "orc_bq_pack_file": (None, [_i, _i, _i, _p, _p, _p, _p, _p]),
            "orc_bq_file_weight": (None, [_i, _i, _i, _p, _p, _p, _p]),
            "orc_qgemm": (None, [_p, _i, _p, _i, _i, _i, _p, _i, _i, _p, _i, _f, _p, _p, _p]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        self.L = L

    # ---- formats -------------------------------------------------------------------------------
    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.L.orc_f32_to_f16_n(x.ctypes.data, out.ctypes.data, x.size)
        return out

    def f32_to_bf16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.L.orc_f32_to_bf16_n(x.ctypes.data, out.ctypes.data, x.size)
        return out

    def quantize_int8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        codes = np.empty(x.shape, dtype=np.int8)
        scales = np.empty(x.shape[:-1] + (x.shape[-1] // 64,), dtype=np.uint16)
        self.L.orc_quantize_int8(x.ctypes.data, x.size, codes.ctypes.data, scales.ctypes.data)
        return codes, scales

    def rope_table(self, pos_begin, count, theta=1e7, rotary_dim=64):
        out = np.empty((count, rotary_dim), dtype=np.float32)
        self.L.orc_rope_table(pos_begin, count, theta, rotary_dim, out.ctypes.data)
        return out

    def rms_offset_norm(self, x, w, eps=1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        y = np.empty_like(x)
        self.L.orc_rms_offset_norm(x.ctypes.data, x.size, w.ctypes.data, eps, y.ctypes.data)
        return y

    # ---- step pieces ---------------------------------------------------------------------------
    def qk_norm_rope_append(self, proj, ld_proj, tok_pos, tok_seq, seq_slot, q_norm, k_norm, nq, nkv, pool, kv_dtype,
                            block_table, eps=1e-6, theta=1e7):
        """proj uint16 [M][ld]; pool uint8 (one layer) updated in place; returns q fp16 bits [M][nq][256]."""
        M = len(tok_pos)
        q = np.zeros((M, nq, 256), dtype=np.uint16)
        tok_pos = np.ascontiguousarray(tok_pos, dtype=np.int32)
        tok_seq = np.ascontiguousarray(tok_seq, dtype=np.int32)
        seq_slot = np.ascontiguousarray(seq_slot, dtype=np.int32)
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        self.L.orc_qk_norm_rope_append(_ptr(np.ascontiguousarray(proj)), ld_proj, M, _ptr(tok_pos), _ptr(tok_seq),
                                       _ptr(seq_slot), _ptr(np.ascontiguousarray(q_norm, dtype=np.float32)),
                                       _ptr(np.ascontiguousarray(k_norm, dtype=np.float32)), eps, theta, 64, nq, nkv,
                                       q.ctypes.data, pool.ctypes.data, kv_dtype, bt.ctypes.data, bt.shape[1])
        return q

    def fill_rows(self, k_rows, v_rows, pos0, slot, nkv, pool, kv_dtype, block_table):
        k_rows = np.ascontiguousarray(k_rows, dtype=np.float32)
        v_rows = np.ascontiguousarray(v_rows, dtype=np.float32)
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        self.L.orc_fill_rows(k_rows.ctypes.data, v_rows.ctypes.data, k_rows.shape[0], pos0, slot, nkv,
                             pool.ctypes.data, kv_dtype, bt.ctypes.data, bt.shape[1])

    def read_back(self, pool, kv_dtype, nkv, block_table, slot, length):
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        k = np.zeros((nkv, length, 256), dtype=np.float32)
        v = np.zeros_like(k)
        self.L.orc_read_back(pool.ctypes.data, kv_dtype, nkv, bt.ctypes.data, bt.shape[1], slot, length,
                             k.ctypes.data, v.ctypes.data)
        return k, v

    def attention_token(self, q, gate, pos, k, v, nq, nkv):
        q = np.ascontiguousarray(q, dtype=np.float32)
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        out = np.empty(nq * 256, dtype=np.float32)
        self.L.orc_attention_token(nq, nkv, q.ctypes.data, gate.ctypes.data, pos, k.ctypes.data, v.ctypes.data,
                                   k.shape[1], out.ctypes.data)
        return out

    def attention_ragged(self, nq, nkv, seq_start, seq_slot, tok_pos, q16, gate_rows, ld_gate, pool, kv_dtype,
                         block_table):
        """q16 [M][nq][256] fp16 bits; gate_rows uint16 with row stride ld_gate; returns bf16 bits [M][nq*256]."""
        M = len(tok_pos)
        out = np.zeros((M, nq * 256), dtype=np.uint16)
        seq_start = np.ascontiguousarray(seq_start, dtype=np.int32)
        seq_slot = np.ascontiguousarray(seq_slot, dtype=np.int32)
        tok_pos = np.ascontiguousarray(tok_pos, dtype=np.int32)
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        self.L.orc_attention_ragged(nq, nkv, len(seq_slot), seq_start.ctypes.data, seq_slot.ctypes.data,
                                    tok_pos.ctypes.data, _ptr(np.ascontiguousarray(q16)),
                                    _ptr(np.ascontiguousarray(gate_rows)), ld_gate, pool.ctypes.data, kv_dtype,
                                    bt.ctypes.data, bt.shape[1], out.ctypes.data)
        return out


    # ---- BQ weights and projection GEMMs -------------------------------------------------------
    def bq_pack_file(self, bits, codes, scales):
        """codes int8 [n][k] (signed), scales bf16 bits [n][k/64] -> the reference file planes
        (lo, hi or None, scales)."""
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        n, k = codes.shape
        lo = np.zeros(n * k // 2, np.uint8)
        hb = {4: 0, 5: 128, 6: 256}[bits]
        hi = np.zeros((n // 64) * (k // 16) * hb, np.uint8) if hb else None
        sc = np.zeros(n * (k // 64), np.uint16)
        self.L.orc_bq_pack_file(bits, n, k, codes.ctypes.data, scales.ctypes.data, lo.ctypes.data, _ptr(hi),
                                sc.ctypes.data)
        return lo, hi, sc

    def bq_file_weight(self, bits, n, k, lo, hi, sc):
        w = np.empty((n, k), np.float32)
        self.L.orc_bq_file_weight(bits, n, k, lo.ctypes.data, _ptr(hi), sc.ctypes.data, w.ctypes.data)
        return w

    def qgemm(self, a, w, kind=0, n_store=0, partials_in=None, hidden=0, eps=1e-6, residual=None):
        """a bf16 bits [m][k], w fp32 [n][k]. Returns out (bf16 bits or fp32 [m][n]) or, for the residual
        epilogue, (residual, xbf, partials_out)."""
        a = np.ascontiguousarray(a, dtype=np.uint16)
        w = np.ascontiguousarray(w, dtype=np.float32)
        m, k = a.shape
        n = w.shape[0]
        pin = None if partials_in is None else np.ascontiguousarray(partials_in, dtype=np.float32)
        if kind == 2:
            res = np.array(residual, dtype=np.float32, copy=True)
            xbf = np.zeros((m, n), np.uint16)
            pout = np.zeros((m, n // 128), np.float32)
            self.L.orc_qgemm(a.ctypes.data, m, w.ctypes.data, n, k, 2, None, n, n, None, 0, eps, res.ctypes.data,
                             xbf.ctypes.data, pout.ctypes.data)
            return res, xbf, pout
        out = np.zeros((m, n), np.float32 if kind == 3 else np.uint16)
        self.L.orc_qgemm(a.ctypes.data, m, w.ctypes.data, n, k, kind, out.ctypes.data, n, n_store or n, _ptr(pin),
                         hidden, eps, None, None, None)
        return out


class Reference:
    """The reference's own src/ref/ops.cpp, built from /root/reference into oracle/_ref/."""

    def __init__(self, path=REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing (needs /root/reference and `make -C oracle ref`)")
        L = ctypes.CDLL(path)
        sig = {
            "refx_qk_norm_rope_append_token": (None, [_i, _i, _i, _d, _f, _p, _i, _p, _p, _p, _p, _p, _i, _i]),
            "refx_int8_group_roundtrip": (None, [_p, _i]),
            "refx_store_new": (_p, [_i, _i]),
            "refx_store_free": (None, [_p]),
            "refx_store_k": (ctypes.POINTER(_f), [_p]),
            "refx_store_v": (ctypes.POINTER(_f), [_p]),
            "refx_attention_token": (None, [_p, _i, _i, _p, _p, _i, _p, _i]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        self.L = L

    def qk_norm_rope_append_token(self, nq, nkv, proj_row, pos, q_norm, k_norm, kv_dtype, eps=1e-6, theta=1e7,
                                  exact=False):
        proj_row = np.ascontiguousarray(proj_row, dtype=np.float32)
        q = np.empty((nq, 256), dtype=np.float32)
        k = np.empty((nkv, 256), dtype=np.float32)
        v = np.empty((nkv, 256), dtype=np.float32)
        self.L.refx_qk_norm_rope_append_token(nq, nkv, 64, theta, eps, proj_row.ctypes.data, pos,
                                              _ptr(np.ascontiguousarray(q_norm, dtype=np.float32)),
                                              _ptr(np.ascontiguousarray(k_norm, dtype=np.float32)), q.ctypes.data,
                                              k.ctypes.data, v.ctypes.data, kv_dtype, int(exact))
        return q, k, v

    def int8_group_roundtrip(self, x):
        x = np.array(x, dtype=np.float32, copy=True)
        self.L.refx_int8_group_roundtrip(x.ctypes.data, x.size)
        return x

    def store(self, nkv, cap):
        return RefStore(self, nkv, cap)


class RefStore:
    """A reference KvStore: k/v [nkv][cap][256] float views (dequantized values)."""

    def __init__(self, ref, nkv, cap):
        self.ref, self.nkv, self.cap = ref, nkv, cap
        self.h = ref.L.refx_store_new(nkv, cap)
        n = nkv * cap * 256
        self.k = np.ctypeslib.as_array(ref.L.refx_store_k(self.h), shape=(n,)).reshape(nkv, cap, 256)
        self.v = np.ctypeslib.as_array(ref.L.refx_store_v(self.h), shape=(n,)).reshape(nkv, cap, 256)

    def attention_token(self, nq, q, gate, pos, exact=False):
        q = np.ascontiguousarray(q, dtype=np.float32)
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        out = np.empty(nq * 256, dtype=np.float32)
        self.ref.L.refx_attention_token(self.h, nq, self.nkv, q.ctypes.data, gate.ctypes.data, pos, out.ctypes.data,
                                        int(exact))
        return out

    def close(self):
        if self.h:
            self.ref.L.refx_store_free(self.h)
            self.h = None

    def __del__(self):
        self.close()
