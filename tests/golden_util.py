"""Loads tests/golden/config1.npz (written by tests/golden/make_config1.py from the reference's
own CPU ops) and lays its prior K/V into a paged pool with the reference byte layout."""
import os

import numpy as np

import q38a

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz")
NQ, NKV, HD, CTX = 24, 4, 256, 130
BLOCK_TABLE = np.array([[2, 0, 1]], np.int32)  # positions 0..130 on permuted pages


def load():
    return dict(np.load(GOLDEN, allow_pickle=False))


def put_row(pool, pos, codes_k, scales_k, codes_v, scales_v):
    pb = q38a.page_bytes(q38a.KV_INT8, NKV)
    page = pool[BLOCK_TABLE[0, pos // 64] * pb:(BLOCK_TABLE[0, pos // 64] + 1) * pb]
    for h in range(NKV):
        k, v, ks, vs = q38a.kv_offsets(q38a.KV_INT8, NKV, h, pos % 64)
        page[k:k + HD] = codes_k[h].view(np.uint8)
        page[v:v + HD] = codes_v[h].view(np.uint8)
        page[ks:ks + 8] = scales_k[h].view(np.uint8)
        page[vs:vs + 8] = scales_v[h].view(np.uint8)


def prior_pool(g):
    pool = np.zeros(q38a.page_bytes(q38a.KV_INT8, NKV) * 3, np.uint8)
    for pos in range(CTX):
        put_row(pool, pos, g["prior_k_codes"][pos], g["prior_k_scales"][pos], g["prior_v_codes"][pos],
                g["prior_v_scales"][pos])
    return pool


def expected_pool(g):
    pool = prior_pool(g)
    put_row(pool, CTX, g["k_codes"], g["k_scales"], g["v_codes"], g["v_scales"])
    return pool
