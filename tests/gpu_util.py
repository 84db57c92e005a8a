"""Device-side helpers for the GPU parity tests: torch tensors as plain device buffers, and the
descriptor structs of the C ABI filled from them. Every computation goes through libq38a."""
import numpy as np
import torch

import q38a

NQ, NKV, HD = 24, 4, 256
LD = 2 * (NQ + NKV) * HD  # proj row: q | gate | k | v


def dev(a):
    """numpy array -> device tensor with the same bytes (uint16 travels as int16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def stream():
    return torch.cuda.current_stream().cuda_stream


class Batch:
    """Ragged batch metadata on the device: seqs = [(slot, pos0, n), ...]."""

    def __init__(self, seqs):
        self.seqs = list(seqs)
        self.seq_start = np.zeros(len(seqs) + 1, np.int32)
        self.seq_slot = np.array([s for s, _, _ in seqs], np.int32)
        self.seq_pos0 = np.array([p for _, p, _ in seqs], np.int32)
        tok_pos, tok_seq = [], []
        for b, (_, p0, n) in enumerate(seqs):
            self.seq_start[b + 1] = self.seq_start[b] + n
            tok_pos += list(range(p0, p0 + n))
            tok_seq += [b] * n
        self.tok_pos = np.array(tok_pos, np.int32)
        self.tok_seq = np.array(tok_seq, np.int32)
        self._d = [dev(x) for x in (self.seq_start, self.seq_slot, self.seq_pos0, self.tok_pos, self.tok_seq)]
        self.M = int(self.seq_start[-1])
        self.desc = q38a.BatchDesc(len(seqs), self.M, max(n for _, _, n in seqs),
                                   *[t.data_ptr() for t in self._d])


class Pool:
    """A page pool of `layers` attention layers in a torch buffer, plus its block table."""

    def __init__(self, dtype, num_pages, block_table, layers=1, nkv=NKV, fill=None):
        self.dtype, self.nkv, self.layers, self.num_pages = dtype, nkv, layers, num_pages
        self.page_bytes = q38a.page_bytes(dtype, nkv)
        self.layer_stride = self.page_bytes * num_pages
        self.bt = np.ascontiguousarray(block_table, np.int32)
        if fill is None:
            self.host = np.zeros(self.layer_stride * layers, np.uint8)
        else:
            self.host = np.ascontiguousarray(fill, np.uint8).copy()
        self.t = dev(self.host)
        self.bt_t = dev(self.bt)
        self.desc = q38a.KvCacheDesc(self.t.data_ptr(), dtype, nkv, num_pages, self.page_bytes, self.layer_stride,
                                     self.bt_t.data_ptr(), self.bt.shape[1])

    def layer_host(self, layer=0):
        return self.host[layer * self.layer_stride:(layer + 1) * self.layer_stride]

    def download(self, layer=0):
        a = host(self.t)
        return a[layer * self.layer_stride:(layer + 1) * self.layer_stride]


def rope_dev(rows, theta=1e7):
    return dev(q38a.rope_table(0, rows, theta))


def append_params(proj_t, q_norm_t, k_norm_t, q_out_t, rope_t, layer=0, nq=NQ, nkv=NKV, ld=LD, eps=1e-6):
    return q38a.QkNormRopeParams(proj_t.data_ptr(), ld, q_norm_t.data_ptr(), k_norm_t.data_ptr(), eps, 1e7, nq, nkv,
                                 q_out_t.data_ptr(), layer, rope_t.data_ptr(), rope_t.shape[0])


def attention_params(q_t, proj_t, out_t, scratch_t, max_splits, layer=0, nq=NQ, nkv=NKV, ld=LD):
    gate_ptr = proj_t.data_ptr() + nq * HD * 2
    return q38a.AttentionParams(q_t.data_ptr(), gate_ptr, ld, out_t.data_ptr(), nq, nkv, layer,
                                scratch_t.data_ptr() if scratch_t is not None else None, max_splits)


def paged_layout(rng, lengths, extra_pages=0):
    """Block table [B][max_pages] mapping each sequence's pages to a random permutation of the pool."""
    pages = [max(1, -(-n // 64)) for n in lengths]
    total = sum(pages) + extra_pages
    perm = rng.permutation(total).astype(np.int32)
    bt = np.zeros((len(lengths), max(pages)), np.int32)
    o = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[o:o + p]
        o += p
    return bt, total


_hip = None


def memcpy(dst, src, nbytes):
    """Synchronous copy between raw addresses (host or device) through the HIP runtime torch loaded."""
    global _hip
    import ctypes
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    torch.cuda.synchronize()
    rc = _hip.hipMemcpy(dst, src, nbytes, 4)  # hipMemcpyDefault
    assert rc == 0, f"hipMemcpy failed: {rc}"


def to_device_ptr(ptr, array):
    a = np.ascontiguousarray(array)
    memcpy(ptr, a.ctypes.data, a.nbytes)


def from_device_ptr(ptr, shape, dtype):
    a = np.empty(shape, dtype)
    memcpy(a.ctypes.data, ptr, a.nbytes)
    return a
