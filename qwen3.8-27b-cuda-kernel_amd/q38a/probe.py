"""ctypes binding of the measurement probes (include/q38a_probe.h): the MFMA issue ceiling and the
HBM read ceiling of the GPU the library runs on."""
import ctypes

from . import _check, lib

_p, _i, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_SIGS = {
    "q38a_probe_mfma": (_i, [_p, _i, _p, ctypes.POINTER(ctypes.c_double)]),
    "q38a_probe_read": (_i, [_p, _sz, _p, _i, _p]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args

EXPORTED = sorted(_SIGS)


def mfma(sink_ptr, iters, stream=0):
    """Launches the MFMA probe; returns the launch's dense fp16 flops."""
    flops = ctypes.c_double()
    _check(lib.q38a_probe_mfma(sink_ptr, iters, stream, ctypes.byref(flops)))
    return flops.value


def read(buf_ptr, nbytes, sink_ptr, sink_len, stream=0):
    """Launches the read probe over nbytes of device memory."""
    _check(lib.q38a_probe_read(buf_ptr, nbytes, sink_ptr, sink_len, stream))
