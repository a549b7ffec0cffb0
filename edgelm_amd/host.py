"""ctypes bindings to ``libedgelm_host.so`` (the C API in ``include/edgelm_host.h``)."""
import ctypes as C
import os

import numpy as np

from .elmh import LIB_DIR, lib as _elmh_lib

HOST_SO = os.path.join(LIB_DIR, "libedgelm_host.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_SO):
            raise RuntimeError(f"host library missing: {HOST_SO} (run __graft_entry__.build())")
        _elmh_lib()  # libelmh first: the host library links against it
        _lib = C.CDLL(HOST_SO)
    return _lib


def _threads(threads):
    return threads or min(16, os.cpu_count() or 1)


def quantize_q8(w, threads=0):
    """edgelm quantize_q8: int8 [N,K] + f32 scale per row."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().elm_quantize_q8(C.c_void_p(w.ctypes.data), C.c_int64(n), C.c_int64(k), C.c_void_p(q.ctypes.data),
                          C.c_void_p(s.ctypes.data), C.c_int(_threads(threads)))
    return q, s


def quantize_q4(w, threads=0):
    """edgelm quantize_q4: u8 [N,K/2] (16 bytes per 32-group) + f32 scale per (row, group)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    if k % 32:
        raise ValueError("q4 needs K % 32 == 0")
    q = np.empty((n, k // 2), np.uint8)
    s = np.empty((n, k // 32), np.float32)
    lib().elm_quantize_q4(C.c_void_p(w.ctypes.data), C.c_int64(n), C.c_int64(k), C.c_void_p(q.ctypes.data),
                          C.c_void_p(s.ctypes.data), C.c_int(_threads(threads)))
    return q, s
