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
    rc = lib().elm_quantize_q8(C.c_void_p(w.ctypes.data), C.c_int64(n), C.c_int64(k), C.c_void_p(q.ctypes.data),
                               C.c_void_p(s.ctypes.data), C.c_int(_threads(threads)))
    if rc != 0:
        raise ValueError(f"elm_quantize_q8 refused shape {w.shape}")
    return q, s


def quantize_q4(w, threads=0):
    """edgelm quantize_q4: u8 [N,K/2] (16 bytes per 32-group) + f32 scale per (row, group)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, max(k, 0) // 2), np.uint8)
    s = np.empty((n, max(k, 0) // 32), np.float32)
    rc = lib().elm_quantize_q4(C.c_void_p(w.ctypes.data), C.c_int64(n), C.c_int64(k), C.c_void_p(q.ctypes.data),
                               C.c_void_p(s.ctypes.data), C.c_int(_threads(threads)))
    if rc != 0:
        raise ValueError(f"elm_quantize_q4 refused shape {w.shape} (K must be a positive multiple of 32)")
    return q, s


# ------------------------------------------------------------------ models and sessions

def _err():
    return lib().elm_last_error().decode()


def _setup():
    L = lib()
    if getattr(L, "_elm_typed", False):
        return L
    L.elm_last_error.restype = C.c_char_p
    L.elm_model_load.restype = C.c_void_p
    L.elm_model_load.argtypes = [C.c_char_p]
    L.elm_model_free.argtypes = [C.c_void_p]
    L.elm_session_create.restype = C.c_void_p
    L.elm_session_create.argtypes = [C.c_void_p, C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    L.elm_session_destroy.argtypes = [C.c_void_p]
    for f in ("elm_session_forward", "elm_session_prefill"):
        getattr(L, f).argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
    L.elm_session_reset.argtypes = [C.c_void_p]
    L.elm_session_pos.argtypes = [C.c_void_p]
    L.elm_session_describe.argtypes = [C.c_void_p, C.c_char_p, C.c_int]
    L.elm_session_generate.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_double),
                                       C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_void_p]
    L.elm_model_config.argtypes = [C.c_void_p, C.c_void_p]
    L.elm_model_fusion.argtypes = [C.c_void_p, C.c_void_p]
    L.elm_model_plan.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
    L.elm_model_partition.argtypes = [C.c_void_p, C.c_char_p, C.c_int, C.c_char_p, C.c_int]
    L._elm_typed = True
    return L


def partition_counts(desc):
    """{backend: (ops, partitions)} from the first line of describe_partitions
    ("<n> partitions | <backend>: <ops> ops in <parts> | ...")."""
    out = {}
    for part in desc.splitlines()[0].split(" | ")[1:]:
        name, rest = part.split(": ")
        w = rest.split()
        out[name] = (int(w[0]), int(w[3]))
    return out


class Model:
    """An .elm file loaded (memory-mapped) by the host library."""

    def __init__(self, path):
        L = _setup()
        self.h = L.elm_model_load(path.encode())
        if not self.h:
            raise RuntimeError(_err())
        cfg = np.zeros(10, np.int32)
        L.elm_model_config(self.h, cfg.ctypes.data)
        keys = ["vocab", "dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "max_seq", "dtype", "tied"]
        self.cfg = dict(zip(keys, (int(v) for v in cfg)))

    def fusion(self):
        o = np.zeros(6, np.int32)
        if _setup().elm_model_fusion(self.h, o.ctypes.data):
            raise RuntimeError(_err())
        return dict(zip(["swiglu", "shared_input", "residual", "rope", "ops_before", "ops_after"], (int(v) for v in o)))

    def plan(self, T, L=1, fuse=True):
        a, n = C.c_int64(), C.c_int64()
        rc = _setup().elm_model_plan(self.h, int(fuse), T, L, C.byref(a), C.byref(n))
        if rc < 0:
            raise RuntimeError(_err())
        return bool(rc), a.value, n.value

    def partition(self, backends, fuse=True):
        buf = C.create_string_buffer(4096)
        n = _setup().elm_model_partition(self.h, backends.encode(), int(fuse), buf, 4096)
        if n < 0:
            raise RuntimeError(_err())
        return n, buf.value.decode()

    def convert(self, dtype, threads=0):
        """Model::convert_weights: f32 weight matrices to "q8" or "q4" in memory (edgelm model.cpp:220-251)."""
        L = _setup()
        L.elm_model_convert.argtypes = [C.c_void_p, C.c_int, C.c_int]
        if L.elm_model_convert(self.h, {"f32": 0, "q8": 1, "q4": 2}[dtype], _threads(threads)):
            raise RuntimeError(_err())
        self.cfg["dtype"] = {"f32": 0, "q8": 1, "q4": 2}[dtype] if dtype != "f32" else self.cfg["dtype"]

    def prefault(self):
        L = _setup()
        L.elm_model_prefault.argtypes = [C.c_void_p]
        if L.elm_model_prefault(self.h):
            raise RuntimeError(_err())

    def write_device_image(self, path, threads=0):
        """Every q8 / q4 weight in the hip delegate's HBM layout, cached in one file; returns the count."""
        L = _setup()
        L.elm_model_write_device_image.argtypes = [C.c_void_p, C.c_char_p, C.c_int]
        n = L.elm_model_write_device_image(self.h, os.fsencode(path), _threads(threads))
        if n < 0:
            raise RuntimeError(_err())
        return n

    def attach_device_image(self, path):
        """Sessions made afterwards upload the weights from the image at `path`; False if it is missing or
        was written for other weights."""
        L = _setup()
        L.elm_model_attach_device_image.argtypes = [C.c_void_p, C.c_char_p]
        r = L.elm_model_attach_device_image(self.h, os.fsencode(path))
        if r < 0:
            raise RuntimeError(_err())
        return r == 1

    def weight(self, name):
        """(dtype, data, scales) of weight `name` as stored (after any conversion)."""
        L = _setup()
        L.elm_model_weight.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_void_p,
                                       C.c_void_p]
        rows, cols = C.c_int64(), C.c_int64()
        dt = L.elm_model_weight(self.h, name.encode(), C.byref(rows), C.byref(cols), None, None)
        if dt < 0:
            raise KeyError(name)
        r, c = rows.value, cols.value
        data = np.empty((r, c) if dt != 2 else (r, c // 2), {0: np.float32, 1: np.int8, 2: np.uint8}[dt])
        scales = None if dt == 0 else np.empty(r if dt == 1 else (r, c // 32), np.float32)
        L.elm_model_weight(self.h, name.encode(), None, None, data.ctypes.data, None if scales is None else scales.ctypes.data)
        return dt, data, scales

    def close(self):
        if self.h:
            _setup().elm_model_free(self.h)
            self.h = None


class Session:
    """edgelm Session on this build's runtime: backends e.g. "hip,cpu" (reference appended last)."""

    def __init__(self, model, backends="hip,cpu", threads=1, max_ctx=256, max_batch=128, all_logits=False,
                 act_quant=False, fuse=True):
        L = _setup()
        self.model = model
        self.vocab = model.cfg["vocab"]
        self.all_logits = all_logits
        self.max_batch = max_batch
        self.h = L.elm_session_create(model.h, backends.encode(), threads, max_ctx, max_batch, int(all_logits),
                                      int(act_quant), int(fuse))
        if not self.h:
            raise RuntimeError(_err())

    def forward(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = len(tokens) if self.all_logits else 1
        out = np.empty((rows, self.vocab), np.float32)
        if _setup().elm_session_forward(self.h, tokens.ctypes.data, len(tokens), out.ctypes.data):
            raise RuntimeError(_err())
        return out

    def reset(self):
        _setup().elm_session_reset(self.h)

    def pos(self):
        return _setup().elm_session_pos(self.h)

    def describe(self):
        buf = C.create_string_buffer(4096)
        n = _setup().elm_session_describe(self.h, buf, 4096)
        return n, buf.value.decode()

    def greedy(self, tokens):
        """Session::greedy: forward the tokens, then the argmax of the last logits row."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        nxt = C.c_int32()
        L = _setup()
        L.elm_session_greedy.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(C.c_int32)]
        if L.elm_session_greedy(self.h, tokens.ctypes.data, len(tokens), C.byref(nxt)):
            raise RuntimeError(_err())
        return nxt.value

    def greedy_steps(self, first, n):
        """Session::greedy_steps: n greedy decode steps from token `first`; the n tokens."""
        out = np.empty(n, np.int32)
        L = _setup()
        L.elm_session_greedy_steps.argtypes = [C.c_void_p, C.c_int32, C.c_int, C.c_void_p]
        if L.elm_session_greedy_steps(self.h, int(first), n, out.ctypes.data):
            raise RuntimeError(_err())
        return out

    def bench(self, prompt, warmup, steps):
        """bench.py's protocol (elm_session_bench): TTFT of the prompt, `warmup` untimed greedy decode steps,
        then `steps` timed ones."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        L = _setup()
        L.elm_session_bench.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double),
                                        C.POINTER(C.c_double), C.c_void_p]
        tt, dm = C.c_double(), C.c_double()
        toks = np.empty(1 + warmup + steps, np.int32)
        if L.elm_session_bench(self.h, prompt.ctypes.data, len(prompt), warmup, steps, C.byref(tt), C.byref(dm),
                               toks.ctypes.data):
            raise RuntimeError(_err())
        return dict(ttft_ms=tt.value, decode_ms=dm.value, tokens=toks)

    def generate(self, prompt, gen):
        """edgelm's bench protocol: prefill, argmax (TTFT), `gen` greedy decode steps."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        pm, tm, dm = C.c_double(), C.c_double(), C.c_double()
        toks = np.empty(gen + 1, np.int32)
        if _setup().elm_session_generate(self.h, prompt.ctypes.data, len(prompt), gen, C.byref(pm), C.byref(tm),
                                         C.byref(dm), toks.ctypes.data):
            raise RuntimeError(_err())
        return dict(prefill_ms=pm.value, ttft_ms=tm.value, decode_ms=dm.value, tokens=toks)

    def close(self):
        if self.h:
            _setup().elm_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
