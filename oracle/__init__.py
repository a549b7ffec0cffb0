"""TEST INFRASTRUCTURE ONLY: ctypes bindings to the CPU oracle.

Two libraries, both built by ``oracle/Makefile`` (called from ``__graft_entry__.build()``):

* ``liboracle.so`` — this build's plain-C restatement of edgelm's algorithms for the
  quantized-matmul path (``oracle/oracle.c``; each function cites reference file:line).
* ``_ref/libedgelm_ref.so`` — edgelm's own C++ compiled from its sources (plus the
  ``ref_shim.cpp`` C wrappers). Present only where it was built; the built file travels with
  the tree.
* ``_ref/libedgelm_ref_hip.so`` — the same, with the ``hip`` delegate registered in edgelm's
  ``make_backend`` at link time (``ref_hip_registration.cpp``): edgelm's own Session, partitioner
  and backends driving the delegate, for the boundary tests.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package, and only as the checker or the CPU baseline. The product (``edgelm_amd``)
never imports it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libedgelm_ref.so")
REF_HIP_SO = os.path.join(HERE, "_ref", "libedgelm_ref_hip.so")

F32, Q8, Q4 = 0, 1, 2

_P = C.c_void_p
_I64 = C.c_int64


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class _OrcWeight(C.Structure):
    _fields_ = [("dtype", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64), ("data", C.c_void_p),
                ("scales", C.c_void_p)]


_orc = None
_ref = None
_ref_hip = None


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (run __graft_entry__.build())")
        _orc = C.CDLL(ORACLE_SO)
        _orc.orc_round_away.restype = C.c_float
        _orc.orc_round_away.argtypes = [C.c_float]
        _orc.orc_silu.restype = C.c_float
        _orc.orc_silu.argtypes = [C.c_float]
        _orc.orc_argmax.restype = C.c_int32
    return _orc


def ref_available():
    return os.path.exists(REF_SO)


def _type_ref(lib):
    lib.eref_pool_create.restype = C.c_void_p
    lib.eref_pool_create.argtypes = [C.c_int, C.c_int, C.c_int64]
    lib.eref_pool_destroy.argtypes = [C.c_void_p]
    lib.eref_session_create.restype = C.c_void_p
    lib.eref_session_create.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    for f in ("eref_session_destroy", "eref_session_reset", "eref_session_vocab"):
        getattr(lib, f).argtypes = [C.c_void_p]
    lib.eref_last_error.restype = C.c_char_p
    lib.eref_argmax.restype = C.c_int32
    return lib


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference build missing: {REF_SO}")
        _ref = _type_ref(C.CDLL(REF_SO))
    return _ref


def ref_hip_available():
    return os.path.exists(REF_HIP_SO)


def ref_hip():
    """edgelm's own runtime with the hip delegate registered (loads libelmh.so, which needs no GPU to load)."""
    global _ref_hip
    if _ref_hip is None:
        if not ref_hip_available():
            raise RuntimeError(f"reference build with the hip backend missing: {REF_HIP_SO}")
        _ref_hip = _type_ref(C.CDLL(REF_HIP_SO))
        _ref_hip.erefhip_partition.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_char_p, C.c_int]
    return _ref_hip


def partition_counts(desc):
    """{backend: (ops, partitions)} from edgelm's describe_partitions (backends.cpp:184-201):
    "<n> partitions: <backend> <ops> ops in <parts>; ..."."""
    head = desc.splitlines()[0].split(":", 1)[1]
    out = {}
    for part in head.split(";"):
        w = part.split()
        if len(w) >= 5:
            out[w[0]] = (int(w[1]), int(w[4]))
    return out


def ref_convert_weight(path, dtype, name, data_cap=1 << 26, scale_cap=1 << 24):
    """edgelm's Model::load + convert_weights(dtype: 1 q8, 2 q4) on the file, then weight `name` as edgelm
    holds it: (dtype, data bytes, scale bytes)."""
    lib = ref()
    lib.eref_convert_weight.argtypes = [C.c_char_p, C.c_int, C.c_char_p, C.c_void_p, C.POINTER(C.c_int64), C.c_void_p,
                                        C.POINTER(C.c_int64)]
    data, scales = np.empty(data_cap, np.uint8), np.empty(scale_cap, np.uint8)
    nd, ns = C.c_int64(data_cap), C.c_int64(scale_cap)
    dt = lib.eref_convert_weight(path.encode(), dtype, name.encode(), data.ctypes.data, C.byref(nd), scales.ctypes.data,
                                 C.byref(ns))
    if dt < 0:
        raise RuntimeError(lib.eref_last_error().decode())
    return dt, data[:nd.value].copy(), scales[:ns.value].copy()


def ref_hip_partition(path, backends, fuse=True):
    """edgelm's partition_graph over the model with the delegate's claims (planning only, no device)."""
    buf = C.create_string_buffer(4096)
    n = ref_hip().erefhip_partition(path.encode(), backends.encode(), int(fuse), buf, 4096)
    if n < 0:
        raise RuntimeError("erefhip_partition failed")
    return n, buf.value.decode()


class Weight:
    """A quantized (or f32) weight held in host numpy arrays, in edgelm's export layout."""

    def __init__(self, dtype, rows, cols, data, scales=None):
        self.dtype, self.rows, self.cols = dtype, int(rows), int(cols)
        self.data = np.ascontiguousarray(data)
        self.scales = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)

    def orc(self):
        return _OrcWeight(self.dtype, self.rows, self.cols, self.data.ctypes.data,
                          None if self.scales is None else self.scales.ctypes.data)


# ------------------------------------------------------------------ C restatement

def quantize_q8(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    orc().orc_quantize_q8(_ptr(w), _I64(n), _I64(k), _ptr(q), _ptr(s))
    return q, s


def quantize_q4(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k // 2), np.uint8)
    s = np.empty((n, k // 32), np.float32)
    orc().orc_quantize_q4(_ptr(w), _I64(n), _I64(k), _ptr(q), _ptr(s))
    return q, s


def make_weight(w, dtype):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    if dtype == F32:
        return Weight(F32, n, k, w)
    q, s = quantize_q8(w) if dtype == Q8 else quantize_q4(w)
    return Weight(dtype, n, k, q, s)


def dequantize(wt):
    out = np.empty((wt.rows, wt.cols), np.float32)
    ow = wt.orc()
    for r in range(wt.rows):
        orc().orc_dequantize_row(C.byref(ow), _I64(r), _ptr(out[r]))
    return out


def quantize_act(x):
    """Per-row, per-32-block int8 activations: (q int8 [T,K], d f32 [T,K/32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    d = np.empty((T, K // 32), np.float32)
    for t in range(T):
        orc().orc_quantize_act_row(_ptr(x[t]), _I64(K), _ptr(q[t]), _ptr(d[t]))
    return q, d


def quantize_act_token(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    d = np.empty(T, np.float32)
    for t in range(T):
        orc().orc_quantize_act_row_token(_ptr(x[t]), _I64(K), _ptr(q[t]), _ptr(d[t:t + 1]))
    return q, d


def ref_matmul(x, w, residual=None, act_quant=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, w.rows), np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    ow = w.orc()
    orc().orc_ref_matmul(_ptr(x), C.c_int(T), C.byref(ow), _ptr(y), _ptr(res), C.c_int(int(act_quant)))
    return y


def ref_swiglu(x, wg, wu, act_quant=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, wg.rows), np.float32)
    g, u = wg.orc(), wu.orc()
    orc().orc_ref_swiglu(_ptr(x), C.c_int(T), C.byref(g), C.byref(u), _ptr(y), C.c_int(int(act_quant)))
    return y


def cpu_matmul(x, weights, residuals=None, act_quant=False):
    """edgelm cpu::matmul (x86 scalar path) over targets; returns a list of outputs."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    n = len(weights)
    arr = (_OrcWeight * n)(*[w.orc() for w in weights])
    ys = [np.empty((T, w.rows), np.float32) for w in weights]
    yp = (C.c_void_p * n)(*[y.ctypes.data for y in ys])
    if residuals is not None:
        residuals = [None if r is None else np.ascontiguousarray(r, dtype=np.float32) for r in residuals]
        rp = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in residuals])
    else:
        rp = None
    orc().orc_cpu_matmul(_ptr(x), C.c_int(T), C.c_int(n), arr, yp, rp, C.c_int(int(act_quant)))
    return ys


def cpu_swiglu(x, wg, wu, act_quant=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, wg.rows), np.float32)
    g, u = wg.orc(), wu.orc()
    orc().orc_cpu_swiglu(_ptr(x), C.c_int(T), C.byref(g), C.byref(u), _ptr(y), C.c_int(int(act_quant)))
    return y


def block_sums(xq, w):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    T = xq.shape[0]
    S = np.empty((T, w.rows, w.cols // 32), np.int32)
    ow = w.orc()
    orc().orc_block_sums(_ptr(xq), C.c_int(T), C.byref(ow), _ptr(S))
    return S


def matmul_a8_token(x, w, residual=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, w.rows), np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    ow = w.orc()
    orc().orc_matmul_a8_token(_ptr(x), C.c_int(T), C.byref(ow), _ptr(y), _ptr(res))
    return y


def silu(v):
    return orc().orc_silu(C.c_float(v))


# ------------------------------------------------------------------ layer ops (cpu backend)

def _layer_call(lib, prefix, q, k, v, pos0, n_heads, n_kv, kc, vc, rope_arg):
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    T = q.shape[0]
    hd = q.shape[1] // n_heads
    out = np.empty_like(q)
    args = [_ptr(q), _ptr(k), _ptr(v), _ptr(out), C.c_int(T), C.c_int(pos0), C.c_int(n_heads), C.c_int(n_kv),
            C.c_int(hd), _ptr(kc), _ptr(vc), C.c_int(kc.shape[1])] + rope_arg
    getattr(lib, prefix + "_attention")(*args)
    return out


def rope_table(head_dim, max_pos, theta):
    """kernels_ref.cpp:11-21: (cos, sin) [max_pos, head_dim/2]."""
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    orc().orc_rope_table(C.c_int(head_dim), C.c_int(max_pos), C.c_float(theta), _ptr(c), _ptr(s))
    return c, s


def rmsnorm(x, w, eps):
    """cpu::rmsnorm (kernels_cpu.cpp:326-335), x86 scalar dot_f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    orc().orc_rmsnorm(_ptr(x), _ptr(w), _ptr(y), C.c_int(x.shape[0]), C.c_int(x.shape[1]), C.c_float(eps))
    return y


def attention(q, k, v, pos0, n_heads, n_kv, kc, vc, rope=None):
    """cpu::attention (kernels_cpu.cpp:417-488). kc/vc: float32 [n_kv, max_ctx, hd] caches, updated
    in place. rope: (cos, sin) from rope_table, or None."""
    r = [None, None] if rope is None else [np.ascontiguousarray(rope[0]), np.ascontiguousarray(rope[1])]
    return _layer_call(orc(), "orc", q, k, v, pos0, n_heads, n_kv, kc, vc, [_ptr(r[0]), _ptr(r[1])])


# ------------------------------------------------------------------ edgelm's own C++ (oracle/_ref)

def rq_rope_table(head_dim, max_pos, theta):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    ref().eref_rope_table(C.c_int(head_dim), C.c_int(max_pos), C.c_float(theta), _ptr(c), _ptr(s))
    return c, s


def rq_rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    ref().eref_rmsnorm(_ptr(x), _ptr(w), _ptr(y), C.c_int(x.shape[0]), C.c_int(x.shape[1]), C.c_float(eps))
    return y


def rq_attention(q, k, v, pos0, n_heads, n_kv, kc, vc, theta=None):
    """edgelm's cpu::attention; theta None: no rotary embedding, else a RopeTable(hd, max_ctx, theta)."""
    return _layer_call(ref(), "eref", q, k, v, pos0, n_heads, n_kv, kc, vc,
                       [C.c_int(0 if theta is None else 1), C.c_float(0.0 if theta is None else theta)])


def rq_quantize_q8(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    ref().eref_quantize_q8(_ptr(w), _I64(n), _I64(k), _ptr(q), _ptr(s))
    return q, s


def rq_quantize_q4(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k // 2), np.uint8)
    s = np.empty((n, k // 32), np.float32)
    ref().eref_quantize_q4(_ptr(w), _I64(n), _I64(k), _ptr(q), _ptr(s))
    return q, s


def rq_quantize_act(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    d = np.empty((T, K // 32), np.float32)
    for t in range(T):
        ref().eref_quantize_act_row(_ptr(x[t]), _I64(K), _ptr(q[t]), _ptr(d[t]))
    return q, d


def rq_ref_matmul(x, w, residual=None, act_quant=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, w.rows), np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    ref().eref_ref_matmul(_ptr(x), C.c_int(T), C.c_int(w.dtype), _I64(w.rows), _I64(w.cols), _ptr(w.data),
                          _ptr(w.scales), _ptr(y), _ptr(res), C.c_int(int(act_quant)))
    return y


def rq_ref_swiglu(x, wg, wu, act_quant=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, wg.rows), np.float32)
    ref().eref_ref_swiglu(_ptr(x), C.c_int(T), C.c_int(wg.dtype), C.c_int(wu.dtype), _I64(wg.rows), _I64(wg.cols),
                          _ptr(wg.data), _ptr(wg.scales), _ptr(wu.data), _ptr(wu.scales), _ptr(y),
                          C.c_int(int(act_quant)))
    return y


class RefPool:
    """edgelm ThreadPool + per-thread scratch, sized for max_T tokens and max_k."""

    def __init__(self, threads, max_T, max_k):
        self.h = ref().eref_pool_create(threads, max_T, max_k)

    def close(self):
        if self.h:
            ref().eref_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rq_cpu_matmul(pool, x, weights, residuals=None, act_quant=False, out=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    n = len(weights)
    K = weights[0].cols
    dt = (C.c_int * n)(*[w.dtype for w in weights])
    rows = (C.c_int64 * n)(*[w.rows for w in weights])
    data = (C.c_void_p * n)(*[w.data.ctypes.data for w in weights])
    sc = (C.c_void_p * n)(*[None if w.scales is None else w.scales.ctypes.data for w in weights])
    ys = out if out is not None else [np.empty((T, w.rows), np.float32) for w in weights]
    yp = (C.c_void_p * n)(*[y.ctypes.data for y in ys])
    rp = None
    if residuals is not None:
        rp = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in residuals])
    rc = ref().eref_cpu_matmul(C.c_void_p(pool.h), _ptr(x), C.c_int(T), C.c_int(n), dt, rows, _I64(K), data, sc, yp,
                               rp, C.c_int(int(act_quant)))
    if rc:
        raise RuntimeError(ref().eref_last_error().decode())
    return ys


def rq_cpu_swiglu(pool, x, wg, wu, act_quant=False, out=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = out if out is not None else np.empty((T, wg.rows), np.float32)
    rc = ref().eref_cpu_swiglu(C.c_void_p(pool.h), _ptr(x), C.c_int(T), C.c_int(wg.dtype), C.c_int(wu.dtype),
                               _I64(wg.rows), _I64(wg.cols), _ptr(wg.data), _ptr(wg.scales), _ptr(wu.data),
                               _ptr(wu.scales), _ptr(y), C.c_int(int(act_quant)))
    if rc:
        raise RuntimeError(ref().eref_last_error().decode())
    return y


def rq_time_cpu_op(threads, x, weights, residuals=None, act_quant=True, swiglu=False, warm=1, min_reps=3,
                   max_reps=200, budget_s=0.3):
    """edgelm's cpu::matmul over `weights` (MATMUL / MATMUL_N / MATMUL_ADD), or cpu::swiglu of weights[0]
    (gate) and weights[1] (up), on edgelm's ThreadPool of `threads`, timed in C (eref_time_cpu_op): `warm`
    untimed calls, then calls for `budget_s` seconds (min_reps .. max_reps); (median ms per call, calls)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    n = len(weights)
    dt = (C.c_int * n)(*[w.dtype for w in weights])
    rows = (C.c_int64 * n)(*[w.rows for w in weights])
    data = (C.c_void_p * n)(*[w.data.ctypes.data for w in weights])
    sc = (C.c_void_p * n)(*[None if w.scales is None else w.scales.ctypes.data for w in weights])
    ys = [np.empty((T, w.rows), np.float32) for w in weights]
    yp = (C.c_void_p * n)(*[y.ctypes.data for y in ys])
    rp = None
    if residuals is not None:
        rp = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in residuals])
    med, reps = C.c_double(), C.c_int()
    rc = ref().eref_time_cpu_op(C.c_int(1 if swiglu else 0), C.c_int(threads), _ptr(x), C.c_int(T), C.c_int(n), dt,
                                rows, _I64(weights[0].cols), data, sc, yp, rp, C.c_int(int(act_quant)), C.c_int(warm),
                                C.c_int(min_reps), C.c_int(max_reps), C.c_double(budget_s), C.byref(med),
                                C.byref(reps))
    if rc:
        raise RuntimeError(ref().eref_last_error().decode())
    return med.value, reps.value


class RefSession:
    """edgelm's own Session over an .elm file (loader, fusion passes, partitioner, backends)."""

    def __init__(self, path, backends="cpu", threads=1, max_ctx=256, max_batch=128, all_logits=False,
                 act_quant=False, fuse=True, with_hip=False):
        """with_hip: edgelm's runtime built with the hip delegate registered (libedgelm_ref_hip.so), so
        backends may name "hip" / "hip-matmul" next to edgelm's own "cpu", "matmul-only", "reference"."""
        self.lib = ref_hip() if with_hip else ref()
        self.h = self.lib.eref_session_create(path.encode(), backends.encode(), threads, max_ctx, max_batch,
                                              int(all_logits), int(act_quant), int(fuse))
        if not self.h:
            raise RuntimeError(self.lib.eref_last_error().decode())
        self.vocab = self.lib.eref_session_vocab(C.c_void_p(self.h))
        self.all_logits = all_logits

    def forward(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        rows = n if self.all_logits else 1
        out = np.empty((rows, self.vocab), np.float32)
        if self.lib.eref_session_forward(C.c_void_p(self.h), _ptr(tokens), C.c_int(n), _ptr(out)):
            raise RuntimeError(self.lib.eref_last_error().decode())
        return out

    def reset(self):
        self.lib.eref_session_reset(C.c_void_p(self.h))

    def bench(self, prompt, warmup, steps):
        """bench.py's protocol on edgelm's Session, timed in C (eref_session_bench)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        tt, dm = C.c_double(), C.c_double()
        toks = np.empty(1 + warmup + steps, np.int32)
        self.lib.eref_session_bench.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                                C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_void_p]
        if self.lib.eref_session_bench(C.c_void_p(self.h), _ptr(prompt), len(prompt), warmup, steps, C.byref(tt),
                                       C.byref(dm), _ptr(toks)):
            raise RuntimeError(self.lib.eref_last_error().decode())
        return dict(ttft_ms=tt.value, decode_ms=dm.value, tokens=toks)

    def describe(self):
        buf = C.create_string_buffer(4096)
        nops = self.lib.eref_session_describe(C.c_void_p(self.h), buf, 4096)
        return nops, buf.value.decode()

    def close(self):
        if self.h:
            self.lib.eref_session_destroy(C.c_void_p(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def argmax(x):
    """argmax of each row of x (tokenizer.cpp:187-189, restated in orc_argmax)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    return np.array([orc().orc_argmax(_ptr(r), _I64(x.shape[1])) for r in x], np.int32)


def rq_argmax(x):
    """edgelm's own argmax (oracle/_ref) on each row of x."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    return np.array([ref().eref_argmax(_ptr(r), C.c_int(x.shape[1])) for r in x], np.int32)
