"""ctypes bindings to ``libelmh.so`` (the C ABI in ``include/elmh.h``).

The HIP library is required: loading fails loudly if it is missing, and there is no CPU
fallback anywhere in this package.
"""
import ctypes as C
import os

import numpy as np

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
ELMH_SO = os.path.join(LIB_DIR, "libelmh.so")

OK, ERR_ARG, ERR_HIP, ERR_NODEV, ERR_UNSUPPORTED, ERR_OOM = range(6)
F32, Q8, Q4 = 0, 1, 2
ACT_F32, ACT_INT8, ACT_INT8_TOKEN = 0, 1, 2
EXACT, FAST = 0, 1

_lib = None


class ElmhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"elmh error {code}: {msg}")
        self.code = code


def lib():
    """The loaded libelmh; raises if the HIP library was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(ELMH_SO):
            raise RuntimeError(f"HIP library missing: {ELMH_SO} (run __graft_entry__.build())")
        L = C.CDLL(ELMH_SO)
        L.elmh_last_error.restype = C.c_char_p
        L.elmh_last_error.argtypes = [C.c_void_p]
        L.elmh_device_arch.restype = C.c_char_p
        L.elmh_device_arch.argtypes = [C.c_void_p]
        L.elmh_stream.restype = C.c_void_p
        L.elmh_stream.argtypes = [C.c_void_p]
        L.elmh_weight_bytes.restype = C.c_size_t
        L.elmh_weight_bytes.argtypes = [C.c_void_p]
        L.elmh_destroy.argtypes = [C.c_void_p]
        L.elmh_destroy.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def device_count():
    n = C.c_int(0)
    lib().elmh_device_count(C.byref(n))
    return n.value


def weight_layout(dtype, rows, cols):
    """(H, data bytes, scale bytes) of a weight's repacked HBM layout (pure host call, no GPU)."""
    H, db, sb = C.c_int(), C.c_size_t(), C.c_size_t()
    rc = lib().elmh_weight_layout(C.c_int(dtype), C.c_int64(rows), C.c_int64(cols), C.byref(H), C.byref(db), C.byref(sb))
    if rc:
        raise ElmhError(rc, lib().elmh_last_error(None).decode())
    return H.value, db.value, sb.value


def repack_host(dtype, rows, cols, data, scales):
    """edgelm's export layout -> the repacked HBM layout, on the CPU: (data bytes, scales) as numpy arrays."""
    _, db, sb = weight_layout(dtype, rows, cols)
    data, scales = np.ascontiguousarray(data), np.ascontiguousarray(scales, dtype=np.float32)
    out, out_s = np.empty(db, np.uint8), np.empty(sb // 4, np.float32)
    rc = lib().elmh_repack_host(C.c_int(dtype), C.c_int64(rows), C.c_int64(cols), _p(data), _p(scales), _p(out), _p(out_s))
    if rc:
        raise ElmhError(rc, lib().elmh_last_error(None).decode())
    return out, out_s


class DevWeight:
    """A weight resident in HBM (repacked). ``free()`` or context teardown releases it."""

    def __init__(self, ctx, handle, dtype, rows, cols):
        self.ctx, self.h, self.dtype, self.rows, self.cols = ctx, handle, dtype, rows, cols

    @property
    def nbytes(self):
        return lib().elmh_weight_bytes(self.h)

    def free(self):
        if self.h:
            lib().elmh_free_weight(self.ctx.h, self.h)
            self.h = None


class DevBuffer:
    """Raw device memory owned by a context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        ctx._check(lib().elmh_malloc(ctx.h, C.c_size_t(self.nbytes), C.byref(p)))
        self.ptr = p.value

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        self.ctx._check(lib().elmh_memcpy_h2d(self.ctx.h, C.c_void_p(self.ptr), _p(arr), C.c_size_t(arr.nbytes)))
        return self

    def download(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        self.ctx._check(lib().elmh_memcpy_d2h(self.ctx.h, _p(out), C.c_void_p(self.ptr), C.c_size_t(out.nbytes)))
        return out

    def free(self):
        if self.ptr:
            lib().elmh_free(self.ctx.h, C.c_void_p(self.ptr))
            self.ptr = None


class Context:
    """One device + one HIP stream (``elmh_create``)."""

    def __init__(self, device=0):
        h = C.c_void_p()
        rc = lib().elmh_create(C.c_int(device), C.byref(h))
        if rc:
            raise ElmhError(rc, lib().elmh_last_error(None).decode())
        self.h = h

    def close(self):
        if self.h:
            lib().elmh_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc:
            raise ElmhError(rc, lib().elmh_last_error(self.h).decode())

    @property
    def arch(self):
        return lib().elmh_device_arch(self.h).decode()

    # ---- weights
    def upload(self, dtype, rows, cols, data, scales):
        data = np.ascontiguousarray(data)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        h = C.c_void_p()
        self._check(lib().elmh_upload_weight(self.h, C.c_int(dtype), C.c_int64(rows), C.c_int64(cols), _p(data),
                                             _p(scales), C.byref(h)))
        return DevWeight(self, h, dtype, rows, cols)

    # ---- host-pointer ops (synchronous)
    def upload_image(self, dtype, rows, cols, data, scales):
        """A weight already in the repacked layout (repack_host's output)."""
        data = np.ascontiguousarray(data)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        h = C.c_void_p()
        self._check(lib().elmh_upload_weight_image(self.h, C.c_int(dtype), C.c_int64(rows), C.c_int64(cols), _p(data),
                                                   _p(scales), C.byref(h)))
        return DevWeight(self, h, dtype, rows, cols)

    def download_image(self, w):
        """(data bytes, scales) of a weight's repacked layout in HBM."""
        _, db, sb = weight_layout(w.dtype, w.rows, w.cols)
        out, out_s = np.empty(db, np.uint8), np.empty(sb // 4, np.float32)
        self._check(lib().elmh_download_weight_image(self.h, w.h, _p(out), _p(out_s)))
        return out, out_s

    def matmul(self, x, weights, residuals=None, act=ACT_INT8, mode=EXACT):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, K = x.shape
        n = len(weights)
        ys = [np.empty((T, w.rows), np.float32) for w in weights]
        wp = (C.c_void_p * n)(*[w.h.value if isinstance(w.h, C.c_void_p) else w.h for w in weights])
        yp = (C.c_void_p * n)(*[y.ctypes.data for y in ys])
        rp = None
        if residuals is not None:
            residuals = [None if r is None else np.ascontiguousarray(r, dtype=np.float32) for r in residuals]
            rp = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in residuals])
        self._check(lib().elmh_matmul(self.h, _p(x), C.c_int(T), C.c_int64(K), C.c_int(n), wp, yp, rp, C.c_int(act),
                                      C.c_int(mode)))
        return ys

    def swiglu(self, x, wg, wu, act=ACT_INT8, mode=EXACT):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, K = x.shape
        y = np.empty((T, wg.rows), np.float32)
        self._check(lib().elmh_swiglu(self.h, _p(x), C.c_int(T), C.c_int64(K), wg.h, wu.h, _p(y), C.c_int(act),
                                      C.c_int(mode)))
        return y

    def quantize_act(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, K = x.shape
        q = np.empty((T, K), np.int8)
        d = np.empty((T, K // 32), np.float32)
        self._check(lib().elmh_quantize_act(self.h, _p(x), C.c_int(T), C.c_int64(K), _p(q), _p(d)))
        return q, d

    def block_sums(self, xq, w):
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        T = xq.shape[0]
        S = np.empty((T, w.rows, w.cols // 32), np.int32)
        self._check(lib().elmh_block_sums(self.h, _p(xq), C.c_int(T), w.h, _p(S)))
        return S

    # ---- device-resident ops (asynchronous on the context stream)
    def reserve(self, max_T, max_K):
        self._check(lib().elmh_reserve(self.h, C.c_int(max_T), C.c_int64(max_K)))

    def matmul_dev(self, x_ptr, T, K, weights, y_ptrs, res_ptrs=None, act=ACT_INT8, mode=EXACT):
        n = len(weights)
        wp = (C.c_void_p * n)(*[w.h.value for w in weights])
        yp = (C.c_void_p * n)(*y_ptrs)
        rp = None if res_ptrs is None else (C.c_void_p * n)(*res_ptrs)
        self._check(lib().elmh_matmul_dev(self.h, C.c_void_p(x_ptr), C.c_int(T), C.c_int64(K), C.c_int(n), wp, yp, rp,
                                          C.c_int(act), C.c_int(mode)))

    def matmul_noalloc_dev(self, x_ptr, T, K, weights, y_ptrs, res_ptrs=None, act=ACT_INT8, mode=EXACT):
        """elmh_matmul_noalloc_dev: matmul_dev with the activation in the library's fixed scratch array."""
        n = len(weights)
        wp = (C.c_void_p * n)(*[w.h.value for w in weights])
        yp = (C.c_void_p * n)(*y_ptrs)
        rp = None if res_ptrs is None else (C.c_void_p * n)(*res_ptrs)
        self._check(lib().elmh_matmul_noalloc_dev(self.h, C.c_void_p(x_ptr), C.c_int(T), C.c_int64(K), C.c_int(n), wp,
                                                  yp, rp, C.c_int(act), C.c_int(mode)))

    def swiglu_dev(self, x_ptr, T, K, wg, wu, y_ptr, act=ACT_INT8, mode=EXACT):
        self._check(lib().elmh_swiglu_dev(self.h, C.c_void_p(x_ptr), C.c_int(T), C.c_int64(K), wg.h, wu.h,
                                          C.c_void_p(y_ptr), C.c_int(act), C.c_int(mode)))

    def swiglu_quant_dev(self, x_ptr, T, K, wg, wu, y_ptr, q_ptr, d_ptr, s_ptr):
        """FFN_SWIGLU (int8 activations, exact) into y, and y quantized as quantize_act_dev would (q, d, s)."""
        self._check(lib().elmh_swiglu_quant_dev(self.h, C.c_void_p(x_ptr), C.c_int(T), C.c_int64(K), wg.h, wu.h,
                                                C.c_void_p(y_ptr), C.c_void_p(q_ptr), C.c_void_p(d_ptr),
                                                C.c_void_p(s_ptr)))

    def ffn_dev(self, x_ptr, T, K, wg, wu, h_ptr, wd, y_ptr, res_ptr=None, norm_w_ptr=None, eps=1e-5, act=ACT_INT8,
                mode=EXACT):
        """FFN_SWIGLU (after RMSNORM with norm_w) into h, then MATMUL(_ADD) of h by wd into y; returns whether
        the SwiGLU launch quantized h for the down projection."""
        self._check(lib().elmh_ffn_dev(self.h, C.c_void_p(x_ptr), C.c_void_p(norm_w_ptr), C.c_float(eps), C.c_int(T),
                                       C.c_int64(K), wg.h, wu.h, C.c_void_p(h_ptr), wd.h, C.c_void_p(y_ptr),
                                       C.c_void_p(res_ptr), C.c_int(act), C.c_int(mode)))
        return bool(lib().elmh_ffn_fused(self.h))

    def quantize_act_dev(self, x_ptr, T, K, q_ptr, d_ptr, s_ptr):
        self._check(lib().elmh_quantize_act_dev(self.h, C.c_void_p(x_ptr), C.c_int(T), C.c_int64(K), C.c_void_p(q_ptr),
                                                C.c_void_p(d_ptr), C.c_void_p(s_ptr)))

    def gemv_a8_dev(self, q_ptr, d_ptr, s_ptr, T, K, weights, y_ptrs, res_ptrs=None):
        n = len(weights)
        wp = (C.c_void_p * n)(*[w.h.value for w in weights])
        yp = (C.c_void_p * n)(*y_ptrs)
        rp = None if res_ptrs is None else (C.c_void_p * n)(*res_ptrs)
        self._check(lib().elmh_gemv_a8_dev(self.h, C.c_void_p(q_ptr), C.c_void_p(d_ptr), C.c_void_p(s_ptr), C.c_int(T),
                                           C.c_int64(K), C.c_int(n), wp, yp, rp))

    # ---- the rest of a layer (device pointers; same float order as edgelm's cpu backend)
    def embed_dev(self, tok_ptr, T, table, y_ptr):
        self._check(lib().elmh_embed_dev(self.h, C.c_void_p(tok_ptr), C.c_int(T), table.h, C.c_void_p(y_ptr)))

    def rmsnorm_dev(self, x_ptr, w_ptr, y_ptr, rows, dim, eps):
        self._check(lib().elmh_rmsnorm_dev(self.h, C.c_void_p(x_ptr), C.c_void_p(w_ptr), C.c_void_p(y_ptr),
                                           C.c_int(rows), C.c_int(dim), C.c_float(eps)))

    def rmsnorm_matmul_dev(self, x_ptr, nw_ptr, eps, T, K, weights, y_ptrs, res_ptrs=None, act=ACT_INT8, mode=EXACT):
        n = len(weights)
        wp = (C.c_void_p * n)(*[w.h.value for w in weights])
        yp = (C.c_void_p * n)(*y_ptrs)
        rp = None if res_ptrs is None else (C.c_void_p * n)(*res_ptrs)
        self._check(lib().elmh_rmsnorm_matmul_dev(self.h, C.c_void_p(x_ptr), C.c_void_p(nw_ptr), C.c_float(eps),
                                                  C.c_int(T), C.c_int64(K), C.c_int(n), wp, yp, rp, C.c_int(act),
                                                  C.c_int(mode)))

    def rmsnorm_swiglu_dev(self, x_ptr, nw_ptr, eps, T, K, wg, wu, y_ptr, act=ACT_INT8, mode=EXACT):
        self._check(lib().elmh_rmsnorm_swiglu_dev(self.h, C.c_void_p(x_ptr), C.c_void_p(nw_ptr), C.c_float(eps),
                                                  C.c_int(T), C.c_int64(K), wg.h, wu.h, C.c_void_p(y_ptr),
                                                  C.c_int(act), C.c_int(mode)))

    def attention_dev(self, q_ptr, k_ptr, v_ptr, out_ptr, T, pos0, n_heads, n_kv, head_dim, kc_ptr, vc_ptr, max_ctx,
                      cos_ptr=None, sin_ptr=None):
        self._check(lib().elmh_attention_dev(
            self.h, C.c_void_p(q_ptr), C.c_void_p(k_ptr), C.c_void_p(v_ptr), C.c_void_p(out_ptr), C.c_int(T),
            C.c_int(pos0), C.c_int(n_heads), C.c_int(n_kv), C.c_int(head_dim), C.c_void_p(kc_ptr), C.c_void_p(vc_ptr),
            C.c_int(max_ctx), C.c_void_p(cos_ptr), C.c_void_p(sin_ptr)))

    def attention_step_dev(self, q_ptr, k_ptr, v_ptr, out_ptr, pos_ptr, n_heads, n_kv, head_dim, kc_ptr, vc_ptr, max_ctx,
                           cos_ptr=None, sin_ptr=None):
        self._check(lib().elmh_attention_step_dev(
            self.h, C.c_void_p(q_ptr), C.c_void_p(k_ptr), C.c_void_p(v_ptr), C.c_void_p(out_ptr), C.c_void_p(pos_ptr),
            C.c_int(n_heads), C.c_int(n_kv), C.c_int(head_dim), C.c_void_p(kc_ptr), C.c_void_p(vc_ptr), C.c_int(max_ctx),
            C.c_void_p(cos_ptr), C.c_void_p(sin_ptr)))

    def attention_matmul_dev(self, q_ptr, k_ptr, v_ptr, out_ptr, T, pos0, n_heads, n_kv, head_dim, kc_ptr, vc_ptr,
                             max_ctx, cos_ptr, sin_ptr, weight, y_ptr, res_ptr=None, act=ACT_INT8, mode=EXACT):
        self._check(lib().elmh_attention_matmul_dev(
            self.h, C.c_void_p(q_ptr), C.c_void_p(k_ptr), C.c_void_p(v_ptr), C.c_void_p(out_ptr), C.c_int(T),
            C.c_int(pos0), C.c_int(n_heads), C.c_int(n_kv), C.c_int(head_dim), C.c_void_p(kc_ptr), C.c_void_p(vc_ptr),
            C.c_int(max_ctx), C.c_void_p(cos_ptr), C.c_void_p(sin_ptr), weight.h, C.c_void_p(y_ptr),
            C.c_void_p(res_ptr), C.c_int(act), C.c_int(mode)))

    def attention_matmul_fused(self):
        """True if the last attention_matmul_dev call had the attention kernel write the GEMM's operand."""
        return bool(lib().elmh_attention_matmul_fused(self.h))

    def argmax_dev(self, x_ptr, rows, n, out_ptr):
        self._check(lib().elmh_argmax_dev(self.h, C.c_void_p(x_ptr), C.c_int(rows), C.c_int64(n), C.c_void_p(out_ptr)))

    def argmax_step_dev(self, x_ptr, n, out_ptr, pos_ptr, ring_ptr, ring_len):
        """elmh_argmax_step_dev: *out = argmax(x[:n]); ring[*pos % ring_len] = *out; *pos += 1 (device pointers)."""
        self._check(lib().elmh_argmax_step_dev(self.h, C.c_void_p(x_ptr), C.c_int64(n), C.c_void_p(out_ptr),
                                               C.c_void_p(pos_ptr), C.c_void_p(ring_ptr), C.c_int(ring_len)))

    def memcpy_d2d(self, dst_ptr, src_ptr, nbytes):
        self._check(lib().elmh_memcpy_d2d(self.h, C.c_void_p(dst_ptr), C.c_void_p(src_ptr), C.c_size_t(nbytes)))

    def memset_dev(self, dst_ptr, value, nbytes):
        self._check(lib().elmh_memset_dev(self.h, C.c_void_p(dst_ptr), C.c_int(value), C.c_size_t(nbytes)))

    def read_sweep_dev(self, src_ptr, nbytes, sink_ptr):
        """elmh_read_sweep_dev: every 16-byte word of src read once (a read-bandwidth ceiling)."""
        self._check(lib().elmh_read_sweep_dev(self.h, C.c_void_p(src_ptr), C.c_size_t(nbytes), C.c_void_p(sink_ptr)))

    def rescale_ceiling_dev(self, mode, blocks, iters, sink_ptr, sink_bytes):
        """elmh_rescale_ceiling_dev: MFMA blocks with the per-block rescale of mode 0 / 1 (q8) / 2 (q4)."""
        self._check(lib().elmh_rescale_ceiling_dev(self.h, C.c_int(mode), C.c_int(blocks), C.c_int(iters),
                                                   C.c_void_p(sink_ptr), C.c_size_t(sink_bytes)))

    @staticmethod
    def read_sweep_sink_bytes():
        lib().elmh_read_sweep_sink_bytes.restype = C.c_size_t
        return int(lib().elmh_read_sweep_sink_bytes())

    def buffer(self, nbytes):
        return DevBuffer(self, nbytes)

    def synchronize(self):
        self._check(lib().elmh_synchronize(self.h))

    # ---- events and graphs
    def event(self):
        e = C.c_void_p()
        self._check(lib().elmh_event_create(self.h, C.byref(e)))
        return e

    def record(self, ev):
        self._check(lib().elmh_event_record(self.h, ev))

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        self._check(lib().elmh_event_elapsed(self.h, a, b, C.byref(ms)))
        return ms.value

    def destroy_event(self, ev):
        lib().elmh_event_destroy(self.h, ev)

    def graph_begin(self):
        self._check(lib().elmh_graph_begin(self.h))

    def graph_end(self):
        g = C.c_void_p()
        self._check(lib().elmh_graph_end(self.h, C.byref(g)))
        return g

    def graph_launch(self, g):
        self._check(lib().elmh_graph_launch(self.h, g))

    def graph_destroy(self, g):
        lib().elmh_graph_destroy(self.h, g)
