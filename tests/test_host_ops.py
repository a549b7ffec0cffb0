"""CPU: the host ops a partition leaves on the CPU (libedgelm_host.so's host_ops.cpp, through the
elm_host_* test hooks) against edgelm's own ops compiled from its sources (oracle/_ref): the reference
backend's ref::rmsnorm / rope / attention / add / mul / silu and RopeTable (kernels_ref.cpp:11-21,
41-57, 82-151) and the cpu backend's cpu::rmsnorm / attention on the x86 scalar path
(kernels_cpu.cpp:326-335, 417-488), bit for bit, KV caches included."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from edgelm_amd import host
from conftest import bits_equal

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")
P = C.c_void_p


def _p(a):
    return a.ctypes.data_as(P)


def _lib():
    L = host.lib()
    L.elm_last_error.restype = C.c_char_p
    L.elm_host_elementwise.argtypes = [C.c_int, P, P, P, C.c_int64]
    return L


def _attn_inputs(rng, T, pos0, nh, nkv, hd, max_ctx):
    q = rng.standard_normal((T, nh * hd), dtype=np.float32)
    k = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    kc = np.full((nkv, max_ctx, hd), np.nan, np.float32)
    vc = np.full((nkv, max_ctx, hd), np.nan, np.float32)
    kc[:, :pos0] = rng.standard_normal((nkv, pos0, hd), dtype=np.float32)
    vc[:, :pos0] = rng.standard_normal((nkv, pos0, hd), dtype=np.float32)
    return q, k, v, kc, vc


def _host_attention(q, k, v, kc, vc, pos0, nh, nkv, hd, rope, theta, flavor, threads):
    out = np.empty_like(q)
    rc = _lib().elm_host_attention(_p(q), _p(k), _p(v), _p(out), C.c_int(q.shape[0]), C.c_int(pos0), C.c_int(nh),
                                   C.c_int(nkv), C.c_int(hd), _p(kc), _p(vc), C.c_int(kc.shape[1]), C.c_int(rope),
                                   C.c_float(theta), C.c_int(flavor), C.c_int(threads))
    assert rc == 0, _lib().elm_last_error()
    return out


def _ref_attention(fn, q, k, v, kc, vc, pos0, nh, nkv, hd, rope, theta, *extra):
    out = np.empty_like(q)
    getattr(O.ref(), fn)(_p(q), _p(k), _p(v), _p(out), C.c_int(q.shape[0]), C.c_int(pos0), C.c_int(nh), C.c_int(nkv),
                         C.c_int(hd), _p(kc), _p(vc), C.c_int(kc.shape[1]), C.c_int(rope), C.c_float(theta),
                         *[C.c_int(e) for e in extra])
    return out


# (T, pos0, n_heads, n_kv, head_dim, max_ctx): prefill, decode, a chunk after a prefix, GQA and MHA, head
# sizes with and without a tail past the last multiple of 4 (18: two elements into the first sum)
CASES = [(16, 0, 9, 3, 64, 40), (1, 37, 9, 3, 64, 64), (5, 11, 4, 2, 18, 24), (3, 0, 2, 2, 6, 8), (1, 0, 6, 1, 32, 4)]


@needs_ref
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("rope", [0, 1])
def test_attention_both_flavors(case, rope):
    T, pos0, nh, nkv, hd, mc = case
    theta = 10000.0
    rng = np.random.default_rng(T * 1000 + pos0 * 10 + hd + rope)
    q, k, v, kc0, vc0 = _attn_inputs(rng, T, pos0, nh, nkv, hd, mc)
    # reference backend: ref::attention
    kc_a, vc_a, kc_b, vc_b = kc0.copy(), vc0.copy(), kc0.copy(), vc0.copy()
    got = _host_attention(q, k, v, kc_a, vc_a, pos0, nh, nkv, hd, rope, theta, 0, 1)
    want = _ref_attention("eref_ref_attention", q, k, v, kc_b, vc_b, pos0, nh, nkv, hd, rope, theta)
    assert bits_equal(got, want)
    assert np.array_equal(kc_a.view(np.int32), kc_b.view(np.int32))
    assert np.array_equal(vc_a.view(np.int32), vc_b.view(np.int32))
    # cpu backend: cpu::attention, serial and over a pool
    for threads in (1, 4):
        kc_a, vc_a, kc_b, vc_b = kc0.copy(), vc0.copy(), kc0.copy(), vc0.copy()
        got = _host_attention(q, k, v, kc_a, vc_a, pos0, nh, nkv, hd, rope, theta, 1, threads)
        want = _ref_attention("eref_cpu_attention_pool", q, k, v, kc_b, vc_b, pos0, nh, nkv, hd, rope, theta, threads)
        assert bits_equal(got, want)
        assert np.array_equal(kc_a.view(np.int32), kc_b.view(np.int32))
        assert np.array_equal(vc_a.view(np.int32), vc_b.view(np.int32))


@needs_ref
def test_flavors_differ():
    """The bit-exact checks above tell the flavors apart: on a long enough row the two accumulation orders
    give different bits, so a host op running the other backend's order would fail them."""
    T, pos0, nh, nkv, hd, mc = 4, 60, 4, 2, 64, 64
    q, k, v, kc, vc = _attn_inputs(np.random.default_rng(9), T, pos0, nh, nkv, hd, mc)
    a = _host_attention(q, k, v, kc.copy(), vc.copy(), pos0, nh, nkv, hd, 1, 10000.0, 0, 1)
    b = _host_attention(q, k, v, kc.copy(), vc.copy(), pos0, nh, nkv, hd, 1, 10000.0, 1, 1)
    assert not bits_equal(a, b) and np.allclose(a, b, rtol=1e-4, atol=1e-5)
    x = np.random.default_rng(2).standard_normal((8, 576), dtype=np.float32)
    w = np.ones(576, np.float32)
    ys = []
    for flavor in (0, 1):
        y = np.empty_like(x)
        assert _lib().elm_host_rmsnorm(_p(x), _p(w), _p(y), 8, 576, C.c_float(1e-5), flavor, 1) == 0
        ys.append(y)
    assert not bits_equal(*ys)


@needs_ref
def test_attention_context_overflow_refused():
    q, k, v, kc, vc = _attn_inputs(np.random.default_rng(1), 4, 6, 2, 1, 8, 8)
    out = np.empty_like(q)
    for flavor in (0, 1):
        rc = _lib().elm_host_attention(_p(q), _p(k), _p(v), _p(out), 4, 6, 2, 1, 8, _p(kc), _p(vc), 8, 1,
                                       C.c_float(10000.0), flavor, 1)
        assert rc == -1 and b"context overflow" in _lib().elm_last_error()


@needs_ref
@pytest.mark.parametrize("rows,dim", [(1, 576), (13, 576), (3, 7), (9, 13), (2, 1)])
def test_rmsnorm_both_flavors(rows, dim):
    rng = np.random.default_rng(rows * 100 + dim)
    x = (rng.standard_normal((rows, dim), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    x[0, 0] = np.float32(1e-20)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    eps = 1e-5
    for flavor, threads, fn in ((0, 1, "eref_ref_rmsnorm"), (1, 1, "eref_rmsnorm"), (1, 4, "eref_rmsnorm")):
        y = np.empty_like(x)
        assert _lib().elm_host_rmsnorm(_p(x), _p(w), _p(y), rows, dim, C.c_float(eps), flavor, threads) == 0
        want = np.empty_like(x)
        getattr(O.ref(), fn)(_p(x), _p(w), _p(want), C.c_int(rows), C.c_int(dim), C.c_float(eps))
        assert bits_equal(y, want), (flavor, threads)


@needs_ref
@pytest.mark.parametrize("hd,max_pos,theta", [(64, 300, 1e5), (18, 50, 10000.0), (2, 7, 500000.0)])
def test_rope_table_and_rope(hd, max_pos, theta):
    c = np.empty((max_pos, hd // 2), np.float32)
    s = np.empty_like(c)
    assert _lib().elm_host_rope_table(hd, max_pos, C.c_float(theta), _p(c), _p(s)) == 0
    rc_, rs_ = O.rq_rope_table(hd, max_pos, theta)
    assert bits_equal(c, rc_) and bits_equal(s, rs_)
    rng = np.random.default_rng(hd)
    T, nh, pos0 = 3, 4, max_pos - 3
    x = rng.standard_normal((T, nh * hd), dtype=np.float32)
    y, want = np.empty_like(x), np.empty_like(x)
    assert _lib().elm_host_rope(_p(x), _p(y), T, nh, hd, pos0, max_pos, C.c_float(theta)) == 0
    O.ref().eref_ref_rope(_p(x), _p(want), C.c_int(T), C.c_int(nh), C.c_int(hd), C.c_int(pos0), C.c_int(max_pos),
                          C.c_float(theta))
    assert bits_equal(y, want)
    assert _lib().elm_host_rope(_p(x), _p(y), T, nh, hd, pos0 + 1, max_pos, C.c_float(theta)) == -1
    assert b"beyond rope table" in _lib().elm_last_error()


@needs_ref
def test_elementwise():
    rng = np.random.default_rng(3)
    a = (rng.standard_normal(4099) * 30).astype(np.float32)
    a[:6] = [0.0, -0.0, 88.8, -88.8, -104.0, 1e-30]
    b = rng.standard_normal(4099).astype(np.float32)
    O.ref().eref_ref_elementwise.argtypes = [C.c_int, P, P, P, C.c_int64]
    for op in (0, 1, 2):
        y, want = np.empty_like(a), np.empty_like(a)
        assert _lib().elm_host_elementwise(op, _p(a), _p(b), _p(y), a.size) == 0
        O.ref().eref_ref_elementwise(op, _p(a), _p(b), _p(want), a.size)
        assert bits_equal(y, want), op
