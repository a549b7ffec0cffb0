"""GPU: elmh_matmul_noalloc_dev (the entry point that allocates nothing) against elmh_matmul_dev, bit for bit,
through the C ABI, on calls in a row where the second is smaller than the first (the fixed scratch array keeps
the first call's contents), on every path that uses scratch (block-scale GEMM fragments, per-token fragments,
the row-major quantizer of the streaming GEMV) and on paths that use none (small GEMV, f32 activations); the
context's own scratch is never touched (its generation counter stays put), and a call too large for the array
fails before running."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import elmh as E

pytestmark = pytest.mark.gpu


def gen(ctx):
    E.lib().elmh_scratch_generation.restype = C.c_uint64
    return int(E.lib().elmh_scratch_generation(ctx.h))


def run_both(ctx, r, ws, dws, T, K, act, with_res):
    x = r.normal(0, 1, (T, K)).astype(np.float32)
    res = [r.normal(0, 1, (T, w.rows)).astype(np.float32) if with_res and i == 0 else None for i, w in enumerate(ws)]
    bx = ctx.buffer(x.nbytes)
    bx.upload(x)
    bres = [None if a is None else ctx.buffer(a.nbytes) for a in res]
    for b, a in zip(bres, res):
        if b is not None:
            b.upload(a)
    ya = [ctx.buffer(T * w.rows * 4) for w in ws]
    yb = [ctx.buffer(T * w.rows * 4) for w in ws]
    rp = [0 if b is None else b.ptr for b in bres] if with_res else None
    ctx.matmul_dev(bx.ptr, T, K, dws, [b.ptr for b in ya], rp, act=act)
    g0 = gen(ctx)
    ctx.matmul_noalloc_dev(bx.ptr, T, K, dws, [b.ptr for b in yb], rp, act=act)
    ctx.synchronize()
    assert gen(ctx) == g0, "the no-allocation entry point reallocated context scratch"
    for i, w in enumerate(ws):
        a = ya[i].download((T, w.rows), np.float32)
        b = yb[i].download((T, w.rows), np.float32)
        assert bits_equal(a, b), f"target {i} T={T} K={K} act={act}: max diff {np.abs(a - b).max()}"
        if act == E.ACT_INT8 and T * w.rows * K <= 40_000_000:
            assert bits_equal(b, O.cpu_matmul(x, [w], [res[i]], act_quant=True)[0])
    for buf in [bx] + [b for b in bres if b is not None] + ya + yb:
        buf.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_noalloc_matches_matmul_dev_big_then_small(ctx, dt):
    r = np.random.default_rng(77 + dt)
    # (T, K, act, targets): each case is followed by a smaller one on the same array
    cases = [
        (512, 4096, E.ACT_INT8, (512, 136)),       # block-scale GEMM fragments: 2 MiB + scales
        (37, 576, E.ACT_INT8, (96, 40)),           # smaller GEMM on the same array
        (300, 1536, E.ACT_INT8_TOKEN, (200,)),     # per-token fragments
        (65, 576, E.ACT_INT8_TOKEN, (72,)),
        (2, 14336, E.ACT_INT8, (64, 36)),          # row-major quantizer + streaming GEMV
        (1, 8192, E.ACT_INT8, (40,)),
        (1, 576, E.ACT_INT8, (960,)),              # small GEMV: no scratch
        (3, 576, E.ACT_F32, (100,)),               # f32 activations: no scratch
    ]
    for T, K, act, rows in cases:
        print(f"[gpu] noalloc dt={dt} T={T} K={K} act={act} rows={rows}", flush=True)
        ws = [O.make_weight(r.normal(0, 0.05, (n, K)).astype(np.float32), dt) for n in rows]
        dws = [ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales) for w in ws]
        run_both(ctx, r, ws, dws, T, K, act, with_res=True)
        for d in dws:
            d.free()


def test_noalloc_rejects_calls_beyond_its_array(ctx):
    r = np.random.default_rng(78)
    w = O.make_weight(r.normal(0, 0.05, (64, 16384)).astype(np.float32), O.Q8)
    dw = ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)
    T, K = 640, 16384  # 640 * 16384 fragment bytes: more than 8 MiB
    bx, by = ctx.buffer(T * K * 4), ctx.buffer(T * 64 * 4)
    g0 = gen(ctx)
    with pytest.raises(E.ElmhError) as e:
        ctx.matmul_noalloc_dev(bx.ptr, T, K, [dw], [by.ptr], act=E.ACT_INT8)
    assert e.value.code == E.ERR_ARG and "no-allocation" in str(e.value)
    assert gen(ctx) == g0
    bx.free(), by.free(), dw.free()
