"""GPU parity: the HIP kernels through the C ABI against the CPU oracle (oracle/), which restates
edgelm's cpu backend on its x86 scalar path and its reference backend.

Bars (mirroring edgelm's own tests, tests/test_ops.cpp:119-240):
  * int8 activations, block sums and every ELMH_EXACT f32 output: bit-identical to the cpu backend;
  * vs the reference backend (ref::matmul / ref::swiglu): rel_err < 1e-5 (test_ops.cpp:228,232);
  * ELMH_FAST GEMM: rel_err < 1e-5 against the exact result.
"""
import os

import numpy as np
import pytest

import oracle as O
from edgelm_amd import elmh as E
from conftest import bits_equal, rel_err

pytestmark = pytest.mark.gpu

# ragged shapes from the reference's tests plus the SmolLM2-135M matmul shapes
SHAPES = [(48, 64), (37, 96), (130, 160), (70, 160), (960, 576), (576, 1536), (1536, 576)]
TOKENS = [1, 2, 3, 4, 5, 9, 17, 64, 65, 128]


def rng(seed):
    return np.random.default_rng(seed)


def weight(r, n, k, dt, sd=0.05):
    return O.make_weight(r.normal(0, sd, (n, k)).astype(np.float32), dt)


def up(ctx, w):
    return ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)


def test_act_quant_bit_exact(ctx):
    r = rng(1)
    xa = r.normal(0, 1, (3, 96)).astype(np.float32)
    xa[1, 40] = 25.0  # the outlier case of the reference's int8 test (make_tiny.py:448-450)
    cases = [xa, r.normal(0, 1, (7, 576)).astype(np.float32), r.normal(0, 3, (2, 14336)).astype(np.float32)]
    z = r.normal(0, 1, (4, 128)).astype(np.float32)
    z[1] = 0.0           # all-zero row: d = 0, q = 0
    z[2, :32] = -0.0     # signed zeros
    z[3, 32:64] = 1e-30  # tiny block
    z[0, 64:96] = np.float32(3e38)  # huge block
    cases.append(z)
    for x in cases:
        print(f"[gpu] act_quant shape={x.shape}", flush=True)
        q, d = ctx.quantize_act(x)
        qo, do = O.quantize_act(x)
        assert np.array_equal(q, qo)
        assert bits_equal(d, do)
    q, d = ctx.quantize_act(xa)
    assert d[1, 1] >= 25.0 / 127.0 and d[1, 0] < 0.1  # outlier isolated to its block (test_ops.cpp:205-207)


def near_half_activations(r, T, K):
    """Rows whose values sit within a few ulp of the rounding points (m - 1/2) s of their block
    (s = amax / 127), where a quotient one ulp off the correctly rounded one would round the
    other way; one value per block is the block's amax."""
    nb = K // 32
    amax = np.exp(r.uniform(-8, 8, (T, nb, 1))).astype(np.float32)
    s = amax / np.float32(127)
    m = r.integers(1, 128, (T, nb, 32)).astype(np.float32)
    base = ((m - np.float32(0.5)) * s).astype(np.float32)
    off = r.integers(-3, 4, (T, nb, 32)).astype(np.int32)
    x = (base.view(np.int32) + off).view(np.float32)
    x = np.minimum(x, amax) * np.where(r.random((T, nb, 32)) < 0.5, -1, 1).astype(np.float32)
    pos = r.integers(0, 32, (T, nb))
    np.put_along_axis(x, pos[..., None], amax, axis=2)
    return x.reshape(T, K).astype(np.float32)


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_act_quant_near_half_points(ctx, dt):
    """Every int8 quantizer (row-major, in-workgroup, GEMM fragments) on values at the rounding
    boundaries: bit-identical to edgelm's per-value division."""
    r = rng(11)
    x = near_half_activations(r, 4, 1536)
    q, d = ctx.quantize_act(x)
    qo, do = O.quantize_act(x)
    assert np.array_equal(q, qo) and bits_equal(d, do)
    for T, K, N in [(1, 576, 1536), (3, 1536, 576), (2, 2048, 256), (64, 576, 256), (130, 576, 256)]:
        print(f"[gpu] near-half matmul dt={dt} T={T} K={K} N={N}", flush=True)
        x = near_half_activations(r, T, K)
        w = weight(r, N, K, dt)
        got = ctx.matmul(x, [up(ctx, w)])[0]
        assert bits_equal(got, O.cpu_matmul(x, [w], None, act_quant=True)[0]), f"T={T} K={K}"


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_block_sums_exact(ctx, dt):
    r = rng(2)
    for n, k in [(70, 160), (960, 576), (37, 96), (130, 1536)]:
        w = weight(r, n, k, dt)
        xq = r.integers(-127, 128, (3, k)).astype(np.int8)
        xq[0, :32] = 127
        xq[1, :32] = -127
        print(f"[gpu] block_sums dt={dt} {n}x{k}", flush=True)
        S = ctx.block_sums(xq, up(ctx, w))
        assert np.array_equal(S, O.block_sums(xq, w))


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
@pytest.mark.parametrize("shape", SHAPES)
def test_matmul_a8_exact(ctx, dt, shape):
    n, k = shape
    r = rng(100 + n + k + dt)
    w = weight(r, n, k, dt)
    dw = up(ctx, w)
    for T in TOKENS:
        print(f"[gpu] matmul a8 dt={dt} {n}x{k} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = r.normal(0, 1, (T, n)).astype(np.float32)
        want = O.cpu_matmul(x, [w], [res], act_quant=True)[0]
        got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8, mode=E.EXACT)[0]
        assert bits_equal(got, want), f"T={T} max diff {np.abs(got - want).max()}"
        got0 = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.EXACT)[0]
        assert bits_equal(got0, O.cpu_matmul(x, [w], None, act_quant=True)[0])
        if n * k * T <= 2_000_000:
            ref = O.ref_matmul(x, w, res, act_quant=True)
            assert rel_err(got, ref) < 1e-5
    dw.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
@pytest.mark.parametrize("shape", [(70, 160), (1536, 576), (130, 160)])
def test_swiglu_a8_exact(ctx, dt, shape):
    n, k = shape
    r = rng(200 + n + dt)
    wg, wu = weight(r, n, k, dt), weight(r, n, k, dt)
    dg, du = up(ctx, wg), up(ctx, wu)
    for T in [1, 3, 4, 9, 64, 128]:
        print(f"[gpu] swiglu a8 dt={dt} {n}x{k} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        got = ctx.swiglu(x, dg, du, act=E.ACT_INT8)
        want = O.cpu_swiglu(x, wg, wu, act_quant=True)
        assert bits_equal(got, want), f"T={T} max diff {np.abs(got - want).max()}"
        if n * k * T <= 2_000_000:
            assert rel_err(got, O.ref_swiglu(x, wg, wu, act_quant=True)) < 1e-5


def test_matmul_n_mixed_targets(ctx):
    """MATMUL_N (fused QKV) equals separate matmuls (test_ops.cpp:173-189), q8 and q4 mixed."""
    r = rng(3)
    ws = [weight(r, 96, 64, O.Q8), weight(r, 32, 64, O.Q4), weight(r, 32, 64, O.Q8), weight(r, 40, 64, O.Q4),
          weight(r, 24, 64, O.Q4)]
    dws = [up(ctx, w) for w in ws]
    for act in (E.ACT_INT8, E.ACT_F32):
        for T in [1, 6, 70]:
            print(f"[gpu] matmul_n act={act} T={T}", flush=True)
            x = r.normal(0, 1, (T, 64)).astype(np.float32)
            res = [r.normal(0, 1, (T, w.rows)).astype(np.float32) if i % 2 else None for i, w in enumerate(ws)]
            got = ctx.matmul(x, dws, res, act=act)
            want = O.cpu_matmul(x, ws, res, act_quant=act == E.ACT_INT8)
            for g, wnt in zip(got, want):
                assert bits_equal(g, wnt)
            for i, (g, w) in enumerate(zip(got, ws)):
                sep = ctx.matmul(x, [dws[i]], [res[i]], act=act)[0]
                assert bits_equal(g, sep)


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_matmul_f32act_exact(ctx, dt):
    r = rng(4 + dt)
    shapes = [(48, 64), (37, 96), (130, 160), (960, 576)] + ([(37, 50), (20, 7), (8200, 64)] if dt == O.Q8 else
                                                              [(576, 1536), (70, 4096)])
    for n, k in shapes:
        w = weight(r, n, k, dt)
        dw = up(ctx, w)
        wu = weight(r, n, k, dt)
        du = up(ctx, wu)
        for T in [1, 3, 4, 17]:
            print(f"[gpu] f32act dt={dt} {n}x{k} T={T}", flush=True)
            x = r.normal(0, 1, (T, k)).astype(np.float32)
            res = r.normal(0, 1, (T, n)).astype(np.float32)
            got = ctx.matmul(x, [dw], [res], act=E.ACT_F32)[0]
            assert bits_equal(got, O.cpu_matmul(x, [w], [res], act_quant=False)[0])
            assert rel_err(got, O.ref_matmul(x, w, res)) < 1e-5
            # act_quant requested but K % 32 != 0: edgelm falls back to f32 activations
            if k % 32:
                got2 = ctx.matmul(x, [dw], [res], act=E.ACT_INT8)[0]
                assert bits_equal(got2, got)
            sg = ctx.swiglu(x, dw, du, act=E.ACT_F32)
            assert bits_equal(sg, O.cpu_swiglu(x, w, wu, act_quant=False))
            # MATMUL_N: targets of different row counts in one launch
            w2 = weight(r, n // 2 + 3, k, dt)
            dw2 = up(ctx, w2)
            got = ctx.matmul(x, [dw, dw2], [res, None], act=E.ACT_F32)
            want = O.cpu_matmul(x, [w, w2], [res, None], act_quant=False)
            assert bits_equal(got[0], want[0]) and bits_equal(got[1], want[1])
            dw2.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_gemm_fast_mode_tolerance(ctx, dt):
    r = rng(5 + dt)
    w = weight(r, 576, 1536, dt)
    dw = up(ctx, w)
    for T in [9, 128]:
        x = r.normal(0, 1, (T, 1536)).astype(np.float32)
        exact = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.EXACT)[0]
        fast = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.FAST)[0]
        assert rel_err(fast, exact) < 1e-5


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_token_scale_extension(ctx, dt):
    """ELMH_ACT_INT8_TOKEN (no edgelm counterpart): bit-exact against the oracle's restatement."""
    r = rng(6 + dt)
    for n, k in [(130, 160), (960, 576)]:
        w = weight(r, n, k, dt)
        dw = up(ctx, w)
        for T in [1, 5, 64, 100]:
            print(f"[gpu] token-scale dt={dt} {n}x{k} T={T}", flush=True)
            x = r.normal(0, 1, (T, k)).astype(np.float32)
            res = r.normal(0, 1, (T, n)).astype(np.float32)
            got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8_TOKEN)[0]
            assert bits_equal(got, O.matmul_a8_token(x, w, res))


def test_zero_rows_and_weights(ctx):
    r = rng(7)
    for dt in (O.Q8, O.Q4):
        wf = r.normal(0, 0.05, (70, 160)).astype(np.float32)
        wf[3] = 0.0  # zero row: scale 0
        w = O.make_weight(wf, dt)
        dw = up(ctx, w)
        for T in [1, 4, 64]:
            x = r.normal(0, 1, (T, 160)).astype(np.float32)
            x[0] = 0.0
            got = ctx.matmul(x, [dw], None, act=E.ACT_INT8)[0]
            assert bits_equal(got, O.cpu_matmul(x, [w], None, act_quant=True)[0])


def test_errors(ctx):
    r = rng(8)
    w = weight(r, 32, 64, O.Q8)
    dw = up(ctx, w)
    with pytest.raises(E.ElmhError) as e:
        ctx.matmul(np.zeros((1, 96), np.float32), [dw])
    assert e.value.code == E.ERR_ARG
    with pytest.raises(E.ElmhError) as e:
        ctx.upload(O.Q4, 4, 48, np.zeros((4, 24), np.uint8), np.zeros((4, 1), np.float32))
    assert e.value.code == E.ERR_ARG
    with pytest.raises(E.ElmhError) as e:
        ctx.upload(O.F32, 4, 64, np.zeros((4, 64), np.float32), np.zeros(4, np.float32))
    assert e.value.code == E.ERR_UNSUPPORTED


# Long rows (K > 2048): the streaming decode GEMV (pre-quantized activation, 4- to 32-row tiles)
# and the GEMM on the same layout. Ragged row counts exercise partial tiles.
LONG = [(512, 4096), (264, 14336), (130, 8192)]


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
@pytest.mark.parametrize("shape", LONG)
def test_matmul_a8_long_rows(ctx, dt, shape):
    n, k = shape
    r = rng(300 + n + k + dt)
    w = weight(r, n, k, dt)
    dw = up(ctx, w)
    for T in [1, 2, 3, 4, 5, 33]:
        print(f"[gpu] matmul a8 long dt={dt} {n}x{k} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = r.normal(0, 1, (T, n)).astype(np.float32)
        want = O.cpu_matmul(x, [w], [res], act_quant=True)[0]
        got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8, mode=E.EXACT)[0]
        assert bits_equal(got, want), f"T={T} max diff {np.abs(got - want).max()}"
    dw.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_matmul_n_and_swiglu_long_rows(ctx, dt):
    """QKV-shaped MATMUL_N (three targets, one with a residual) and FFN_SWIGLU at K = 4096."""
    r = rng(7 + dt)
    k = 4096
    ws = [weight(r, 512, k, dt), weight(r, 128, k, dt), weight(r, 136, k, dt)]
    dws = [up(ctx, w) for w in ws]
    for T in [1, 2, 4]:
        print(f"[gpu] matmul_n long dt={dt} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = [None, r.normal(0, 1, (T, 128)).astype(np.float32), None]
        got = ctx.matmul(x, dws, res, act=E.ACT_INT8)
        want = O.cpu_matmul(x, ws, res, act_quant=True)
        for i, (g, wv) in enumerate(zip(got, want)):
            assert bits_equal(g, wv), f"T={T} target {i}"
    wg, wu = weight(r, 300, k, dt), weight(r, 300, k, dt)
    dg, du = up(ctx, wg), up(ctx, wu)
    for T in [1, 2, 3, 4, 9]:
        print(f"[gpu] swiglu long dt={dt} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        got = ctx.swiglu(x, dg, du, act=E.ACT_INT8)
        assert bits_equal(got, O.cpu_swiglu(x, wg, wu, act_quant=True)), f"T={T}"
    for d in dws + [dg, du]:
        d.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_matmul_n_and_swiglu_fold_wave_rows(ctx, dt):
    """Rows of more than 256 blocks (K = 14336, decode): the GEMV folds in a wave of its own while
    the weights stream; MATMUL_N with ragged targets and a residual, and FFN_SWIGLU."""
    r = rng(11 + dt)
    k = 14336
    ws = [weight(r, 260, k, dt), weight(r, 36, k, dt), weight(r, 68, k, dt)]
    dws = [up(ctx, w) for w in ws]
    print(f"[gpu] matmul_n fold-wave dt={dt}", flush=True)
    x = r.normal(0, 1, (1, k)).astype(np.float32)
    res = [None, r.normal(0, 1, (1, 36)).astype(np.float32), None]
    got = ctx.matmul(x, dws, res, act=E.ACT_INT8)
    want = O.cpu_matmul(x, ws, res, act_quant=True)
    for i, (g, wv) in enumerate(zip(got, want)):
        assert bits_equal(g, wv), f"target {i}"
    wg, wu = weight(r, 132, k, dt), weight(r, 132, k, dt)
    dg, du = up(ctx, wg), up(ctx, wu)
    print(f"[gpu] swiglu fold-wave dt={dt}", flush=True)
    got = ctx.swiglu(x, dg, du, act=E.ACT_INT8)
    assert bits_equal(got, O.cpu_swiglu(x, wg, wu, act_quant=True))
    for d in dws + [dg, du]:
        d.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_matmul_f32act_long_rows(ctx, dt):
    """f32 activations at K > 2048 (taller row tiles): GEMV and dequantizing GEMM."""
    r = rng(400 + dt)
    for n, k in [(130, 4096), (66, 14336)]:
        w = weight(r, n, k, dt)
        dw = up(ctx, w)
        for T in [1, 3, 17]:
            print(f"[gpu] matmul f32act long dt={dt} {n}x{k} T={T}", flush=True)
            x = r.normal(0, 1, (T, k)).astype(np.float32)
            res = r.normal(0, 1, (T, n)).astype(np.float32)
            got = ctx.matmul(x, [dw], [res], act=E.ACT_F32)[0]
            assert bits_equal(got, O.cpu_matmul(x, [w], [res], act_quant=False)[0]), f"T={T}"
        dw.free()
    # SwiGLU at K from 16288 to 16384 (H = 8 for q4): the group-parallel q4 GEMV takes one-row tiles there,
    # and its LDS check must size them, not the layout's 8-row tiles, at one token as at several
    for k in (16288, 16384):
        wg, wu = weight(r, 40, k, dt), weight(r, 40, k, dt)
        dg, du = up(ctx, wg), up(ctx, wu)
        for T in [1, 3]:
            print(f"[gpu] swiglu f32act long dt={dt} 40x{k} T={T}", flush=True)
            x = r.normal(0, 1, (T, k)).astype(np.float32)
            assert bits_equal(ctx.swiglu(x, dg, du, act=E.ACT_F32), O.cpu_swiglu(x, wg, wu, act_quant=False)), f"T={T}"
        dg.free(), du.free()


@pytest.mark.parametrize("tile", ["64", "128"])
@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_gemm_token_tiles(ctx, dt, tile, monkeypatch):
    """Both GEMM tile heights (64 and 128 tokens, picked by shape unless ELMH_GEMM_TOKEN_TILE forces
    one) over several token tiles with a ragged last one and a partial last row tile: per-block
    int8 (exact, fast, residual), per-token int8 (block groups with a partial last group: K = 576
    is 18 blocks), MATMUL_N and FFN_SWIGLU. The tile height is forced with four and with eight waves
    per workgroup (ELMH_GEMM_WAVES; eight serve the block-scale modes without SwiGLU), and the
    per-block ring with one barrier per block (ELMH_GEMM_KB=1) as well as per group of six blocks."""
    for waves in ("8", "4"):
        monkeypatch.setenv("ELMH_GEMM_WAVES", waves)
        for kb in ("6", "1"):
            monkeypatch.setenv("ELMH_GEMM_KB", kb)
            check_token_tiles(ctx, dt, tile, monkeypatch)


def check_token_tiles(ctx, dt, tile, monkeypatch):
    monkeypatch.setenv("ELMH_GEMM_TOKEN_TILE", tile)
    r = rng(500 + dt)
    n, k = 300, 576
    w, w2 = weight(r, n, k, dt), weight(r, 72, k, dt)
    wg, wu = weight(r, n, k, dt), weight(r, n, k, dt)
    dw, dw2, dg, du = up(ctx, w), up(ctx, w2), up(ctx, wg), up(ctx, wu)
    for T in [65, 130, 257, 512]:
        print(f"[gpu] gemm tile={tile} waves={os.environ.get('ELMH_GEMM_WAVES')} kb={os.environ.get('ELMH_GEMM_KB')} "
              f"dt={dt} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = r.normal(0, 1, (T, n)).astype(np.float32)
        got = ctx.matmul(x, [dw, dw2], [res, None], act=E.ACT_INT8, mode=E.EXACT)
        want = O.cpu_matmul(x, [w, w2], [res, None], act_quant=True)
        assert bits_equal(got[0], want[0]) and bits_equal(got[1], want[1])
        fast = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.FAST)[0]
        assert rel_err(fast, O.cpu_matmul(x, [w], None, act_quant=True)[0]) < 1e-5
        assert bits_equal(ctx.swiglu(x, dg, du, act=E.ACT_INT8), O.cpu_swiglu(x, wg, wu, act_quant=True))
        tok = ctx.matmul(x, [dw, dw2], [res, None], act=E.ACT_INT8_TOKEN)
        assert bits_equal(tok[0], O.matmul_a8_token(x, w, res)) and bits_equal(tok[1], O.matmul_a8_token(x, w2))
        if T == 65:
            g, u = O.matmul_a8_token(x, wg), O.matmul_a8_token(x, wu)
            want_sw = np.array([O.silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape) * u
            assert bits_equal(ctx.swiglu(x, dg, du, act=E.ACT_INT8_TOKEN), want_sw)
    for d in (dw, dw2, dg, du):
        d.free()


@pytest.mark.parametrize("kernel", ["lds16", "wave", "wave32", "ring"])
@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_gemm_kernels_small_and_ragged(ctx, dt, kernel, monkeypatch):
    """Every GEMM kernel forced (ELMH_GEMM_KERNEL): one wave per 16x16 tile with the workgroup's
    operands staged in LDS (what small problems select; at K = 1568 the q8 SwiGLU's operands do not
    fit and it falls back to the next), the same loading from L2, one wave per 32x32 tile, and the
    LDS-ring kernel. Ragged rows and tokens (partial tiles), MATMUL_N with a residual, FFN_SWIGLU,
    per-block exact and fast, per-token, and an odd block count."""
    monkeypatch.setenv("ELMH_GEMM_KERNEL", kernel)
    r = rng(700 + dt)
    for n, n2, k in [(300, 40, 576), (70, 33, 1568)]:
        w, w2 = weight(r, n, k, dt), weight(r, n2, k, dt)
        wg, wu = weight(r, n, k, dt), weight(r, n, k, dt)
        dw, dw2, dg, du = up(ctx, w), up(ctx, w2), up(ctx, wg), up(ctx, wu)
        for T in [5, 33, 128, 130]:
            print(f"[gpu] gemm kernel={kernel} dt={dt} {n}x{k} T={T}", flush=True)
            x = r.normal(0, 1, (T, k)).astype(np.float32)
            res = r.normal(0, 1, (T, n)).astype(np.float32)
            got = ctx.matmul(x, [dw, dw2], [res, None], act=E.ACT_INT8, mode=E.EXACT)
            want = O.cpu_matmul(x, [w, w2], [res, None], act_quant=True)
            assert bits_equal(got[0], want[0]) and bits_equal(got[1], want[1])
            fast = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.FAST)[0]
            assert rel_err(fast, O.cpu_matmul(x, [w], None, act_quant=True)[0]) < 1e-5
            assert bits_equal(ctx.swiglu(x, dg, du, act=E.ACT_INT8), O.cpu_swiglu(x, wg, wu, act_quant=True))
            tok = ctx.matmul(x, [dw, dw2], [res, None], act=E.ACT_INT8_TOKEN)
            assert bits_equal(tok[0], O.matmul_a8_token(x, w, res)) and bits_equal(tok[1], O.matmul_a8_token(x, w2))
            g, u = O.matmul_a8_token(x, wg), O.matmul_a8_token(x, wu)
            want_sw = np.array([O.silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape) * u
            assert bits_equal(ctx.swiglu(x, dg, du, act=E.ACT_INT8_TOKEN), want_sw)
        for d in (dw, dw2, dg, du):
            d.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_gemm_ring_short_rows(ctx, dt, monkeypatch):
    """The LDS-ring GEMM in edgelm's per-block mode at rows shorter than one group of six blocks
    (K = 32, 64: the only group is partial) and one full group plus a partial one (K = 224),
    grouped and with one barrier per block (ELMH_GEMM_KB=1), exact and fast."""
    monkeypatch.setenv("ELMH_GEMM_KERNEL", "ring")
    r = rng(800 + dt)
    for kb in ("6", "1"):
        monkeypatch.setenv("ELMH_GEMM_KB", kb)
        for n, k in [(72, 32), (130, 64), (200, 224)]:
            w = weight(r, n, k, dt)
            dw = up(ctx, w)
            for T in [65, 130]:
                print(f"[gpu] gemm ring short rows kb={kb} dt={dt} {n}x{k} T={T}", flush=True)
                x = r.normal(0, 1, (T, k)).astype(np.float32)
                res = r.normal(0, 1, (T, n)).astype(np.float32)
                got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8, mode=E.EXACT)[0]
                assert bits_equal(got, O.cpu_matmul(x, [w], [res], act_quant=True)[0]), f"{n}x{k} T={T}"
                fast = ctx.matmul(x, [dw], None, act=E.ACT_INT8, mode=E.FAST)[0]
                assert rel_err(fast, O.cpu_matmul(x, [w], None, act_quant=True)[0]) < 1e-5
            dw.free()


@pytest.mark.parametrize("tile", ["64", "128"])
def test_gemm_token_odd_block_count(ctx, tile, monkeypatch):
    """Per-token q8 GEMM at K = 1568 (49 blocks): the last group of 4 (64-token tiles) or 2
    (128-token tiles) blocks per barrier holds one real block and repeats of it that must add
    nothing."""
    monkeypatch.setenv("ELMH_GEMM_TOKEN_TILE", tile)
    r = rng(600)
    n, k = 200, 1568
    w = weight(r, n, k, O.Q8)
    dw = up(ctx, w)
    for T in [130, 257]:
        print(f"[gpu] gemm per-token odd nb tile={tile} T={T}", flush=True)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = r.normal(0, 1, (T, n)).astype(np.float32)
        got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8_TOKEN)[0]
        assert bits_equal(got, O.matmul_a8_token(x, w, res))
    dw.free()


def test_dev_pointer_unaligned_input(ctx):
    """elmh_matmul_dev takes any 4-byte-aligned device pointer for x (here 4 bytes past a 256-byte
    boundary): the same bits as the host-pointer call, on the GEMV and both GEMM quantizers."""
    r = rng(600)
    n, k = 200, 576
    w = weight(r, n, k, O.Q8)
    dw = up(ctx, w)
    for T in [2, 9, 70]:
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        bx = ctx.buffer(x.nbytes + 16)
        bx.upload(np.concatenate([np.zeros(1, np.float32), x.ravel()]))
        by = ctx.buffer(T * n * 4)
        for act in (E.ACT_INT8, E.ACT_INT8_TOKEN):
            print(f"[gpu] unaligned x T={T} act={act}", flush=True)
            ctx.matmul_dev(bx.ptr + 4, T, k, [dw], [by.ptr], act=act)
            got = by.download((T, n), np.float32)
            assert bits_equal(got, ctx.matmul(x, [dw], None, act=act)[0])
        bx.free()
        by.free()
    dw.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_rmsnorm_fused_block_gemm_wide_values(ctx, dt):
    """RMSNORM fused into the block-scale GEMM's quantizer launch over ragged token counts, one and
    several 64-token chunks, K from one block to 24, and values spread over 24 binades (block scales
    far apart, quotients near the rounding points): bit-identical to edgelm's cpu::rmsnorm then the
    cpu backend's matmul / SwiGLU (through the oracle)."""
    r = rng(23)
    for T, K, N in [(5, 576, 64), (64, 576, 960), (65, 768, 48), (128, 576, 576), (200, 64, 32), (127, 512, 192),
                    (33, 32, 16)]:
        print(f"[gpu] rmsnorm block gemm dt={dt} T={T} K={K} N={N}", flush=True)
        x = (r.normal(0, 1, (T, K)) * np.exp2(r.integers(-12, 12, (T, K)))).astype(np.float32)
        nw = r.normal(1, 0.3, K).astype(np.float32)
        res = r.normal(0, 1, (T, N)).astype(np.float32)
        w, w2 = weight(r, N, K, dt), weight(r, N // 2, K, dt)
        xn = O.rmsnorm(x, nw, 1e-5)
        bx, bnw, bres = ctx.buffer(x.nbytes), ctx.buffer(nw.nbytes), ctx.buffer(res.nbytes)
        bx.upload(x)
        bnw.upload(nw)
        bres.upload(res)
        by, by2 = ctx.buffer(T * N * 4), ctx.buffer(T * (N // 2) * 4)
        dw, dw2 = up(ctx, w), up(ctx, w2)
        ctx.rmsnorm_matmul_dev(bx.ptr, bnw.ptr, 1e-5, T, K, [dw, dw2], [by.ptr, by2.ptr], [bres.ptr, 0])
        want = O.cpu_matmul(xn, [w, w2], [res, None], act_quant=True)
        assert bits_equal(by.download((T, N), np.float32), want[0]), f"T={T} K={K}"
        assert bits_equal(by2.download((T, N // 2), np.float32), want[1]), f"T={T} K={K}"
        wg, wu = weight(r, N, K, dt), weight(r, N, K, dt)
        dg, du = up(ctx, wg), up(ctx, wu)
        ctx.rmsnorm_swiglu_dev(bx.ptr, bnw.ptr, 1e-5, T, K, dg, du, by.ptr)
        assert bits_equal(by.download((T, N), np.float32), O.cpu_swiglu(xn, wg, wu, act_quant=True)), f"T={T} K={K}"
        for b in (bx, bnw, bres, by, by2, dw, dw2, dg, du):
            b.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_rmsnorm_fused_f32act(ctx, dt):
    """f32 activations: at one token the q4 GEMV's workgroups normalize x themselves (q8, and q4
    at T > 1, go through scratch); values spread over 24 binades so that the sum of squares'
    order shows. Bit-identical to edgelm's cpu::rmsnorm then the cpu backend's f32-activation
    matmul / SwiGLU (through the oracle)."""
    r = rng(25)
    for T, K, N in [(1, 576, 960), (1, 32, 40), (1, 1536, 576), (1, 4096, 130), (1, 8192, 48), (2, 576, 64),
                    (3, 64, 96)]:
        print(f"[gpu] rmsnorm f32act dt={dt} T={T} K={K} N={N}", flush=True)
        x = (r.normal(0, 1, (T, K)) * np.exp2(r.integers(-12, 12, (T, K)))).astype(np.float32)
        nw = r.normal(1, 0.3, K).astype(np.float32)
        res = r.normal(0, 1, (T, N)).astype(np.float32)
        w, w2 = weight(r, N, K, dt), weight(r, N // 2 + 3, K, dt)
        xn = O.rmsnorm(x, nw, 1e-5)
        bx, bnw, bres = ctx.buffer(x.nbytes), ctx.buffer(nw.nbytes), ctx.buffer(res.nbytes)
        bx.upload(x)
        bnw.upload(nw)
        bres.upload(res)
        by, by2 = ctx.buffer(T * N * 4), ctx.buffer(T * (N // 2 + 3) * 4)
        dw, dw2 = up(ctx, w), up(ctx, w2)
        ctx.rmsnorm_matmul_dev(bx.ptr, bnw.ptr, 1e-5, T, K, [dw, dw2], [by.ptr, by2.ptr], [bres.ptr, 0],
                               act=E.ACT_F32)
        want = O.cpu_matmul(xn, [w, w2], [res, None], act_quant=False)
        assert bits_equal(by.download((T, N), np.float32), want[0]), f"T={T} K={K}"
        assert bits_equal(by2.download((T, N // 2 + 3), np.float32), want[1]), f"T={T} K={K}"
        wg, wu = weight(r, N, K, dt), weight(r, N, K, dt)
        dg, du = up(ctx, wg), up(ctx, wu)
        ctx.rmsnorm_swiglu_dev(bx.ptr, bnw.ptr, 1e-5, T, K, dg, du, by.ptr, act=E.ACT_F32)
        assert bits_equal(by.download((T, N), np.float32), O.cpu_swiglu(xn, wg, wu, act_quant=False)), f"T={T} K={K}"
        for b in (bx, bnw, bres, by, by2, dw, dw2, dg, du):
            b.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_rmsnorm_fused_into_matmul(ctx, dt):
    """elmh_rmsnorm_matmul_dev / elmh_rmsnorm_swiglu_dev: bit-identical to RMSNORM then the matmul
    (edgelm's cpu::rmsnorm and cpu backend matmul, through the oracle) on every path: each GEMV
    workgroup normalizing its rows (T <= 4, K <= 2048), the GEMM's quantizer normalizing them
    (T > 4, K <= 2048, ragged token counts), and the rows going through scratch first."""
    r = rng(21)
    for T, K, N in [(1, 576, 960), (2, 576, 64), (4, 1536, 576), (3, 2048, 96), (5, 576, 64), (1, 4096, 64),
                    (33, 576, 96), (130, 1536, 64), (64, 2048, 32), (9, 4096, 64)]:
        print(f"[gpu] rmsnorm+matmul dt={dt} T={T} K={K} N={N}", flush=True)
        x = r.normal(0, 2, (T, K)).astype(np.float32)
        nw = r.normal(1, 0.2, K).astype(np.float32)
        res = r.normal(0, 1, (T, N)).astype(np.float32)
        w, w2 = weight(r, N, K, dt), weight(r, N // 2, K, dt)
        xn = O.rmsnorm(x, nw, 1e-5)
        bx, bnw, bres = ctx.buffer(x.nbytes), ctx.buffer(nw.nbytes), ctx.buffer(res.nbytes)
        bx.upload(x)
        bnw.upload(nw)
        bres.upload(res)
        by, by2 = ctx.buffer(T * N * 4), ctx.buffer(T * (N // 2) * 4)
        dw, dw2 = up(ctx, w), up(ctx, w2)
        ctx.rmsnorm_matmul_dev(bx.ptr, bnw.ptr, 1e-5, T, K, [dw, dw2], [by.ptr, by2.ptr], [bres.ptr, 0])
        want = O.cpu_matmul(xn, [w, w2], [res, None], act_quant=True)
        assert bits_equal(by.download((T, N), np.float32), want[0]), f"T={T} K={K}"
        assert bits_equal(by2.download((T, N // 2), np.float32), want[1]), f"T={T} K={K}"
        wg, wu = weight(r, N, K, dt), weight(r, N, K, dt)
        dg, du = up(ctx, wg), up(ctx, wu)
        ctx.rmsnorm_swiglu_dev(bx.ptr, bnw.ptr, 1e-5, T, K, dg, du, by.ptr)
        assert bits_equal(by.download((T, N), np.float32), O.cpu_swiglu(xn, wg, wu, act_quant=True)), f"T={T} K={K}"
        for b in (bx, bnw, bres, by, by2, dw, dw2, dg, du):
            b.free()


# (dt, N, K, T): the streaming SwiGLU quantizing its own output (q4 at K = 4096, the 8B shape among
# them; q8 at K = 2048 with more than 4 MB of weights), and calls that take the SwiGLU and then the
# quantizer launch (two tokens; the small GEMV)
SWQ_CASES = [(O.Q4, 320, 4096, 1), (O.Q4, 14336, 4096, 1), (O.Q8, 1024, 2048, 1), (O.Q4, 320, 4096, 2),
             (O.Q8, 1536, 576, 1)]


@pytest.mark.parametrize("case", SWQ_CASES)
def test_swiglu_quant_exact(ctx, case):
    """elmh_swiglu_quant_dev: y bit-identical to edgelm's cpu::swiglu with int8 activations, and q / d / s
    to quantize_act_row of that y (the down projection's input), block sums included."""
    dt, n, k, T = case
    r = rng(500 + n + k + dt + T)
    wg, wu = weight(r, n, k, dt), weight(r, n, k, dt)
    dg, du = up(ctx, wg), up(ctx, wu)
    x = r.normal(0, 1, (T, k)).astype(np.float32)
    bx, by, bq, bd, bs = (ctx.buffer(T * k * 4), ctx.buffer(T * n * 4), ctx.buffer(T * n), ctx.buffer(T * n // 8),
                          ctx.buffer(T * n // 8))
    bx.upload(x)
    print(f"[gpu] swiglu_quant dt={dt} {n}x{k} T={T}", flush=True)
    ctx.swiglu_quant_dev(bx.ptr, T, k, dg, du, by.ptr, bq.ptr, bd.ptr, bs.ptr)
    ctx.synchronize()
    y = by.download((T, n), np.float32)
    q = bq.download((T, n), np.int8)
    d = bd.download((T, n // 32), np.float32)
    s = bs.download((T, n // 32), np.int32)
    want = O.cpu_swiglu(x, wg, wu, act_quant=True)
    assert bits_equal(y, want)
    qw, dw = O.quantize_act(want)
    assert np.array_equal(q, qw) and bits_equal(d, dw)
    assert np.array_equal(s, qw.reshape(T, n // 32, 32).astype(np.int32).sum(-1))
    for b in (bx, by, bq, bd, bs, dg, du):
        b.free()


def test_swiglu_quant_refuses_partial_blocks(ctx):
    r = rng(77)
    wg, wu = weight(r, 40, 4096, O.Q4), weight(r, 40, 4096, O.Q4)
    dg, du = up(ctx, wg), up(ctx, wu)
    bufs = [ctx.buffer(4096 * 4), ctx.buffer(40 * 4), ctx.buffer(64), ctx.buffer(8), ctx.buffer(8)]
    with pytest.raises(RuntimeError, match="multiple of 32"):
        ctx.swiglu_quant_dev(bufs[0].ptr, 1, 4096, dg, du, *[b.ptr for b in bufs[1:]])
    for b in bufs + [dg, du]:
        b.free()


# (dt, N, K, T, norm, residual, fused): elmh_ffn_dev, the FFN pair as one call; fused: the SwiGLU
# launch hands h to the down projection quantized (one token on the streaming GEMV; the GEMM's
# fragments on the 16 x 16 wave path, T > 4 and K <= 1536)
FFN_CASES = [(O.Q4, 1024, 4096, 1, False, True, True), (O.Q4, 1024, 4096, 1, True, True, True),
             (O.Q4, 2048, 2560, 1, True, False, True), (O.Q8, 1024, 2048, 1, False, True, True),
             (O.Q4, 1024, 4096, 2, True, True, False), (O.Q4, 1536, 576, 1, True, True, False),
             (O.Q4, 1536, 576, 9, False, True, True), (O.Q4, 1536, 576, 128, True, True, True),
             (O.Q8, 1536, 576, 70, False, True, True), (O.Q8, 160, 96, 33, True, True, True),
             (O.Q4, 2048, 2560, 64, True, False, False)]


@pytest.mark.parametrize("case", FFN_CASES)
def test_ffn_pair_exact(ctx, case):
    """elmh_ffn_dev: h and y bit-identical to edgelm's cpu backend (RMSNORM, then cpu::swiglu, then
    cpu::matmul with the residual), int8 activations; whether the quantized handoff ran."""
    dt, n, k, T, norm, resid, fused = case
    r = rng(900 + n + k + T + dt + 2 * norm)
    wg, wu, wd = weight(r, n, k, dt), weight(r, n, k, dt), weight(r, k, n, dt)
    dg, du, dd = up(ctx, wg), up(ctx, wu), up(ctx, wd)
    x = r.normal(0, 1, (T, k)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    res = r.normal(0, 1, (T, k)).astype(np.float32)
    bx, bn, bh, by, br = (ctx.buffer(T * k * 4), ctx.buffer(k * 4), ctx.buffer(T * n * 4), ctx.buffer(T * k * 4),
                          ctx.buffer(T * k * 4))
    bx.upload(x)
    bn.upload(nw)
    br.upload(res)
    print(f"[gpu] ffn pair dt={dt} {n}x{k} T={T} norm={norm} res={resid}", flush=True)
    got_fused = ctx.ffn_dev(bx.ptr, T, k, dg, du, bh.ptr, dd, by.ptr, br.ptr if resid else None,
                            bn.ptr if norm else None, 1e-5)
    ctx.synchronize()
    assert got_fused == fused
    xin = O.rmsnorm(x, nw, 1e-5) if norm else x
    hw = O.cpu_swiglu(xin, wg, wu, act_quant=True)
    yw = O.cpu_matmul(hw, [wd], [res] if resid else None, act_quant=True)[0]
    assert bits_equal(bh.download((T, n), np.float32), hw)
    assert bits_equal(by.download((T, k), np.float32), yw)
    for b in (bx, bn, bh, by, br, dg, du, dd):
        b.free()
