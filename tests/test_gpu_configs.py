"""GPU parity at the benchmark's configurations: the shapes and token
counts bench.py reports, through the C ABI, against the CPU oracle (edgelm's cpu backend on its x86 scalar
path; the per-token extension against its pinned restatement).

The oracle is serial, so the biggest problems are checked on a stripe of output rows: every output row of a
matmul depends only on its own weight row and x, so the oracle run on the stripe's rows must give exactly the
GPU's values in those columns. Stripes take the first and last row tiles (partial-tile and XCD edges) and
random rows between.

Bars: per-block int8 activations (ELMH_ACT_INT8, ELMH_EXACT) bit-identical to edgelm's cpu backend; the
per-token extension bit-identical to orc_matmul_a8_token; q4 scales and activation blocks of any magnitude
(subnormal included) bit-identical too.
"""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import elmh as E

pytestmark = pytest.mark.gpu


def up(ctx, w):
    return ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)


def rows_of(w, idx):
    """The weight restricted to rows idx (same dtype and layout)."""
    return O.Weight(w.dtype, len(idx), w.cols, w.data[idx], w.scales[idx])


def stripe(r, n, extra=256):
    if n <= 1024:
        return np.arange(n)
    mid = r.choice(np.arange(512, n - 256), size=extra, replace=False)
    return np.unique(np.concatenate([np.arange(512), mid, np.arange(n - 256, n)]))


def weight(r, n, k, dt, sd=0.02):
    return O.make_weight(r.normal(0, sd, (n, k)).astype(np.float32), dt)


def check_cols(got, want, idx, what):
    assert bits_equal(np.ascontiguousarray(got[:, idx]), want), f"{what}: max diff {np.abs(got[:, idx] - want).max()}"


# ------------------------------------------------------------------ SmolLM2-135M prefill GEMMs

SMOL_T = [32, 128, 512]


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_smollm2_prefill_shapes(ctx, dt):
    """MATMUL_N QKV 576+192+192 x 576, FFN_SWIGLU 2 x 1536 x 576, MATMUL_ADD 576 x 1536 + residual and the
    q8 LM head 49152 x 576, at T = 32 / 128 / 512, per-block exact and per-token."""
    r = np.random.default_rng(9000 + dt)
    qkv = [weight(r, n, 576, dt) for n in (576, 192, 192)]
    wg, wu = weight(r, 1536, 576, dt), weight(r, 1536, 576, dt)
    wd = weight(r, 576, 1536, dt)
    head = weight(r, 49152, 576, O.Q8)
    d_qkv = [up(ctx, w) for w in qkv]
    dg, du, dd, dh = up(ctx, wg), up(ctx, wu), up(ctx, wd), up(ctx, head)
    hidx = stripe(r, 49152)
    head_s = rows_of(head, hidx)
    for T in SMOL_T:
        x = r.normal(0, 1, (T, 576)).astype(np.float32)
        xf = r.normal(0, 1, (T, 1536)).astype(np.float32)
        res = r.normal(0, 1, (T, 576)).astype(np.float32)
        for act in (E.ACT_INT8, E.ACT_INT8_TOKEN):
            print(f"[gpu] smollm2 dt={dt} T={T} act={act}: qkv, swiglu, down", flush=True)
            got = ctx.matmul(x, d_qkv, None, act=act)
            if act == E.ACT_INT8:
                want = O.cpu_matmul(x, qkv, None, act_quant=True)
            else:
                want = [O.matmul_a8_token(x, w) for w in qkv]
            for i, (g, wv) in enumerate(zip(got, want)):
                assert bits_equal(g, wv), f"qkv target {i} T={T} act={act}"
            sw = ctx.swiglu(x, dg, du, act=act)
            if act == E.ACT_INT8:
                assert bits_equal(sw, O.cpu_swiglu(x, wg, wu, act_quant=True)), f"swiglu T={T}"
            else:
                g, u = O.matmul_a8_token(x, wg), O.matmul_a8_token(x, wu)
                want_sw = np.array([O.silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape) * u
                assert bits_equal(sw, want_sw), f"swiglu token T={T}"
            down = ctx.matmul(xf, [dd], [res], act=act)[0]
            want_d = (O.cpu_matmul(xf, [wd], [res], act_quant=True)[0] if act == E.ACT_INT8
                      else O.matmul_a8_token(xf, wd, res))
            assert bits_equal(down, want_d), f"down T={T} act={act}"
            print(f"[gpu] smollm2 dt={dt} T={T} act={act}: lm head ({len(hidx)} of 49152 rows checked)", flush=True)
            lg = ctx.matmul(x, [dh], None, act=act)[0]
            want_h = (O.cpu_matmul(x, [head_s], None, act_quant=True)[0] if act == E.ACT_INT8
                      else O.matmul_a8_token(x, head_s))
            check_cols(lg, want_h, hidx, f"lm head T={T} act={act}")
    for d in d_qkv + [dg, du, dd, dh]:
        d.free()


# ------------------------------------------------------------------ Llama-3-8B-shaped layer

@pytest.mark.parametrize("dt", [O.Q4, O.Q8])
def test_llama8b_layer_shapes(ctx, dt):
    """QKV 4096+1024+1024 x 4096 (MATMUL_N), gate+up 2 x 14336 x 4096 (FFN_SWIGLU) and down 4096 x 14336 +
    residual at T = 1 (streaming GEMV) and T = 512 (int8 MFMA GEMM), per-block exact; per-token at T = 512."""
    r = np.random.default_rng(9100 + dt)
    print(f"[gpu] llama8b dt={dt}: quantizing weights", flush=True)
    qkv = [weight(r, n, 4096, dt) for n in (4096, 1024, 1024)]
    wg, wu = weight(r, 14336, 4096, dt), weight(r, 14336, 4096, dt)
    wd = weight(r, 4096, 14336, dt)
    d_qkv = [up(ctx, w) for w in qkv]
    dg, du, dd = up(ctx, wg), up(ctx, wu), up(ctx, wd)
    qidx = [stripe(r, w.rows, 128) for w in qkv]
    qkv_s = [rows_of(w, i) for w, i in zip(qkv, qidx)]
    fidx = stripe(r, 14336, 128)
    wg_s, wu_s = rows_of(wg, fidx), rows_of(wu, fidx)
    didx = stripe(r, 4096, 128)
    wd_s = rows_of(wd, didx)
    for T in (1, 512):
        x = r.normal(0, 1, (T, 4096)).astype(np.float32)
        xf = r.normal(0, 1, (T, 14336)).astype(np.float32)
        res = r.normal(0, 1, (T, 4096)).astype(np.float32)
        acts = (E.ACT_INT8,) if T == 1 else (E.ACT_INT8, E.ACT_INT8_TOKEN)
        for act in acts:
            tok = act == E.ACT_INT8_TOKEN
            print(f"[gpu] llama8b dt={dt} T={T} act={act}: qkv", flush=True)
            got = ctx.matmul(x, d_qkv, None, act=act)
            for i, (g, ws, idx) in enumerate(zip(got, qkv_s, qidx)):
                want = O.matmul_a8_token(x, ws) if tok else O.cpu_matmul(x, [ws], None, act_quant=True)[0]
                check_cols(g, want, idx, f"qkv target {i} T={T} act={act}")
            print(f"[gpu] llama8b dt={dt} T={T} act={act}: gate+up", flush=True)
            sw = ctx.swiglu(x, dg, du, act=act)
            if tok:
                g, u = O.matmul_a8_token(x, wg_s), O.matmul_a8_token(x, wu_s)
                want = np.array([O.silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape) * u
            else:
                want = O.cpu_swiglu(x, wg_s, wu_s, act_quant=True)
            check_cols(sw, want, fidx, f"swiglu T={T} act={act}")
            print(f"[gpu] llama8b dt={dt} T={T} act={act}: down", flush=True)
            down = ctx.matmul(xf, [dd], [res], act=act)[0]
            rs = np.ascontiguousarray(res[:, didx])
            want = O.matmul_a8_token(xf, wd_s, rs) if tok else O.cpu_matmul(xf, [wd_s], [rs], act_quant=True)[0]
            check_cols(down, want, didx, f"down T={T} act={act}")
    for d in d_qkv + [dg, du, dd]:
        d.free()


# ------------------------------------------------------------------ q4 scales and activations of any magnitude

def tiny_case(r, n, k, dt):
    """Weights whose rows include tiny and subnormal scales, and activations whose 32-blocks include
    blocks so small that ws * xd falls below 2^-122 and below the normal range, next to ordinary ones."""
    w = r.normal(0, 0.05, (n, k)).astype(np.float32)
    w[1] *= np.float32(1e-30)
    w[2] *= np.float32(1e-36)
    w[3] = np.float32(3e-39) * np.sign(w[3])  # subnormal weights: subnormal q4 scales
    W = O.make_weight(w, dt)
    return W


def tiny_acts(r, T, k):
    x = r.normal(0, 1, (T, k)).astype(np.float32)
    nb = k // 32
    for t in range(T):
        for b in range(nb):
            m = (t * 7 + b * 3) % 5
            if m == 1:
                x[t, b * 32:(b + 1) * 32] *= np.float32(1e-33)
            elif m == 2:
                x[t, b * 32:(b + 1) * 32] *= np.float32(1e-38)
            elif m == 3:
                x[t, b * 32:(b + 1) * 32] = np.float32(2e-42) * np.sign(x[t, b * 32:(b + 1) * 32])
    return x


@pytest.mark.parametrize("dt", [O.Q4, O.Q8])
def test_tiny_scales_and_blocks_bit_exact(ctx, dt, monkeypatch):
    """Products ws * xd below 2^-122 (and subnormal) go through every path bit-identically: the small and
    the streaming GEMV, the three GEMM kernels, SwiGLU, the per-token mode and f32 activations."""
    r = np.random.default_rng(9200 + dt)
    for n, k in [(96, 576), (40, 4096), (36, 14336)]:
        W, Wu = tiny_case(r, n, k, dt), tiny_case(r, n, k, dt)
        dw, du = up(ctx, W), up(ctx, Wu)
        Ts = [1, 2, 4] + ([5, 33, 130] if k <= 4096 else [])
        for T in Ts:
            x = tiny_acts(r, T, k)
            res = r.normal(0, 1e-30, (T, n)).astype(np.float32)
            kernels = ["wave", "wave32", "ring"] if T > 4 else [None]
            for kern in kernels:
                if kern:
                    monkeypatch.setenv("ELMH_GEMM_KERNEL", kern)
                print(f"[gpu] tiny dt={dt} {n}x{k} T={T} kernel={kern}", flush=True)
                got = ctx.matmul(x, [dw], [res], act=E.ACT_INT8)[0]
                assert bits_equal(got, O.cpu_matmul(x, [W], [res], act_quant=True)[0]), f"T={T} {kern}"
                sw = ctx.swiglu(x, dw, du, act=E.ACT_INT8)
                assert bits_equal(sw, O.cpu_swiglu(x, W, Wu, act_quant=True)), f"swiglu T={T} {kern}"
                tok = ctx.matmul(x, [dw], [res], act=E.ACT_INT8_TOKEN)[0]
                assert bits_equal(tok, O.matmul_a8_token(x, W, res)), f"token T={T} {kern}"
            monkeypatch.delenv("ELMH_GEMM_KERNEL", raising=False)
            if T <= 33:
                f32 = ctx.matmul(x, [dw], [res], act=E.ACT_F32)[0]
                assert bits_equal(f32, O.cpu_matmul(x, [W], [res], act_quant=False)[0]), f"f32 T={T}"
        dw.free()
        du.free()
