"""CPU: pins the oracle (oracle/oracle.c) before anything is checked against it.

  1. against edgelm's own C++ compiled from the reference sources (oracle/_ref), bit for bit;
  2. against the committed fixtures written by that build (tests/golden/gen_fixtures.py);
  3. against what the mathematics fixes, independently of the oracle's code: quantizer error
     bounds and extreme values, zero rows, integer block sums by numpy brute force, and the
     int8-activation f32 fold re-derived with numpy float32 arithmetic in block order.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from conftest import bits_equal, rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "edgelm_ref_vectors.npz")
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_fixture_quantizers(golden):
    w = golden["quant.w"]
    q8, s8 = O.quantize_q8(w)
    q4, s4 = O.quantize_q4(w)
    assert np.array_equal(q8, golden["quant.q8"]) and bits_equal(s8, golden["quant.q8s"])
    assert np.array_equal(q4, golden["quant.q4"]) and bits_equal(s4, golden["quant.q4s"])


def test_fixture_act_quant(golden):
    q, d = O.quantize_act(golden["actq.x"])
    assert np.array_equal(q, golden["actq.q"]) and bits_equal(d, golden["actq.d"])


def test_fixture_matmuls(golden):
    i = 0
    n_cases = 0
    while f"mm{i}.meta" in golden:
        p = f"mm{i}."
        dt, n, k, T, aq = (int(v) for v in golden[p + "meta"])
        W, Wu = O.make_weight(golden[p + "w"], dt), O.make_weight(golden[p + "wu"], dt)
        x, res = golden[p + "x"], golden[p + "res"]
        assert bits_equal(O.cpu_matmul(x, [W], [res], aq)[0], golden[p + "cpu"]), p
        assert bits_equal(O.cpu_swiglu(x, W, Wu, aq), golden[p + "cpu_sw"]), p
        assert bits_equal(O.ref_matmul(x, W, res, aq), golden[p + "ref"]), p
        assert bits_equal(O.ref_swiglu(x, W, Wu, aq), golden[p + "ref_sw"]), p
        i += 1
        n_cases += 1
    assert n_cases == 32


@needs_ref
def test_oracle_equals_reference_build():
    r = np.random.default_rng(11)
    pool = O.RefPool(3, 40, 1536)
    try:
        for n, k in [(48, 64), (130, 160), (960, 576), (576, 1536)]:
            w = r.normal(0, 0.05, (n, k)).astype(np.float32)
            for dt in (O.Q8, O.Q4):
                W, Wu = O.make_weight(w, dt), O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
                qa, sa = O.quantize_q8(w) if dt == O.Q8 else O.quantize_q4(w)
                qb, sb = O.rq_quantize_q8(w) if dt == O.Q8 else O.rq_quantize_q4(w)
                assert np.array_equal(qa, qb) and bits_equal(sa, sb)
                for T in (1, 4, 33):
                    x = r.normal(0, 1, (T, k)).astype(np.float32)
                    res = r.normal(0, 1, (T, n)).astype(np.float32)
                    for aq in (False, True):
                        assert bits_equal(O.cpu_matmul(x, [W], [res], aq)[0], O.rq_cpu_matmul(pool, x, [W], [res], aq)[0])
                        assert bits_equal(O.cpu_swiglu(x, W, Wu, aq), O.rq_cpu_swiglu(pool, x, W, Wu, aq))
                        if n * k * T < 3e6:
                            assert bits_equal(O.ref_matmul(x, W, res, aq), O.rq_ref_matmul(x, W, res, aq))
    finally:
        pool.close()


def test_quantizer_closed_forms():
    """Error bounds of test_ops.cpp:156-171, plus extremes the mathematics fixes."""
    r = np.random.default_rng(3)
    n, k = 64, 256
    w = r.normal(0, 0.05, (n, k)).astype(np.float32)
    w[0] = 0.0
    q8, s8 = O.quantize_q8(w)
    q4, s4 = O.quantize_q4(w)
    d8 = O.dequantize(O.Weight(O.Q8, n, k, q8, s8))
    d4 = O.dequantize(O.Weight(O.Q4, n, k, q4, s4))
    amax = np.abs(w).max()
    e8, e4 = np.abs(d8 - w).max(), np.abs(d4 - w).max()
    assert e8 <= amax / 127 * 0.5 + 1e-7 and e4 <= amax / 8 + 1e-7 and e4 > e8
    assert s8[0] == 0 and np.all(q8[0] == 0) and np.all(s4[0] == 0) and np.all(q4[0] == 0x88)
    # q8: the row's max-magnitude element maps to +-127
    for row in range(1, n):
        j = int(np.argmax(np.abs(w[row])))
        assert abs(int(q8[row, j])) == 127
        assert s8[row] == np.float32(np.abs(w[row]).max() / np.float32(127))
    # q4: the group's first max-magnitude element maps to -8 (stored 0); low/high nibble layout
    g = w[1, :32]
    j = int(np.argmax(np.abs(g)))
    nib = (q4[1, j] & 0x0F) if j < 16 else (q4[1, j - 16] >> 4)
    assert nib == 0 and s4[1, 0] == np.float32(g[j] / np.float32(-8))


def test_act_quant_closed_forms():
    r = np.random.default_rng(4)
    x = r.normal(0, 1, (5, 256)).astype(np.float32)
    x[1, 40] = 25.0
    x[2, :32] = 0.0
    q, d = O.quantize_act(x)
    blocks = x.reshape(5, 8, 32)
    qb = q.reshape(5, 8, 32).astype(np.int32)
    assert np.all(d == (np.abs(blocks).max(axis=2) / np.float32(127)).astype(np.float32))
    nz = d > 0
    assert np.all(np.abs(qb).max(axis=2)[nz] == 127) and np.all(qb[~nz] == 0)
    err = np.abs(qb * d[..., None] - blocks)
    assert np.all(err <= d[..., None] * 0.5 * (1 + 1e-6))
    assert d[1, 1] >= 25 / 127 and d[1, 0] < 0.1  # outlier stays in its block (test_ops.cpp:205-207)


def test_block_sums_brute_force():
    r = np.random.default_rng(5)
    for dt in (O.Q8, O.Q4):
        W = O.make_weight(r.normal(0, 0.05, (37, 96)).astype(np.float32), dt)
        xq = r.integers(-127, 128, (3, 96)).astype(np.int8)
        if dt == O.Q8:
            wq = W.data.astype(np.int64)
        else:
            p = W.data.reshape(37, 3, 16).astype(np.int64)
            wq = np.concatenate([(p & 15) - 8, (p >> 4) - 8], axis=2).reshape(37, 96)
        S = np.einsum("tbi,nbi->tnb", xq.astype(np.int64).reshape(3, 3, 32), wq.reshape(37, 3, 32))
        assert np.array_equal(O.block_sums(xq, W), S)


def test_a8_fold_rederived_with_numpy():
    """out = sum_b float(S_b) * xd_b (* ws) folded in block order with single-rounding float32 ops."""
    r = np.random.default_rng(6)
    for dt in (O.Q8, O.Q4):
        n, k, T = 70, 160, 3
        W = O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        xq, xd = O.quantize_act(x)
        S = O.block_sums(xq, W).astype(np.float32)  # exact: |S| < 2^24
        acc = np.zeros((T, n), np.float32)
        for b in range(k // 32):
            if dt == O.Q8:
                p = S[:, :, b] * xd[:, b:b + 1]
            else:
                p = S[:, :, b] * (W.scales[None, :, b] * xd[:, b:b + 1])
            acc = acc + p
        want = acc * W.scales[None, :] if dt == O.Q8 else acc
        assert bits_equal(O.cpu_matmul(x, [W], None, act_quant=True)[0], want)
        # int8 activations perturb the result, but only a little (test_ops.cpp:235-238)
        e = rel_err(O.ref_matmul(x, W, act_quant=True), O.ref_matmul(x, W, act_quant=False))
        assert 0 < e < 2e-2


def test_matmul_n_equals_separate():
    r = np.random.default_rng(7)
    ws = [O.make_weight(r.normal(0, 1, (m, 64)).astype(np.float32), d) for m, d in [(96, O.Q8), (32, O.Q4), (32, O.F32)]]
    for T in (1, 6):
        x = r.normal(0, 1, (T, 64)).astype(np.float32)
        fused = O.cpu_matmul(x, ws, None, act_quant=False)
        for y, w in zip(fused, ws):
            assert bits_equal(y, O.cpu_matmul(x, [w], None, act_quant=False)[0])
            assert rel_err(y, O.ref_matmul(x, w)) < 1e-5


def test_silu_matches_libm_definition():
    for v in (-10.0, -1.5, -0.0, 0.0, 0.3, 2.0, 30.0):
        v32 = np.float32(v)
        want = v32 / (np.float32(1) + np.exp(-v32, dtype=np.float32))
        assert abs(O.silu(float(v32)) - float(want)) <= 2e-7 * max(1.0, abs(float(want)))


def test_device_expf_matches_libm_exhaustively(tmp_path):
    """elm_expf (the expf the device SwiGLU epilogue uses) equals the host libm expf on all 2^32 inputs."""
    src = tmp_path / "expf_check.c"
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src.write_text(
        "#include <math.h>\n#include <stdio.h>\n#include <string.h>\n#include <stdint.h>\n"
        "#define ELM_HOSTDEV\n#include \"elm_expf.h\"\n"
        "int main(void){unsigned long bad=0;for(uint64_t u=0;u<=0xFFFFFFFFull;++u){uint32_t v=(uint32_t)u;float x;"
        "memcpy(&x,&v,4);float a=expf(x),b=elm_expf(x);if(isnan(a)&&isnan(b))continue;"
        "if(memcmp(&a,&b,4))bad++;}printf(\"%lu\\n\",bad);return bad!=0;}\n")
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", os.path.join(root, "edgelm_amd", "csrc"), str(src), "-o",
                    str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout


@needs_ref
def test_act_quant_applies_against_reference_build():
    """act_quant_applies (kernels.hpp:46-48): with K % 32 != 0, or f32 weights, int8 activations do not apply and
    edgelm's cpu and reference backends take the f32 path; the oracle must agree with edgelm's build there."""
    r = np.random.default_rng(12)
    pool = O.RefPool(2, 9, 200)
    try:
        for k, dt in [(40, O.Q8), (72, O.Q8), (200, O.Q8), (64, O.F32), (96, O.F32)]:
            n = 37
            W = O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
            Wu = O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
            for T in (1, 9):
                x = r.normal(0, 1, (T, k)).astype(np.float32)
                res = r.normal(0, 1, (T, n)).astype(np.float32)
                a8 = O.cpu_matmul(x, [W], [res], True)[0]
                assert bits_equal(a8, O.rq_cpu_matmul(pool, x, [W], [res], True)[0]), (k, dt, T)
                assert bits_equal(a8, O.cpu_matmul(x, [W], [res], False)[0]), (k, dt, T)
                assert bits_equal(O.ref_matmul(x, W, res, True), O.rq_ref_matmul(x, W, res, True)), (k, dt, T)
                assert bits_equal(O.cpu_swiglu(x, W, Wu, True), O.rq_cpu_swiglu(pool, x, W, Wu, True)), (k, dt, T)
    finally:
        pool.close()


# ---- the per-token activation mode (an extension: edgelm has no such mode, so nothing of edgelm's pins it
# directly; these checks tie it to the pinned per-block quantizer and matmul, and to integer brute force) ----

def _rows_with_shared_block_max(r, T, K):
    """Rows where every 32-block holds the row's largest magnitude (both signs occur), so the per-block
    scales all equal the per-row one."""
    x = r.normal(0, 1, (T, K)).astype(np.float32)
    amax = np.float32(5.0) + np.abs(x).max()
    for t in range(T):
        for b in range(K // 32):
            x[t, b * 32 + r.integers(0, 32)] = amax if (t + b) % 2 else -amax
    return x


def test_token_quantizer_equals_block_quantizer_when_block_maxima_agree():
    r = np.random.default_rng(21)
    x = _rows_with_shared_block_max(r, 6, 256)
    q, d = O.quantize_act_token(x)
    qb, db = O.quantize_act(x)
    assert np.array_equal(q, qb) and np.all(db == d[:, None])
    if O.ref_available():
        qr, dr = O.rq_quantize_act(x)
        assert np.array_equal(q, qr) and np.all(dr == d[:, None])


def test_token_quantizer_closed_forms():
    r = np.random.default_rng(22)
    x = r.normal(0, 1, (7, 160)).astype(np.float32)
    x[2] = 0.0
    x[3, 17] = -40.0  # an outlier sets the whole row's scale
    q, d = O.quantize_act_token(x)
    assert d[2] == 0 and np.all(q[2] == 0)
    nz = d > 0
    assert np.all(d == (np.abs(x).max(axis=1) / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q[nz].astype(np.int32)).max(axis=1) == 127)
    err = np.abs(q.astype(np.float64) * d[:, None].astype(np.float64) - x)
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-6))
    assert q[3, 17] == -127 and np.abs(q[3]).astype(np.int32).sum() < np.abs(q[4]).astype(np.int32).sum()


def _int_weights(W):
    if W.dtype == O.Q8:
        return W.data.astype(np.int64)
    p = W.data.reshape(W.rows, W.cols // 32, 16).astype(np.int64)
    return np.concatenate([(p & 15) - 8, (p >> 4) - 8], axis=2).reshape(W.rows, W.cols)


def test_token_matmul_integer_sums_brute_force():
    """q8: one int32 sum over all of K (numpy int64 brute force), then (float(S) * d) * ws;
    q4: int32 sums per 32-group, folded in group order as float(S_g) * ws_g, then * d."""
    r = np.random.default_rng(23)
    for dt in (O.Q8, O.Q4):
        n, k, T = 53, 224, 5
        W = O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
        x = r.normal(0, 1, (T, k)).astype(np.float32)
        res = r.normal(0, 1, (T, n)).astype(np.float32)
        xq, d = O.quantize_act_token(x)
        wq = _int_weights(W)
        if dt == O.Q8:
            S = xq.astype(np.int64) @ wq.T
            assert np.abs(S).max() < 2 ** 24
            want = (S.astype(np.float32) * d[:, None]) * W.scales[None, :]
        else:
            Sg = np.einsum("tgi,ngi->tng", xq.astype(np.int64).reshape(T, k // 32, 32), wq.reshape(n, k // 32, 32))
            acc = np.zeros((T, n), np.float32)
            for g in range(k // 32):
                acc = acc + Sg[:, :, g].astype(np.float32) * W.scales[None, :, g]
            want = acc * d[:, None]
        assert bits_equal(O.matmul_a8_token(x, W), want), dt
        assert bits_equal(O.matmul_a8_token(x, W, res), res + want), dt


def test_token_matmul_equals_edgelm_where_the_modes_coincide():
    """With a single nonzero 32-block per row the per-block fold has one term, and with a power-of-two scale
    (block max 127 * 2^-3) every rescale is exact: the per-token result then equals edgelm's per-block
    cpu::matmul bit for bit."""
    r = np.random.default_rng(24)
    for dt in (O.Q8, O.Q4):
        n, k, T = 41, 192, 4
        W = O.make_weight(r.normal(0, 0.05, (n, k)).astype(np.float32), dt)
        x = np.zeros((T, k), np.float32)
        for t in range(T):
            b = (2 * t + 1) % (k // 32)
            blk = r.normal(0, 0.03, 32).astype(np.float32)
            blk[r.integers(0, 32)] = np.float32(127 * 0.125) * (1 if t % 2 else -1)
            x[t, b * 32:(b + 1) * 32] = blk
        _, d = O.quantize_act_token(x)
        assert np.all(d == np.float32(0.125))
        want = O.cpu_matmul(x, [W], None, act_quant=True)[0]
        assert bits_equal(O.matmul_a8_token(x, W), want), dt


@needs_ref
def test_oracle_tiny_magnitudes_against_reference_build():
    """Scales and activation blocks near and below the normal range: the oracle keeps edgelm's float order there
    too (q4: float(S) * (ws * xd) per block, subnormal products included)."""
    r = np.random.default_rng(13)
    pool = O.RefPool(2, 40, 576)
    try:
        for dt in (O.Q8, O.Q4):
            w = r.normal(0, 0.05, (40, 576)).astype(np.float32)
            w[1] *= np.float32(1e-30)
            w[2] *= np.float32(1e-36)
            w[3] = np.float32(3e-39) * np.sign(w[3])
            W = O.make_weight(w, dt)
            Wu = O.make_weight(r.normal(0, 0.05, (40, 576)).astype(np.float32), dt)
            for T in (1, 5, 33):
                x = r.normal(0, 1, (T, 576)).astype(np.float32)
                x[:, 32:64] *= np.float32(1e-33)
                x[:, 96:128] *= np.float32(1e-38)
                x[:, 160:192] = np.float32(2e-42)
                res = r.normal(0, 1e-30, (T, 40)).astype(np.float32)
                for aq in (False, True):
                    assert bits_equal(O.cpu_matmul(x, [W], [res], aq)[0], O.rq_cpu_matmul(pool, x, [W], [res], aq)[0])
                    assert bits_equal(O.cpu_swiglu(x, W, Wu, aq), O.rq_cpu_swiglu(pool, x, W, Wu, aq))
    finally:
        pool.close()
