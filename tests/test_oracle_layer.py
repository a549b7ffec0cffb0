"""CPU: pins the oracle's restatement of the non-matmul layer ops (RopeTable, cpu::rmsnorm,
cpu::attention; oracle/oracle.c) before the GPU kernels are checked against it:

  1. bit for bit against the committed fixtures written by edgelm's own C++ (tests/golden);
  2. bit for bit against that C++ itself (oracle/_ref) where it is built;
  3. against what the mathematics fixes: one visible position returns v exactly, position 0
     leaves q and k unrotated, a zero row normalizes to zero, a one-hot row to a closed form,
     and the rotation preserves the norm of each (x_i, x_{i+hd/2}) pair.
"""
import os

import numpy as np
import pytest

import oracle as O
from conftest import bits_equal

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "edgelm_ref_vectors.npz")
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")
NH, NKV, HD, MC = 9, 3, 64, 24
ATTN_CALLS = [(0, 5), (5, 1), (6, 3)]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_fixture_rope_table(golden):
    c, s = O.rope_table(64, 40, 100000.0)
    assert bits_equal(c, golden["rope.cos"]) and bits_equal(s, golden["rope.sin"])


def test_fixture_rmsnorm(golden):
    for i in range(3):
        p = f"rms{i}."
        assert bits_equal(O.rmsnorm(golden[p + "x"], golden[p + "w"], 1e-5), golden[p + "y"]), p


def test_fixture_attention(golden):
    for rope in (0, 1):
        kc = np.zeros((NKV, MC, HD), np.float32)
        vc = np.zeros_like(kc)
        tab = O.rope_table(HD, MC, 100000.0) if rope else None
        for j, (pos0, T) in enumerate(ATTN_CALLS):
            p = f"attn{rope}.{j}."
            got = O.attention(golden[p + "q"], golden[p + "k"], golden[p + "v"], pos0, NH, NKV, kc, vc, tab)
            assert bits_equal(got, golden[p + "out"]), p
        assert bits_equal(kc, golden[f"attn{rope}.kc"]) and bits_equal(vc, golden[f"attn{rope}.vc"])


@needs_ref
def test_layer_ops_equal_reference_build():
    r = np.random.default_rng(21)
    for dim in (576, 577, 1, 64):
        x = r.normal(0, 2, (5, dim)).astype(np.float32)
        w = r.normal(1, 0.2, dim).astype(np.float32)
        assert bits_equal(O.rmsnorm(x, w, 1e-6), O.rq_rmsnorm(x, w, 1e-6))
    c1, s1 = O.rope_table(128, 64, 10000.0)
    c2, s2 = O.rq_rope_table(128, 64, 10000.0)
    assert bits_equal(c1, c2) and bits_equal(s1, s2)
    for nh, nkv, hd, mc in [(9, 3, 64, 64), (4, 4, 32, 40), (8, 1, 128, 33)]:
        for rope in (False, True):
            k1 = np.zeros((nkv, mc, hd), np.float32)
            v1, k2, v2 = np.zeros_like(k1), np.zeros_like(k1), np.zeros_like(k1)
            tab = O.rope_table(hd, mc, 100000.0) if rope else None
            pos = 0
            for T in (7, 1, 1, 4, 13):
                if pos + T > mc:
                    break
                q = r.normal(0, 1, (T, nh * hd)).astype(np.float32)
                k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
                v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
                a = O.attention(q, k, v, pos, nh, nkv, k1, v1, tab)
                b = O.rq_attention(q, k, v, pos, nh, nkv, k2, v2, 100000.0 if rope else None)
                assert bits_equal(a, b), (nh, nkv, hd, rope, pos, T)
                pos += T
            assert bits_equal(k1, k2) and bits_equal(v1, v2)


def test_attention_closed_forms():
    r = np.random.default_rng(22)
    q = r.normal(0, 1, (1, NH * HD)).astype(np.float32)
    k = r.normal(0, 1, (1, NKV * HD)).astype(np.float32)
    v = r.normal(0, 1, (1, NKV * HD)).astype(np.float32)
    for tab in (None, O.rope_table(HD, MC, 100000.0)):
        kc = np.zeros((NKV, MC, HD), np.float32)
        vc = np.zeros_like(kc)
        out = O.attention(q, k, v, 0, NH, NKV, kc, vc, tab)
        # one visible position: softmax weight exactly 1, out = that position's value (GQA mapping h -> h / 3)
        want = np.concatenate([v[0, (h // (NH // NKV)) * HD:(h // (NH // NKV) + 1) * HD] for h in range(NH)])
        assert bits_equal(out[0], want)
        # position 0: cos = 1, sin = 0, so the cached key is the key itself
        assert bits_equal(kc[:, 0, :].reshape(-1), k[0])


def test_rmsnorm_and_rope_closed_forms():
    w = np.linspace(0.5, 1.5, 8).astype(np.float32)
    assert bits_equal(O.rmsnorm(np.zeros((1, 8), np.float32), w, 1e-5), np.zeros((1, 8), np.float32))
    x = np.zeros((1, 8), np.float32)
    x[0, 3] = 2.0
    inv = np.float32(1.0) / np.sqrt(np.float32(4.0) / np.float32(8) + np.float32(1e-5), dtype=np.float32)
    want = np.zeros((1, 8), np.float32)
    want[0, 3] = np.float32(2.0) * inv * w[3]
    assert bits_equal(O.rmsnorm(x, w, 1e-5), want)
    c, s = O.rope_table(HD, MC, 100000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=1e-6)


def argmax_cases(r):
    """Rows that exercise std::max_element's rules: ties, signed zeros, NaNs at and after index 0."""
    rows = [r.normal(0, 1, 49152).astype(np.float32), r.normal(0, 1, 1).astype(np.float32),
            np.full(37, 2.5, np.float32), np.array([-0.0, 0.0, -0.0], np.float32),
            np.array([0.0, -0.0], np.float32), np.array([-np.inf, -np.inf, -3.0, -np.inf], np.float32)]
    x = r.normal(0, 1, 1000).astype(np.float32)
    x[[5, 700]] = 9.0  # tie: the first wins
    rows.append(x)
    x = r.normal(0, 1, 1000).astype(np.float32)
    x[0] = np.nan  # NaN at index 0: nothing compares greater, index 0 stays
    x[3] = 50.0
    rows.append(x)
    x = r.normal(0, 1, 1000).astype(np.float32)
    x[[1, 400, 999]] = np.nan  # later NaNs never replace the best
    rows.append(x)
    rows.append(np.array([1.0] + [np.nan] * 9, np.float32))
    return rows


def test_argmax_closed_forms():
    r = np.random.default_rng(30)
    rows = argmax_cases(r)
    want = [None, 0, 0, 0, 0, 2, 5, 0, None, 0]
    for x, w in zip(rows, want):
        got = int(O.argmax(x)[0])
        if w is not None:
            assert got == w, (x[:8], got, w)
        finite = x[~np.isnan(x)]
        if x.size and not np.isnan(x[0]):
            # NaN-free view: the first index of the maximum, as numpy's argmax defines it
            assert x[got] == finite.max() and got == int(np.flatnonzero(x == finite.max())[0])


@needs_ref
def test_argmax_equals_reference_build():
    r = np.random.default_rng(31)
    for x in argmax_cases(r) + [r.normal(0, 3, (5, 4099)).astype(np.float32)]:
        x = np.atleast_2d(x)
        assert np.array_equal(O.argmax(x), O.rq_argmax(x))
