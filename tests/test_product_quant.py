"""CPU: the product's load-time weight quantizers (libedgelm_host: elm_quantize_q8 / elm_quantize_q4) against
edgelm's own quantize_q8 / quantize_q4 (model.cpp:150-190) — the committed fixtures written by edgelm's build,
and edgelm's build itself where oracle/_ref is present — byte for byte, at several thread counts. Every
benchmarked and end-to-end model is quantized by these functions, so a session-level comparison (both sides
read the same file) could not catch a quantizer bug."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import host as H

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "edgelm_ref_vectors.npz")
THREADS = (1, 3, 8, 16)


def test_product_quantizers_equal_golden_vectors():
    g = np.load(GOLDEN, allow_pickle=False)
    w = g["quant.w"]
    for th in THREADS:
        q8, s8 = H.quantize_q8(w, threads=th)
        q4, s4 = H.quantize_q4(w, threads=th)
        assert np.array_equal(q8, g["quant.q8"]) and bits_equal(s8, g["quant.q8s"]), th
        assert np.array_equal(q4, g["quant.q4"]) and bits_equal(s4, g["quant.q4s"]), th


def _hard_rows(r, n, k):
    """Normal rows plus the cases the rounding rule decides: zero rows, ties at +-x.5 steps, equal-magnitude
    maxima of both signs (q4 keeps the FIRST one), subnormal and huge values."""
    w = r.normal(0, 0.02, (n, k)).astype(np.float32)
    w[0] = 0
    w[1, :] = np.float32(0.5) * (np.arange(k) % 17 - 8).astype(np.float32)
    w[2, 5], w[2, 9] = np.float32(-0.3), np.float32(0.3)
    w[3] = np.float32(1e-41) * (np.arange(k) % 5 - 2).astype(np.float32)
    w[4, ::7] = np.float32(3e38)
    w[5, :32] = np.float32(-1.0)
    return w


@pytest.mark.parametrize("dtype", ["q8", "q4"])
def test_product_quantizers_equal_oracle_and_reference(dtype):
    r = np.random.default_rng(31)
    for n, k in [(37, 96), (300, 576), (64, 1536)]:
        w = _hard_rows(r, n, k)
        want = O.quantize_q8(w) if dtype == "q8" else O.quantize_q4(w)
        ref = None
        if O.ref_available():
            ref = O.rq_quantize_q8(w) if dtype == "q8" else O.rq_quantize_q4(w)
            assert np.array_equal(want[0], ref[0]) and bits_equal(want[1], ref[1])
        for th in THREADS:
            got = H.quantize_q8(w, threads=th) if dtype == "q8" else H.quantize_q4(w, threads=th)
            assert np.array_equal(got[0], want[0]) and bits_equal(got[1], want[1]), (n, k, th)


def test_q4_rejects_k_not_multiple_of_32():
    w = np.ones((3, 40), np.float32)
    with pytest.raises(ValueError):
        H.quantize_q4(w)
    with pytest.raises(ValueError):
        H.quantize_q4(np.ones((3, 16), np.float32))
    q, s = H.quantize_q8(w)  # q8 takes any K
    assert np.all(q == 127) and np.all(s == np.float32(1) / np.float32(127))
