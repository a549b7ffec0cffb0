"""Writes tests/golden/edgelm_ref_vectors.npz: inputs and outputs of edgelm's own C++ (compiled from
the reference sources into oracle/_ref by oracle/Makefile) for the quantized-matmul path.

The fixtures let the CPU suite pin the C oracle (oracle/oracle.c) on machines where the reference
build is absent. Inputs come from numpy's default_rng with the seeds below; outputs from:
  quantize_q8 / quantize_q4       (model.cpp:150-190)
  quantize_act_row                (kernels_ref.cpp:23-37), including the outlier row of the
                                  reference's own int8 test (make_tiny.py:448-450)
  cpu::matmul / cpu::swiglu       (kernels_cpu.cpp:339-411), act f32 and int8, x86 scalar path
  ref::matmul / ref::swiglu       (kernels_ref.cpp:58-80, 153-160)
  RopeTable, cpu::rmsnorm, cpu::attention (kernels_ref.cpp:11-21, kernels_cpu.cpp:326-335, 417-488)
Shapes and token counts follow tests/test_ops.cpp:119-154 and 192-240.

    python tests/golden/gen_fixtures.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "edgelm_ref_vectors.npz")


ATTN_CALLS = [(0, 5), (5, 1), (6, 3)]  # (pos0, T): prefill, decode, chunk


def layer_fixtures(out):
    """RopeTable (kernels_ref.cpp:11-21), cpu::rmsnorm (kernels_cpu.cpp:326-335) and cpu::attention
    (kernels_cpu.cpp:417-488) on SmolLM2-135M's head shape (9 query / 3 KV heads of 64)."""
    rng = np.random.default_rng(20260102)
    out["rope.cos"], out["rope.sin"] = O.rq_rope_table(64, 40, 100000.0)
    for i, (rows, dim) in enumerate([(4, 578), (3, 576), (2, 7)]):
        x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
        w = rng.normal(1, 0.1, dim).astype(np.float32)
        out[f"rms{i}.x"], out[f"rms{i}.w"] = x, w
        out[f"rms{i}.y"] = O.rq_rmsnorm(x, w, 1e-5)
    nh, nkv, hd, mc = 9, 3, 64, 24
    for rope in (0, 1):
        kc = np.zeros((nkv, mc, hd), np.float32)
        vc = np.zeros_like(kc)
        for j, (pos0, T) in enumerate(ATTN_CALLS):
            p = f"attn{rope}.{j}."
            q = rng.normal(0, 1, (T, nh * hd)).astype(np.float32)
            k = rng.normal(0, 1, (T, nkv * hd)).astype(np.float32)
            v = rng.normal(0, 1, (T, nkv * hd)).astype(np.float32)
            out[p + "q"], out[p + "k"], out[p + "v"] = q, k, v
            out[p + "out"] = O.rq_attention(q, k, v, pos0, nh, nkv, kc, vc, 100000.0 if rope else None)
        out[f"attn{rope}.kc"], out[f"attn{rope}.vc"] = kc, vc


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libedgelm_ref.so not built (needs /root/reference; run make -C oracle)")
    rng = np.random.default_rng(20260101)
    out = {}
    pool = O.RefPool(4, 32, 2048)
    # quantizers
    w = rng.normal(0, 0.05, (37, 96)).astype(np.float32)
    w[5] = 0.0
    w[6, 7] = 0.3  # a dominant element
    w[7, 3] = -0.3
    out["quant.w"] = w
    out["quant.q8"], out["quant.q8s"] = O.rq_quantize_q8(w)
    out["quant.q4"], out["quant.q4s"] = O.rq_quantize_q4(w)
    # activation quantizer
    xa = rng.normal(0, 1, (3, 96)).astype(np.float32)
    xa[1, 40] = 25.0
    xa[2, 64:96] = 0.0
    out["actq.x"] = xa
    out["actq.q"], out["actq.d"] = O.rq_quantize_act(xa)
    # matmuls
    cases = [("f32act", d, n, k, T) for d in (O.Q8, O.Q4) for (n, k) in [(48, 64), (37, 96), (130, 160)]
             for T in (1, 3, 4, 17)]
    cases += [("a8", d, 70, 160, T) for d in (O.Q8, O.Q4) for T in (1, 3, 4, 9)]
    for i, (kind, dt, n, k, T) in enumerate(cases):
        wf = rng.normal(0, 1, (n, k)).astype(np.float32)
        wuf = rng.normal(0, 1, (n, k)).astype(np.float32)
        x = rng.normal(0, 1, (T, k)).astype(np.float32)
        res = rng.normal(0, 1, (T, n)).astype(np.float32)
        W, Wu = O.make_weight(wf, dt), O.make_weight(wuf, dt)
        aq = kind == "a8"
        p = f"mm{i}."
        out[p + "meta"] = np.array([dt, n, k, T, int(aq)], np.int64)
        out[p + "w"], out[p + "wu"], out[p + "x"], out[p + "res"] = wf, wuf, x, res
        out[p + "cpu"] = O.rq_cpu_matmul(pool, x, [W], [res], aq)[0]
        out[p + "cpu_sw"] = O.rq_cpu_swiglu(pool, x, W, Wu, aq)
        out[p + "ref"] = O.rq_ref_matmul(x, W, res, aq)
        out[p + "ref_sw"] = O.rq_ref_swiglu(x, W, Wu, aq)
    pool.close()
    layer_fixtures(out)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
