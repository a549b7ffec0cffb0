"""GPU: the delegate inside edgelm's own runtime. oracle/_ref/libedgelm_ref_hip.so is edgelm compiled from the
reference sources with `hip` / `hip-matmul` registered in make_backend at link time (the INTEGRATION.md patch
to backends.cpp:158-163); edgelm's Session, fusion passes, partitioner, cpu / matmul-only / reference backends
and ExecContext are edgelm's own, and its Backend has none of this build's optional hooks, so the delegate
runs its un-hooked path: every run() uploads its inputs from edgelm's host arena and copies its outputs back
(hip_backend.cpp, unprepared()).

Bar (test_e2e.cpp:33-75): logits bit-identical to edgelm's own cpu Session on the same file, fused and
unfused graphs (SessionOptions::fuse, test_e2e.cpp:48), f32 and int8 activations, prefill / chunked / decode,
and with edgelm's matmul-only backend ahead of or behind the delegate in the preference list."""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import synth as S

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not O.ref_hip_available(), reason="needs oracle/_ref (edgelm's own build)")]


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny_gpu_boundary")
    TINY_SEED = 4321
    paths = {}
    for dt in ("q8", "q4"):
        p = str(d / f"tiny.{dt}.elm")
        S.write_model(p, S.TINY, dt, seed=TINY_SEED, sd=0.15, embed_sd=0.5)
        paths[dt] = p
    return paths


def run_all(sess, ids, prefill, batch):
    out = []
    for i in range(0, prefill, batch):
        out.append(sess.forward(ids[i:min(prefill, i + batch)]))
    for t in ids[prefill:]:
        out.append(sess.forward(np.array([t], np.int32)))
    return np.concatenate(out)


VARIANTS = [("full prefill", 128, 40), ("chunked prefill (7)", 7, 40), ("prefill 5 + decode", 128, 5)]


@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("act", [False, True])
@pytest.mark.parametrize("dt", ["q8", "q4"])
@pytest.mark.parametrize("backends", ["hip,cpu", "hip-matmul,cpu", "matmul-only,hip,cpu"])
def test_edgelm_session_runs_the_delegate(tiny, backends, dt, act, fuse):
    ids = np.random.default_rng(8).integers(0, 320, 40).astype(np.int32)
    for name, batch, prefill in VARIANTS:
        print(f"[gpu] edgelm session {backends} {dt} act_int8={act} fuse={fuse} {name}", flush=True)
        kw = dict(threads=3, max_ctx=64, max_batch=batch, all_logits=True, act_quant=act, fuse=fuse)
        mine = O.RefSession(tiny[dt], backends, with_hip=True, **kw)
        ref = O.RefSession(tiny[dt], "cpu", **kw)
        nops, desc = mine.describe()
        assert ("hip" in desc), desc
        got, want = run_all(mine, ids, prefill, batch), run_all(ref, ids, prefill, batch)
        assert bits_equal(got, want), f"{name}: max diff {np.abs(got - want).max()}\n{desc}"
        mine.close(), ref.close()


def test_edgelm_session_smollm2_shape(tmp_path):
    """configs[3] through edgelm's own Session: the 128-token LCG prompt and greedy decode steps on the
    SmolLM2-135M-shaped random model (q4 + q8 embedding, int8 activations), delegate un-hooked."""
    p = str(tmp_path / "smollm2.q4.elm")
    print("[gpu] writing SmolLM2-135M-shaped random q4 model", flush=True)
    S.write_model(p, S.SMOLLM2_135M, "q4", embed_dtype="q8", seed=20260101, sd=0.05, embed_sd=0.5)
    prompt = S.lcg_prompt(128, 49152)
    for backends in ("hip,cpu", "hip-matmul,cpu"):
        mine = O.RefSession(p, backends, threads=8, max_ctx=160, max_batch=128, act_quant=True, with_hip=True)
        ref = O.RefSession(p, "cpu", threads=16, max_ctx=160, max_batch=128, act_quant=True)
        print(f"[gpu] edgelm session smollm2 {backends} prefill", flush=True)
        a, b = mine.forward(prompt), ref.forward(prompt)
        assert bits_equal(a, b)
        tok = int(O.rq_argmax(b)[0])
        for step in range(6):
            a, b = mine.forward(np.array([tok], np.int32)), ref.forward(np.array([tok], np.int32))
            assert bits_equal(a, b), f"{backends} decode step {step}"
            tok = int(O.rq_argmax(b)[0])
        mine.close(), ref.close()
