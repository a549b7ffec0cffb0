"""CPU: the host runtime around the delegate — .elm writing/loading, fusion passes, memory planner,
partitioner — against edgelm's own loader and passes (oracle/_ref) and the expectations of edgelm's
tests (test_graph.cpp:182-339)."""
import os

import numpy as np
import pytest

import oracle as O
from edgelm_amd import synth as S
from edgelm_amd import host

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny")
    TINY_SEED = 1234
    paths = {}
    for dt in ("f32", "q8", "q4"):
        p = str(d / f"tiny.{dt}.elm")
        S.write_model(p, S.TINY, dt, seed=TINY_SEED, sd=0.15, embed_sd=0.5)
        paths[dt] = p
    return paths


def test_loader_config_and_graph(tiny):
    for dt, code in (("f32", 0), ("q8", 1), ("q4", 2)):
        m = host.Model(tiny[dt])
        assert m.cfg["vocab"] == 320 and m.cfg["dim"] == 64 and m.cfg["n_layers"] == 2 and m.cfg["tied"] == 1
        assert m.cfg["dtype"] == code
    with pytest.raises(RuntimeError):
        host.Model(os.path.join(os.path.dirname(tiny["q8"]), "missing.elm"))
    bad = os.path.join(os.path.dirname(tiny["q8"]), "bad.elm")
    with open(bad, "wb") as f:
        f.write(b"definitely not an elm file" + b"." * 200)
    with pytest.raises(RuntimeError):
        host.Model(bad)
    # record counts the graph section cannot hold (u32 n_tensors at byte 8, n_ops at byte 12) are refused as
    # a malformed file before anything is allocated for them
    with open(tiny["q8"], "rb") as f:
        blob = bytearray(f.read())
    for at in (8, 12):
        huge = bytearray(blob)
        huge[at:at + 4] = (0xFFFFFFFF).to_bytes(4, "little")
        with open(bad, "wb") as f:
            f.write(huge)
        with pytest.raises(RuntimeError, match="malformed .elm file"):
            host.Model(bad)


def test_fusion_and_planner(tiny):
    m = host.Model(tiny["q4"])
    fz = m.fusion()
    assert (fz["swiglu"], fz["shared_input"], fz["residual"], fz["rope"]) == (2, 2, 4, 2)
    assert fz["ops_before"] == 1 + 2 * 16 + 3 and fz["ops_after"] == 1 + 2 * 7 + 3
    for fuse in (False, True):
        for T in (1, 16, 128):
            ok, arena, naive = m.plan(T, 1, fuse)
            assert ok and arena < naive and arena >= T * 64 * 4


@needs_ref
def test_reference_loader_reads_our_files(tiny):
    for dt in ("q8", "q4"):
        r = O.RefSession(tiny[dt], "cpu", threads=1, max_ctx=32, max_batch=8)
        nops, desc = r.describe()
        assert nops == 18 and "reference 2 ops" in desc
        r.close()


def test_partitioner_hip_claims(tiny):
    for dt in ("q8", "q4"):
        m = host.Model(tiny[dt])
        # hip-matmul: exactly the quantized matmuls (per layer 4, plus the LM head)
        n, desc = m.partition("hip-matmul,cpu")
        c = host.partition_counts(desc)
        assert c["hip-matmul"][0] == 9 and c["cpu"][0] == 7 and c["reference"][0] == 2, desc
        n2, desc2 = m.partition("hip-matmul")  # no cpu: the reference backend takes the rest
        c2 = host.partition_counts(desc2)
        assert c2["hip-matmul"][0] == 9 and c2["reference"][0] == 9, desc2
        # hip: the whole quantized model (EMBED, RMSNORM, ATTENTION, LAST_ROWS too) in one partition
        n3, desc3 = m.partition("hip,cpu")
        assert n3 == 1 and host.partition_counts(desc3) == {"hip": (18, 1)}, desc3
    # f32 weights: not claimed, and no host backend of this build runs a matmul -> loud failure
    m = host.Model(tiny["f32"])
    with pytest.raises(RuntimeError, match="no backend claims"):
        m.partition("hip,cpu")


@needs_ref
@pytest.mark.parametrize("dtype", ["q8", "q4"])
def test_convert_weights_equals_edgelm(tiny, dtype):
    """Model::convert_weights (load-time quantization of an f32 file, edgelm model.cpp:220-251, main.cpp:53-60)
    byte for byte against edgelm's own on the same file: every weight matrix converted, norm vectors kept f32;
    the converted model then partitions onto the delegate like a quantized file."""
    m = host.Model(tiny["f32"])
    m.convert(dtype, threads=3)
    code = {"q8": 1, "q4": 2}[dtype]
    names = ["model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight", "model.layers.1.mlp.down_proj.weight",
             "model.layers.1.mlp.gate_proj.weight", "model.norm.weight", "model.layers.0.input_layernorm.weight"]
    for name in names:
        dt, data, scales = m.weight(name)
        rdt, rdata, rscales = O.ref_convert_weight(tiny["f32"], code, name)
        assert dt == rdt, name
        assert np.array_equal(data.view(np.uint8).ravel(), rdata), name
        if scales is None:
            assert dt == 0 and rscales.size == 0, name
        else:
            assert np.array_equal(scales.view(np.uint8).ravel(), rscales), name
    n, desc = m.partition("hip,cpu")
    assert n == 1 and host.partition_counts(desc) == {"hip": (18, 1)}, desc
    with pytest.raises(RuntimeError):
        m.convert("f32")  # a quantized model cannot go back


def test_session_without_gpu_fails_loudly(tiny):
    from edgelm_amd import elmh
    if elmh.device_count() > 0:
        pytest.skip("a GPU is present")
    m = host.Model(tiny["q4"])
    with pytest.raises(RuntimeError, match="hip backend unavailable"):
        host.Session(m, "hip,cpu")


def test_lcg_prompt_matches_edgelm_bench():
    # main.cpp:178-184 with vocab 49152 (lo = 1000): first ids recomputed with Python integers
    p = S.lcg_prompt(4, 49152)
    x, want = 12345, []
    for _ in range(4):
        x = (x * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        want.append(1000 + (x >> 33) % (49152 - 1000))
    assert list(p) == want and p.dtype == np.int32
