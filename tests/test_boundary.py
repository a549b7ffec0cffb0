"""CPU: the drop-in boundary inside edgelm itself. oracle/_ref/libedgelm_ref_hip.so is edgelm's own runtime
compiled from the reference sources with the `hip` delegate registered in make_backend at link time (the
INTEGRATION.md patch, reference src/backends.cpp:158-163); edgelm's partition_graph (backends.cpp:165-182)
then places the delegate in the preference list beside its own cpu / matmul-only / reference backends.

Checked here without a GPU: which ops edgelm's partitioner gives the delegate (its claims, planned without a
device), that they agree with this build's runtime, and that an edgelm Session asked for "hip" on a host
without a usable gfx950 fails loudly instead of computing the matmuls on the CPU. The same sessions run on
the GPU in tests/test_gpu_boundary.py."""
import numpy as np
import pytest

import oracle as O
from edgelm_amd import synth as S
from edgelm_amd import host

needs_ref_hip = pytest.mark.skipif(not O.ref_hip_available(), reason="oracle/_ref not built (no /root/reference here)")


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny_boundary")
    TINY_SEED = 4321
    paths = {}
    for dt in ("q8", "q4"):
        p = str(d / f"tiny.{dt}.elm")
        S.write_model(p, S.TINY, dt, seed=TINY_SEED, sd=0.15, embed_sd=0.5)
        paths[dt] = p
    return paths


counts = O.partition_counts  # edgelm's describe_partitions format


@needs_ref_hip
@pytest.mark.parametrize("fuse", [True, False])
def test_edgelm_partitioner_places_the_delegate(tiny, fuse):
    # fused graph, per layer: RMSNORM, MATMUL_N, ATTENTION, MATMUL_ADD, RMSNORM, FFN_SWIGLU, MATMUL_ADD;
    # then EMBED first and LAST_ROWS, RMSNORM, MATMUL (lm head) last: 1 + 2 * 7 + 3 = 18 ops
    n, d = O.ref_hip_partition(tiny["q4"], "hip,cpu", fuse)
    c = counts(d)
    if fuse:
        assert n == 1 and c == {"hip": (18, 1)}, d
    else:  # ROPE (2 per layer), ADD (2), SILU, MUL stay on the cpu backend: 6 per layer
        assert c["cpu"][0] == 2 * 6 and c["hip"][0] == 1 + 2 * 10 + 3, d
    n, d = O.ref_hip_partition(tiny["q4"], "hip-matmul,cpu", fuse)
    c = counts(d)
    mm = (2 * 4 + 1) if fuse else (2 * 7 + 1)  # matmul-family ops per layer (fused: 4) and the lm head
    assert c["hip-matmul"][0] == mm, d
    assert c["reference"][0] == 2, d  # EMBED and LAST_ROWS: edgelm's cpu backend leaves them to reference


@needs_ref_hip
def test_edgelm_partitioner_with_matmul_only(tiny):
    """The delegate beside edgelm's own matmul-only backend (backends.cpp:137-150: MATMUL / MATMUL_N /
    MATMUL_ADD with f32 or q8 weights), in both orders: the first backend in the list that claims an op
    gets it."""
    _, d = O.ref_hip_partition(tiny["q8"], "matmul-only,hip,cpu")
    c = counts(d)
    assert c["matmul-only"][0] == 2 * 3 + 1, d  # MATMUL_N, two MATMUL_ADD per layer, the lm head
    assert c["hip"][0] == 18 - 7, d             # the rest, FFN_SWIGLU included
    _, d = O.ref_hip_partition(tiny["q4"], "matmul-only,hip,cpu")
    assert "matmul-only" not in counts(d), d    # q4 weights: matmul-only claims nothing
    _, d = O.ref_hip_partition(tiny["q8"], "hip,matmul-only,cpu")
    assert counts(d) == {"hip": (18, 1)}, d


@needs_ref_hip
@pytest.mark.parametrize("backends", ["hip,cpu", "hip-matmul,cpu"])
def test_edgelm_and_this_runtime_partition_alike(tiny, backends):
    for dt in ("q8", "q4"):
        for fuse in (True, False):
            n_ref, d_ref = O.ref_hip_partition(tiny[dt], backends, fuse)
            m = host.Model(tiny[dt])
            n_mine, d_mine = m.partition(backends, fuse)
            assert n_ref == n_mine and counts(d_ref) == host.partition_counts(d_mine), (d_ref, d_mine)


@needs_ref_hip
def test_edgelm_session_with_hip_fails_loudly_without_a_gpu(tiny):
    from edgelm_amd import elmh
    if elmh.device_count() > 0:
        pytest.skip("a GPU is present: tests/test_gpu_boundary.py runs these sessions")
    with pytest.raises(RuntimeError) as e:
        O.RefSession(tiny["q4"], "hip,cpu", with_hip=True)
    assert "hip backend unavailable" in str(e.value)
