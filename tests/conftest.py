import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library through its C ABI")


@pytest.fixture(scope="session")
def ctx():
    """The elmh context on device 0. Fails loudly (no skip) when the HIP library or GPU is missing."""
    from edgelm_amd import elmh
    print(f"[gpu] creating elmh context on device 0", flush=True)
    c = elmh.Context(0)
    assert c.arch.startswith("gfx950"), c.arch
    yield c
    c.close()


def rel_err(a, b):
    """max |a - b| / max(1, max |b|) — edgelm's tolerance metric (tests/common.hpp:68-76)."""
    import numpy as np
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)) / max(1.0, float(np.max(np.abs(b)))))


def bits_equal(a, b):
    import numpy as np
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.int32), b.view(np.int32)))
