"""CPU: the C-ABI libraries load and export every symbol their headers declare; calls that need a
device fail cleanly (with a status code and message, no crash) on a host without one."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(elm[a-z]*_[a-z0-9_]+)\s*\(", text)))


def test_elmh_exports_every_declared_symbol():
    from edgelm_amd import elmh
    lib = elmh.lib()
    names = declared("elmh.h")
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_elmh_fails_cleanly_without_device():
    from edgelm_amd import elmh
    if elmh.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(elmh.ElmhError) as e:
        elmh.Context(0)
    assert e.value.code == elmh.ERR_NODEV
    # null-context calls report an argument error instead of crashing
    lib = elmh.lib()
    assert lib.elmh_synchronize(None) == elmh.ERR_ARG
    assert lib.elmh_matmul(None, None, 1, 32, 0, None, None, None, 1, 0) == elmh.ERR_ARG
    assert b"null" in lib.elmh_last_error(None)


@pytest.mark.skipif(not os.path.isdir("/root/reference/include/edgelm"), reason="edgelm's headers are not on this host")
def test_hip_backend_compiles_against_edgelm_headers():
    """The delegate's Backend (edgelm_amd/host/src/hip_backend.cpp) is the file a maintainer drops
    into edgelm's src/: it must compile against edgelm's own headers, not only against the
    restated ones the host runtime here uses."""
    import shutil
    import subprocess
    cxx = shutil.which("g++") or "g++"
    src = os.path.join(ROOT, "edgelm_amd", "host", "src", "hip_backend.cpp")
    p = subprocess.run([cxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                        "-I/root/reference/include", f"-I{INCLUDE}", src], capture_output=True, text=True)
    assert p.returncode == 0, p.stderr


def test_attention_step_support_is_a_pure_query():
    """elmh_attention_step_supported needs no device: every cache length runs (score rows past LDS live in a
    device buffer); only head sizes the kernels do not take and empty caches are refused."""
    from edgelm_amd import elmh as E
    f = E.lib().elmh_attention_step_supported
    assert f(64, 2048) == 1 and f(64, 16384) == 1 and f(64, 20000) == 1 and f(64, 40000) == 1 and f(64, 1 << 20) == 1
    assert f(62, 128) == 0 and f(64, 0) == 0 and f(260, 128) == 0
