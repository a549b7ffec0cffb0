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
