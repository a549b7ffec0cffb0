"""In-tree build of the native libraries (no JIT cache, no pip install).

* ``edgelm_amd/lib/libelmh.so`` — the HIP kernels for gfx950 plus the C ABI of ``include/elmh.h``.
* ``edgelm_amd/lib/libedgelm_host.so`` — the C++17 host runtime (edgelm's Backend / partitioner / Session
  interfaces, implemented here, with the ``hip`` backend that calls libelmh), linked against libelmh.

Run ``python -m edgelm_amd.build`` (or ``__graft_entry__.build()``). Always recompiles.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "edgelm_amd")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
HOST_INC = os.path.join(HOST, "include")
LIB = os.path.join(PKG, "lib")
OBJ = os.path.join(PKG, "_build")
INC = os.path.join(ROOT, "include")

ARCH = "gfx950"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Device code: IEEE divide, no FP contraction (fused multiply-adds are written explicitly),
# and no packed-FP32 instructions (they are switched off for gfx950 here on purpose).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INC}", f"-I{CSRC}",
]
# Host code: the reference's default build (-O2/-O3, no -march) keeps the x86-64 baseline ISA (SSE2, no
# FMA), so host float arithmetic rounds like edgelm's scalar path; contraction stays off regardless.
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra", "-pthread", f"-I{INC}",
              f"-I{HOST_INC}"]

ELMH_SRCS = ["elmh_kernels.hip", "elmh_layer.hip", "elmh_api.cpp"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the device-only feature flag; keep other diagnostics
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _compile_hip(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_elmh():
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(ELMH_SRCS)) as ex:
        objs = list(ex.map(_compile_hip, ELMH_SRCS))
    out = os.path.join(LIB, "libelmh.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def host_sources():
    src = os.path.join(HOST, "src")
    if not os.path.isdir(src):
        return []
    return sorted(os.path.join(src, f) for f in os.listdir(src) if f.endswith(".cpp"))


def build_host():
    srcs = host_sources()
    if not srcs:
        return None
    os.makedirs(OBJ, exist_ok=True)
    cxx = shutil.which("g++") or "g++"
    rocm = "/opt/rocm"

    def one(s):
        obj = os.path.join(OBJ, "host_" + os.path.basename(s) + ".o")
        _run([cxx, *HOST_FLAGS, "-c", s, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(one, srcs))
    out = os.path.join(LIB, "libedgelm_host.so")
    tmp = out + ".tmp"
    _run([cxx, "-shared", "-fPIC", "-pthread", "-o", tmp, *objs, f"-L{LIB}", "-lelmh",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{rocm}/lib"])
    os.replace(tmp, out)
    return out


def build():
    libs = [build_elmh()]
    h = build_host()
    if h:
        libs.append(h)
    return libs


if __name__ == "__main__":
    for lib in build():
        print("built", os.path.relpath(lib, ROOT))
