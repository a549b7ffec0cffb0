"""Seeded random-init models for the tests and the benchmark (no checkpoints exist offline).

``write_model`` asks the host library (``elm_write_random_model``, include/edgelm_host.h) to write an
.elm file: the unfused Llama graph edgelm's exporter emits, random weights quantized with edgelm's
quantizers. ``lcg_prompt`` is the prompt of edgelm's bench protocol.
"""
import ctypes as C

from . import host

# The two model shapes the tests and the benchmark use.
TINY = dict(vocab=320, dim=64, hidden=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, max_seq=128,
            rope_theta=10000.0, norm_eps=1e-5, bos=0, eos=0, tied=True)
SMOLLM2_135M = dict(vocab=49152, dim=576, hidden=1536, n_layers=30, n_heads=9, n_kv_heads=3, head_dim=64,
                    max_seq=2048, rope_theta=100000.0, norm_eps=1e-5, bos=1, eos=2, tied=True)

DTYPES = {"f32": 0, "q8": 1, "q4": 2}


class _Spec(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                         "max_seq")] + \
               [("rope_theta", C.c_float), ("norm_eps", C.c_float), ("bos", C.c_int32), ("eos", C.c_int32),
                ("tied", C.c_int32), ("weight_dtype", C.c_int32), ("embed_dtype", C.c_int32), ("seed", C.c_uint64),
                ("sd", C.c_float), ("embed_sd", C.c_float), ("norm_sd", C.c_float), ("threads", C.c_int32)]


def write_model(path, cfg, dtype="q4", embed_dtype=None, seed=20260101, sd=0.02, embed_sd=None, norm_sd=0.1,
                threads=0):
    """Writes a random-init model of shape ``cfg``: weight matrices N(0, sd) as ``dtype``, the embedding
    N(0, embed_sd or sd) as ``embed_dtype`` (default: dtype), norm vectors 1 + N(0, norm_sd) in f32."""
    s = _Spec(**{k: cfg[k] for k in ("vocab", "dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                      "max_seq", "rope_theta", "norm_eps", "bos", "eos")})
    s.tied = int(cfg["tied"])
    s.weight_dtype = DTYPES[dtype]
    s.embed_dtype = DTYPES[embed_dtype] if embed_dtype else -1
    s.seed, s.sd, s.norm_sd = seed, sd, norm_sd
    s.embed_sd = embed_sd if embed_sd is not None else sd
    s.threads = host._threads(threads)
    L = host.lib()
    L.elm_write_random_model.argtypes = [C.c_char_p, C.POINTER(_Spec)]
    L.elm_last_error.restype = C.c_char_p
    if L.elm_write_random_model(path.encode(), C.byref(s)) != 0:
        raise RuntimeError(L.elm_last_error().decode())
    return path


def lcg_prompt(n, vocab, seed=12345):
    """The prompt of edgelm's bench protocol (main.cpp:178-184): x = x * 6364136223846793005 +
    1442695040888963407 (mod 2^64), id = lo + (x >> 33) % (vocab - lo), lo = 1000 when vocab > 2000."""
    import numpy as np
    lo = 1000 if vocab > 2000 else 0
    x, ids = seed, np.empty(n, np.int32)
    for i in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        ids[i] = lo + (x >> 33) % (vocab - lo)
    return ids
