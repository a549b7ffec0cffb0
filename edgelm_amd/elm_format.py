"""Writer for edgelm's .elm model files and the seeded random-init models this build benchmarks.

The layout is edgelm's (reference tools/elm.py:1-9, 207-276): a 128-byte little-endian header,
tensor records, op records, a tokenizer section and 64-byte aligned weight blobs. The graph is the
unfused Llama graph edgelm exports (elm.py:105-161), so edgelm's own loader and fusion passes accept
the files, and a session of this build and one of edgelm see the same op sequence. Weights are
quantized with edgelm's quantizers (through libedgelm_host, bit-identical to model.cpp:150-190).
"""
import concurrent.futures as cf
import os
import struct

import numpy as np

from . import host

MAGIC = b"ELM1"
ALIGN = 64
DT_F32, DT_Q8, DT_Q4, DT_I32 = 0, 1, 2, 3
KIND_WEIGHT, KIND_ACT, KIND_INPUT, KIND_OUTPUT = 0, 1, 2, 3
ROWS_CONST, ROWS_T, ROWS_L = 0, 1, 2
OPS = dict(EMBED=0, RMSNORM=1, MATMUL=2, ROPE=3, ATTENTION=4, ADD=5, SILU=6, MUL=7, LAST_ROWS=8)

# The model configurations used by the tests and the benchmark.
TINY = dict(vocab=320, dim=64, hidden=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, max_seq=128,
            rope_theta=10000.0, norm_eps=1e-5, bos=0, eos=0, tied=True)
SMOLLM2_135M = dict(vocab=49152, dim=576, hidden=1536, n_layers=30, n_heads=9, n_kv_heads=3, head_dim=64,
                    max_seq=2048, rope_theta=100000.0, norm_eps=1e-5, bos=1, eos=2, tied=True)


class _Graph:
    def __init__(self):
        self.tensors, self.ops = [], []

    def tensor(self, name, kind, dtype, rows_sym, rows, cols, array=None):
        self.tensors.append(dict(name=name, kind=kind, dtype=dtype, rows_sym=rows_sym, rows=rows, cols=cols,
                                 array=array))
        return len(self.tensors) - 1

    def act(self, name, cols, rows_sym=ROWS_T):
        return self.tensor(name, KIND_ACT, DT_F32, rows_sym, 0, cols)

    def op(self, kind, name, ins, outs, iattr=(), fattr=()):
        self.ops.append(dict(type=OPS[kind], name=name, ins=list(ins), outs=list(outs),
                             iattr=list(iattr) + [0] * (4 - len(iattr)), fattr=list(fattr) + [0.0] * (2 - len(fattr))))


def llama_graph(cfg, weights):
    """The unfused Llama graph over T tokens, tensor and op order as edgelm's exporter writes it."""
    g = _Graph()
    D, H, nh, nkv, hd = cfg["dim"], cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    eps, theta = cfg["norm_eps"], cfg["rope_theta"]

    def w(name):
        a = weights[name]
        if a.ndim == 1:
            return g.tensor(name, KIND_WEIGHT, DT_F32, ROWS_CONST, 1, a.shape[0], a)
        return g.tensor(name, KIND_WEIGHT, DT_F32, ROWS_CONST, a.shape[0], a.shape[1], a)

    tokens = g.tensor("tokens", KIND_INPUT, DT_I32, ROWS_T, 0, 1)
    emb = w("model.embed_tokens.weight")
    x = g.act("x.embed", D)
    g.op("EMBED", "embed", [tokens, emb], [x])
    for l in range(cfg["n_layers"]):
        p, L = f"model.layers.{l}.", f"L{l}."
        h = g.act(L + "attn_in", D)
        g.op("RMSNORM", L + "attn_norm", [x, w(p + "input_layernorm.weight")], [h], fattr=[eps])
        q, k, v = g.act(L + "q", nh * hd), g.act(L + "k", nkv * hd), g.act(L + "v", nkv * hd)
        g.op("MATMUL", L + "wq", [h, w(p + "self_attn.q_proj.weight")], [q])
        g.op("MATMUL", L + "wk", [h, w(p + "self_attn.k_proj.weight")], [k])
        g.op("MATMUL", L + "wv", [h, w(p + "self_attn.v_proj.weight")], [v])
        qr, kr = g.act(L + "q_rope", nh * hd), g.act(L + "k_rope", nkv * hd)
        g.op("ROPE", L + "rope_q", [q], [qr], iattr=[nh, hd], fattr=[theta])
        g.op("ROPE", L + "rope_k", [k], [kr], iattr=[nkv, hd], fattr=[theta])
        a = g.act(L + "attn", nh * hd)
        g.op("ATTENTION", L + "attention", [qr, kr, v], [a], iattr=[l, nh, nkv, 0], fattr=[theta])
        o = g.act(L + "attn_out", D)
        g.op("MATMUL", L + "wo", [a, w(p + "self_attn.o_proj.weight")], [o])
        x1 = g.act(L + "x_attn", D)
        g.op("ADD", L + "residual_attn", [x, o], [x1])
        h2 = g.act(L + "ffn_in", D)
        g.op("RMSNORM", L + "ffn_norm", [x1, w(p + "post_attention_layernorm.weight")], [h2], fattr=[eps])
        gt, up = g.act(L + "gate", H), g.act(L + "up", H)
        g.op("MATMUL", L + "w_gate", [h2, w(p + "mlp.gate_proj.weight")], [gt])
        g.op("MATMUL", L + "w_up", [h2, w(p + "mlp.up_proj.weight")], [up])
        gs = g.act(L + "gate_silu", H)
        g.op("SILU", L + "silu", [gt], [gs])
        m = g.act(L + "ffn_mid", H)
        g.op("MUL", L + "gate_mul", [gs, up], [m])
        d = g.act(L + "ffn_out", D)
        g.op("MATMUL", L + "w_down", [m, w(p + "mlp.down_proj.weight")], [d])
        x2 = g.act(L + "x_out", D)
        g.op("ADD", L + "residual_ffn", [x1, d], [x2])
        x = x2
    xl = g.act("x.last", D, ROWS_L)
    g.op("LAST_ROWS", "last_rows", [x], [xl])
    xn = g.act("x.final_norm", D, ROWS_L)
    g.op("RMSNORM", "final_norm", [xl, w("model.norm.weight")], [xn], fattr=[eps])
    head = emb if cfg["tied"] else w("lm_head.weight")
    logits = g.tensor("logits", KIND_OUTPUT, DT_F32, ROWS_L, 0, cfg["vocab"])
    g.op("MATMUL", "lm_head", [xn, head], [logits])
    return g


def _pad(buf):
    buf.extend(b"\0" * ((-len(buf)) % ALIGN))


def write_elm(path, cfg, weights, dtype="q4", embed_dtype=None):
    """Serializes the model; 2-D weights are quantized to `dtype`, the (tied) embedding to
    `embed_dtype` (default: dtype), 1-D norm weights stay f32."""
    g = llama_graph(cfg, weights)
    codes = {"f32": DT_F32, "q8": DT_Q8, "q4": DT_Q4}
    qdt, edt = codes[dtype], codes[embed_dtype or dtype]
    blob = bytearray()
    recs = []
    for t in g.tensors:
        r = dict(t, data_off=0, data_bytes=0, scale_off=0, scale_bytes=0, group=0)
        a = t["array"]
        if t["kind"] == KIND_WEIGHT:
            want = (edt if t["name"] == "model.embed_tokens.weight" else qdt) if a.ndim == 2 else DT_F32
            if want == DT_Q8:
                data, scale = host.quantize_q8(a)
                r["dtype"], r["group"] = DT_Q8, a.shape[1]
            elif want == DT_Q4:
                data, scale = host.quantize_q4(a)
                r["dtype"], r["group"] = DT_Q4, 32
            else:
                data, scale = np.ascontiguousarray(a, dtype=np.float32), None
            _pad(blob)
            r["data_off"], r["data_bytes"] = len(blob), data.nbytes
            blob.extend(np.ascontiguousarray(data).tobytes())
            if scale is not None:
                _pad(blob)
                r["scale_off"], r["scale_bytes"] = len(blob), scale.nbytes
                blob.extend(np.ascontiguousarray(scale, dtype=np.float32).tobytes())
        recs.append(r)
    gb = bytearray()
    for r in recs:
        nm = r["name"].encode()
        gb += struct.pack("<H", len(nm)) + nm
        gb += struct.pack("<BBBBqqQQQQI", r["kind"], r["dtype"], r["rows_sym"], 0, r["rows"], r["cols"],
                          r["data_off"], r["data_bytes"], r["scale_off"], r["scale_bytes"], r["group"])
    for o in g.ops:
        gb += struct.pack("<BBBB", o["type"], len(o["ins"]), len(o["outs"]), 0)
        gb += struct.pack(f"<{len(o['ins'])}i", *o["ins"]) + struct.pack(f"<{len(o['outs'])}i", *o["outs"])
        gb += struct.pack("<4i2f", *o["iattr"], *o["fattr"])
        nm = o["name"].encode()
        gb += struct.pack("<H", len(nm)) + nm
    # tokenizer section: one single-byte token per id, no merges (the benchmarks feed token ids)
    tk = bytearray(struct.pack("<II", cfg["vocab"], 1))
    for i in range(cfg["vocab"]):
        tk += struct.pack("<HBB", 1, i % 256, 0)
    tk += struct.pack("<I", 0)
    graph_off = 128
    tok_off = graph_off + len(gb)
    w_off = tok_off + len(tk)
    w_off += (-w_off) % ALIGN
    hdr = MAGIC + struct.pack("<III", 1, len(g.tensors), len(g.ops))
    hdr += struct.pack("<QQQQQQ", graph_off, len(gb), tok_off, len(tk), w_off, len(blob))
    hdr += struct.pack("<8I", cfg["vocab"], cfg["dim"], cfg["hidden"], cfg["n_layers"], cfg["n_heads"],
                       cfg["n_kv_heads"], cfg["head_dim"], cfg["max_seq"])
    hdr += struct.pack("<ffII", cfg["rope_theta"], cfg["norm_eps"], cfg["bos"], cfg["eos"])
    hdr += struct.pack("<III", qdt, 32 if qdt == DT_Q4 else 0, 1 if cfg["tied"] else 0)
    hdr += b"\0" * (128 - len(hdr))
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(gb)
        f.write(tk)
        f.write(b"\0" * (w_off - tok_off - len(tk)))
        f.write(blob)
    return w_off + len(blob)


def _randn(rng_seed, shape, sd):
    r = np.random.default_rng(rng_seed)
    return (r.standard_normal(shape, dtype=np.float32) * np.float32(sd)).astype(np.float32)


def random_weights(cfg, seed, sd=0.02, embed_sd=None, norm_sd=0.1):
    """Seeded random-init Llama weights (HF naming): linears N(0, sd), embedding N(0, embed_sd or sd),
    norms 1 + N(0, norm_sd). Each tensor has its own generator (seed, index), filled in parallel."""
    D, H, V = cfg["dim"], cfg["hidden"], cfg["vocab"]
    qd, kd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    spec = [("model.embed_tokens.weight", (V, D), embed_sd or sd, 0.0)]
    spec.append(("model.norm.weight", (D,), norm_sd, 1.0))
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}."
        spec += [(p + "input_layernorm.weight", (D,), norm_sd, 1.0),
                 (p + "post_attention_layernorm.weight", (D,), norm_sd, 1.0),
                 (p + "self_attn.q_proj.weight", (qd, D), sd, 0.0), (p + "self_attn.k_proj.weight", (kd, D), sd, 0.0),
                 (p + "self_attn.v_proj.weight", (kd, D), sd, 0.0), (p + "self_attn.o_proj.weight", (D, qd), sd, 0.0),
                 (p + "mlp.gate_proj.weight", (H, D), sd, 0.0), (p + "mlp.up_proj.weight", (H, D), sd, 0.0),
                 (p + "mlp.down_proj.weight", (D, H), sd, 0.0)]

    def make(i):
        name, shape, s, base = spec[i]
        a = _randn((seed, i), shape, s)
        return name, (a + np.float32(base)).astype(np.float32) if base else a

    with cf.ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as ex:
        return dict(ex.map(make, range(len(spec))))


def lcg_prompt(n, vocab, seed=12345):
    """edgelm's bench prompt (main.cpp:178-184): x = x*6364136223846793005 + 1442695040888963407,
    id = lo + (x >> 33) % (vocab - lo), lo = 1000 when vocab > 2000."""
    x = seed
    lo = 1000 if vocab > 2000 else 0
    out = []
    for _ in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        out.append(lo + (x >> 33) % (vocab - lo))
    return np.asarray(out, dtype=np.int32)
