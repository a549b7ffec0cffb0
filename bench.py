#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul delegate (one GPU).

Headline workload: a random-init SmolLM2-135M-shaped model (30 layers, q4 group-32
weights with a q8 embedding, int8 activations) through this build's Session with the `hip` delegate running
the whole model on the GPU; edgelm's bench protocol: a 128-token LCG prompt, then greedy decode. A "step" is
one decode token; value = decode tok/s over exactly --steps timed steps after --warmup untimed ones.

Also reported (extra keys): TTFT and cold TTFT, the matmul-only flavour, per-kernel event timings and the HBM
roofline of the step's dominant kernel, the decode matmul chain alone, the 8B-shaped W4A8 decode
sweep (configs[4]: 8 Llama-3-8B layers round-robin, > 256 MB Infinity Cache), the int8 GEMMs at T=128 / 512
(configs[2], configs[4]), and the CPU baseline: edgelm's own Session (compiled from the reference sources into
oracle/_ref) on this host's cores, same model file and protocol.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, published
METRIC = "decode tok/s + W4A8 GEMV achieved HBM GB/s; prefill tok/s at T=128"

D, HID, L, VOCAB, KV = 576, 1536, 30, 49152, 192


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def q_bytes(dt, n, k):
    return n * k // 2 + n * (k // 32) * 4 if dt == 2 else n * k + n * 4


def randn(seed, n, k, sd=0.02, threads=None):
    """N(0, sd) float32 [n, k] from numpy generators spawned off one seed, filled by threads."""
    import concurrent.futures as cf
    threads = threads or min(16, os.cpu_count() or 1)
    out = np.empty((n, k), np.float32)
    seqs = np.random.SeedSequence(seed).spawn(threads)
    rows = (n + threads - 1) // threads

    def fill(i):
        a, b = i * rows, min(n, (i + 1) * rows)
        if a < b:
            np.random.default_rng(seqs[i]).standard_normal((b - a, k), dtype=np.float32, out=out[a:b])
            out[a:b] *= np.float32(sd)

    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(fill, range(threads)))
    return out


class Model:
    """Random-init weights, quantized with edgelm's quantizers, uploaded to HBM."""

    def __init__(self, ctx, seed, shapes, dtype):
        from edgelm_amd import host
        self.ctx = ctx
        self.w = {}
        for i, (name, (n, k)) in enumerate(shapes.items()):
            f = randn(seed * 1000 + i, n, k)
            dt = dtype(name)
            q, s = host.quantize_q4(f) if dt == 2 else host.quantize_q8(f)
            self.w[name] = ctx.upload(dt, n, k, q, s)
            del f, q, s

    def free(self):
        for w in self.w.values():
            w.free()


def smollm_shapes():
    sh = {}
    for l in range(L):
        sh.update({f"{l}.q": (D, D), f"{l}.k": (KV, D), f"{l}.v": (KV, D), f"{l}.o": (D, D), f"{l}.g": (HID, D),
                   f"{l}.u": (HID, D), f"{l}.d": (D, HID)})
    sh["head"] = (VOCAB, D)
    return sh


def time_graph(ctx, fn, reps, warm=2, inner=1):
    """Captures fn() `inner` times into one HIP graph, replays it `reps` times between two events on
    the library's stream; ms per fn(). A replay must carry far more GPU work than the ~0.1 ms of host
    time one graph launch costs, or the events time the host; `inner` repeats short ops for that."""
    fn()  # eager once: allocates scratch outside capture
    ctx.synchronize()
    ctx.graph_begin()
    for _ in range(inner):
        fn()
    g = ctx.graph_end()
    for _ in range(warm):
        ctx.graph_launch(g)
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps):
        ctx.graph_launch(g)
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1) / (reps * inner)
    ctx.destroy_event(e0)
    ctx.destroy_event(e1)
    ctx.graph_destroy(g)
    return ms


def time_eager(ctx, fn, reps, warm=2, inner=1):
    """time_graph's measurement with plain launches (no graph): events around reps * inner calls.
    Host-bound for short kernels; used only to run the bench under a kernel tracer."""
    for _ in range(warm):
        fn()
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps * inner):
        fn()
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1) / (reps * inner)
    ctx.destroy_event(e0)
    ctx.destroy_event(e1)
    return ms


def decode_step_bench(ctx, E, steps, warmup, eager=False):
    log("building SmolLM2-135M-shaped W4A8 weights")
    t0 = time.time()
    m = Model(ctx, 1234, smollm_shapes(), lambda n: 1 if n == "head" else 2)
    log(f"weights ready in {time.time() - t0:.1f}s")
    W = m.w
    f4 = 4
    bufs = {}

    def buf(name, n):
        bufs[name] = ctx.buffer(n * f4)
        return bufs[name].ptr

    r = np.random.default_rng(7)
    x = [buf(f"x{l}", D) for l in range(L + 1)]
    bufs["x0"].upload(r.standard_normal(D, dtype=np.float32))
    q = [buf(f"q{l}", D) for l in range(L)]
    kk = [buf(f"k{l}", KV) for l in range(L)]
    vv = [buf(f"v{l}", KV) for l in range(L)]
    x1 = [buf(f"x1{l}", D) for l in range(L)]
    h = [buf(f"h{l}", HID) for l in range(L)]
    logits = buf("logits", VOCAB)
    ctx.reserve(4, HID)

    def qkv(l):
        ctx.matmul_dev(x[l], 1, D, [W[f"{l}.q"], W[f"{l}.k"], W[f"{l}.v"]], [q[l], kk[l], vv[l]], act=E.ACT_INT8)

    def oproj(l):  # q stands in for the attention output (same shape)
        ctx.matmul_dev(q[l], 1, D, [W[f"{l}.o"]], [x1[l]], [x[l]], act=E.ACT_INT8)

    def ffn(l):
        ctx.swiglu_dev(x1[l], 1, D, W[f"{l}.g"], W[f"{l}.u"], h[l], act=E.ACT_INT8)

    def down(l):
        ctx.matmul_dev(h[l], 1, HID, [W[f"{l}.d"]], [x[l + 1]], [x1[l]], act=E.ACT_INT8)

    def head():
        ctx.matmul_dev(x[L], 1, D, [W["head"]], [logits], act=E.ACT_INT8)

    def step():
        for l in range(L):
            qkv(l)
            oproj(l)
            ffn(l)
            down(l)
        head()

    # whole decode step as one graph: warmup, then exactly `steps` timed replays (eager mode:
    # plain launches, host-bound, for kernel tracing)
    step()
    ctx.synchronize()
    if not eager:
        ctx.graph_begin()
        step()
        g = ctx.graph_end()
    run = (lambda: ctx.graph_launch(g)) if not eager else step
    for _ in range(warmup):
        run()
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.synchronize()
    ctx.record(e0)
    for _ in range(steps):
        run()
    ctx.record(e1)
    ms_step = ctx.elapsed_ms(e0, e1) / steps
    if not eager:
        ctx.graph_destroy(g)
    log(f"decode step {ms_step * 1e3:.1f} us -> {1e3 / ms_step:.1f} tok/s" + (" (eager launches)" if eager else ""))

    # per-op kernel time: a graph holding 16 x (the op for all 30 layers, distinct weights),
    # replayed; time per call (one kernel per call: the GEMV kernels quantize x themselves)
    timer = time_eager if eager else time_graph
    per = {}
    ops = {
        "MATMUL_N qkv": (qkv, q_bytes(2, D + 2 * KV, D) + D * 4 + (D + 2 * KV) * 4, 2 * (D + 2 * KV) * D),
        "MATMUL_ADD o": (oproj, q_bytes(2, D, D) + D * 4 + 2 * D * 4, 2 * D * D),
        "FFN_SWIGLU": (ffn, 2 * q_bytes(2, HID, D) + D * 4 + HID * 4, 4 * HID * D),
        "MATMUL_ADD down": (down, q_bytes(2, D, HID) + HID * 4 + 2 * D * 4, 2 * D * HID),
    }
    for name, (fn, nbytes, ops_) in ops.items():
        ms = timer(ctx, lambda: [fn(l) for l in range(L)], 10, inner=16) / L
        per[name] = {"us": ms * 1e3, "bytes": nbytes, "GBs": nbytes / (ms * 1e-3) / 1e9, "calls_per_step": L,
                     "kernels_per_call": 1}
    hb = q_bytes(1, VOCAB, D) + D * 4 + VOCAB * 4
    ms = timer(ctx, lambda: [head() for _ in range(8)], 10, inner=16) / 8
    per["MATMUL lm_head q8"] = {"us": ms * 1e3, "bytes": hb, "GBs": hb / (ms * 1e-3) / 1e9, "calls_per_step": 1,
                                "kernels_per_call": 1}
    for k, v in per.items():
        log(f"  {k:20s} {v['us']:8.2f} us  {v['GBs']:8.1f} GB/s")
    for b in bufs.values():
        b.free()
    m.free()
    return ms_step, per


def b8_shapes(layers=8):
    sh = {}
    for l in range(layers):
        sh.update({f"{l}.q": (4096, 4096), f"{l}.k": (1024, 4096), f"{l}.v": (1024, 4096), f"{l}.g": (14336, 4096),
                   f"{l}.u": (14336, 4096), f"{l}.d": (4096, 14336)})
    return sh


def sweep_8b(ctx, E, reps=10, eager=False):
    """8 distinct Llama-3-8B layers, W4A8 decode GEMVs round-robin (1.007 GB per sweep)."""
    log("building 8B-shaped W4A8 weights (8 layers, ~1 GB)")
    t0 = time.time()
    m = Model(ctx, 99, b8_shapes(), lambda n: 2)
    log(f"weights ready in {time.time() - t0:.1f}s")
    W = m.w
    bx = ctx.buffer(14336 * 4)
    bx.upload(np.random.default_rng(5).standard_normal(14336, dtype=np.float32))
    by = [ctx.buffer(14336 * 4) for _ in range(3)]
    ctx.reserve(4, 14336)
    total = sum(q_bytes(2, w.rows, w.cols) for w in W.values())

    # the FFN pair as the hip backend runs it (elmh_ffn_dev): FFN_SWIGLU into h, whose launch also
    # quantizes h (edgelm quantizes the down projection's input once, cpu::matmul's quantize_act_row),
    # then the down GEMV on the quantized h
    hq, hd, hs = ctx.buffer(14336), ctx.buffer(448 * 4), ctx.buffer(448 * 4)

    def sweep():
        for l in range(8):
            ctx.matmul_dev(bx.ptr, 1, 4096, [W[f"{l}.q"], W[f"{l}.k"], W[f"{l}.v"]],
                           [by[0].ptr, by[1].ptr, by[2].ptr], act=E.ACT_INT8)
            ctx.ffn_dev(bx.ptr, 1, 4096, W[f"{l}.g"], W[f"{l}.u"], by[0].ptr, W[f"{l}.d"], by[1].ptr)

    ms = (time_eager if eager else time_graph)(ctx, sweep, reps)
    gbs = total / (ms * 1e-3) / 1e9
    log(f"8B sweep {ms * 1e3:.1f} us for {total / 1e9:.3f} GB -> {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of peak)")
    # each op type alone over the 8 layers (includes the activation quantization: inside the GEMV
    # for K = 4096; for the down GEMV's K = 14336 either in the SwiGLU launch before it, as the sweep
    # runs it, or, for MATMUL down on an f32 activation, a separate launch before it)
    per_op = {}
    ops8 = {
        "MATMUL_N qkv 6144x4096": (lambda l: ctx.matmul_dev(bx.ptr, 1, 4096, [W[f"{l}.q"], W[f"{l}.k"], W[f"{l}.v"]],
                                                            [by[0].ptr, by[1].ptr, by[2].ptr], act=E.ACT_INT8),
                                   sum(q_bytes(2, W[f"0.{n}"].rows, 4096) for n in "qkv")),
        "FFN_SWIGLU 2x14336x4096": (lambda l: ctx.swiglu_dev(bx.ptr, 1, 4096, W[f"{l}.g"], W[f"{l}.u"], by[0].ptr,
                                                             act=E.ACT_INT8), 2 * q_bytes(2, 14336, 4096)),
        "FFN_SWIGLU 2x14336x4096 + quantized h": (
            lambda l: ctx.swiglu_quant_dev(bx.ptr, 1, 4096, W[f"{l}.g"], W[f"{l}.u"], by[0].ptr, hq.ptr, hd.ptr,
                                           hs.ptr), 2 * q_bytes(2, 14336, 4096)),
        "MATMUL down 4096x14336": (lambda l: ctx.matmul_dev(bx.ptr, 1, 14336, [W[f"{l}.d"]], [by[1].ptr], act=E.ACT_INT8),
                                   q_bytes(2, 4096, 14336)),
    }
    timer = time_eager if eager else time_graph
    for name, (fn, nbytes) in ops8.items():
        ums = timer(ctx, lambda: [fn(l) for l in range(8)], reps, inner=8) / 8
        per_op[name] = {"us": ums * 1e3, "weight_bytes": nbytes, "GBs": nbytes / (ums * 1e-3) / 1e9,
                        "kernels_per_call": 2 if name.startswith("MATMUL down") else 1}
        log(f"  8B {name:26s} {ums * 1e3:8.2f} us  {per_op[name]['GBs']:7.0f} GB/s (weights+scales / time, incl. act quant)")

    # the down GEMV alone, pre-quantized activation (pure kernel time), all 8 layers
    q = ctx.buffer(14336)
    d = ctx.buffer(448 * 4)
    s = ctx.buffer(448 * 4)
    ctx.quantize_act_dev(bx.ptr, 1, 14336, q.ptr, d.ptr, s.ptr)
    dms = timer(ctx, lambda: [ctx.gemv_a8_dev(q.ptr, d.ptr, s.ptr, 1, 14336, [W[f"{l}.d"]], [by[1].ptr])
                              for l in range(8)], reps, inner=8) / 8
    dbytes = q_bytes(2, 4096, 14336) + 14336 + 448 * 8 + 4096 * 4
    dgbs = dbytes / (dms * 1e-3) / 1e9
    log(f"8B down GEMV {dms * 1e3:.2f} us -> {dgbs:.0f} GB/s")
    for b in [bx, q, d, s, hq, hd, hs] + by:
        b.free()
    m.free()
    return {"sweep_us": ms * 1e3, "bytes": total, "GBs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "per_op": per_op,
            "down_gemv_us": dms * 1e3, "down_gemv_bytes": dbytes, "down_gemv_GBs": dgbs}


def gemm_bench(ctx, E, T, shapes, dt=1, act=None, reps=10, eager=False):
    """Prefill int8 GEMMs at T tokens: int ops / time."""
    act = E.ACT_INT8 if act is None else act
    sh = {f"{i}": s for i, s in enumerate(shapes)}
    m = Model(ctx, 5 + T, sh, lambda n: dt)
    W = m.w
    kmax = max(k for _, k in shapes)
    nmax = max(n for n, _ in shapes)
    bx = ctx.buffer(T * kmax * 4)
    bx.upload(np.random.default_rng(3).standard_normal(T * kmax, dtype=np.float32))
    by = ctx.buffer(T * nmax * 4)
    ctx.reserve(T, kmax)
    out = {}
    for i, (n, k) in enumerate(shapes):
        ms = (time_eager if eager else time_graph)(ctx, lambda: ctx.matmul_dev(bx.ptr, T, k, [W[f"{i}"]], [by.ptr],
                                                                               act=act), reps, inner=16)
        ops = 2.0 * T * n * k
        out[f"{n}x{k}"] = {"us": ms * 1e3, "TOPs": ops / (ms * 1e-3) / 1e12,
                           "frac_int8_peak": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS}
    bx.free()
    by.free()
    m.free()
    return out


class HostWeight:
    """One weight quantized on the host with edgelm's quantizers (the product's host.quantize_*), kept in the
    export layout so the same bytes feed the GPU upload and edgelm's cpu backend."""

    def __init__(self, seed, n, k, dtype):
        from edgelm_amd import host
        f = randn(seed, n, k)
        self.dtype, self.rows, self.cols = dtype, n, k
        self.data, self.scales = host.quantize_q4(f) if dtype == 2 else host.quantize_q8(f)

    def rows_sample(self, m):
        """The first m rows (the CPU baseline's bounded sample: edgelm's work per row is the same for every row)."""
        h = HostWeight.__new__(HostWeight)
        h.dtype, h.rows, h.cols = self.dtype, m, self.cols
        h.data = np.ascontiguousarray(self.data[:m])
        h.scales = np.ascontiguousarray(self.scales[:m])
        return h


def measured_ceilings(ctx, E, reps=10):
    """Read and copy bandwidth this GPU reaches, for the roofline next to the nominal 8 TB/s: elmh_read_sweep_dev
    over 4 GiB (far past the 256 MB Infinity Cache: HBM) and over 128 MiB read again and again (past the 8 x 4 MB
    of L2, inside the Infinity Cache), and a 2 GiB device-to-device copy (read + write bytes)."""
    sinkn = E.Context.read_sweep_sink_bytes()
    sink = ctx.buffer(sinkn)
    out = {}
    for name, n, inner in (("hbm_read_GBs", 4 << 30, 1), ("infinity_cache_read_GBs", 128 << 20, 16)):
        b = ctx.buffer(n)
        ctx.memset_dev(b.ptr, 1, n)
        ms = time_graph(ctx, lambda: ctx.read_sweep_dev(b.ptr, n, sink.ptr), reps, inner=inner)
        out[name] = n / (ms * 1e-3) / 1e9
        out[name.replace("_GBs", "_bytes")] = n
        b.free()
    n = 2 << 30
    src, dst = ctx.buffer(n), ctx.buffer(n)
    ctx.memset_dev(src.ptr, 1, n)
    ms = time_eager(ctx, lambda: ctx.memcpy_d2d(dst.ptr, src.ptr, n), reps)
    out["hbm_copy_GBs"] = 2 * n / (ms * 1e-3) / 1e9
    out["hbm_copy_bytes"] = n
    for b in (src, dst, sink):
        b.free()
    log("measured ceilings: HBM read {hbm_read_GBs:.0f} GB/s, Infinity Cache read {infinity_cache_read_GBs:.0f} GB/s, "
        "HBM copy {hbm_copy_GBs:.0f} GB/s (read + write)".format(**out))
    return out


def rescale_ceiling(ctx, E, iters=20000, cus=256):
    """The per-32-block exact rescale's ceiling (SURVEY's per-block epilogue question), measured without memory
    traffic by elmh_rescale_ceiling_dev: int8 MFMA blocks alone, then with the q8 and the q4 rescale of every
    block's 32 x 32 int32 sums, at 1, 2 and 4 four-wave workgroups per CU (1, 2, 4 waves per SIMD); int ops /
    time as a fraction of the int8 peak."""
    out = {}
    for wpc in (1, 2, 4):
        blocks = cus * wpc
        sink = ctx.buffer(blocks * 1024)
        for mode, name in ((0, "mfma_only"), (1, "q8_exact_rescale"), (2, "q4_exact_rescale")):
            ms = time_eager(ctx, lambda: ctx.rescale_ceiling_dev(mode, blocks, iters, sink.ptr, sink.nbytes), 5)
            tops = blocks * 4 * iters * 2 * 65536 / (ms * 1e-3) / 1e12
            out.setdefault(name, {})[f"{wpc}_workgroups_per_cu"] = {"TOPs": tops, "frac_int8_peak": tops / INT8_PEAK_TOPS}
        sink.free()
    log("rescale ceiling (fraction of int8 peak, 1 / 2 / 4 workgroups per CU): " + "; ".join(
        f"{k} " + " / ".join("%.3f" % v["frac_int8_peak"] for v in d.values()) for k, d in out.items()))
    return out


def cpu_op_baseline(op, T, threads_list=(1, 4, 16), macs_per_thread=30e6, budget_s=0.3):
    """CPU-baseline leg for one op: edgelm's own cpu::matmul / cpu::swiglu (oracle/_ref, compiled from the
    reference sources; its ThreadPool, x86 scalar path) on the op's host weights and a seeded x, timed in C.
    A call is bounded to about macs_per_thread multiply-adds per thread: bigger ops run on the first rows of
    each weight (edgelm's cost per row is the same for every row) and their time is scaled to the whole op;
    `sample` says which."""
    import oracle as O
    if not O.ref_available():
        return None
    ws, kind = op["weights"], op["kind"]
    K = ws[0].cols
    full = sum(w.rows for w in (ws[:1] if kind == "swiglu" else ws)) * (2 if kind == "swiglu" else 1) * T * K
    x = np.random.default_rng(3).standard_normal((T, K), dtype=np.float32)
    out = {}
    for th in threads_list:
        # at least two of edgelm's 16-row blocks per thread, so the sample keeps every thread busy
        f = min(1.0, macs_per_thread * th / full)
        sw = [w if f >= 1.0 else w.rows_sample(min(w.rows, max(32 * th, int(round(w.rows * f / 16)) * 16))) for w in ws]
        done = sum(w.rows for w in (sw[:1] if kind == "swiglu" else sw)) * (2 if kind == "swiglu" else 1) * T * K
        res = None
        if op.get("residual"):
            res = [np.random.default_rng(4).standard_normal((T, w.rows), dtype=np.float32) for w in sw]
        med, reps = O.rq_time_cpu_op(th, x, sw, res, act_quant=op["act"] != "f32", swiglu=kind == "swiglu",
                                     budget_s=budget_s)
        us = med * 1e3 * full / done
        out[str(th)] = {"us": us, "reps": reps,
                        "sample": "whole op" if done == full else f"first {sw[0].rows} of {ws[0].rows} rows "
                                                                  f"per weight, time scaled by {full / done:.2f}"}
    return out


def pair_rates(entry, nbytes=None, ops=None, ceil=None):
    """Adds GB/s (nbytes) or TOP/s (ops) and roofline fractions to a {gpu_us, cpu: {threads: {us}}} entry."""
    def rate(us):
        return (nbytes / (us * 1e-6) / 1e9) if nbytes else (ops / (us * 1e-6) / 1e12)
    g = entry["gpu_us"]
    if nbytes:
        entry.update(unit="GB/s", algorithmic_bytes=nbytes, gpu_GBs=rate(g), gpu_frac_hbm_peak=rate(g) / HBM_PEAK_GBS)
        if ceil:
            entry["gpu_frac_hbm_read_measured"] = rate(g) / ceil["hbm_read_GBs"]
            entry["gpu_frac_infinity_cache_read_measured"] = rate(g) / ceil["infinity_cache_read_GBs"]
    else:
        entry.update(unit="TOP/s", int_ops=ops, gpu_TOPs=rate(g), gpu_frac_int8_peak=rate(g) / INT8_PEAK_TOPS)
    for v in (entry.get("cpu") or {}).values():
        v["GBs" if nbytes else "TOPs"] = rate(v["us"])
    if entry.get("cpu"):
        best = min(v["us"] for v in entry["cpu"].values())
        entry["gpu_speedup_vs_best_cpu"] = best / g
    return entry


def config_pairs(ctx, E, per_decode, per_8b, ceil, cpu=True, reps=10):
    """Every BASELINE config on the GPU beside edgelm's cpu backend at 1 / 4 / 16 threads, same inputs:
    configs[0] (q8 GEMV 960x576, f32 activations), configs[1] (the SmolLM2 W4A8 decode ops: GPU times from the
    decode chain), configs[2] (the SmolLM2 ops at T = 32 / 128 / 512, W8A8 in edgelm's per-block mode, epilogues
    fused), configs[4] (the 8B W4A8 ops at T = 1: GPU times from the 8-layer sweep; and at T = 512)."""
    out = {}
    copies = 30  # T = 1 ops cycle through 30 distinct weights, as a decode step's 30 layers do

    def gpu_time(fn, T, inner):
        return time_graph(ctx, fn, reps, inner=inner) * 1e3

    # configs[0]
    w0 = [HostWeight(700 + i, 960, 576, 1) for i in range(copies)]
    d0 = [ctx.upload(1, 960, 576, w.data, w.scales) for w in w0]
    bx = ctx.buffer(512 * 14336 * 4)  # x of every op below: at most T = 512 rows of K = 14336
    bx.upload(np.random.default_rng(3).standard_normal(512 * 14336, dtype=np.float32))
    ctx.reserve(512, 14336)
    y0 = ctx.buffer(960 * 4)
    us = time_graph(ctx, lambda: [ctx.matmul_dev(bx.ptr, 1, 576, [d], [y0.ptr], act=E.ACT_F32) for d in d0],
                    reps, inner=4) * 1e3 / copies
    y0.free()
    e = {"op": "MATMUL q8 960x576 (fused QKV rows as one weight), f32 activations, T=1", "gpu_us": us,
         "cpu": cpu_op_baseline({"weights": w0[:1], "kind": "matmul", "act": "f32"}, 1) if cpu else None}
    out["configs[0] q8 GEMV 960x576 f32-act"] = pair_rates(e, nbytes=q_bytes(1, 960, 576) + 576 * 4 + 960 * 4,
                                                         ceil=ceil)
    for d in d0:
        d.free()
    cpu_us = " / ".join("%.1f" % v["us"] for v in e["cpu"].values()) if e["cpu"] else ""
    log(f"  configs[0] q8 GEMV f32-act 960x576: GPU {us:.2f} us" + (f", CPU 1/4/16 threads {cpu_us} us" if cpu_us else ""))

    # configs[1] (GPU per-op times from the decode chain, 30 distinct layers)
    sm = {"MATMUL_N qkv": ([(D, D), (KV, D), (KV, D)], "matmul", False), "FFN_SWIGLU": ([(HID, D), (HID, D)], "swiglu", False),
          "MATMUL_ADD down": ([(D, HID)], "matmul", True), "MATMUL lm_head q8": ([(VOCAB, D)], "matmul", False)}
    if per_decode:
        for name, (shapes, kind, resid) in sm.items():
            dt = 1 if "lm_head" in name else 2
            ws = [HostWeight(800 + i, n, k, dt) for i, (n, k) in enumerate(shapes)]
            p = per_decode[name]
            e = {"op": f"{name} W4A8 T=1" if dt == 2 else f"{name} W8A8 T=1", "gpu_us": p["us"],
                 "cpu": cpu_op_baseline({"weights": ws, "kind": kind, "act": "int8", "residual": resid}, 1)
                 if cpu else None}
            out[f"configs[1] {name}"] = pair_rates(e, nbytes=p["bytes"], ceil=ceil)

    def fused_op(T, K, shapes, kind, resid, dws):
        """The op's call and its int ops; every output buffer (and the residual) at exactly its size."""
        outs = [ctx.buffer(T * n * 4) for n, _ in shapes[:1 if kind == "swiglu" else len(shapes)]]
        rb = ctx.buffer(T * shapes[0][0] * 4) if resid else None
        if rb:
            rb.upload(np.random.default_rng(4).standard_normal(T * shapes[0][0], dtype=np.float32))
        if kind == "swiglu":
            fn = lambda: ctx.swiglu_dev(bx.ptr, T, K, dws[0], dws[1], outs[0].ptr, act=E.ACT_INT8)
            ops = 2 * T * K * shapes[0][0] * 2
        else:
            fn = lambda: ctx.matmul_dev(bx.ptr, T, K, dws, [o.ptr for o in outs], [rb.ptr] if rb else None,
                                        act=E.ACT_INT8)
            ops = 2 * T * K * sum(n for n, _ in shapes)
        assert T * K * 4 <= bx.nbytes
        return fn, ops, outs + ([rb] if rb else [])

    # W8A8 (edgelm's per-block mode), T = 32 / 128 / 512, epilogues fused
    for T in (32, 128, 512):
        for name, (shapes, kind, resid) in sm.items():
            ws = [HostWeight(900 + i, n, k, 1) for i, (n, k) in enumerate(shapes)]
            dws = [ctx.upload(1, w.rows, w.cols, w.data, w.scales) for w in ws]
            fn, ops, bufs = fused_op(T, shapes[0][1], shapes, kind, resid, dws)
            log(f"  configs[2] {name} T={T} on the GPU")
            us = gpu_time(fn, T, 16 if T < 512 else 4)
            e = {"op": f"{name} W8A8 (per-32-block activation scales) T={T}", "gpu_us": us,
                 "cpu": cpu_op_baseline({"weights": ws, "kind": kind, "act": "int8", "residual": resid}, T)
                 if cpu else None}
            out[f"configs[2] {name} T={T}"] = pair_rates(e, ops=ops)
            for d in dws + bufs:
                d.free()
        log(f"  configs[2] T={T}: " + ", ".join(f"{n} {out[f'configs[2] {n} T={T}']['gpu_us']:.1f} us" for n in sm))

    # 8B W4A8 at T = 1 (GPU per-op times from the sweep) and T = 512
    b8 = {"MATMUL_N qkv 6144x4096": ([(4096, 4096), (1024, 4096), (1024, 4096)], "matmul"),
          "FFN_SWIGLU 2x14336x4096": ([(14336, 4096), (14336, 4096)], "swiglu"),
          "MATMUL down 4096x14336": ([(4096, 14336)], "matmul")}
    for name, (shapes, kind) in b8.items():
        ws = [HostWeight(950 + i, n, k, 2) for i, (n, k) in enumerate(shapes)]
        if per_8b:
            p = per_8b[name]
            e = {"op": f"{name} W4A8 T=1 (8 distinct layers round-robin on the GPU)", "gpu_us": p["us"],
                 "cpu": cpu_op_baseline({"weights": ws, "kind": kind, "act": "int8"}, 1) if cpu else None}
            out[f"configs[4] {name} T=1"] = pair_rates(e, nbytes=p["weight_bytes"], ceil=ceil)
        dws = [ctx.upload(2, w.rows, w.cols, w.data, w.scales) for w in ws]
        T = 512
        fn, ops, bufs = fused_op(T, shapes[0][1], shapes, kind, False, dws)
        log(f"  configs[4] {name} T=512 on the GPU")
        us = gpu_time(fn, T, 2)
        e = {"op": f"{name} W4A8 (per-32-block activation scales) T=512", "gpu_us": us,
             "cpu": cpu_op_baseline({"weights": ws, "kind": kind, "act": "int8"}, T) if cpu else None}
        out[f"configs[4] {name} T=512"] = pair_rates(e, ops=ops)
        log(f"  configs[4] {name} T=512: GPU {us:.1f} us")
        for d in dws + bufs:
            d.free()
    bx.free()
    return out


E2E_SD, E2E_EMBED_SD = 0.05, 0.5  # weight scales of the e2e model: greedy tokens differ step to step


def write_e2e_model(path):
    from edgelm_amd import synth as S
    t0 = time.time()
    S.write_model(path, S.SMOLLM2_135M, "q4", embed_dtype="q8", seed=20260101, sd=E2E_SD, embed_sd=E2E_EMBED_SD)
    log(f"e2e model written in {time.time() - t0:.1f}s ({os.path.getsize(path) / 1e6:.1f} MB)")


def e2e_headline(path, steps, warmup, P=128):
    """the random-init SmolLM2-135M-shaped model (q4 g32 + q8 embedding, int8 activations) through
    this build's Session with backends "hip,cpu" (the whole model on the GPU, decode steps replayed as HIP
    graphs, greedy argmax on the device): edgelm's bench protocol (main.cpp:173-233) with the LCG prompt of P
    tokens; after two untimed reps (the backend runs the first prompt of a length op by op, captures the second
    into a HIP graph and replays it for later ones, as it does for decode steps), one timed rep: TTFT of the
    prompt, `warmup` untimed decode steps, then exactly
    `steps` timed greedy decode steps queued back to back (Session::greedy_steps: each step's token id goes
    from the device argmax into the next step on the device and is copied back asynchronously; the clock stops
    once every token id is on the host). `ttft_ms` is the median over that rep's prompt and four more reps of
    the prompt alone (one prompt's TTFT varies by a few percent from run to run); `ttft_samples_ms` lists them."""
    from edgelm_amd import synth as S
    from edgelm_amd import host
    prompt = S.lcg_prompt(P, 49152)
    threads = min(8, os.cpu_count() or 1)
    t0 = time.perf_counter()
    m = host.Model(path)
    m.prefault()
    s = host.Session(m, "hip,cpu", threads=threads, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=True)
    cold = s.bench(prompt, 0, 1)  # first use: weight upload and repack, buffers, graph capture on later steps
    cold_ms = (time.perf_counter() - t0) * 1e3 - cold["decode_ms"]
    s.bench(prompt, 2, 4)  # warm-up rep (the cold rep above was the first)
    r = s.bench(prompt, warmup, steps)
    ttfts = [r["ttft_ms"]] + [s.bench(prompt, 0, 1)["ttft_ms"] for _ in range(4)]
    ttft = float(np.median(ttfts))
    s.close()
    m.close()
    # the same cold start with the weights' device image (the repacked HBM layout cached on disk next
    # to the .elm file): written once, then a new model and session map it and upload from it
    img = path + ".gfx950.img"
    t0 = time.perf_counter()
    mw = host.Model(path)
    mw.write_device_image(img, threads=threads)
    mw.close()
    write_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    m = host.Model(path)
    attached = m.attach_device_image(img)  # the upload reads the image, so the .elm is not prefaulted
    s = host.Session(m, "hip,cpu", threads=threads, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=True)
    cold_img = s.bench(prompt, 0, 1)
    cold_img_ms = (time.perf_counter() - t0) * 1e3 - cold_img["decode_ms"]
    img_tokens_match = bool(np.array_equal(cold_img["tokens"], r["tokens"][:len(cold_img["tokens"])]))
    s.close()
    log(f"e2e cold TTFT {cold_ms:.0f} ms from the .elm file, {cold_img_ms:.0f} ms with its device image "
        f"(attached: {attached}, image written in {write_ms:.0f} ms)")
    out = {"decode_tok_s": steps / (r["decode_ms"] / 1e3), "ms_per_step": r["decode_ms"] / steps,
           "ttft_ms": ttft, "ttft_samples_ms": [round(t, 4) for t in ttfts], "prefill_tok_s": P / (ttft / 1e3),
           "prompt": P, "steps": steps,
           "warmup": warmup, "backends": "hip,cpu", "host_threads": threads,
           "cold_ttft_ms": cold_ms, "cold_ttft_note": "model load + prefault + session creation + first prompt "
                                                      "(weight upload and repack included) to the first token",
           "cold_ttft_device_image_ms": cold_img_ms, "device_image_attached": attached,
           "device_image_write_ms": write_ms, "device_image_tokens_match": img_tokens_match,
           "greedy_tokens": [int(t) for t in r["tokens"]]}
    log(f"e2e hip,cpu: decode {out['decode_tok_s']:.1f} tok/s ({out['ms_per_step'] * 1e3:.0f} us/token), "
        f"TTFT {out['ttft_ms']:.2f} ms, prefill {out['prefill_tok_s']:.0f} tok/s, cold TTFT {cold_ms:.0f} ms")
    # the matmul-only flavour (configs[3] as BASELINE words it: MATMUL* on the GPU, the rest on the host)
    s = host.Session(m, "hip-matmul,cpu", threads=threads, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=True)
    s.bench(prompt, 2, 4)
    s.bench(prompt, 2, 4)
    rm = s.bench(prompt, warmup, steps)
    s.close()
    out["matmul_only"] = {"decode_tok_s": steps / (rm["decode_ms"] / 1e3), "ttft_ms": rm["ttft_ms"],
                          "backends": "hip-matmul,cpu",
                          "greedy_tokens_match": bool(np.array_equal(rm["tokens"], r["tokens"]))}
    log(f"e2e hip-matmul,cpu: decode {out['matmul_only']['decode_tok_s']:.1f} tok/s, TTFT {rm['ttft_ms']:.2f} ms, "
        f"tokens match: {out['matmul_only']['greedy_tokens_match']}")
    # edgelm's f32-activation mode (act_quant off: the f32 x dequantized-weight dot products), whole model
    # on the GPU as above; its tokens follow other numerics than the int8 run's, so they are not compared
    s = host.Session(m, "hip,cpu", threads=threads, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=False)
    s.bench(prompt, 2, 4)
    s.bench(prompt, 2, 4)
    rf = s.bench(prompt, warmup, steps)
    s.close()
    out["f32_activations"] = {"decode_tok_s": steps / (rf["decode_ms"] / 1e3), "ttft_ms": rf["ttft_ms"],
                              "backends": "hip,cpu", "act_quant": False}
    log(f"e2e hip,cpu f32 activations: decode {out['f32_activations']['decode_tok_s']:.1f} tok/s, "
        f"TTFT {rf['ttft_ms']:.2f} ms")
    m.close()
    return out, r["tokens"]


def host_cpu():
    """CPU model, logical CPUs the process may use, and physical cores of the host."""
    model, cores = "unknown", set()
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"model": model, "usable_logical_cpus": usable, "physical_cores": len(cores) or None}


def cpu_baseline(path, tokens_gpu, steps, warmup, P=128, budget_s=15.0):
    """edgelm's own Session (compiled from the reference sources into oracle/_ref; cpu backend, its x86 scalar
    path since this host has no NEON, act int8) on the same model file and protocol as the headline, timed
    inside C (eref_session_bench). Bounded: repeated timed reps for about budget_s seconds at 16 threads
    (this box's CPU share), then one rep each at 1 and 4 threads (4 is edgelm's CLI default)."""
    import oracle as O
    from edgelm_amd import synth as S
    if not O.ref_available():
        log("cpu baseline skipped: oracle/_ref not built")
        return None, None
    prompt = S.lcg_prompt(P, 49152)
    ct = min(16, os.cpu_count() or 1)
    r = O.RefSession(path, "cpu", threads=ct, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=True)
    r.bench(prompt, 2, 4)
    reps, t_end = [], time.time() + budget_s
    while time.time() < t_end or not reps:
        reps.append(r.bench(prompt, warmup, steps))
    r.close()
    dec = sorted(steps / (x["decode_ms"] / 1e3) for x in reps)
    med = dec[len(dec) // 2]
    match = bool(np.array_equal(reps[0]["tokens"], tokens_gpu))
    log(f"cpu baseline (edgelm session, {ct} threads): decode {med:.1f} tok/s over {len(reps)} reps, "
        f"TTFT {reps[0]['ttft_ms']:.0f} ms, greedy tokens match the GPU's: {match}")
    by_threads = {}
    for th in (1, 4):
        r = O.RefSession(path, "cpu", threads=th, max_ctx=P + warmup + steps + 8, max_batch=P, act_quant=True)
        x = r.bench(prompt, 2, min(steps, 32))
        by_threads[str(th)] = {"decode_tok_s": min(steps, 32) / (x["decode_ms"] / 1e3), "ttft_ms": x["ttft_ms"]}
        r.close()
    cpu = host_cpu()
    base = {"value": med, "unit": "tok/s", "cores": ct, "kind": "reference",
            "sample": f"{len(reps)} timed reps of the headline protocol ({P}-token prompt, {warmup} untimed + {steps} "
                      f"timed greedy decode steps) on edgelm's own Session, cpu backend, act int8, {ct} threads, "
                      f"~{budget_s:.0f} s",
            "cpu_model": cpu["model"], "usable_logical_cpus": cpu["usable_logical_cpus"],
            "physical_cores": cpu["physical_cores"], "path": "x86 scalar (EDGELM_NEON=0)"}
    extra = {"ttft_ms": reps[0]["ttft_ms"], "greedy_tokens_match_gpu": match, "by_threads": by_threads}
    return base, extra


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")


def pmc_workload(ctx, E):
    """The roofline kernels alone, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes: eager launches
    of the SmolLM2 FFN_SWIGLU and MATMUL_ADD down GEMVs (the candidates for the headline roofline
    kernel; 30 distinct layers each) and of the 8B down GEMV on a pre-quantized activation (8
    distinct layers), 4 rounds each, plus a 64 MiB device copy of known size whose counter readings
    calibrate the others."""
    m = Model(ctx, 1234, {f"{l}.{n}": (HID, D) for l in range(L) for n in "gu"} |
              {f"{l}.d": (D, HID) for l in range(L)}, lambda n: 2)
    bx = ctx.buffer(14336 * 4)
    bx.upload(np.random.default_rng(5).standard_normal(14336, dtype=np.float32))
    by = ctx.buffer(14336 * 4)
    bres = ctx.buffer(D * 4)
    bres.upload(np.random.default_rng(6).standard_normal(D, dtype=np.float32))
    for _ in range(4):
        for l in range(L):
            ctx.swiglu_dev(bx.ptr, 1, D, m.w[f"{l}.g"], m.w[f"{l}.u"], by.ptr, act=E.ACT_INT8)
    ctx.synchronize()
    for _ in range(4):
        for l in range(L):
            ctx.matmul_dev(bx.ptr, 1, HID, [m.w[f"{l}.d"]], [by.ptr], [bres.ptr], act=E.ACT_INT8)
    ctx.synchronize()
    bres.free()
    m.free()
    m = Model(ctx, 11, {f"{l}.d": (4096, 14336) for l in range(8)}, lambda n: 2)
    q, d, s = ctx.buffer(14336), ctx.buffer(448 * 4), ctx.buffer(448 * 4)
    ctx.quantize_act_dev(bx.ptr, 1, 14336, q.ptr, d.ptr, s.ptr)
    for _ in range(4):
        for l in range(8):
            ctx.gemv_a8_dev(q.ptr, d.ptr, s.ptr, 1, 14336, [m.w[f"{l}.d"]], [by.ptr])
    ctx.synchronize()
    m.free()
    # the 8B gate+up SwiGLU that also quantizes h (32-row workgroups), 8 distinct layers
    m = Model(ctx, 12, {f"{l}.{n}": (14336, 4096) for l in range(8) for n in "gu"}, lambda n: 2)
    for _ in range(4):
        for l in range(8):
            ctx.swiglu_quant_dev(bx.ptr, 1, 4096, m.w[f"{l}.g"], m.w[f"{l}.u"], by.ptr, q.ptr, d.ptr, s.ptr)
    ctx.synchronize()
    m.free()
    n = 64 << 20
    src, dst = ctx.buffer(n), ctx.buffer(n)
    ctx.memset_dev(src.ptr, 1, n)
    for _ in range(4):
        ctx.memcpy_d2d(dst.ptr, src.ptr, n)
    ctx.synchronize()
    for b in (bx, by, q, d, s, src, dst):
        b.free()
    log("pmc workload done")


def pmc_gemm_workload(ctx, E):
    """The configs[4] T = 512 prefill GEMMs alone (q8 weights with the per-token scale, then with edgelm's
    per-block scales, then q4 weights with per-block scales), four eager launches per shape, for rocprofv3
    --pmc passes (MFMA busy cycles, LDS bank conflicts, VALU and MFMA instruction counts)."""
    b8 = [(4096, 4096), (14336, 4096), (4096, 14336)]
    bx = ctx.buffer(512 * 14336 * 4)
    bx.upload(np.random.default_rng(3).standard_normal(512 * 14336, dtype=np.float32))
    by = ctx.buffer(512 * 14336 * 4)
    ctx.reserve(512, 14336)
    for dt, acts in ((1, (E.ACT_INT8_TOKEN, E.ACT_INT8)), (2, (E.ACT_INT8,))):
        m = Model(ctx, 5, {f"{i}": sh for i, sh in enumerate(b8)}, lambda n: dt)
        for act in acts:
            for i, (n, k) in enumerate(b8):
                for _ in range(4):
                    ctx.matmul_dev(bx.ptr, 512, k, [m.w[f"{i}"]], [by.ptr], act=act)
                ctx.synchronize()
        m.free()
    bx.free()
    by.free()
    log("pmc gemm workload done")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(kernel)
    return None if k is None else int(k["fetch_bytes"] + k["write_bytes"])


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed greedy decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed greedy decode steps before them")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-8b", action="store_true", help="skip the 8B-shaped sweep")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMMs")
    ap.add_argument("--no-chain", action="store_true", help="skip the decode matmul chain and its per-op timers")
    ap.add_argument("--no-pairs", action="store_true",
                    help="skip the per-config GPU / CPU pairs (configs[0], [1], [2], [4] beside edgelm's cpu backend)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the roofline kernels and a calibration copy (for rocprofv3 counter passes)")
    ap.add_argument("--pmc-gemm", action="store_true",
                    help="run only the T = 512 prefill GEMMs (for rocprofv3 counter passes)")
    ap.add_argument("--eager", action="store_true",
                    help="no HIP graphs, in the benchmarks or the e2e sessions (for kernel tracing): the step "
                         "rate becomes host-bound, per-kernel event timings are unchanged")
    args = ap.parse_args()
    if args.eager:  # the e2e sessions' decode graphs too
        os.environ["EDGELM_HIP_GRAPHS"] = "0"
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (this delegate has no multi-GPU path); got --gpus {args.gpus}, "
              f"WORLD_SIZE {world}", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)

    from edgelm_amd import elmh as E
    if args.pmc_workload or args.pmc_gemm:
        ctx = E.Context(0)
        (pmc_workload if args.pmc_workload else pmc_gemm_workload)(ctx, E)
        ctx.close()
        return

    import tempfile
    extra = {}
    with tempfile.TemporaryDirectory() as tmp:
        model_path = os.path.join(tmp, "smollm2-135m-random.q4.elm")
        write_e2e_model(model_path)
        head, tokens = e2e_headline(model_path, args.steps, args.warmup)

        ctx = E.Context(0)
        log(f"device {ctx.arch}")
        ceil = measured_ceilings(ctx, E)
        extra["measured_ceilings"] = ceil
        per = None
        if not args.no_chain:
            ms_chain, per = decode_step_bench(ctx, E, 200, 20, args.eager)
            extra["decode_matmul_chain"] = {"us_per_token": ms_chain * 1e3, "tok_s": 1e3 / ms_chain,
                                            "what": "the 121 matmul-family calls of a decode step alone (configs[1] "
                                                    "shapes, W4A8, device-resident, one HIP graph per step)",
                                            "per_op": per}
        if not args.no_8b:
            extra["gemv_8b_w4a8"] = sweep_8b(ctx, E, eager=args.eager)
        if not args.no_gemm:
            sm = [(D + 2 * KV, D), (HID, D), (D, HID), (VOCAB, D)]
            b8 = [(4096, 4096), (14336, 4096), (4096, 14336)]
            # BASELINE configs[2] read literally: W8A8, int8 per-channel weights, one int8 scale per token
            # (ELMH_ACT_INT8_TOKEN, an extension: edgelm's mode is per 32-block, timed in configs[2] below)
            extra["gemm_w8a8_token_T128"] = gemm_bench(ctx, E, 128, sm, act=E.ACT_INT8_TOKEN, eager=args.eager)
            extra["gemm_w8a8_token_T512_8b"] = gemm_bench(ctx, E, 512, b8, act=E.ACT_INT8_TOKEN, eager=args.eager)
            # edgelm's parity mode: per-32-block activation scales, block-order f32 rescale (VALU-bound)
            extra["gemm_w8a8_T512_8b"] = gemm_bench(ctx, E, 512, b8, eager=args.eager)
            # W4A8 prefill (the e2e model's layers), parity mode
            extra["gemm_w4a8_T512_8b"] = gemm_bench(ctx, E, 512, b8, dt=2, eager=args.eager)
        if not args.no_gemm:
            extra["gemm_rescale_ceiling"] = rescale_ceiling(ctx, E)
        if not args.no_pairs:
            log("per-config GPU / CPU pairs")
            extra["config_pairs"] = config_pairs(ctx, E, per, extra.get("gemv_8b_w4a8", {}).get("per_op"), ceil,
                                                 cpu=not args.no_cpu)
        ctx.close()

        roof = None
        if per:
            # dominant kernel of the headline decode step: gemv_small_kernel<q4, 1 token, no SwiGLU, no norm> runs the
            # o projection and the down projection of every layer (the largest share of the step's GPU time in
            # the kernel trace); its per-launch time comes from HIP events around graph replays on the library's
            # stream, and its algorithmic bytes are the down projection's (the larger of its two calls)
            dom_name = "MATMUL_ADD down"
            dom = per[dom_name]
            roof = {"kernel": "gemv_small_kernel<2, 1, false, false, false> (" + dom_name + " 576x1536 q4 + residual, T=1)",
                    "bound": "hbm", "achieved": round(dom["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(dom["GBs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom_name),
                    "algorithmic_bytes_per_launch": dom["bytes"], "avg_launch_us": round(dom["us"], 3),
                    "peak_hbm_read_measured": round(ceil["hbm_read_GBs"], 1),
                    "frac_hbm_read_measured": round(dom["GBs"] / ceil["hbm_read_GBs"], 4),
                    "peak_infinity_cache_read_measured": round(ceil["infinity_cache_read_GBs"], 1),
                    "frac_infinity_cache_read_measured": round(dom["GBs"] / ceil["infinity_cache_read_GBs"], 4),
                    "note": "SmolLM2-sized weights stay in L2 / Infinity Cache and each call is a few microseconds: "
                            "latency-bound; roofline_8b_down_gemv is the HBM-bound kernel (configs[4])"}
        if "gemv_8b_w4a8" in extra:
            g8 = extra["gemv_8b_w4a8"]
            extra["roofline_8b_down_gemv"] = {
                "kernel": "gemv_stream_kernel (8B down 4096x14336, W4A8, T=1)", "bound": "hbm",
                "achieved": round(g8["down_gemv_GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(g8["down_gemv_GBs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic("8B down GEMV"),
                "algorithmic_bytes_per_launch": g8["down_gemv_bytes"], "avg_launch_us": round(g8["down_gemv_us"], 3),
                "peak_hbm_read_measured": round(ceil["hbm_read_GBs"], 1),
                "frac_hbm_read_measured": round(g8["down_gemv_GBs"] / ceil["hbm_read_GBs"], 4),
                "sweep_frac_hbm_read_measured": round(g8["GBs"] / ceil["hbm_read_GBs"], 4)}
        cpu = None
        if not args.no_cpu:
            cpu, cpu_extra = cpu_baseline(model_path, tokens, args.steps, args.warmup)
            if cpu_extra:
                head["cpu_reference"] = cpu_extra
                head["greedy_tokens_match_edgelm"] = cpu_extra["greedy_tokens_match_gpu"]

    line = {
        "metric": METRIC, "value": round(head["decode_tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 (W4A8: q4 g32 weights x per-32-block int8 activations, int32 acc, f32 rescale)",
        "data": f"synthetic (random-init SmolLM2-135M-shaped model, weights N(0,{E2E_SD}), embedding "
                f"N(0,{E2E_EMBED_SD}), quantized with edgelm's quantizers; LCG prompt of edgelm's bench)",
        "config": {"workload": "configs[3]: end-to-end SmolLM2-135M-shaped decode (30 layers, q4 g32 + q8 embedding, "
                               "int8 activations), backends hip,cpu, 128-token prompt then greedy decode; a step is one "
                               "token", "parallelism": "single GPU",
                   "timing": "eager launches (kernel-trace mode; step rate host-bound)" if args.eager else
                             "host clock around exactly `steps` greedy steps queued back to back; stops once every "
                             "step's token id is on the host"},
        "roofline": roof, "cpu_baseline": cpu, "e2e_smollm2_w4a8": head, **extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
