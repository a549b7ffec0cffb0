"""GPU parity of the non-matmul layer ops (edgelm_amd/csrc/elmh_layer.hip through the C ABI)
against the CPU oracle, which restates edgelm's cpu backend and is pinned against edgelm's own
C++ (tests/test_oracle_layer.py). Bar: bit-identical outputs and KV caches.
"""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import elmh as E

pytestmark = pytest.mark.gpu


def dev(ctx, a):
    a = np.ascontiguousarray(a)
    b = ctx.buffer(max(a.nbytes, 4))
    b.upload(a)
    return b


@pytest.mark.parametrize("dim", [576, 578, 1, 64, 1536])
def test_rmsnorm_bit_exact(ctx, dim):
    r = np.random.default_rng(dim)
    for rows in (1, 3, 130):
        print(f"[gpu] rmsnorm dim={dim} rows={rows}", flush=True)
        x = r.normal(0, 2, (rows, dim)).astype(np.float32)
        x[0, : min(dim, 5)] = 0.0
        w = r.normal(1, 0.2, dim).astype(np.float32)
        bx, bw, by = dev(ctx, x), dev(ctx, w), ctx.buffer(x.nbytes)
        ctx.rmsnorm_dev(bx.ptr, bw.ptr, by.ptr, rows, dim, 1e-5)
        assert bits_equal(by.download(x.shape, np.float32), O.rmsnorm(x, w, 1e-5))
        for b in (bx, bw, by):
            b.free()


ATTN_SHAPES = [(9, 3, 64, 160, (17, 1, 1, 5, 1, 9)), (4, 4, 32, 48, (17, 1, 1, 5, 1, 9)),
               (8, 1, 128, 40, (17, 1, 1, 5, 1, 9)),
               # head_dim 20: value chunks of 204 whole positions; more positions than threads
               (6, 2, 20, 320, (257, 1, 30, 1)),
               # a long prefill: several value chunks and score rows per thread
               (9, 3, 64, 420, (400, 1, 1))]


@pytest.mark.parametrize("shape", ATTN_SHAPES, ids=[f"{s[0]}x{s[1]}x{s[2]}" for s in ATTN_SHAPES])
@pytest.mark.parametrize("rope", [False, True])
def test_attention_bit_exact(ctx, shape, rope):
    """A session's sequence of calls: prefill, decodes and a chunk, KV cache carried on the GPU."""
    nh, nkv, hd, mc, steps = shape
    r = np.random.default_rng(nh * 100 + hd + int(rope))
    tab = O.rope_table(hd, mc, 100000.0) if rope else None
    kc = np.zeros((nkv, mc, hd), np.float32)
    vc = np.zeros_like(kc)
    bkc, bvc = dev(ctx, kc), dev(ctx, vc)
    bcos, bsin = (dev(ctx, tab[0]), dev(ctx, tab[1])) if rope else (None, None)
    pos = 0
    for T in steps:
        if pos + T > mc:
            break
        print(f"[gpu] attention {shape[:4]} rope={rope} pos0={pos} T={T}", flush=True)
        q = r.normal(0, 1, (T, nh * hd)).astype(np.float32)
        k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        bq, bk, bv, bo = dev(ctx, q), dev(ctx, k), dev(ctx, v), ctx.buffer(q.nbytes)
        ctx.attention_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, T, pos, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                          bcos.ptr if rope else None, bsin.ptr if rope else None)
        want = O.attention(q, k, v, pos, nh, nkv, kc, vc, tab)
        assert bits_equal(bo.download(q.shape, np.float32), want), f"pos0={pos} T={T}"
        for b in (bq, bk, bv, bo):
            b.free()
        pos += T
    assert bits_equal(bkc.download(kc.shape, np.float32), kc)
    assert bits_equal(bvc.download(vc.shape, np.float32), vc)
    for b in [bkc, bvc] + ([bcos, bsin] if rope else []):
        b.free()


# (n_heads, n_kv, head_dim, max_ctx, cached positions): score rows past what LDS holds (about 20K positions at
# head size 64, fewer at 20), through the head-size-64 and the generic instantiation
LONG_SHAPES = [(9, 3, 64, 33024, 32760), (6, 2, 20, 40000, 39950)]


@pytest.mark.parametrize("shape", LONG_SHAPES, ids=[f"{s[0]}x{s[1]}x{s[2]}" for s in LONG_SHAPES])
def test_attention_past_lds_score_rows(ctx, shape):
    """Contexts longer than a workgroup's LDS can hold a score row of: a chunk of prompt tokens, a decode
    step, and decode steps with the position read from device memory (the graph-replayed form, its rows
    sized for the whole cache), each bit-identical to edgelm's cpu attention (the oracle), KV caches
    included. The rows live in a device buffer; the in-order sum of the exponentials crosses chunk
    boundaries of the LDS staging."""
    nh, nkv, hd, mc, p0 = shape
    r = np.random.default_rng(hd + mc)
    tab = O.rope_table(hd, mc, 100000.0)
    kc = r.normal(0, 1, (nkv, mc, hd)).astype(np.float32)
    vc = r.normal(0, 1, (nkv, mc, hd)).astype(np.float32)
    kc[:, p0:] = np.nan  # never read before the step that writes them
    vc[:, p0:] = np.nan
    bkc, bvc = dev(ctx, kc), dev(ctx, vc)
    bcos, bsin = dev(ctx, tab[0]), dev(ctx, tab[1])
    bpos = ctx.buffer(4)
    pos = p0
    for T, step in [(5, False), (1, False), (1, True), (1, True)]:
        print(f"[gpu] attention past LDS {shape} pos0={pos} T={T} step={step}", flush=True)
        q = r.normal(0, 1, (T, nh * hd)).astype(np.float32)
        k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        bq, bk, bv, bo = dev(ctx, q), dev(ctx, k), dev(ctx, v), ctx.buffer(q.nbytes)
        if step:
            bpos.upload(np.array([pos], np.int32))
            ctx.attention_step_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, bpos.ptr, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                                   bcos.ptr, bsin.ptr)
        else:
            ctx.attention_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, T, pos, nh, nkv, hd, bkc.ptr, bvc.ptr, mc, bcos.ptr,
                              bsin.ptr)
        want = O.attention(q, k, v, pos, nh, nkv, kc, vc, tab)
        assert bits_equal(bo.download(q.shape, np.float32), want), f"pos0={pos} T={T}"
        for b in (bq, bk, bv, bo):
            b.free()
        pos += T
    assert bits_equal(bkc.download(kc.shape, np.float32), kc)
    assert bits_equal(bvc.download(vc.shape, np.float32), vc)
    assert E.lib().elmh_attention_step_supported(hd, mc) == 1
    for b in (bkc, bvc, bcos, bsin, bpos):
        b.free()


@pytest.mark.parametrize("rope", [False, True])
def test_attention_long_cache_decode_steps(ctx, rope):
    """Decode steps with the position read from device memory (the form a captured graph replays) over a
    cache of 16,384 positions, whose score row the step kernel keeps whole in LDS (more than 64 KB: the
    kernel's LDS limit is raised to gfx950's 160 KB), at positions around the 320-position value chunks."""
    nh, nkv, hd, mc = 9, 3, 64, 16384
    r = np.random.default_rng(77 + int(rope))
    tab = O.rope_table(hd, mc, 100000.0) if rope else None
    kc = np.zeros((nkv, mc, hd), np.float32)
    vc = np.zeros_like(kc)
    bkc, bvc = dev(ctx, kc), dev(ctx, vc)
    bcos, bsin = (dev(ctx, tab[0]), dev(ctx, tab[1])) if rope else (None, None)
    bpos = ctx.buffer(4)
    pos = 0
    for T, step in [(318, False), (1, True), (1, True), (1, True), (318, False), (1, True), (1, True)]:
        print(f"[gpu] long-cache attention rope={rope} pos0={pos} T={T} step={step}", flush=True)
        q = r.normal(0, 1, (T, nh * hd)).astype(np.float32)
        k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        bq, bk, bv, bo = dev(ctx, q), dev(ctx, k), dev(ctx, v), ctx.buffer(q.nbytes)
        if step:
            bpos.upload(np.array([pos], np.int32))
            ctx.attention_step_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, bpos.ptr, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                                   bcos.ptr if rope else None, bsin.ptr if rope else None)
        else:
            ctx.attention_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, T, pos, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                              bcos.ptr if rope else None, bsin.ptr if rope else None)
        want = O.attention(q, k, v, pos, nh, nkv, kc, vc, tab)
        assert bits_equal(bo.download(q.shape, np.float32), want), f"pos0={pos} T={T}"
        for b in (bq, bk, bv, bo):
            b.free()
        pos += T
    assert bits_equal(bkc.download(kc.shape, np.float32), kc)
    for b in [bkc, bvc, bpos] + ([bcos, bsin] if rope else []):
        b.free()


@pytest.mark.parametrize("rope", [False, True])
def test_attention_decode_steps_across_row_chunks(ctx, rope):
    """Decode steps (position in device memory) of the head-size-64 decode kernel, which moves the cached
    rows into LDS 256 at a time: the first position, positions on both sides of 256 and 512 cached rows
    (one and several chunks of keys and values) and the cache's last position. Rows past the step's
    position hold NaN: the kernel reads such rows ahead and must never use them."""
    nh, nkv, hd, mc = 9, 3, 64, 1100
    r = np.random.default_rng(91 + int(rope))
    tab = O.rope_table(hd, mc, 100000.0) if rope else None
    kc = np.full((nkv, mc, hd), np.nan, np.float32)
    vc = np.full_like(kc, np.nan)
    bkc, bvc = dev(ctx, kc), dev(ctx, vc)
    bcos, bsin = (dev(ctx, tab[0]), dev(ctx, tab[1])) if rope else (None, None)
    bpos = ctx.buffer(4)
    pos = 0
    plan = [(1, True), (1, True), (253, False)] + [(1, True)] * 5 + [(250, False)] + [(1, True)] * 4 + \
           [(585, False), (1, True)]
    for T, step in plan:
        print(f"[gpu] chunked decode attention rope={rope} pos0={pos} T={T} step={step}", flush=True)
        q = r.normal(0, 1, (T, nh * hd)).astype(np.float32)
        k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        bq, bk, bv, bo = dev(ctx, q), dev(ctx, k), dev(ctx, v), ctx.buffer(q.nbytes)
        if step:
            bpos.upload(np.array([pos], np.int32))
            ctx.attention_step_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, bpos.ptr, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                                   bcos.ptr if rope else None, bsin.ptr if rope else None)
        else:
            ctx.attention_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, T, pos, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                              bcos.ptr if rope else None, bsin.ptr if rope else None)
        want = O.attention(q, k, v, pos, nh, nkv, kc, vc, tab)
        got = bo.download(q.shape, np.float32)
        assert not np.isnan(got).any(), f"pos0={pos} T={T}"
        assert bits_equal(got, want), f"pos0={pos} T={T}"
        for b in (bq, bk, bv, bo):
            b.free()
        pos += T
    assert pos == mc
    assert bits_equal(bkc.download(kc.shape, np.float32), kc)
    assert bits_equal(bvc.download(vc.shape, np.float32), vc)
    for b in [bkc, bvc, bpos] + ([bcos, bsin] if rope else []):
        b.free()


FUSED_ATTN = [(9, 3, 64, 300, (128, 1, 33, 7, 3)), (4, 4, 32, 64, (17, 5))]


@pytest.mark.parametrize("shape", FUSED_ATTN, ids=[f"{s[0]}x{s[1]}x{s[2]}" for s in FUSED_ATTN])
@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_attention_fused_into_matmul(ctx, shape, dt):
    """elmh_attention_matmul_dev: out and the KV caches as ATTENTION, and y bit-identical to the o
    projection (MATMUL_ADD with the residual, then plain MATMUL) on edgelm's cpu backend over the
    attention's output, for a session's calls: chunks where the attention kernel writes the GEMM's
    quantized operand (T = 128, then T = 33 and 7 over the token slots the first call left past T), a
    decode token and a short chunk on the GEMV, and head size 32, which never fuses; each call's path
    is asserted through elmh_attention_matmul_fused."""
    nh, nkv, hd, mc, steps = shape
    r = np.random.default_rng(nh + hd + dt)
    tab = O.rope_table(hd, mc, 100000.0)
    kc = np.zeros((nkv, mc, hd), np.float32)
    vc = np.zeros_like(kc)
    bkc, bvc, bcos, bsin = dev(ctx, kc), dev(ctx, vc), dev(ctx, tab[0]), dev(ctx, tab[1])
    D, N = nh * hd, 96
    w = O.make_weight(r.normal(0, 0.05, (N, D)).astype(np.float32), dt)
    dw = ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)
    pos = 0
    for i, T in enumerate(steps):
        print(f"[gpu] attention+matmul {shape[:4]} dt={dt} pos0={pos} T={T}", flush=True)
        q = r.normal(0, 1, (T, D)).astype(np.float32)
        k = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        v = r.normal(0, 1, (T, nkv * hd)).astype(np.float32)
        res = r.normal(0, 1, (T, N)).astype(np.float32) if i % 2 == 0 else None
        bq, bk, bv, bo, by = dev(ctx, q), dev(ctx, k), dev(ctx, v), ctx.buffer(q.nbytes), ctx.buffer(T * N * 4)
        bres = dev(ctx, res) if res is not None else None
        ctx.attention_matmul_dev(bq.ptr, bk.ptr, bv.ptr, bo.ptr, T, pos, nh, nkv, hd, bkc.ptr, bvc.ptr, mc,
                                 bcos.ptr, bsin.ptr, dw, by.ptr, bres.ptr if bres else None)
        # the path taken: the attention kernel writes the GEMM's operand for chunks of head size 64 that
        # go to the block-scale GEMM (more than 4 tokens at these shapes: T = 128, 33, 7); decode tokens
        # and chunks of up to 4 tokens use the GEMV, head size 32 the separate quantizer
        assert ctx.attention_matmul_fused() == (hd == 64 and T > 4), f"pos0={pos} T={T}"
        att = O.attention(q, k, v, pos, nh, nkv, kc, vc, tab)
        assert bits_equal(bo.download(q.shape, np.float32), att), f"pos0={pos} T={T}"
        want = O.cpu_matmul(att, [w], [res], act_quant=True)[0]
        assert bits_equal(by.download((T, N), np.float32), want), f"pos0={pos} T={T}"
        for b in (bq, bk, bv, bo, by) + ((bres,) if bres else ()):
            b.free()
        pos += T
    assert bits_equal(bkc.download(kc.shape, np.float32), kc)
    assert bits_equal(bvc.download(vc.shape, np.float32), vc)
    for b in (bkc, bvc, bcos, bsin, dw):
        b.free()


def test_attention_rejects_bad_shapes(ctx):
    from edgelm_amd import elmh as E
    b = ctx.buffer(4096)
    for args in [(1, 8, 9, 3, 64, 8),    # pos0 + T > max_ctx
                 (1, 0, 9, 4, 64, 8),    # heads not a multiple of kv heads
                 (1, 0, 9, 3, 62, 8)]:   # head_dim not a multiple of 4
        T, pos0, nh, nkv, hd, mc = args
        with pytest.raises(E.ElmhError) as e:
            ctx.attention_dev(b.ptr, b.ptr, b.ptr, b.ptr, T, pos0, nh, nkv, hd, b.ptr, b.ptr, mc)
        assert e.value.code == E.ERR_ARG
    b.free()


def test_attention_matmul_rejects_bad_arguments(ctx):
    """elmh_attention_matmul_dev checks the attention's arguments as elmh_attention_dev does, and
    the weight against the attention's output width (n_heads * head_dim), before any launch."""
    from edgelm_amd import elmh as E
    b = ctx.buffer(1 << 16)
    r = np.random.default_rng(5)
    w = O.make_weight(r.normal(0, 0.05, (32, 9 * 64)).astype(np.float32), O.Q8)
    dw = ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)
    for T, pos0, nh, act in [(8, 0, 8, E.ACT_INT8),    # weight width 576 != 8 * 64
                             (4, 10, 9, E.ACT_INT8),   # pos0 + T > max_ctx
                             (8, 0, 9, 7)]:            # no such activation mode
        with pytest.raises(E.ElmhError) as e:
            ctx.attention_matmul_dev(b.ptr, b.ptr, b.ptr, b.ptr, T, pos0, nh, 1 if nh == 8 else 3, 64, b.ptr, b.ptr,
                                     12, None, None, dw, b.ptr, None, act=act)
        assert e.value.code == E.ERR_ARG, e.value
    b.free()
    dw.free()


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_embed_bit_exact(ctx, dt):
    r = np.random.default_rng(30 + dt)
    rows, cols = 300, 576
    w = O.make_weight(r.normal(0, 0.5, (rows, cols)).astype(np.float32), dt)
    dw = ctx.upload(w.dtype, w.rows, w.cols, w.data, w.scales)
    full = O.dequantize(w)
    for toks in ([0], [rows - 1, 5, 5, 123], list(r.integers(0, rows, 70))):
        print(f"[gpu] embed dt={dt} T={len(toks)}", flush=True)
        t = np.array(toks, np.int32)
        bt, by = dev(ctx, t), ctx.buffer(len(toks) * cols * 4)
        ctx.embed_dev(bt.ptr, len(toks), dw, by.ptr)
        assert bits_equal(by.download((len(toks), cols), np.float32), full[t])
        bt.free()
        by.free()
    dw.free()


def test_fill_and_copy(ctx):
    b = ctx.buffer(1031)
    b.upload(np.arange(1031, dtype=np.uint8))
    ctx.memset_dev(b.ptr + 3, 0xAB, 1021)
    got = b.download((1031,), np.uint8)
    want = np.arange(1031, dtype=np.uint8)
    want[3:1024] = 0xAB
    assert np.array_equal(got, want)
    c = ctx.buffer(1031)
    ctx.memcpy_d2d(c.ptr, b.ptr, 1031)
    assert np.array_equal(c.download((1031,), np.uint8), want)
    b.free()
    c.free()


def test_read_sweep_reads_every_word(ctx):
    """elmh_read_sweep_dev (the benchmark's read ceiling) folds every 16-byte word of its source by XOR, one
    fold per wave: the XOR of all the folds is the XOR of all the source's 32-bit words, for sizes around
    the kernel's unrolled-loop and grid boundaries; unaligned sizes are refused."""
    nsink = E.Context.read_sweep_sink_bytes()
    sink = ctx.buffer(nsink)
    r = np.random.default_rng(11)
    for n16 in (1, 255, 2048 * 256, 2048 * 256 * 8 - 1, 2048 * 256 * 8 + 17, 3 * 2048 * 256 * 8 + 5):
        print(f"[gpu] read sweep {n16 * 16} bytes", flush=True)
        words = r.integers(0, 2 ** 32, n16 * 4, dtype=np.uint32)
        src = ctx.buffer(n16 * 16)
        src.upload(words)
        ctx.memset_dev(sink.ptr, 0, nsink)
        ctx.read_sweep_dev(src.ptr, n16 * 16, sink.ptr)
        folds = sink.download((nsink // 4,), np.uint32)
        assert np.bitwise_xor.reduce(folds) == np.bitwise_xor.reduce(words)
        src.free()
    src = ctx.buffer(64)
    with pytest.raises(E.ElmhError):
        ctx.read_sweep_dev(src.ptr, 40, sink.ptr)
    src.free()
    sink.free()


def test_rescale_ceiling_runs_every_mode(ctx):
    """elmh_rescale_ceiling_dev (the benchmark's per-block rescale ceiling) runs each mode to completion, writes
    one finite value per thread, the same on a second run, and refuses a sink too small for its grid."""
    blocks, iters = 8, 64
    sink = ctx.buffer(blocks * 1024)
    for mode in (0, 1, 2):
        print(f"[gpu] rescale ceiling mode {mode}", flush=True)
        runs = []
        for _ in range(2):
            ctx.memset_dev(sink.ptr, 0xFF, sink.nbytes)
            ctx.rescale_ceiling_dev(mode, blocks, iters, sink.ptr, sink.nbytes)
            runs.append(sink.download((blocks * 256,), np.float32))
        assert np.all(np.isfinite(runs[0])) and np.array_equal(runs[0].view(np.int32), runs[1].view(np.int32))
    with pytest.raises(E.ElmhError):
        ctx.rescale_ceiling_dev(1, blocks + 1, iters, sink.ptr, sink.nbytes)
    sink.free()


def test_argmax_step_feeds_the_next_step(ctx):
    """elmh_argmax_step_dev: the argmax into the next step's token slot, into the ring slot of the step's
    position (mod the ring length), and the device position one up, call after call."""
    r = np.random.default_rng(33)
    ring_len, V = 8, 49152
    bx, bo, bpos, bring = ctx.buffer(V * 4), ctx.buffer(4), ctx.buffer(4), ctx.buffer(ring_len * 4)
    bring.upload(np.full(ring_len, -1, np.int32))
    pos = 13
    bpos.upload(np.array([pos], np.int32))
    want = {}
    for step in range(11):
        x = r.normal(0, 1, V).astype(np.float32)
        bx.upload(x)
        print(f"[gpu] argmax step pos={pos}", flush=True)
        ctx.argmax_step_dev(bx.ptr, V, bo.ptr, bpos.ptr, bring.ptr, ring_len)
        tok = int(O.argmax(x)[0])
        assert int(bo.download((1,), np.int32)[0]) == tok
        want[pos % ring_len] = tok
        pos += 1
        assert int(bpos.download((1,), np.int32)[0]) == pos
    ring = bring.download((ring_len,), np.int32)
    for slot, tok in want.items():
        assert ring[slot] == tok
    with pytest.raises(E.ElmhError):
        ctx.argmax_step_dev(bx.ptr, V, bo.ptr, bpos.ptr, bring.ptr, 6)  # not a power of two
    with pytest.raises(E.ElmhError):
        ctx.argmax_step_dev(bx.ptr, 64 * 4096 + 1, bo.ptr, bpos.ptr, bring.ptr, ring_len)
    for b in (bx, bo, bpos, bring):
        b.free()


def test_argmax_matches_edgelm(ctx):
    """Greedy sampling on the device (argmax, tokenizer.cpp:187-189) against the oracle's
    restatement of std::max_element: ties, signed zeros, NaNs at and after index 0, and row lengths
    around the workgroup size and the SmolLM2 vocabulary."""
    from test_oracle_layer import argmax_cases
    r = np.random.default_rng(32)
    rows = argmax_cases(r) + [r.normal(0, 1, n).astype(np.float32) for n in (1023, 1024, 1025, 100003)]
    for x in rows:
        print(f"[gpu] argmax n={x.size}", flush=True)
        bx, bo = dev(ctx, x), ctx.buffer(4)
        ctx.argmax_dev(bx.ptr, 1, x.size, bo.ptr)
        assert int(bo.download((1,), np.int32)[0]) == int(O.argmax(x)[0])
        bx.free()
        bo.free()
    # one row is split into workgroup slices of up to 4096 values: ties, NaNs and maxima across slices
    x = r.normal(0, 1, 9000).astype(np.float32)
    x[[5, 4096 + 7]] = 9.0  # a tie across slices: the first wins
    y = r.normal(0, 1, 9000).astype(np.float32)
    y[4100:8192] = np.nan  # a whole slice of NaNs posts no candidate
    y[8500] = 20.0
    z = r.normal(0, 1, 12289).astype(np.float32)
    z[0] = np.nan  # NaN at index 0 stands against a larger value in a later slice
    z[12288] = 99.0
    u = r.normal(0, 1, 262144).astype(np.float32)  # 64 slices, the maximum in the last value
    u[-1] = 50.0
    for x in (x, y, z, u, r.normal(0, 1, 4097).astype(np.float32), r.normal(0, 1, 49151).astype(np.float32)):
        print(f"[gpu] argmax across slices n={x.size}", flush=True)
        bx, bo = dev(ctx, x), ctx.buffer(4)
        for _ in range(2):  # the second launch finds the counter the first one left zero
            ctx.argmax_dev(bx.ptr, 1, x.size, bo.ptr)
            assert int(bo.download((1,), np.int32)[0]) == int(O.argmax(x)[0])
        bx.free()
        bo.free()
    x = r.normal(0, 1, (6, 49152)).astype(np.float32)
    x[2, 17] = x[2].max()  # a tie with a later maximum
    print("[gpu] argmax rows=6", flush=True)
    bx, bo = dev(ctx, x), ctx.buffer(6 * 4)
    ctx.argmax_dev(bx.ptr, 6, 49152, bo.ptr)
    assert np.array_equal(bo.download((6,), np.int32), O.argmax(x))
    bx.free()
    bo.free()
