"""GPU: device images of weights (the cached repacked layout of the load path).

elmh_repack_host (the CPU) must write the bytes the device upload's repack writes, for every tile height
the layout uses (8, 16 and 32 rows) and both dtypes; a weight uploaded from that image must multiply
bit-identically; and a session of this runtime on a model with an attached device image must give
edgelm's own Session's logits bit for bit (the weights then never pass through the export layout on the
device)."""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from edgelm_amd import elmh as E
from edgelm_amd import host
from edgelm_amd import synth as S

pytestmark = pytest.mark.gpu

SHAPES = [(70, 576), (960, 576), (64, 2560), (100, 4096), (33, 8192), (40, 14336), (9, 100)]


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
def test_host_repack_equals_device_repack(ctx, dt):
    r = np.random.default_rng(40 + dt)
    for rows, cols in SHAPES:
        if dt == O.Q4 and cols % 32:
            continue
        H, _, _ = E.weight_layout(dt, rows, cols)
        print(f"[gpu] device image dt={dt} {rows}x{cols} H={H}", flush=True)
        w = O.make_weight(r.normal(0, 0.1, (rows, cols)).astype(np.float32), dt)
        dw = ctx.upload(dt, rows, cols, w.data, w.scales)
        dev, dev_s = ctx.download_image(dw)
        img, img_s = E.repack_host(dt, rows, cols, w.data, w.scales)
        assert np.array_equal(dev, img), f"{rows}x{cols}: data"
        assert np.array_equal(dev_s.view(np.uint32), img_s.view(np.uint32)), f"{rows}x{cols}: scales"
        dwi = ctx.upload_image(dt, rows, cols, img, img_s)
        x = r.normal(0, 1, (3, cols)).astype(np.float32)
        for act in (E.ACT_INT8, E.ACT_F32):
            assert bits_equal(ctx.matmul(x, [dwi], None, act=act)[0], ctx.matmul(x, [dw], None, act=act)[0])
        dw.free()
        dwi.free()


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref (edgelm's own build)")
@pytest.mark.parametrize("dt", ["q8", "q4"])
def test_session_on_attached_image_bit_identical_to_edgelm(tmp_path, dt):
    p = str(tmp_path / f"tiny.{dt}.elm")
    S.write_model(p, S.TINY, dt, seed=77, sd=0.15, embed_sd=0.5)
    img = str(tmp_path / "tiny.img")
    m = host.Model(p)
    assert m.write_device_image(img, threads=2) > 0
    assert m.attach_device_image(img)
    ids = np.random.default_rng(6).integers(0, 320, 24).astype(np.int32)
    for backends in ("hip,cpu", "hip-matmul,cpu"):
        print(f"[gpu] session on device image {dt} {backends}", flush=True)
        mine = host.Session(m, backends, threads=2, max_ctx=64, max_batch=16, all_logits=True, act_quant=True)
        ref = O.RefSession(p, "cpu", threads=2, max_ctx=64, max_batch=16, all_logits=True, act_quant=True)
        got = np.concatenate([mine.forward(ids[:16])] + [mine.forward(ids[i:i + 1]) for i in range(16, 24)])
        want = np.concatenate([ref.forward(ids[:16])] + [ref.forward(ids[i:i + 1]) for i in range(16, 24)])
        assert bits_equal(got, want)
        mine.close(), ref.close()
    m.close()
