"""CPU: the device image of a model (the cached repacked layout of the load path).

elmh_repack_host (libelmh, host code) must give the layout the device upload builds; here it is checked
against an independent numpy statement of that layout (item (n, b) at ((n // H) * nb + b) * H + n % H,
q8 rows zero-padded past K and past the last row, q4 padding rows 0x88 with scale 0). The device side is
checked in tests/test_gpu_device_image.py. Model.write_device_image / attach_device_image must take the
image of the same weights and refuse one written for other weights, a truncated file or a missing one,
without touching the model."""
import numpy as np
import pytest

import oracle as O
from edgelm_amd import elmh as E
from edgelm_amd import host
from edgelm_amd import synth as S


def numpy_repack(w):
    H, db, sb = E.weight_layout(w.dtype, w.rows, w.cols)
    nb = (w.cols + 31) // 32
    rows_pad = (w.rows + 63) // 64 * 64
    G = 32 if w.dtype == O.Q8 else 16
    out = np.zeros((rows_pad * nb, G), np.uint8)
    n = np.arange(rows_pad)[:, None]
    b = np.arange(nb)[None, :]
    dst = ((n // H) * nb + b) * H + n % H  # [rows_pad][nb]
    if w.dtype == O.Q8:
        raw = np.zeros((rows_pad, nb * 32), np.uint8)
        raw[:w.rows, :w.cols] = w.data.reshape(w.rows, w.cols).view(np.uint8)
        out[dst.ravel()] = raw.reshape(rows_pad * nb, 32)
        sc = np.zeros(rows_pad, np.float32)
        sc[:w.rows] = w.scales
    else:
        raw = np.full((rows_pad, nb * 16), 0x88, np.uint8)
        raw[:w.rows] = w.data.reshape(w.rows, w.cols // 2)
        out[dst.ravel()] = raw.reshape(rows_pad * nb, 16)
        sc = np.zeros(rows_pad * nb, np.float32)
        src = np.zeros((rows_pad, nb), np.float32)
        src[:w.rows] = w.scales.reshape(w.rows, nb)
        sc[dst.ravel()] = src.ravel()
    assert out.nbytes == db and sc.nbytes == sb
    return out.ravel(), sc


@pytest.mark.parametrize("dt", [O.Q8, O.Q4])
@pytest.mark.parametrize("rows,cols", [(1, 32), (65, 96), (200, 576), (70, 4096), (9, 14336)])
def test_repack_host_matches_the_layout(dt, rows, cols):
    r = np.random.default_rng(rows * 7 + cols + dt)
    w = O.make_weight(r.normal(0, 0.1, (rows, cols)).astype(np.float32), dt)
    got, got_s = E.repack_host(dt, rows, cols, w.data, w.scales)
    want, want_s = numpy_repack(w)
    assert np.array_equal(got, want)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


def test_repack_host_q8_ragged_rows_and_cols():
    r = np.random.default_rng(3)
    w = O.make_weight(r.normal(0, 0.1, (37, 100)).astype(np.float32), O.Q8)  # K not a multiple of 32
    got, got_s = E.repack_host(O.Q8, 37, 100, w.data, w.scales)
    want, want_s = numpy_repack(w)
    assert np.array_equal(got, want) and np.array_equal(got_s, want_s)


def test_repack_host_rejects_bad_shapes():
    with pytest.raises(E.ElmhError):
        E.weight_layout(O.Q4, 8, 48)  # q4 needs K % 32 == 0
    with pytest.raises(E.ElmhError):
        E.weight_layout(0, 8, 64)  # f32 is not uploaded


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("device_image")
    paths = {}
    for name, seed in (("a", 11), ("b", 12)):
        p = str(d / f"tiny_{name}.q4.elm")
        S.write_model(p, S.TINY, "q4", embed_dtype="q8", seed=seed, sd=0.1, embed_sd=0.5)
        paths[name] = p
    return d, paths


def test_write_and_attach(models):
    d, paths = models
    m = host.Model(paths["a"])
    img = str(d / "a.img")
    n = m.write_device_image(img, threads=3)
    # q/k/v/o/gate/up/down per layer and the embedding (the tiny model ties its LM head to it)
    assert n == 7 * S.TINY["n_layers"] + (1 if S.TINY["tied"] else 2)
    assert m.attach_device_image(img)
    # the same file again, from a fresh load of the same model, with a different thread count
    m2 = host.Model(paths["a"])
    img2 = str(d / "a2.img")
    m2.write_device_image(img2, threads=1)
    with open(img, "rb") as f1, open(img2, "rb") as f2:
        assert f1.read() == f2.read()
    assert m2.attach_device_image(img)
    m.close(), m2.close()


def test_attach_refuses_other_weights_and_broken_files(models):
    d, paths = models
    img = str(d / "a3.img")
    host.Model(paths["a"]).write_device_image(img)
    other = host.Model(paths["b"])
    assert not other.attach_device_image(img)             # written for other weights
    assert not other.attach_device_image(str(d / "none"))  # missing
    cut = str(d / "cut.img")
    with open(img, "rb") as f:
        data = f.read()
    with open(cut, "wb") as f:
        f.write(data[: len(data) // 2])
    m = host.Model(paths["a"])
    assert not m.attach_device_image(cut)                  # truncated
    bad = str(d / "bad.img")
    with open(bad, "wb") as f:
        f.write(b"XXXXXXXX" + data[8:])
    assert not m.attach_device_image(bad)                  # not an image
    assert m.attach_device_image(img)
    other.close(), m.close()


@pytest.mark.parametrize("offset,bit", [(100, 0x80), (1031, 0x01), (3000, 0x10)])
def test_attach_refuses_a_one_byte_edit_anywhere(models, offset, bit):
    """A model re-exported to the same path with one weight byte changed (away from any 64-byte sample the
    digest once took, in a high or a low bit of its word) must not attach the image of the old weights."""
    d, paths = models
    img = str(d / f"edit{offset}.img")
    host.Model(paths["a"]).write_device_image(img)
    m = host.Model(paths["a"])
    _, data, _ = m.weight("model.layers.0.mlp.down_proj.weight")
    m.close()
    with open(paths["a"], "rb") as f:
        blob = bytearray(f.read())
    raw = data.view(np.uint8).ravel()
    assert raw.size > offset + 64
    at = blob.find(bytes(raw[:256]))
    assert at > 0 and blob.find(bytes(raw[:256]), at + 1) < 0  # the weight's bytes sit once in the file
    edited = str(d / f"edit{offset}.elm")
    blob[at + offset] ^= bit
    with open(edited, "wb") as f:
        f.write(blob)
    e = host.Model(edited)
    assert not e.attach_device_image(img)
    assert e.weight("model.layers.0.mlp.down_proj.weight")[1].view(np.uint8).ravel()[offset] == raw[offset] ^ bit
    e.close()
    same = host.Model(paths["a"])
    assert same.attach_device_image(img)
    same.close()
