"""GPU runs in tiles and on 8-bit images, and cancellation.

- ien_model_run_tiled (Model::run_float_tiled, realesrgan-native
  lib.rs:216-289): Real-ESRGAN with the 34-pixel margin gives the whole
  image's result bit for bit, as the reference's own GPU test requires
  (realesrgan-native tests/gpu.rs:59-73); SCUNet's tiles equal the model's
  runs on the oracle's tile regions, composed (scunet-native lib.rs:192-247),
  and a wider margin brings them closer to the whole image.
- ien_model_run_u8 (Model::run): Real-ESRGAN and SCUNet bytes equal the
  oracle's to_byte of the tiled float run (tiles of 768 / 896 with margins
  34 / 64); LaMa's equal the oracle's compositing of the float run on
  to_float / the binarised mask; BiRefNet's logits equal the float run on
  the oracle's normalisation.  Against the oracle's CPU run the bytes reach
  the reference's own 48 dB bar (tests/gpu.rs:58).
- Progress counts every tile's steps; a cancel returns IEN_ERR_CANCELLED
  after the step the callback stopped at, issues no further work (tiles
  after it are never written, the run ends early) and leaves the model
  usable.
"""

import time

import numpy as np
import pytest

import synthetic

pytestmark = pytest.mark.gpu


def psnr8(a, b):
    mse = float(np.mean((a.astype(np.float64) - b.astype(np.float64)) ** 2))
    return 10 * np.log10(255.0 ** 2 / max(mse, 1e-30))


@pytest.fixture(scope="module")
def esrgan(ctx):
    import ien

    m = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=synthetic.esrgan_tensors())
    yield m
    m.free()


@pytest.fixture(scope="module")
def scunet(ctx):
    import ien

    m = ien.Model(ctx, ien.MODEL_SCUNET, tensors=synthetic.scunet_tensors(init="fan"))
    yield m
    m.free()


@pytest.mark.parametrize("h,w,tile", [(150, 200, 64), (97, 61, 40), (64, 64, 64)])
def test_esrgan_tiles_equal_the_whole_image(esrgan, h, w, tile):
    image = synthetic.esrgan_image(h, w, seed=h * w)
    whole = esrgan.run(image)
    seen = []
    tiled = esrgan.run_tiled(image, tile, 34, progress=lambda f, u: seen.append(f) or 0)
    tiles = -(-w // tile) * -(-h // tile)
    assert len(seen) == 34 * tiles and seen == sorted(seen) and abs(seen[-1] - 1.0) < 1e-6
    assert np.array_equal(tiled.view(np.uint32), whole.view(np.uint32))


def test_scunet_tiles(esrgan, scunet, oracle):
    h, w, tile, margin = 100, 140, 64, 16
    image = synthetic.scunet_image(h, w, seed=7)
    tiled = scunet.run_tiled(image, tile, margin)
    want = np.zeros_like(tiled)
    for x0, x1, y0, y1, rx0, rx1, ry0, ry1 in oracle.tile_regions(w, h, tile, margin):
        part = scunet.run(np.ascontiguousarray(image[ry0:ry1, rx0:rx1]))
        want[y0:y1, x0:x1] = part[y0 - ry0:y1 - ry0, x0 - rx0:x1 - rx0]
    assert np.array_equal(tiled, want)
    # A random network sees the whole image, so tiles only approach it: a
    # wider margin brings them closer.
    whole = scunet.run(image)
    near = float(np.abs(scunet.run_tiled(image, tile, 48) - whole).mean())
    far = float(np.abs(scunet.run_tiled(image, tile, 0) - whole).mean())
    assert np.isfinite(tiled).all() and near < far, (near, far)


def test_tiled_refuses_other_models_and_tile_zero(ctx, esrgan):
    import ien

    with pytest.raises(ien.IenError) as e:
        esrgan.run_tiled(synthetic.esrgan_image(8, 8), 0, 34)
    assert e.value.status == ien.ERR_INPUT
    lama = ien.Model(ctx, ien.MODEL_LAMA, tensors=synthetic.lama_tensors())
    with pytest.raises(ien.IenError) as e:
        lama.run_tiled(synthetic.lama_image(16, 16), 8, 2)
    assert e.value.status == ien.ERR_INPUT
    lama.free()


def test_esrgan_u8(esrgan, oracle):
    # Wider than one 768-pixel tile: two tiles with the 34-pixel margin.
    h, w = 96, 800
    rng = np.random.default_rng(3)
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    got = esrgan.run_u8(rgb)
    assert got.shape == (4 * h, 4 * w, 3) and got.dtype == np.uint8
    floats = esrgan.run_tiled(oracle.bytes_to_floats(rgb), 768, 34)
    assert np.array_equal(got, oracle.floats_to_bytes(floats))
    cpu = oracle.realesrgan_run(synthetic.esrgan_layers(synthetic.esrgan_tensors()), oracle.bytes_to_floats(rgb))
    assert psnr8(got, oracle.floats_to_bytes(cpu)) > 48.0


def test_scunet_u8(scunet, oracle):
    # Two 896-pixel tiles side by side, margin 64.
    h, w = 64, 960
    rng = np.random.default_rng(4)
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    got = scunet.run_u8(rgb)
    assert got.shape == (h, w, 3) and got.dtype == np.uint8
    floats = scunet.run_tiled(oracle.bytes_to_floats(rgb), 896, 64)
    assert np.array_equal(got, oracle.floats_to_bytes(floats))


def test_lama_u8(ctx, oracle):
    import ien

    t = synthetic.lama_tensors()
    h, w = 72, 96
    rng = np.random.default_rng(5)
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    mask = (synthetic.lama_mask(h, w, seed=9) * rng.choice(np.array([1, 3, 255], np.uint8), (h, w))).astype(np.uint8)
    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=t)
    done = []
    got = model.run_u8(rgb, mask=mask, progress=lambda f, u: done.append(f) or 0)
    assert len(done) == 26 and abs(done[-1] - 1.0) < 1e-6
    pred = model.run(oracle.bytes_to_floats(rgb), mask=oracle.mask_bytes(mask))
    model.free()
    assert np.array_equal(got, oracle.composite_bytes(rgb, mask, pred))
    assert np.array_equal(got[mask == 0], rgb[mask == 0])
    cpu = oracle.lama_run(t, synthetic.lama_names(), oracle.bytes_to_floats(rgb), oracle.mask_bytes(mask))
    assert psnr8(got, oracle.composite_bytes(rgb, mask, cpu)) > 48.0


def test_birefnet_u8(ctx, oracle):
    import ien

    side = 128
    rng = np.random.default_rng(6)
    rgb = rng.integers(0, 256, (side, side, 3), dtype=np.uint8)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=synthetic.birefnet_tensors(init="fan"))
    got = model.run_u8(rgb)
    want = model.run(oracle.normalize_bytes(rgb))
    model.free()
    assert got.shape == (side, side) and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_u8_checks(ctx, esrgan):
    import ien

    with pytest.raises(ien.IenError) as e:
        esrgan.run_u8(np.zeros((4, 4, 3), np.uint8), mask=np.zeros((4, 4), np.uint8))
    assert e.value.status == ien.ERR_INPUT
    lama = ien.Model(ctx, ien.MODEL_LAMA, tensors=synthetic.lama_tensors())
    with pytest.raises(ien.IenError) as e:
        lama.run_u8(np.zeros((16, 16, 3), np.uint8))
    assert e.value.status == ien.ERR_INPUT
    lama.free()


def test_cancel_stops_issuing_tiles(esrgan):
    """A cancel in the first tile: the callback is not called again, the
    later tiles' output is never written, and the next run is whole."""
    import ctypes
    import ien

    h, w, tile = 64, 192, 64
    image = synthetic.esrgan_image(h, w, seed=11)
    out = np.full((4 * h, 4 * w, 3), -7.0, np.float32)
    calls = []

    def stop(done, _user):
        calls.append(done)
        return 1 if len(calls) == 5 else 0

    cb = ien.PROGRESS(stop)
    st = ien.load().ien_model_run_tiled(esrgan.h, image.ctypes.data_as(ctypes.c_void_p), w, h, tile, 34,
                                        out.ctypes.data_as(ctypes.c_void_p), ctypes.cast(cb, ctypes.c_void_p),
                                        None)
    assert st == ien.ERR_CANCELLED and len(calls) == 5
    assert (out[:, 4 * tile:] == -7.0).all()  # tiles 2 and 3 never ran
    assert np.array_equal(esrgan.run_tiled(image, tile, 34), esrgan.run(image))


def test_cancel_ends_the_run_early(ctx):
    """SCUNet at 512 x 768: cancelled after its first block, the run takes
    a fraction of a full run (the remaining 27 blocks are never issued)."""
    import ien

    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=synthetic.scunet_tensors())
    image = synthetic.scunet_image(512, 768)
    model.run(image)

    def timed(progress):
        t = []
        for _ in range(3):
            t0 = time.perf_counter()
            try:
                model.run(image, progress=progress)
            except ien.IenError as e:
                assert e.status == ien.ERR_CANCELLED
            t.append(time.perf_counter() - t0)
        return sorted(t)[1]

    full = timed(lambda f, u: 0)
    cancelled = timed(lambda f, u: 1)
    print(f"SCUNet 512x768 with progress: full {full * 1e3:.2f} ms, cancelled after block 1 {cancelled * 1e3:.2f} ms")
    assert cancelled < 0.6 * full
    first = model.run(image)
    model.free()
    assert np.isfinite(first).all()
