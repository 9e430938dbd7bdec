"""Pins of the oracle's 8-bit image I/O and tiling (oracle/io.c): the
models' to_float / to_byte (realesrgan-native lib.rs:292-300), BiRefNet's
normalisation table (birefnet-native lib.rs:111-116), LaMa's mask and
compositing (lama-native lib.rs:138-155) and the tile grid of
run_float_tiled (realesrgan-native lib.rs:251-265)."""

import numpy as np
import pytest


def test_to_float_every_byte(oracle):
    b = np.arange(256, dtype=np.uint8)
    got = oracle.bytes_to_floats(b)
    want = b.astype(np.float32) / np.float32(255.0)  # IEEE f32 division
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0] == 0.0 and got[255] == 1.0


def test_to_byte_known_answers(oracle):
    cases = {
        0.0: 0, 1.0: 255, -0.0: 0, -1.0: 0, 2.0: 255, float("inf"): 255, float("-inf"): 0,
        float("nan"): 0,
        # 0.5 * 255 = 127.5: ties go away from zero (Rust's round), not to even.
        0.5: 128,
        # 1.5 / 255 rounds in f32 to a value whose product with 255 is 1.5 or
        # just above or below it: the f64 definition decides.
    }
    x = np.array(list(cases), np.float32)
    got = oracle.floats_to_bytes(x)
    assert list(got) == list(cases.values())


def test_to_byte_inverts_to_float(oracle):
    b = np.arange(256, dtype=np.uint8)
    assert np.array_equal(oracle.floats_to_bytes(oracle.bytes_to_floats(b)), b)


def test_to_byte_against_f64_definition(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-0.2, 1.2, 100000),
                        (np.arange(512) + 0.5) / 255.0,  # ties and their neighbours
                        np.nextafter((np.arange(512) + 0.5) / 255.0, 0)]).astype(np.float32)
    got = oracle.floats_to_bytes(x)
    c = np.clip(x, np.float32(0), np.float32(1))
    prod = (c * np.float32(255.0)).astype(np.float32)  # the f32 product
    want = np.floor(prod.astype(np.float64) + 0.5)  # ties away from zero (prod >= 0)
    assert np.array_equal(got, want.astype(np.uint8))


def test_normalize_against_f64(oracle):
    mean = np.array([0.485, 0.456, 0.406])
    std = np.array([0.229, 0.224, 0.225])
    rgb = np.stack(np.meshgrid(np.arange(256), np.arange(256), np.arange(256), indexing="ij"),
                   -1).reshape(-1, 3)[::97].astype(np.uint8)
    got = oracle.normalize_bytes(rgb)
    want = (rgb / 255.0 - mean) / std
    # Three f32 roundings (division, subtraction, division) of values up to 2.7.
    assert np.abs(got - want).max() <= 4e-7 * 4
    # The f32 steps exactly as the table computes them.
    m32, s32 = mean.astype(np.float32), std.astype(np.float32)
    exact = ((rgb.astype(np.float32) / np.float32(255.0)) - m32) / s32
    assert np.array_equal(got.view(np.uint32), exact.astype(np.float32).view(np.uint32))


def test_mask_and_composite_brute_force(oracle):
    rng = np.random.default_rng(1)
    h, w = 13, 17
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    mask = rng.choice(np.array([0, 0, 1, 7, 255], np.uint8), (h, w))
    pred = rng.uniform(-0.1, 1.1, (h, w, 3)).astype(np.float32)
    holes = oracle.mask_bytes(mask)
    assert set(np.unique(holes)) <= {0.0, 1.0} and np.array_equal(holes != 0, mask != 0)
    got = oracle.composite_bytes(rgb, mask, pred)
    for y in range(h):
        for x in range(w):
            for c in range(3):
                want = oracle.lib().or_to_byte(float(pred[y, x, c])) if mask[y, x] else rgb[y, x, c]
                assert got[y, x, c] == want


@pytest.mark.parametrize("width,height,tile,margin", [
    (150, 100, 64, 34), (64, 64, 64, 34), (768, 512, 768, 34), (1000, 129, 896, 64), (7, 300, 4, 0),
    (1, 1, 1, 5)])
def test_tile_regions_partition_the_image(oracle, width, height, tile, margin):
    r = oracle.tile_regions(width, height, tile, margin)
    cols, rows = -(-width // tile), -(-height // tile)
    assert len(r) == cols * rows
    cover = np.zeros((height, width), np.int32)
    for x0, x1, y0, y1, rx0, rx1, ry0, ry1 in r:
        assert x1 - x0 <= tile and y1 - y0 <= tile and x1 > x0 and y1 > y0
        cover[y0:y1, x0:x1] += 1
        assert rx0 == max(0, x0 - margin) and ry0 == max(0, y0 - margin)
        assert rx1 == min(width, x1 + margin) and ry1 == min(height, y1 + margin)
    assert (cover == 1).all()  # every pixel in exactly one tile
    # Equal tiles: sides differ by at most one pixel.
    ws = r[:, 1] - r[:, 0]
    hs = r[:, 3] - r[:, 2]
    assert ws.max() - ws.min() <= 1 and hs.max() - hs.min() <= 1
