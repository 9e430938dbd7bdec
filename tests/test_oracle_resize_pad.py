"""Pins the oracle's resize (birefnet-native decoder.rs:436-522) against
torch's align-corners bilinear interpolation in float64, a linear ramp
(reproduced exactly) and the i0 == i1 corner rule; and the padding helpers
(scunet-native network.rs:356-379, lama-native network.rs:336-370) against
numpy's edge and symmetric padding."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F


@pytest.mark.parametrize("sh,sw,dh,dw", [(5, 7, 9, 13), (8, 8, 16, 16), (16, 16, 8, 8), (1, 5, 3, 9),
                                         (4, 4, 1, 1), (32, 32, 1024, 1024), (256, 256, 1024, 1024)])
def test_resize_matches_torch_align_corners(oracle, sh, sw, dh, dw):
    rng = np.random.default_rng(sh * 100 + dh)
    c = 3 if dh * dw > 10000 else 5
    x = rng.standard_normal((sh, sw, c)).astype(np.float32)
    want = F.interpolate(torch.from_numpy(x.astype(np.float64)).permute(2, 0, 1)[None], size=(dh, dw),
                         mode="bilinear", align_corners=True)[0].permute(1, 2, 0).numpy()
    got = oracle.resize(x, dh, dw)
    assert np.abs(got - want).max() < 2e-5 * (1 + np.abs(want).max())


def test_resize_ramp_and_corner_rule(oracle):
    """A linear ramp comes out as the ramp at the aligned coordinates, and
    the last row and column (i0 == i1, weights 0.5 and 0.5) reproduce the
    source's last row and column exactly."""
    sh, sw, dh, dw = 6, 9, 11, 17
    yy, xx = np.meshgrid(np.arange(sh), np.arange(sw), indexing="ij")
    ramp = (0.5 * yy - 0.25 * xx + 1.0).astype(np.float32)[..., None]
    got = oracle.resize(ramp, dh, dw)[..., 0]
    ty = np.arange(dh)[:, None] * (sh - 1) / (dh - 1)
    tx = np.arange(dw)[None, :] * (sw - 1) / (dw - 1)
    assert np.abs(got - (0.5 * ty - 0.25 * tx + 1.0)).max() < 1e-5
    x = np.random.default_rng(0).standard_normal((sh, sw, 2)).astype(np.float32)
    r = oracle.resize(x, dh, dw)
    assert np.array_equal(r[-1, -1], x[-1, -1]) and np.array_equal(r[0, 0], x[0, 0])


def test_resize_add(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 6, 3)).astype(np.float32)
    base = rng.standard_normal((7, 11, 3)).astype(np.float32)
    assert np.abs(oracle.resize(x, 7, 11, out=base, add=True) - (base + oracle.resize(x, 7, 11))).max() < 1e-6


@pytest.mark.parametrize("h,w,multiple", [(5, 7, 8), (64, 64, 64), (65, 3, 64), (17, 30, 8)])
def test_pad_helpers_match_numpy(oracle, h, w, multiple):
    rng = np.random.default_rng(h + w)
    img = rng.random((h, w, 3)).astype(np.float32)
    m = (rng.random((h, w)) < 0.3).astype(np.float32)
    ph, pw = -(-h // multiple) * multiple, -(-w // multiple) * multiple
    want = np.pad(img, ((0, ph - h), (0, pw - w), (0, 0)), mode="edge")
    assert np.array_equal(oracle.pad_replicate(img, multiple), want)
    if ph - h <= h and pw - w <= w:  # symmetric padding reflects at most the whole side
        masked = np.concatenate([img * (1 - m[..., None]), m[..., None]], axis=2)
        want4 = np.pad(masked, ((0, ph - h), (0, pw - w), (0, 0)), mode="symmetric")
        assert np.array_equal(oracle.masked_rows(img, m, multiple), want4)
