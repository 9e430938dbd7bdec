"""Pins of the oracle's BiRefNet restatement (oracle/birefnet.c) against an
independent torch restatement (tests/birefnet_torch.py): timm-style shifted
windows with padding and the three-slice shift mask, patch merging by
strided slices, the decoder with F.conv2d / F.interpolate, the deformable
ASPP sampling through F.grid_sample, and the full-resolution branch as its
two convolutions (the oracle composes them into a 5x5 inside the edge
ring, as decoder.rs:594-757 does)."""

import numpy as np
import pytest

import synthetic
import birefnet_torch


@pytest.mark.parametrize("window,side,init,offsets,bound", [
    (12, 64, "fan", 0.0, 1e-4),           # the configured window, heavy padding
    (12, 128, "fan", 0.0, 1e-4),
    (12, 64, "trunc_normal", 0.0, 1e-4),  # the configured init
    (7, 64, "fan", 0.0, 1e-4),            # the reference's window
    (7, 64, "fan", 0.3, 1e-3),            # deformable sampling at random offsets
])
def test_birefnet_matches_torch_restatement(oracle, window, side, init, offsets, bound):
    t = synthetic.birefnet_tensors(window=window, init=init, offsets=offsets)
    img = synthetic.birefnet_image(side, seed=side + window)
    want = birefnet_torch.run(t, img, window)
    got = oracle.birefnet_run(t, synthetic.birefnet_names(window), img, window)
    assert got.shape == (side, side)
    assert float(np.abs(want).std()) > 0.1
    assert np.abs(got - want).max() < bound * max(1.0, float(np.abs(want).max()))


def test_birefnet_names_match_the_weights_file():
    names = synthetic.birefnet_names(7)
    d = dict(names)
    assert len(names) == len(d)
    assert d["stage2.block5.position_bias"] == (12, 49, 49)
    assert d["squeeze.conv_in.weight"] == (9 * 2880, 64)
    assert d["block4.gdt.weight"] == (9 * 768, 16) and "block1.gdt.weight" not in d
    assert d["block1.aspp.branch3.offset.weight"] == (49 * 64, 147)
    assert d["patches5.conv1.weight"] == (9 * 3072, 64)
    assert d["stage2.merge.weight"] == (1536, 768) and "stage3.merge.weight" not in d
    assert dict(synthetic.birefnet_names(12))["stage0.block0.position_bias"] == (3, 144, 144)


def test_birefnet_rejects_bad_sides(oracle):
    t = synthetic.birefnet_tensors()
    with pytest.raises(RuntimeError):
        oracle.birefnet_run(t, synthetic.birefnet_names(), np.zeros((96, 96, 3), np.float32), 12)
