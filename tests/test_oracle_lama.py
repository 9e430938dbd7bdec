"""Pins of the oracle's LaMa restatement (oracle/lama.c):

- the Fourier transforms against the f64 definition on the reference's own
  test shapes (crates/lama-native/src/fourier.rs:448-484
  spectrum_matches_definition, bound 1e-5) and its inverse round trip;
- against torch.fft.rfftn / irfftn(norm="ortho") fixtures, including
  non-Hermitian spectra (only the real parts of column 0 and, for even
  widths, the last column are read) and numpy.fft on a 64 x 64 map;
- the phase products of the transposed convolutions against
  F.conv_transpose2d(stride 2, padding 1, output padding 1) + ReLU;
- the whole generator against an independent torch restatement
  (tests/lama_torch.py) on padded and unpadded sizes."""

import math

import numpy as np
import pytest

import synthetic
import lama_torch


def values(n, seed):
    # fourier.rs:442-446
    return (np.sin(np.arange(n) * 0.7 + seed) * 2.0).astype(np.float32)


@pytest.mark.parametrize("h,w,c", [(4, 6, 3), (5, 7, 2), (16, 12, 2), (9, 10, 2), (1, 8, 1)])
def test_spectrum_matches_definition(oracle, h, w, c):
    x = values(h * w * c, 0.3).reshape(h, w, c)
    s = oracle.rfft2(x)
    half = w // 2 + 1
    ky = np.arange(h)[:, None, None, None]
    k = np.arange(half)[None, :, None, None]
    y = np.arange(h)[None, None, :, None]
    xx = np.arange(w)[None, None, None, :]
    ang = -2 * math.pi * (ky * y / h + k * xx / w)
    x64 = x.astype(np.float64)
    norm = 1 / math.sqrt(h * w)
    re = np.einsum("abyx,yxc->abc", np.cos(ang), x64) * norm
    im = np.einsum("abyx,yxc->abc", np.sin(ang), x64) * norm
    assert np.abs(s[..., :c] - re).max() < 1e-5
    assert np.abs(s[..., c:] - im).max() < 1e-5
    back = np.ones_like(x)
    oracle.irfft2_add(s, back)
    assert np.abs(back - 1.0 - x).max() < 1e-5


def test_rfft_matches_torch_fixture(oracle, golden):
    got = oracle.rfft2(golden["rfft_x"])
    assert np.abs(got - golden["rfft_y"]).max() < 1e-5


@pytest.mark.parametrize("name", ["irfft_odd", "irfft_even"])
def test_irfft_matches_torch_fixture(oracle, golden, name):
    s = golden[f"{name}_s"]
    want = golden[f"{name}_y"]
    out = np.zeros(want.shape, np.float32)
    oracle.irfft2_add(s, out)
    assert np.abs(out - want).max() < 1e-5


def test_irfft_drops_imaginary_edge_columns(oracle):
    """After the column transform, the imaginary parts of column 0 and (even
    width) column w / 2 are dropped (irfftn's C2R step): a constant
    imaginary part planted down such a column lands only there and changes
    nothing; one down column 1 does."""
    rng = np.random.default_rng(3)
    h, w, c = 6, 8, 2
    s = rng.standard_normal((h, w // 2 + 1, 2 * c)).astype(np.float32)
    base = oracle.irfft2_add(s, np.zeros((h, w, c), np.float32))
    for col, same in ((0, True), (w // 2, True), (1, False)):
        t = s.copy()
        t[:, col, c:] += 5.0
        got = oracle.irfft2_add(t, np.zeros((h, w, c), np.float32))
        diff = float(np.abs(got - base).max())
        assert (diff < 1e-5) if same else (diff > 0.5), (col, diff)


def test_fourier_matches_numpy_64(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 64, 4)).astype(np.float32)
    s = oracle.rfft2(x)
    ref = np.fft.rfft2(x.astype(np.float64), axes=(0, 1), norm="ortho")
    assert np.abs(s[..., :4] - ref.real).max() < 2e-5
    assert np.abs(s[..., 4:] - ref.imag).max() < 2e-5
    sp = rng.standard_normal(s.shape).astype(np.float32)
    out = oracle.irfft2_add(sp, np.zeros_like(x))
    ref2 = np.fft.irfft2(sp[..., :4] + 1j * sp[..., 4:].astype(np.float64), s=(64, 64), axes=(0, 1),
                         norm="ortho")
    assert np.abs(out - ref2).max() < 2e-5


def phases_from_kernel(wt):
    """export_weights.py's four phase matrices of a [in, out, 3, 3] kernel."""
    out = []
    for p in range(4):
        ys, xs = lama_torch.PHASE_TAPS[p // 2], lama_torch.PHASE_TAPS[p % 2]
        out.append(np.concatenate([wt[:, :, ky, kx] for _, ky in ys for _, kx in xs]))
    return out


def test_transposed_phases_match_conv_transpose(oracle, golden):
    x, wt, b = golden["up_x"], golden["up_w"], golden["up_b"]
    got = oracle.lama_up(phases_from_kernel(wt), [b] * 4, x)
    assert got.shape == golden["up_y"].shape
    assert np.abs(got - golden["up_y"]).max() < 1e-5


def test_lama_names_match_the_weights_file():
    names = synthetic.lama_names()
    assert len(names) == 358 and len({n for n, _ in names}) == 358
    d = dict(names)
    assert d["block17.ffc1.local.weight"] == (9 * 512, 128)
    assert d["block0.ffc0.fourier.weight"] == (384, 384)
    assert d["up0.phase3.weight"] == (4 * 512, 256) and d["up2.phase0.weight"] == (128, 64)
    assert "block0.ffc0.spectral_out.bias" not in d


@pytest.mark.parametrize("h,w", [(64, 64), (44, 60)])
def test_lama_matches_torch_restatement(oracle, h, w):
    t = synthetic.lama_tensors()
    img = synthetic.lama_image(h, w, seed=h + w)
    mask = synthetic.lama_mask(h, w, seed=h * w)
    want = lama_torch.run(t, img, mask)
    got = oracle.lama_run(t, synthetic.lama_names(), img, mask)
    assert got.shape == (h, w, 3)
    # Not saturated: the comparison sees the network, not a clamp.
    assert 0.05 < float(want.std()) and float(want.min()) > 1e-4 and float(want.max()) < 1 - 1e-4
    assert np.abs(got - want).max() < 2e-4
