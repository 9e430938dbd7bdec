"""Pins the oracle's Swin window logic (crates/scunet-native/src/swin.rs,
crates/birefnet-native/src/swin.rs, tools/scunet/export_weights.py):
position-bias gathers decoded from self-describing tables, shift-mask
classes against the standard region mask of a rolled map, window gathers
against torch.roll + window partition, and whole blocks against an
independent torch float64 formulation (tests/golden/make_golden.py)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import ROOT

GOLDEN = np.load(ROOT / "tests" / "golden" / "golden.npz")


@pytest.mark.parametrize("window", [7, 8, 12])
def test_position_bias_decodes_offsets(oracle, window):
    """Tables whose entries name their own cell: the gather must return, for
    tokens (yi, xi), (yj, xj), the cell (yi - yj + W - 1, xi - xj + W - 1) of
    the token pair's head, in both table layouts (a swapped axis, a sign or an
    index slip shows up as a wrong decode)."""
    heads, side, n = 3, 2 * window - 1, window * window
    h, a, b = np.meshgrid(np.arange(heads), np.arange(side), np.arange(side), indexing="ij")
    code = (h * 10000 + a * 100 + b).astype(np.float32)  # [heads][2W-1][2W-1]
    swin = code.reshape(heads, side * side).T.copy()      # [(2W-1)^2][heads]
    yi, xi = np.divmod(np.arange(n), window)
    want = (np.arange(heads)[:, None, None] * 10000 + (yi[:, None] - yi[None, :] + window - 1) * 100
            + (xi[:, None] - xi[None, :] + window - 1)).astype(np.float32)
    assert np.array_equal(oracle.position_bias(code, heads, window, oracle.POS_SCUNET), want)
    assert np.array_equal(oracle.position_bias(swin, heads, window, oracle.POS_SWIN), want)


def standard_region_mask(ph, pw, window, shift):
    """The region ids of a rolled map's windows, as the Swin implementations
    build them (three slices per axis), [windows][N]."""
    img = np.zeros((ph, pw), np.int64)
    cnt = 0
    for hs in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
        for ws in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
            img[hs, ws] = cnt
            cnt += 1
    return img.reshape(ph // window, window, pw // window, window).transpose(0, 2, 1, 3).reshape(-1, window * window)


@pytest.mark.parametrize("window,shift,masked,h,w", [(8, 4, -np.inf, 24, 32), (12, 6, -100.0, 36, 24)])
def test_bias_tables_match_the_standard_shift_mask(oracle, window, shift, masked, h, w):
    """For window = 2 shift (SCUNet 8/4, the configuration's BiRefNet 12/6)
    the class tables must mask exactly the token pairs of different regions
    of the standard mask, window by window."""
    heads, n = 2, window * window
    pos = np.random.default_rng(1).standard_normal((heads, n, n)).astype(np.float32)
    tables = oracle.bias_tables(pos, window, shift, masked)
    assert tables.shape == (4, heads, n, n)
    regions = standard_region_mask(h, w, window, shift)
    for win in range(regions.shape[0]):
        cls = oracle.window_class(win, window, shift, h, w)
        diff = regions[win][:, None] != regions[win][None, :]
        want = pos + np.where(diff, np.float32(masked), np.float32(0))[None]
        assert np.array_equal(tables[cls], want), (win, cls)


def test_bias_tables_unshifted_and_window7(oracle):
    """Unshifted: the position bias alone.  Window 7 / shift 3 (the
    reference's BiRefNet): the reference splits a last window's rows (and
    columns) in two, the first four and the last three (swin.rs:28-30).
    (The standard three-slice mask would also separate the first row from
    the next three; this is where the reference departs from it.)"""
    heads, n = 1, 49
    pos = np.zeros((heads, n, n), np.float32)
    assert np.array_equal(oracle.bias_tables(pos, 7, 0, -100.0), pos[None])
    t = oracle.bias_tables(pos, 7, 3, -100.0)
    y, x = np.divmod(np.arange(n), 7)
    for cls in range(4):
        ry = (y >= 4) if cls & 2 else np.zeros(n, bool)
        rx = (x >= 4) if cls & 1 else np.zeros(n, bool)
        rid = 2 * ry + rx
        want = np.where(rid[:, None] != rid[None, :], -100.0, 0.0).astype(np.float32)
        assert np.array_equal(t[cls, 0], want)


@pytest.mark.parametrize("window,shift,h,w", [(8, 4, 16, 24), (8, 0, 16, 16), (7, 3, 10, 10), (12, 6, 15, 13)])
def test_window_gather_is_roll_then_partition(oracle, window, shift, h, w):
    """Token i of window w is element (w, i) of the map padded to whole
    windows, rolled by -shift and partitioned (padding: -1)."""
    ph, pw = -(-h // window) * window, -(-w // window) * window
    idx = torch.full((ph, pw), -1, dtype=torch.int64)
    idx[:h, :w] = torch.arange(h * w).reshape(h, w)
    if shift:
        idx = torch.roll(idx, shifts=(-shift, -shift), dims=(0, 1))
    want = idx.reshape(ph // window, window, pw // window, window).permute(0, 2, 1, 3).reshape(-1, window * window)
    for win in range(want.shape[0]):
        got = [oracle.window_source(win, i, window, shift, h, w) for i in range(window * window)]
        assert got == want[win].tolist()
    classes = [oracle.window_class(win, window, shift, h, w) for win in range(want.shape[0])]
    wx, wy = pw // window, ph // window
    expect = [0 if not shift else int(k % wx == wx - 1) + 2 * int(k // wx == wy - 1) for k in range(wx * wy)]
    assert classes == expect


@pytest.mark.parametrize("name,window,shift,masked", [("swin_w8s4", 8, 4, -np.inf), ("swin_w8s0", 8, 0, -np.inf),
                                                      ("swin_w12s6", 12, 6, -100.0)])
def test_swin_attend_golden(oracle, name, window, shift, masked):
    g = {k: GOLDEN[f"{name}_{k}"] for k in ("x", "g", "b", "wqkv", "bqkv", "pos", "wproj", "bproj", "y")}
    tables = oracle.bias_tables(g["pos"], window, shift, masked)
    got = oracle.swin_attend(g["x"], window, shift, g["g"], g["b"], g["wqkv"], g["bqkv"], tables, g["wproj"],
                             g["bproj"])
    err = np.abs(got - g["y"])
    assert err.max() < 2e-4 * (1 + np.abs(g["y"]).max()), err.max()


def test_swin_mlp_golden(oracle):
    g = {k: GOLDEN[f"mlp_{k}"] for k in ("x", "g", "b", "w1", "b1", "w2", "b2", "y")}
    got = oracle.swin_mlp(g["x"], g["g"], g["b"], g["w1"], g["b1"], g["w2"], g["b2"])
    assert np.abs(got - g["y"]).max() < 2e-4 * (1 + np.abs(g["y"]).max())
