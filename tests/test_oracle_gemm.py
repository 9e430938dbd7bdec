"""Pins the oracle's product (crates/native-engine/src/gemm.rs multiply):
dense rows, accumulate over row ranges, convolution taps with zero and
reflect padding, strides and transposed-convolution phase offsets -- against
f64 brute force (the reference's own oracle pattern, gemm.rs:680-700) and
torch conv2d / conv_transpose2d fixtures."""

import math

import numpy as np
import pytest

from conftest import ROOT

GOLDEN = np.load(ROOT / "tests" / "golden" / "golden.npz")


def values(n, seed):
    """gemm.rs:674-678: sin-based test values."""
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37) + np.float32(seed)) * 0.5).astype(np.float32)


def close(got, want, tol=1e-4):
    assert np.all(np.abs(got - want) <= tol * (1 + np.abs(want))), np.abs(got - want).max()


@pytest.mark.parametrize("m,k,n", [(1, 3, 1), (7, 40, 17), (13, 1100, 48), (6, 512, 16)])
def test_dense_rows_match_reference(oracle, m, k, n):
    a = values(m * k, 0.3).reshape(m, k)
    w = values(k * n, 1.1).reshape(k, n)
    b = values(n, 2.0)
    got = oracle.multiply_rows(a, w, b)
    close(got, a.astype(np.float64) @ w.astype(np.float64) + b)


def test_row_ranges_accumulate_onto_output(oracle):
    from oracle import oracle as O
    import ctypes

    m, k, n = 20, 70, 33
    a = values(m * k, 0.7).reshape(m, k)
    w = values(k * n, -0.4).reshape(k, n)
    out = np.ones((m, n), np.float32)
    inp = O._rows_input(a, k)
    for r0, r1 in [(0, 5), (5, 17), (17, 20)]:
        part = np.ascontiguousarray(out[r0:r1])
        O.lib().or_multiply(ctypes.byref(inp), r0, r1 - r0, O._p(w), k, n, None, O._p(part), n, O.ACT_NONE, 1)
        out[r0:r1] = part
    close(out, a.astype(np.float64) @ w + 1.0)


def brute_conv(x, w, b, size, step=1, pad="zero", gap=0):
    h, wd, c = x.shape
    n = w.shape[1]
    half = size // 2
    oh, ow = (h - 1) // step + 1, (wd - 1) // step + 1
    out = np.zeros((oh, ow, n))
    for oy in range(oh):
        for ox in range(ow):
            s = b.astype(np.float64).copy()
            for t in range(size * size):
                y, xx = oy * step + t // size - half, ox * step + t % size - half
                if not (0 <= y < h and 0 <= xx < wd):
                    if pad == "zero":
                        continue
                    y = min(abs(y), 2 * (h - 1) - y)
                    xx = min(abs(xx), 2 * (wd - 1) - xx)
                s += x[y, xx].astype(np.float64) @ w[t * c:(t + 1) * c].astype(np.float64)
            out[oy, ox] = s
    return out


@pytest.mark.parametrize("h,w,c,size,n", [(5, 7, 3, 3, 20), (4, 9, 64, 7, 16), (3, 3, 600, 3, 5), (6, 5, 2, 1, 3),
                                          (5, 6, 32, 3, 32)])
def test_same_convolution_matches_brute_force(oracle, h, w, c, size, n):
    """gemm.rs:881-926, with ReLU."""
    x = values(h * w * c, 0.9).reshape(h, w, c)
    wt = values(size * size * c * n, 0.2).reshape(-1, n)
    b = values(n, -1.0)
    got = oracle.multiply_conv(x, wt, b, size=size, act=oracle.ACT_RELU)
    close(got, np.maximum(brute_conv(x, wt, b, size), 0))


@pytest.mark.parametrize("name,size,step,pad", [("conv_3x3_zero", 3, 1, 0), ("conv_7x7_zero", 7, 1, 0),
                                                ("conv_1x1", 1, 1, 0), ("conv_3x3_reflect", 3, 1, 1),
                                                ("conv_3x3_s2_reflect", 3, 2, 1), ("conv_7x7_reflect", 7, 1, 1)])
def test_convolution_golden(oracle, name, size, step, pad):
    g = lambda s: GOLDEN[f"{name}_{s}"]
    got = oracle.multiply_conv(g("x"), g("w"), g("b"), size=size, step=step, pad=pad)
    close(got, g("y"), 1e-5)


def test_reflect_matches_brute_force(oracle):
    x = values(6 * 7 * 5, 0.1).reshape(6, 7, 5)
    wt = values(9 * 5 * 4, 0.5).reshape(45, 4)
    b = values(4, 0.2)
    close(oracle.multiply_conv(x, wt, b, size=3, step=2, pad=oracle.PAD_REFLECT), brute_conv(x, wt, b, 3, 2, "reflect"))


def phase_weights(wt, py, px):
    """One output phase of a stride-2, padding-1, output-padding-1 3x3
    transposed convolution as offset taps: along each axis an even output
    reads kernel tap 1 at offset 0; an odd one reads tap 2 at offset 0 and
    tap 0 at offset 1 (lama-native network.rs:268-271)."""
    axis = {0: [(0, 1)], 1: [(0, 2), (1, 0)]}
    offsets, rows = [], []
    for dy, ky in axis[py]:
        for dx, kx in axis[px]:
            offsets.append((dy, dx))
            rows.append(wt[:, :, ky, kx])  # cin x cout
    return offsets, np.concatenate(rows, 0)


def test_transposed_phases_golden(oracle):
    """Taps::Offsets (gemm.rs:281-285) assembling a transposed convolution,
    against torch conv_transpose2d."""
    x, wt, b, want = GOLDEN["convT_x"], GOLDEN["convT_w"], GOLDEN["convT_b"], GOLDEN["convT_y"]
    h, w, _ = x.shape
    got = np.zeros((2 * h, 2 * w, wt.shape[1]), np.float32)
    for py in (0, 1):
        for px in (0, 1):
            offsets, mat = phase_weights(wt, py, px)
            got[py::2, px::2] = oracle.multiply_conv(x, mat, b, offsets=offsets)
    close(got, want, 1e-5)


def test_gelu_act_and_threads_bit_exact(oracle):
    x = values(9 * 11 * 16, 0.4).reshape(9, 11, 16)
    wt = values(9 * 16 * 24, 0.8).reshape(-1, 24)
    one = oracle.multiply_conv(x, wt, None, act=oracle.ACT_GELU, threads=1)
    many = oracle.multiply_conv(x, wt, None, act=oracle.ACT_GELU, threads=5)
    assert np.array_equal(one, many)
    close(one, oracle.gelu(brute_conv(x, wt, np.zeros(24, np.float32), 3).astype(np.float32)), 1e-5)
