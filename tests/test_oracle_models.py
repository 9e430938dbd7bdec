"""Pins the oracle's window attention (crates/native-engine/src/
attention.rs), Real-ESRGAN network (crates/realesrgan-native/src/
network.rs) and depthwise convolution against f64 definitions and torch
fixtures (tests/golden/make_golden.py)."""

import numpy as np
import pytest

import synthetic
from conftest import ROOT

GOLDEN = np.load(ROOT / "tests" / "golden" / "golden.npz")


@pytest.mark.parametrize("tokens", [49, 64, 144])
def test_attention_golden(oracle, tokens):
    qkv, bias, want = GOLDEN[f"attn{tokens}_qkv"], GOLDEN[f"attn{tokens}_bias"], GOLDEN[f"attn{tokens}_y"]
    got = oracle.attention(qkv, 64, 1, bias)[:, 32:64]
    assert np.abs(got - want).max() < 1e-5


def test_attention_definition_all_heads(oracle):
    """attention.rs:215-247: f64 softmax attention with -100-masked biases."""
    rng = np.random.default_rng(5)
    tokens, c = 49, 96
    qkv = rng.standard_normal((tokens, 3 * c)).astype(np.float32)
    bias = rng.standard_normal((tokens, tokens)).astype(np.float32)
    bias[rng.random((tokens, tokens)) < 0.3] = -100
    got = np.zeros((tokens, c), np.float32)
    for head in range(c // 32):
        got += oracle.attention(qkv, c, head, bias)
    for head in range(c // 32):
        q = qkv[:, head * 32:head * 32 + 32].astype(np.float64) / np.sqrt(32)
        k = qkv[:, c + head * 32:c + head * 32 + 32].astype(np.float64)
        v = qkv[:, 2 * c + head * 32:2 * c + head * 32 + 32].astype(np.float64)
        s = q @ k.T + bias
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.abs(got[:, head * 32:head * 32 + 32] - p @ v).max() < 1e-5


def test_pixel_shuffle_golden(oracle):
    got = oracle.pixel_shuffle_add(GOLDEN["shuffle_last"].reshape(-1, 48), GOLDEN["shuffle_img"])
    assert np.abs(got - GOLDEN["shuffle_y"]).max() < 1e-6


def test_pixel_shuffle_index_map(oracle):
    """network.rs:115-141: channel 16c + 4i + j of pixel (y, x) goes to
    output pixel (4y + i, 4x + j), channel c -- exactly."""
    h, w = 3, 4
    last = np.arange(h * w * 48, dtype=np.float32).reshape(h * w, 48)
    img = np.zeros((h, w, 3), np.float32)
    got = oracle.pixel_shuffle_add(last, img)
    for y in range(h):
        for x in range(w):
            for i in range(4):
                for j in range(4):
                    for c in range(3):
                        assert got[4 * y + i, 4 * x + j, c] == last[y * w + x, 16 * c + 4 * i + j]


def test_realesrgan_golden(oracle):
    """The whole network (Winograd F(4x4) layers, PReLU, shuffle) against an
    independent torch float64 composition of SRVGGNetCompact; the bound is
    the reference's own CPU-vs-PyTorch one (tests/reference.rs:61-79)."""
    tensors = synthetic.esrgan_tensors()
    got = oracle.realesrgan_run(synthetic.esrgan_layers(tensors), GOLDEN["esrgan_img"], threads=4)
    assert np.abs(got - GOLDEN["esrgan_y"]).max() < 5e-4


def test_depthwise_golden(oracle):
    got = oracle.depthwise(GOLDEN["dw_x"], GOLDEN["dw_w"], GOLDEN["dw_b"], threads=3)
    assert np.abs(got - GOLDEN["dw_y"]).max() < 1e-5
