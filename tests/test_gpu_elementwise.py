"""GPU parity of the memory-bound passes against the oracle: half
conversions and the pixel-shuffle index map bit for bit; LayerNorm, GELU,
sigmoid and the depthwise convolution to f16 storage accuracy."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_half_conversions_bit_exact(ctx, oracle):
    import torch
    import ien

    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    x[np.isnan(x)] = 0.0  # NaN payloads are not part of the contract
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504.0, 65520.0, 6e-8, 3e-8, 2.98e-8, 1e-30])])
    xt = torch.from_numpy(x).cuda()
    h = torch.empty(x.size, dtype=torch.int16, device="cuda")
    ien.floats_to_halves(ctx, xt, h)
    allh = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).cuda()
    back = torch.empty(65536, dtype=torch.float32, device="cuda")
    ien.halves_to_floats(ctx, allh, back)
    torch.cuda.synchronize()
    got = h.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.f32_to_half(x))
    want = oracle.half_to_f32(np.arange(65536, dtype=np.uint16))
    g = back.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(g), nan) and np.array_equal(g[~nan].view(np.uint32), want[~nan].view(np.uint32))


# Last-layer strides of 64, 48 (the network's) and 50 halves; a 1 x 1 image.
@pytest.mark.parametrize("h,w,stride", [(3, 5, 64), (64, 96, 64), (256, 384, 48), (1, 1, 48),
                                        (7, 33, 50)])
def test_pixel_shuffle_add_bit_exact(ctx, oracle, h, w, stride):
    import torch
    import ien

    rng = np.random.default_rng(h)
    last = rng.standard_normal((h * w, stride)).astype(np.float16)
    image = rng.random((h, w, 3), dtype=np.float32)
    want = oracle.pixel_shuffle_add(last[:, :48].astype(np.float32), image)
    out = torch.empty((4 * h, 4 * w, 3), dtype=torch.float32, device="cuda")
    ien.pixel_shuffle_add(ctx, torch.from_numpy(last).cuda(), stride, torch.from_numpy(image).cuda(), w, h, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("rows,c", [(1, 32), (77, 96), (300, 768), (5, 3072), (9, 37), (40, 8),
                                    (33, 1536), (7, 2048), (130, 2304), (1000, 96), (64, 384),
                                    (11, 24), (13, 48), (17, 56), (21, 192), (19, 160)])
def test_layer_norm(ctx, oracle, rows, c):
    import torch
    import ien

    rng = np.random.default_rng(c)
    x = (rng.standard_normal((rows, c)) * 3 + 1).astype(np.float16)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    want = oracle.layer_norm(x.astype(np.float32), gamma, beta).reshape(rows, c)
    xt = torch.from_numpy(x).cuda()
    ien.layer_norm(ctx, xt, rows, c, c, torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    got = xt.float().cpu().numpy()
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max() + 2e-3


def test_layer_norm_strided_columns(ctx, oracle):
    """Columns 0..c of rows `stride` apart: normalised in place, the others
    untouched (the level maps of the BiRefNet decoder)."""
    import torch
    import ien

    rows, c, stride = 50, 192, 384
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((rows, stride)) * 2).astype(np.float16)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    want = oracle.layer_norm(x[:, :c].astype(np.float32), gamma, beta).reshape(rows, c)
    xt = torch.from_numpy(x).cuda()
    ien.layer_norm(ctx, xt, rows, c, stride, torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    got = xt.float().cpu().numpy()
    assert np.abs(got[:, :c] - want).max() <= 2e-3 * np.abs(want).max() + 2e-3
    assert np.array_equal(got[:, c:], x[:, c:].astype(np.float32))


def test_gelu_sigmoid(ctx, oracle):
    import torch
    import ien

    x = np.linspace(-10, 10, 4001).astype(np.float16)
    for fn, ref in ((ien.gelu, oracle.gelu), (ien.sigmoid, oracle.sigmoid)):
        xt = torch.from_numpy(x.copy()).cuda()
        fn(ctx, xt)
        torch.cuda.synchronize()
        want = ref(x.astype(np.float32))
        got = xt.float().cpu().numpy()
        assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max() + 1e-3


@pytest.mark.parametrize("layout,size,h,w,c", [(1, 7, 128, 128, 192), (1, 7, 30, 50, 5), (1, 3, 33, 20, 4),
                                               (0, 7, 17, 23, 24), (0, 5, 9, 11, 3)])
def test_depthwise(ctx, oracle, layout, size, h, w, c):
    import torch
    import ien

    rng = np.random.default_rng(size * c)
    x = rng.standard_normal((h, w, c)).astype(np.float16).astype(np.float32)
    wt = rng.standard_normal((size * size, c)).astype(np.float32) / size
    b = rng.standard_normal(c).astype(np.float32)
    want = oracle.depthwise(x, wt, b)
    xin = x.transpose(2, 0, 1).copy() if layout == ien.NCHW else x
    xt = torch.from_numpy(xin).half().cuda()
    y = torch.empty_like(xt)
    ien.depthwise(ctx, xt, h, w, c, layout, torch.from_numpy(wt).cuda(), size, torch.from_numpy(b).cuda(), y)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    if layout == ien.NCHW:
        got = got.transpose(1, 2, 0)
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max() + 2e-3
