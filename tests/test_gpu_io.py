"""GPU parity of the 8-bit image passes (ien_bytes_to_floats,
ien_floats_to_bytes, ien_mask_bytes, ien_normalize_bytes,
ien_composite_bytes: realesrgan-native lib.rs:292-300, lama-native
lib.rs:138-155, birefnet-native lib.rs:111-116) against the oracle, bit for
bit: every byte, special floats, ties, ragged lengths and unaligned
buffers (the scalar paths)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MEAN = (0.485, 0.456, 0.406)
STD = (0.229, 0.224, 0.225)


def special_floats(rng, n):
    base = np.array([0, -0.0, 1, -1, 2, 0.5, np.nan, np.inf, -np.inf, 1e-30, 1 - 1e-7], np.float32)
    ties = ((np.arange(256) + 0.5) / 255.0).astype(np.float32)
    x = np.concatenate([base, ties, np.nextafter(ties, 0), np.nextafter(ties, 1),
                        rng.uniform(-0.2, 1.2, n).astype(np.float32)])
    return x


@pytest.mark.parametrize("n,offset", [(1 << 20, 0), (4097, 0), (1000, 3), (15, 1), (0, 0)])
def test_bytes_and_floats(ctx, oracle, n, offset):
    import torch
    import ien

    rng = np.random.default_rng(n + offset)
    b = rng.integers(0, 256, n + offset, dtype=np.uint8)
    b[offset:offset + min(n, 256)] = np.arange(min(n, 256))
    db = torch.from_numpy(b).cuda()[offset:]
    df = torch.empty(n + offset, dtype=torch.float32, device="cuda")[offset:]
    ien.bytes_to_floats(ctx, db, df)
    torch.cuda.synchronize()
    want = oracle.bytes_to_floats(b[offset:])
    assert np.array_equal(df.cpu().numpy().view(np.uint32), want.view(np.uint32))

    x = special_floats(rng, n)[: n] if n else np.zeros(0, np.float32)
    x = np.concatenate([np.zeros(offset, np.float32), x])
    dx = torch.from_numpy(x).cuda()[offset:]
    dy = torch.empty(len(x), dtype=torch.uint8, device="cuda")[offset:]
    ien.floats_to_bytes(ctx, dx, dy)
    torch.cuda.synchronize()
    assert np.array_equal(dy.cpu().numpy(), oracle.floats_to_bytes(x[offset:]))


@pytest.mark.parametrize("pixels,offset", [(512 * 512, 0), (1001, 0), (333, 5)])
def test_mask_normalize_composite(ctx, oracle, pixels, offset):
    import torch
    import ien

    rng = np.random.default_rng(pixels)
    rgb = rng.integers(0, 256, pixels * 3 + offset, dtype=np.uint8)
    mask = rng.choice(np.array([0, 0, 1, 9, 255], np.uint8), pixels + offset)
    pred = special_floats(rng, pixels * 3)[: pixels * 3]
    pred = np.concatenate([np.zeros(offset, np.float32), pred])
    d_rgb = torch.from_numpy(rgb).cuda()[offset:]
    d_mask = torch.from_numpy(mask).cuda()[offset:]
    d_pred = torch.from_numpy(pred).cuda()[offset:]

    holes = torch.empty(pixels + offset, dtype=torch.float32, device="cuda")[offset:]
    ien.mask_bytes(ctx, d_mask, holes)
    norm = torch.empty(pixels * 3 + offset, dtype=torch.float32, device="cuda")[offset:]
    ien.normalize_bytes(ctx, d_rgb, MEAN, STD, norm)
    out = torch.empty(pixels * 3 + offset, dtype=torch.uint8, device="cuda")[offset:]
    ien.composite_bytes(ctx, d_rgb, d_mask, d_pred, out)
    torch.cuda.synchronize()
    r, m, p = rgb[offset:], mask[offset:], pred[offset:]
    assert np.array_equal(holes.cpu().numpy(), oracle.mask_bytes(m))
    assert np.array_equal(norm.cpu().numpy().view(np.uint32), oracle.normalize_bytes(r).view(np.uint32))
    want = oracle.composite_bytes(r.reshape(-1, 3), m, p.reshape(-1, 3)).reshape(-1)
    assert np.array_equal(out.cpu().numpy(), want)
