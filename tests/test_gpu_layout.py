"""GPU checks of the layout ops behind the U-Net levels, bit for bit against
numpy: the 2x2 gathers in both orders (scunet-native network.rs:403-437,
birefnet-native swin.rs merge), the 2x2 scatter (network.rs:439-478) and the
skip add (one f32 add, one rounding)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("order", [0, 1])
def test_gather_2x2(ctx, order):
    import torch
    import ien

    h, w, c, stride = 6, 10, 24, 40
    x = np.random.default_rng(order).standard_normal((h * w, stride)).astype(np.float16)
    rows = torch.zeros((h // 2 * w // 2, 4 * c), dtype=torch.float16, device="cuda")
    ien.gather_2x2(ctx, torch.from_numpy(x).cuda(), h, w, c, stride, order, rows)
    torch.cuda.synchronize()
    m = x[:, :c].reshape(h, w, c)
    taps = [(0, 0), (0, 1), (1, 0), (1, 1)] if order == 0 else [(0, 0), (1, 0), (0, 1), (1, 1)]
    want = np.concatenate([m[dy::2, dx::2] for dy, dx in taps], axis=2).reshape(-1, 4 * c)
    assert np.array_equal(rows.cpu().numpy(), want)


def test_scatter_2x2_and_add(ctx):
    import torch
    import ien

    h, w, c, rs = 5, 7, 16, 72
    rows = np.random.default_rng(1).standard_normal((h * w, rs)).astype(np.float16)
    out = torch.zeros((4 * h * w, c), dtype=torch.float16, device="cuda")
    ien.scatter_2x2(ctx, torch.from_numpy(rows).cuda(), rs, h, w, c, out, c)
    torch.cuda.synchronize()
    want = np.zeros((2 * h, 2 * w, c), np.float16)
    r = rows[:, :4 * c].reshape(h, w, 4, c)
    for q in range(4):
        want[q // 2::2, q % 2::2] = r[:, :, q]
    assert np.array_equal(out.cpu().numpy().reshape(2 * h, 2 * w, c), want)
    a = np.random.default_rng(2).standard_normal(1003).astype(np.float16)
    b = np.random.default_rng(3).standard_normal(1003).astype(np.float16)
    at = torch.from_numpy(a).cuda()
    ien.add(ctx, at, torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(at.cpu().numpy(), (a.astype(np.float32) + b.astype(np.float32)).astype(np.float16))
