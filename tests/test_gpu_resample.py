"""GPU parity of the resampling passes: the align-corners bilinear resize
(birefnet-native decoder.rs:436-522) against the oracle to f16 storage
accuracy, f16 and f32 outputs, with and without `add`, 1 channel and 8-channel
chunks; the model-input padding (scunet / lama network.rs) and the crop
bit for bit."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sh,sw,dh,dw,c", [(5, 7, 9, 13, 8), (32, 32, 64, 64, 64), (64, 64, 32, 32, 16),
                                           (256, 256, 1024, 1024, 1), (1, 5, 3, 9, 3), (17, 23, 17, 23, 24)])
@pytest.mark.parametrize("out_f32,add", [(False, False), (False, True), (True, False), (True, True)])
def test_resize(ctx, oracle, sh, sw, dh, dw, c, out_f32, add):
    import torch
    import ien

    rng = np.random.default_rng(sh + dh + c)
    sstride, dstride = c + (8 if c % 8 == 0 else 1), c + 8
    x = rng.standard_normal((sh * sw, sstride)).astype(np.float16)
    base = rng.standard_normal((dh * dw, dstride)).astype(np.float32)
    dt = torch.float32 if out_f32 else torch.float16
    dst = torch.from_numpy(base).to(dt).cuda()
    ien.resize(ctx, torch.from_numpy(x).cuda(), sh, sw, sstride, c, dst, dh, dw, dstride, out_f32=out_f32, add=add)
    torch.cuda.synchronize()
    got = dst.float().cpu().numpy()
    src = x[:, :c].astype(np.float32).reshape(sh, sw, c)
    init = base.astype(np.float16).astype(np.float32) if not out_f32 else base
    want = oracle.resize(src, dh, dw, out=init[:, :c].reshape(dh, dw, c), add=add).reshape(dh * dw, c)
    err = np.abs(got[:, :c] - want)
    tol = (2e-3 * np.abs(want) + 2e-3) if not out_f32 else (1e-5 * (1 + np.abs(want)))
    assert (err <= tol).all(), err.max()
    assert np.array_equal(got[:, c:], init[:, c:])  # columns past c untouched


@pytest.mark.parametrize("h,w,multiple", [(5, 7, 8), (65, 30, 64), (17, 30, 8), (64, 64, 64)])
def test_pad_and_crop(ctx, oracle, h, w, multiple):
    import torch
    import ien

    rng = np.random.default_rng(h * w)
    img = rng.random((h, w, 3)).astype(np.float32)
    m = (rng.random((h, w)) < 0.3).astype(np.float32)
    ph, pw = -(-h // multiple) * multiple, -(-w // multiple) * multiple
    out = torch.full((ph * pw, 8), 9.0, dtype=torch.float16, device="cuda")
    ien.pad_image(ctx, ien.PAD_REPLICATE, torch.from_numpy(img).cuda(), None, w, h, multiple, out, 8)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = oracle.pad_replicate(img, multiple).reshape(ph * pw, 3).astype(np.float16)
    assert np.array_equal(got[:, :3], want) and np.all(got[:, 3:] == 9.0)
    if ph - h <= h and pw - w <= w:
        out4 = torch.zeros((ph * pw, 4), dtype=torch.float16, device="cuda")
        ien.pad_image(ctx, ien.PAD_SYMMETRIC_MASKED, torch.from_numpy(img).cuda(), torch.from_numpy(m).cuda(), w, h,
                      multiple, out4, 4)
        torch.cuda.synchronize()
        want4 = oracle.masked_rows(img, m, multiple).reshape(ph * pw, 4).astype(np.float16)
        assert np.array_equal(out4.cpu().numpy(), want4)
    back = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    ien.crop(ctx, out, pw, 8, w, h, 3, back)
    torch.cuda.synchronize()
    assert np.array_equal(back.cpu().numpy(), img.astype(np.float16).astype(np.float32))
