"""GPU parity of the SCUNet U-Net (crates/scunet-native/src/network.rs,
swin.rs) through the C ABI model interface against the oracle's
or_scunet_run, on synthetic weights: the fan-in-scaled init (activations of
order one through the 28 blocks) on images that need padding to 64 and a
crop; the configuration's trunc-normal init; graph replay, progress and
cancel; the configuration's 512 x 768 size through properties."""

import numpy as np
import pytest

import synthetic

pytestmark = pytest.mark.gpu


def psnr(got, want):
    peak = max(1.0, float(np.abs(want).max()))
    mse = float(np.mean((got - want) ** 2))
    return 10 * np.log10(peak * peak / max(mse, 1e-30))


@pytest.fixture(scope="module")
def fan():
    return synthetic.scunet_tensors(init="fan")


@pytest.mark.parametrize("h,w", [(64, 64), (70, 90), (64, 192)])
def test_scunet_matches_oracle(ctx, oracle, fan, h, w):
    import ien

    img = synthetic.scunet_image(h, w, seed=h + w)
    want = oracle.scunet_run(fan, synthetic.scunet_names(), img)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=fan)
    got = model.run(img)
    model.free()
    err = np.abs(got - want)
    scale = max(1.0, float(np.abs(want).max()))
    assert err.max() <= 2e-2 * scale, (err.max(), scale)
    assert psnr(got, want) >= 45.0


def test_scunet_trunc_normal_init(ctx, oracle):
    import ien

    t = synthetic.scunet_tensors()
    img = synthetic.scunet_image(64, 128, seed=3)
    want = oracle.scunet_run(t, synthetic.scunet_names(), img)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=t)
    got = model.run(img)
    model.free()
    assert np.abs(got - want).max() <= 2e-2 and psnr(got, want) >= 45.0


def test_scunet_graph_progress_and_cancel(ctx, fan):
    import torch
    import ien

    h, w = 64, 128
    img = synthetic.scunet_image(h, w, seed=5)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=fan)
    done = []
    eager = model.run(img, progress=lambda f, u: done.append(f) or 0)
    assert len(done) == 28 and abs(done[-1] - 1.0) < 1e-6
    with pytest.raises(ien.IenError) as e:
        model.run(img, progress=lambda f, u: 1)
    assert e.value.status == ien.ERR_CANCELLED
    d_in = torch.from_numpy(img).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(3):
        model.run_device(d_in, w, h, d_out)
        torch.cuda.synchronize()
        assert np.array_equal(d_out.cpu().numpy(), eager)
    model.free()


def test_scunet_config_size_properties(ctx):
    """1 x 3 x 512 x 768 with the configuration's init: finite, deterministic,
    the graph replay equal to the eager run."""
    import torch
    import ien

    h, w = 512, 768
    img = synthetic.scunet_image(h, w)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=synthetic.scunet_tensors())
    d_in = torch.from_numpy(img).cuda()
    a = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    model.run_device(d_in, w, h, a)
    model.set_graph(True)
    model.run_device(d_in, w, h, b)
    model.run_device(d_in, w, h, b)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(a).all()) and torch.equal(a, b)
    model.free()


def test_scunet_graph_first_run_captures(ctx, fan):
    """Graph mode set before any eager run: the first run captures, so every
    block's scratch is sized before the capture starts; the replays equal an
    eager model's output."""
    import torch
    import ien

    h, w = 128, 192
    img = synthetic.scunet_image(h, w, seed=9)
    eager_model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=fan)
    want = eager_model.run(img)
    eager_model.free()
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=fan)
    model.set_graph(True)
    d_in = torch.from_numpy(img).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    for _ in range(2):
        d_out.zero_()
        model.run_device(d_in, w, h, d_out)
        torch.cuda.synchronize()
        assert np.array_equal(d_out.cpu().numpy(), want)
    model.free()
