"""GPU parity of the SCUNet U-Net (crates/scunet-native/src/network.rs,
swin.rs) through the C ABI model interface against the oracle's
or_scunet_run, on synthetic weights: the fan-in-scaled init (activations of
order one through the 28 blocks) on images that need padding to 64 and a
crop; the configuration's trunc-normal init; graph replay, progress and
cancel; the configuration's 512 x 768 size against the oracle with both
inits.  Bounds: the configuration's (max error 2e-2, PSNR 45 dB) and the
output's spread (error RMS <= 1 % of its std, max <= 5 % of its peak)."""

import numpy as np
import pytest

import synthetic
from parity import assert_config_tolerance, assert_spread

pytestmark = pytest.mark.gpu


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
    assert_config_tolerance(got, want, peak=max(1.0, float(np.abs(want).max())), what=f"{h}x{w}")
    assert_spread(got, want, what=f"{h}x{w}")


def test_scunet_trunc_normal_init(ctx, oracle):
    import ien

    t = synthetic.scunet_tensors()
    img = synthetic.scunet_image(64, 128, seed=3)
    want = oracle.scunet_run(t, synthetic.scunet_names(), img)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=t)
    got = model.run(img)
    model.free()
    assert_config_tolerance(got, want, what="trunc-normal 64x128")
    assert_spread(got, want, what="trunc-normal 64x128")


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


@pytest.mark.parametrize("init", ["trunc_normal", "fan"])
def test_scunet_config_size_matches_oracle(ctx, oracle, init):
    """1 x 3 x 512 x 768, the configuration's size, against the oracle with
    the configuration's trunc-normal init (outputs of about 0.1, so the
    spread bounds are the ones that bite) and the fan-in init; the graph
    replay the benchmark times equals the eager run."""
    import torch
    import ien

    h, w = 512, 768
    t = synthetic.scunet_tensors(init=init)
    img = synthetic.scunet_image(h, w)
    print(f"SCUNet {h}x{w} {init}", flush=True)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=t)
    got = model.run(img)
    d_in = torch.from_numpy(img).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    model.run_device(d_in, w, h, d_out)
    model.run_device(d_in, w, h, d_out)
    torch.cuda.synchronize()
    assert np.array_equal(d_out.cpu().numpy(), got)
    model.free()
    want = oracle.scunet_run(t, synthetic.scunet_names(), img)
    assert np.isfinite(got).all()
    assert_config_tolerance(got, want, peak=max(1.0, float(np.abs(want).max())), what=init)
    assert_spread(got, want, what=init)


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
