"""GPU parity of BiRefNet-lite (crates/birefnet-native/src/swin.rs,
decoder.rs, lib.rs run_normalized) through the C ABI model interface
against the oracle's or_birefnet_run: the configured window 12 (padded
grids at every stage) and the reference's window 7, the fan-in and the
configuration's trunc-normal inits; the mask compared after the sigmoid
(max-abs 2e-2, PSNR 45 dB) and the logits within 2 % of their range; the
deformable ASPP at three offset scales; the size checks; progress and graph replay; the
configuration's 1024 x 1024 size against the oracle with both inits.  The
logits are also held to the spread bounds (error RMS <= 1 % of their std,
max <= 5 % of their peak)."""

import numpy as np
import pytest

import synthetic
from parity import assert_config_tolerance, assert_spread

pytestmark = pytest.mark.gpu


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


@pytest.mark.parametrize("window,side,init", [
    (12, 64, "fan"), (12, 128, "fan"), (12, 128, "trunc_normal"), (7, 64, "fan"), (7, 192, "fan")])
def test_birefnet_matches_oracle(ctx, oracle, window, side, init):
    import ien

    t = synthetic.birefnet_tensors(window=window, init=init)
    img = synthetic.birefnet_image(side, seed=side + window)
    want = oracle.birefnet_run(t, synthetic.birefnet_names(window), img, window)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=t)
    got = model.run(img)
    model.free()
    assert got.shape == (side, side)
    check(got, want, f"window {window} side {side} {init}")


def check(got, want, what):
    """Logits within the configuration's bar scaled to their peak and
    within the spread bounds; the mask (sigmoid) within the bar itself."""
    assert_config_tolerance(got, want, peak=max(1.0, float(np.abs(want).max())), what=what + " logits")
    assert_spread(got, want, what=what + " logits")
    assert_config_tolerance(sigmoid(got), sigmoid(want), what=what + " mask")
    # The edge ring, where the full-resolution branch runs its two
    # convolutions instead of the composed one, on its own.
    ring = np.zeros(got.shape, bool)
    ring[0], ring[-1], ring[:, 0], ring[:, -1] = True, True, True, True
    assert_spread(got[ring], want[ring], what=what + " ring logits")


@pytest.mark.parametrize("window,side,offsets", [(7, 64, 0.002), (7, 64, 0.3), (12, 128, 0.01)])
def test_birefnet_deformable_matches_oracle(ctx, oracle, window, side, offsets):
    """The deformable ASPP (decoder.rs:176-313): non-zero offset and
    modulator convolutions, sample points moved within a pixel (0.002),
    a few pixels (0.01) and far outside the map (0.3)."""
    import ien

    t = synthetic.birefnet_tensors(window=window, init="fan", offsets=offsets)
    img = synthetic.birefnet_image(side, seed=side + 3)
    want = oracle.birefnet_run(t, synthetic.birefnet_names(window), img, window)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=t)
    got = model.run(img)
    model.free()
    check(got, want, f"deformable window {window} side {side} offsets {offsets}")


def test_birefnet_rejects_bad_sizes(ctx):
    import ien

    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=synthetic.birefnet_tensors())
    for h, w in ((96, 96), (64, 128)):
        with pytest.raises(ien.IenError) as e:
            model.run(np.zeros((h, w, 3), np.float32))
        assert e.value.status == ien.ERR_INPUT
    model.free()


def test_birefnet_graph_and_progress(ctx):
    import torch
    import ien

    side = 128
    t = synthetic.birefnet_tensors(init="fan")
    img = synthetic.birefnet_image(side, seed=11)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=t)
    done = []
    eager = model.run(img, progress=lambda f, u: done.append(f) or 0)
    assert len(done) == 14 and abs(done[-1] - 1.0) < 1e-6
    d_in = torch.from_numpy(img).cuda()
    d_out = torch.empty((side, side), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(3):
        d_out.zero_()
        model.run_device(d_in, side, side, d_out)
        torch.cuda.synchronize()
        assert np.array_equal(d_out.cpu().numpy(), eager)
    model.free()


# The half-size backbone runs on a branch stream beside the full-size one;
# with every branch on the context's stream (IEN_SERIAL_BRANCHES, read when
# a context opens) the launches are the same, so the logits are the same
# bits, eager and replayed.
def test_birefnet_branches_match_serial(monkeypatch):
    import torch
    import ien

    side = 256
    t = synthetic.birefnet_tensors(init="fan")
    img = synthetic.birefnet_image(side, seed=21)
    got = {}
    for serial in ("0", "1"):
        monkeypatch.setenv("IEN_SERIAL_BRANCHES", serial)
        c = ien.Context(0)
        model = ien.Model(c, ien.MODEL_BIREFNET, tensors=t)
        got[serial, "eager"] = model.run(img)
        d_in = torch.from_numpy(img).cuda()
        d_out = torch.empty((side, side), dtype=torch.float32, device="cuda")
        model.set_graph(True)
        model.run_device(d_in, side, side, d_out)
        torch.cuda.synchronize()
        got[serial, "graph"] = d_out.cpu().numpy()
        model.free()
        c.close()
    ref = got["1", "eager"].view(np.uint32)
    for key, out in got.items():
        assert np.array_equal(out.view(np.uint32), ref), key


@pytest.mark.parametrize("init", ["trunc_normal", "fan"])
def test_birefnet_config_size_matches_oracle(ctx, oracle, init):
    """1 x 3 x 1024 x 1024 N(0, 1), window 12, the configuration's size,
    against the oracle with the configuration's init and the fan-in init;
    the graph replay the benchmark times equals the eager run."""
    import torch
    import ien

    side = 1024
    t = synthetic.birefnet_tensors(init=init)
    img = synthetic.birefnet_image(side)
    print(f"BiRefNet {side} {init}", flush=True)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=t)
    got = model.run(img)
    d_in = torch.from_numpy(img).cuda()
    d_out = torch.empty((side, side), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    model.run_device(d_in, side, side, d_out)
    model.run_device(d_in, side, side, d_out)
    torch.cuda.synchronize()
    assert np.array_equal(d_out.cpu().numpy(), got)
    model.free()
    want = oracle.birefnet_run(t, synthetic.birefnet_names(12), img, 12)
    assert np.isfinite(got).all() and float(want.std()) > 0.1
    check(got, want, f"1024 {init}")
