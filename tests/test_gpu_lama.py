"""GPU parity of Big LaMa's generator (crates/lama-native/src/network.rs,
fourier.rs) through the C ABI model interface against the oracle's
or_lama_run, on synthetic He-normal weights: sizes that need no padding,
padding to multiples of 8 with the mirrored mask, and the smallest side;
progress, cancel and graph replay; the configuration's 512 x 512 size
through properties; the size and mask checks."""

import numpy as np
import pytest

import synthetic

pytestmark = pytest.mark.gpu


def psnr(got, want):
    mse = float(np.mean((got - want) ** 2))
    return 10 * np.log10(1.0 / max(mse, 1e-30))


@pytest.fixture(scope="module")
def tensors():
    return synthetic.lama_tensors()


@pytest.mark.parametrize("h,w", [(64, 64), (44, 60), (9, 23), (96, 128)])
def test_lama_matches_oracle(ctx, oracle, tensors, h, w):
    import ien

    img = synthetic.lama_image(h, w, seed=h + w)
    mask = synthetic.lama_mask(h, w, seed=h * w)
    want = oracle.lama_run(tensors, synthetic.lama_names(), img, mask)
    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=tensors)
    got = model.run(img, mask=mask)
    model.free()
    err = float(np.abs(got - want).max())
    assert err <= 2e-2, err
    assert psnr(got, want) >= 45.0


def test_lama_graph_progress_and_cancel(ctx, tensors):
    import torch
    import ien

    h, w = 64, 96
    img = synthetic.lama_image(h, w, seed=5)
    mask = synthetic.lama_mask(h, w, seed=6)
    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=tensors)
    done = []
    eager = model.run(img, mask=mask, progress=lambda f, u: done.append(f) or 0)
    assert len(done) == 26 and abs(done[-1] - 1.0) < 1e-6
    assert all(a < b for a, b in zip(done, done[1:]))
    with pytest.raises(ien.IenError) as e:
        model.run(img, mask=mask, progress=lambda f, u: 1)
    assert e.value.status == ien.ERR_CANCELLED
    # The model is usable after a cancel.
    assert np.array_equal(model.run(img, mask=mask), eager)
    d_in = torch.from_numpy(img).cuda()
    d_mask = torch.from_numpy(mask).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(3):
        d_out.zero_()
        model.run_device(d_in, w, h, d_out, d_mask=d_mask)
        torch.cuda.synchronize()
        assert np.array_equal(d_out.cpu().numpy(), eager)
    model.free()


def test_lama_config_size_properties(ctx, tensors):
    """1 x 4 x 512 x 512 (RGB plus a ~25 % rectangle mask): finite, in
    (0, 1), deterministic, the graph replay equal to the eager run."""
    import torch
    import ien

    h, w = 512, 512
    img = synthetic.lama_image(h, w)
    mask = synthetic.lama_mask(h, w)
    assert 0.2 < float(mask.mean()) < 0.35
    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=tensors)
    d_in = torch.from_numpy(img).cuda()
    d_mask = torch.from_numpy(mask).cuda()
    a = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    model.run_device(d_in, w, h, a, d_mask=d_mask)
    model.set_graph(True)
    model.run_device(d_in, w, h, b, d_mask=d_mask)
    model.run_device(d_in, w, h, b, d_mask=d_mask)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(a).all()) and torch.equal(a, b)
    assert float(a.min()) >= 0.0 and float(a.max()) <= 1.0 and float(a.std()) > 0.05
    model.free()


def test_lama_checks_size_and_mask(ctx, tensors):
    import ien

    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=tensors)
    img = synthetic.lama_image(8, 20)
    with pytest.raises(ien.IenError) as e:
        model.run(img, mask=np.zeros((8, 20), np.float32))
    assert e.value.status == ien.ERR_INPUT
    with pytest.raises(ien.IenError) as e:
        model.run(synthetic.lama_image(16, 16))
    assert e.value.status == ien.ERR_INPUT
    model.free()
