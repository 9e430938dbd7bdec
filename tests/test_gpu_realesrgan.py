"""GPU parity of Real-ESRGAN general x4v3 (SRVGGNetCompact) through the C
ABI's model entry points against the oracle's restatement of the
reference's CPU f32 path (crates/realesrgan-native/src/network.rs), on the
same seeded input and random-init weights.

Bar (the configuration's tolerance): max |gpu - oracle| <= 2e-2 and PSNR >= 45 dB on
the [0, 1] scale.  The GPU keeps activations in f16 between layers and
sums in f32 on MFMA; the oracle is f32 throughout with Winograd F(4x4, 3x3).
"""

import numpy as np
import pytest

import synthetic
from parity import assert_spread

pytestmark = pytest.mark.gpu


def psnr(a, b):
    mse = float(np.mean((np.asarray(a, np.float64) - np.asarray(b, np.float64)) ** 2))
    return float("inf") if mse == 0 else 10 * np.log10(1.0 / mse)


@pytest.fixture(scope="module")
def tensors():
    return synthetic.esrgan_tensors()


def reference(oracle, tensors, image):
    return oracle.realesrgan_run(synthetic.esrgan_layers(tensors), image)


@pytest.mark.parametrize("h,w", [(16, 24), (37, 53), (64, 96)])
def test_small_images(ctx, oracle, tensors, h, w):
    import ien

    image = synthetic.esrgan_image(h, w, seed=h)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    got = model.run(image)
    want = reference(oracle, tensors, image)
    model.free()
    err = np.abs(got - want).max()
    print(f"{h}x{w}: max err {err:.3g}, PSNR {psnr(got, want):.1f} dB")
    assert err <= 2e-2 and psnr(got, want) >= 45


def test_config_size_device_path_and_graph(ctx, oracle, tensors):
    """1x3x256x384, the benchmark configuration, on device buffers, eager and
    replayed from a HIP graph (each replay checked against the eager result)."""
    import torch
    import ien

    image = synthetic.esrgan_image(256, 384)
    want = reference(oracle, tensors, image)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    d_in = torch.from_numpy(image).cuda()
    d_out = torch.empty((1024, 1536, 3), dtype=torch.float32, device="cuda")
    model.run_device(d_in, 384, 256, d_out)
    torch.cuda.synchronize()
    eager = d_out.cpu().numpy()
    err = np.abs(eager - want).max()
    print(f"256x384: max err {err:.3g}, PSNR {psnr(eager, want):.1f} dB")
    assert err <= 2e-2 and psnr(eager, want) >= 45
    # The network's own part (output minus the repeated input) against its
    # spread: error RMS <= 1 % of its std, max <= 5 % of its peak.
    up = np.repeat(np.repeat(image, 4, axis=0), 4, axis=1)
    assert_spread(eager - up, want - up, what="256x384 residual")
    model.set_graph(True)
    for replay in range(3):
        d_out.zero_()
        torch.cuda.synchronize()
        model.run_device(d_in, 384, 256, d_out)
        torch.cuda.synchronize()
        assert np.array_equal(d_out.cpu().numpy(), eager), f"replay {replay} differs"
    model.free()


def unfused_network(ctx, tensors, image):
    """The network from one-layer products through the C ABI: the input as
    the model stages it (an f16 map of 4 channels, the fourth zero), the
    first layer with its weights expanded to 4 channels (the four-channel
    kernel), the 32 body layers and the last through ien_multiply_ex (the
    resident kernel), then the pixel shuffle."""
    import torch
    import ien

    h, w, _ = image.shape
    layers = synthetic.esrgan_layers(tensors)
    d_img = torch.from_numpy(image).cuda()
    x = torch.zeros((h * w, 4), dtype=torch.float16, device="cuda")
    ien.pad_image(ctx, ien.PAD_REPLICATE, d_img, None, w, h, 1, x, 4)
    maps = [torch.empty((h * w, 64), dtype=torch.float16, device="cuda") for _ in range(2)]
    last = torch.empty((h * w, 48), dtype=torch.float16, device="cuda")
    keep = []
    for i, (wt, b, slope) in enumerate(layers):
        if i == 0:
            w4 = np.zeros((36, wt.shape[1]), np.float32)
            for t in range(9):
                w4[4 * t:4 * t + 3] = wt[3 * t:3 * t + 3]
            wt, src, cin = w4, x, 4
        else:
            src, cin = maps[(i - 1) % 2], 64
        m = ien.Matrix(ctx, wt, b)
        sl = None if slope is None else torch.from_numpy(slope).cuda()
        keep += [m, sl]
        dst = last if i == len(layers) - 1 else maps[i % 2]
        inp = ien.image_input(src, h, w, cin)
        ien.multiply_ex(ctx, inp, 0, h * w, m, dst, dst.shape[1],
                        act=ien.ACT_PRELU if slope is not None else ien.ACT_NONE, slope=sl)
    out = torch.empty((4 * h, 4 * w, 3), dtype=torch.float32, device="cuda")
    ien.pixel_shuffle_add(ctx, last, 48, d_img, w, h, out)
    torch.cuda.synchronize()
    for m in keep[::2]:
        m.free()
    return out.cpu().numpy()


@pytest.mark.parametrize("h,w", [(256, 384), (50, 70), (16, 24), (37, 100)])
def test_body_pairs_equal_single_layers(ctx, tensors, h, w):
    """The model runs its body two layers per launch; the same network from
    one-layer launches gives the same bits (tiles of 16 x 24 at the
    configured size, ragged edge tiles, a single tile)."""
    import ien

    image = synthetic.esrgan_image(h, w, seed=h + w)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    got = model.run(image)
    model.free()
    want = unfused_network(ctx, tensors, image)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), float(np.abs(got - want).max())


@pytest.mark.parametrize("h,w", [(256, 384), (50, 70), (16, 24), (37, 100), (1, 1), (300, 500)])
def test_body_chain_equals_pairs(ctx, tensors, h, w):
    """Without a progress callback the 32 body layers run as one chain of
    pairs (tiles exchanging 2-pixel borders) where every tile fits on the
    device at once (300 x 500 has more tiles than CUs and runs pair by
    pair); with one they run a pair per launch.  Same bits either way."""
    import ien

    image = synthetic.esrgan_image(h, w, seed=h * 7 + w)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    chained = model.run(image)
    paired = model.run(image, progress=lambda done, user: 0)
    model.free()
    assert np.array_equal(chained.view(np.uint32), paired.view(np.uint32)), float(np.abs(chained - paired).max())


def test_body_chain_wait_limit(tensors, monkeypatch):
    """A chain whose waits for neighbours never succeed (the wall-clock limit
    set negative from the host): every tile gives up at its first wait and
    sets the abort word, and every workgroup ends.
    - The host-buffer run sees the failure and repeats the run through the
      pair launches: the same bits as a run with the normal limit.
    - The device path returns at once; ien_model_status then reports the
      failure (IEN_ERR_GPU) once, and a second status call is clean.
    - A context with the normal limit is unaffected, on both paths."""
    import torch
    import ien

    image = synthetic.esrgan_image(256, 384, seed=9)
    calm = ien.Context(0)
    model = ien.Model(calm, ien.MODEL_REALESRGAN, tensors=tensors)
    want = model.run(image, progress=lambda done, user: 0)  # the pair path
    model.free()
    calm.close()

    monkeypatch.setenv("IEN_CHAIN_SPIN_TICKS", "-1")
    hurried = ien.Context(0)
    monkeypatch.delenv("IEN_CHAIN_SPIN_TICKS")
    model = ien.Model(hurried, ien.MODEL_REALESRGAN, tensors=tensors)
    got = model.run(image)  # chain gives up, repeated through pairs
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    model.status()  # the host run's failure was handled and is not reported again
    d_in = torch.from_numpy(image).cuda()
    d_out = torch.zeros((1024, 1536, 3), dtype=torch.float32, device="cuda")
    model.set_graph(False)
    model.run_device(d_in, 384, 256, d_out)
    with pytest.raises(ien.IenError) as e:
        model.status()
    assert e.value.status == ien.ERR_GPU and "timed out" in str(e.value), str(e.value)
    model.status()  # reported once
    model.set_graph(True)
    model.run_device(d_in, 384, 256, d_out)
    model.run_device(d_in, 384, 256, d_out)
    with pytest.raises(ien.IenError):
        model.status()
    again = model.run(image)  # a host run after unreported device failures: still the right bits
    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    model.free()
    hurried.close()

    calm = ien.Context(0)
    model = ien.Model(calm, ien.MODEL_REALESRGAN, tensors=tensors)
    got = model.run(image)
    d_out.zero_()
    model.set_graph(True)
    model.run_device(d_in, 384, 256, d_out)
    model.status()
    dev = d_out.cpu().numpy()
    model.free()
    calm.close()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(dev.view(np.uint32), want.view(np.uint32))


def pair_inputs(ctx, tensors, h, w, seed):
    import torch
    import ien

    (w1, b1, s1), (w2, b2, s2) = synthetic.esrgan_layers(tensors)[1:3]
    x = np.random.default_rng(seed).standard_normal((h, w, 64)).astype(np.float16)
    m1, m2 = ien.Matrix(ctx, w1, b1), ien.Matrix(ctx, w2, b2)
    sl1, sl2 = torch.from_numpy(s1).cuda(), torch.from_numpy(s2).cuda()
    return x, (w1, b1, s1, w2, b2, s2), m1, sl1, m2, sl2


@pytest.mark.parametrize("h,w", [(256, 384), (33, 49), (16, 24), (1, 1)])
def test_conv3_pair_op(ctx, oracle, tensors, h, w):
    """ien_conv3_pair (two body steps of network.rs:96-109 in one launch):
    bit for bit two single-layer ien_multiply_ex launches, and close to the
    oracle's two conv3 + PReLU steps with the intermediate map rounded to
    f16 as the GPU stores it (error RMS <= 0.2 % of the output's spread)."""
    import torch
    import ien

    x, (w1, b1, s1, w2, b2, s2), m1, sl1, m2, sl2 = pair_inputs(ctx, tensors, h, w, seed=h * w)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty_like(dx)
    mid = torch.empty_like(dx)
    ref = torch.empty_like(dx)
    ien.conv3_pair(ctx, dx, dy, h, w, m1, sl1, m2, sl2)
    ien.multiply_ex(ctx, ien.image_input(dx, h, w, 64), 0, h * w, m1, mid, 64, act=ien.ACT_PRELU, slope=sl1)
    ien.multiply_ex(ctx, ien.image_input(mid, h, w, 64), 0, h * w, m2, ref, 64, act=ien.ACT_PRELU, slope=sl2)
    torch.cuda.synchronize()
    got = dy.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), ref.cpu().numpy().view(np.uint16))
    first = oracle.conv3(x, w1, b1, finish=oracle.FINISH_PRELU, slope=s1, threads=8)
    want = oracle.conv3(first.astype(np.float16), w2, b2, finish=oracle.FINISH_PRELU, slope=s2, threads=8)
    assert_spread(got.astype(np.float32), want, rms_frac=2e-3, max_frac=1e-2, what=f"pair {h}x{w}")
    m1.free()
    m2.free()


@pytest.mark.parametrize("h,w,pairs", [(256, 384, 16), (40, 100, 3), (17, 25, 1)])
def test_conv3_chain_op(ctx, tensors, h, w, pairs):
    """ien_conv3_chain: `pairs` pairs of body layers in one launch, bit for
    bit the same number of ien_conv3_pair launches; the output map is the
    first for an even count, the second for an odd one."""
    import torch
    import ien

    layers = synthetic.esrgan_layers(tensors)[1:1 + 2 * pairs]
    mats = [ien.Matrix(ctx, wt, b) for wt, b, _ in layers]
    slopes = [torch.from_numpy(sl).cuda() for _, _, sl in layers]
    x = torch.from_numpy(np.random.default_rng(h + pairs).standard_normal((h, w, 64)).astype(np.float16)).cuda()
    a, b = x.clone(), torch.empty_like(x)
    out = ien.conv3_chain(ctx, a, b, h, w, mats, slopes)
    torch.cuda.synchronize()
    ien.conv3_chain_status(ctx)
    assert out is (a if pairs % 2 == 0 else b)
    ref, tmp = x.clone(), torch.empty_like(x)
    for k in range(pairs):
        ien.conv3_pair(ctx, ref, tmp, h, w, mats[2 * k], slopes[2 * k], mats[2 * k + 1], slopes[2 * k + 1])
        ref, tmp = tmp, ref
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.cpu().numpy().view(np.uint16))
    for m in mats:
        m.free()


def test_conv3_chain_refusals(ctx, tensors):
    """Counts outside 1..16 and maps with more tiles than the device holds
    at once are refused before anything is launched."""
    import torch
    import ien

    layers = synthetic.esrgan_layers(tensors)[1:3]
    mats = [ien.Matrix(ctx, wt, b) for wt, b, _ in layers]
    slopes = [torch.from_numpy(sl).cuda() for _, _, sl in layers]
    big = torch.zeros((1024, 1024, 64), dtype=torch.float16, device="cuda")
    other = torch.zeros_like(big)
    with pytest.raises(ien.IenError) as e:
        ien.conv3_chain(ctx, big, other, 1024, 1024, mats, slopes)
    assert e.value.status == ien.ERR_INPUT and "tiles" in str(e.value), str(e.value)
    with pytest.raises(ien.IenError) as e:
        ien.conv3_chain(ctx, big, other, 64, 64, [], [])
    assert e.value.status == ien.ERR_INPUT and "pairs" in str(e.value), str(e.value)
    for m in mats:
        m.free()


def test_conv3_pair_refusals(ctx, tensors):
    """Overlapping maps, misaligned maps and layers that are not 3x3 64->64
    are refused before anything is launched."""
    import torch
    import ien

    h, w = 8, 8
    x, _, m1, sl1, m2, sl2 = pair_inputs(ctx, tensors, h, w, seed=1)
    buf = torch.zeros(3 * h * w * 64, dtype=torch.float16, device="cuda")
    last_w, last_b, _ = synthetic.esrgan_layers(tensors)[-1]
    m_last = ien.Matrix(ctx, last_w, last_b)
    cases = ((buf[: h * w * 64], buf[h * w * 32: h * w * 96], m2, "overlap"),
             (buf[1: 1 + h * w * 64], buf[2 * h * w * 64:], m2, "aligned"),
             (buf[: h * w * 64], buf[2 * h * w * 64:], m_last, "k 576, n 48"))
    for src, dst, second, message in cases:
        with pytest.raises(ien.IenError) as e:
            ien.conv3_pair(ctx, src, dst, h, w, m1, sl1, second, sl2)
        assert e.value.status == ien.ERR_INPUT and message in str(e.value), str(e.value)
    for m in (m1, m2, m_last):
        m.free()


def test_progress_and_cancel(ctx, tensors):
    """lib.rs:168-188: progress after each of the 34 layers, monotone, ending
    at 1; breaking cancels, the model stays usable and the next run is
    bit-identical."""
    import ien

    image = synthetic.esrgan_image(20, 28, seed=5)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    seen = []

    def report(done, _user):
        seen.append(done)
        return 0

    first = model.run(image, progress=report)
    assert len(seen) == 34 and seen == sorted(seen) and abs(seen[-1] - 1.0) < 1e-6
    calls = []

    def stop(done, _user):
        calls.append(done)
        return 1 if len(calls) == 13 else 0

    with pytest.raises(ien.IenError) as e:
        model.run(image, progress=stop)
    assert e.value.status == ien.ERR_CANCELLED and len(calls) == 13
    assert np.array_equal(model.run(image), first)
    model.free()


def test_weights_errors(ctx, tensors):
    import ien

    bad = dict(tensors)
    bad["body.0.weight"] = bad["body.0.weight"][:-1]
    with pytest.raises(ien.IenError) as e:
        ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=bad)
    assert e.value.status == ien.ERR_WEIGHTS and "body.0.weight" in str(e.value)
    extra = dict(tensors)
    extra["unused"] = np.zeros(3, np.float32)
    with pytest.raises(ien.IenError) as e:
        ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=extra)
    assert "not used" in str(e.value)
    missing = dict(tensors)
    del missing["body.66.bias"]
    with pytest.raises(ien.IenError) as e:
        ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=missing)
    assert "missing" in str(e.value)
