"""GPU parity of the fused FFC spectral branch (ien_spectral_run,
crates/lama-native/src/network.rs:205-245) against the oracle's products and
transforms composed in the reference's order, with f16 rounding where the
GPU stores f16 (the spectral map, the spectrum, the filtered spectrum, the
updated spectral map and the output), and against the unfused GPU chain
(ien_multiply and the Fourier units).  Shapes: LaMa's 64 x 64 eighth scale,
odd and even sides, sides of one, rectangles.  Weights: one FFC of the
synthetic LaMa network (He-normal).  The input is a 512-channel map whose
last 384 channels are the global part; the output's 384 global channels
hold a cross output to accumulate onto, inside a 512-channel map whose
local channels must stay untouched."""

import numpy as np
import pytest

import synthetic
from parity import spread_errors

pytestmark = pytest.mark.gpu

LOCAL, GLOBAL, CHANNELS, SPECTRAL = 128, 384, 512, 192
SHAPES = [(64, 64), (8, 8), (6, 8), (2, 3), (12, 16), (33, 17), (1, 1), (64, 5), (7, 64), (40, 36)]


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.fixture(scope="module")
def weights():
    t = synthetic.lama_tensors()
    n = "block3.ffc0"
    return {k: t[f"{n}.{k}"] for k in ("spectral_in.weight", "spectral_in.bias", "fourier.weight",
                                       "fourier.bias", "spectral_out.weight")}


def oracle_chain(oracle, x_global, cross, wt):
    """network.rs:205-245 on the oracle, rounded to f16 where the GPU stores."""
    from oracle.oracle import ACT_RELU

    h, w, _ = x_global.shape
    rows = x_global.reshape(h * w, GLOBAL)
    spectral = f16(oracle.multiply_rows(rows, wt["spectral_in.weight"], wt["spectral_in.bias"],
                                        act=ACT_RELU)).reshape(h, w, SPECTRAL)
    spectrum = f16(oracle.rfft2(spectral))
    half = w // 2 + 1
    filtered = f16(oracle.multiply_rows(spectrum.reshape(h * half, 2 * SPECTRAL), wt["fourier.weight"],
                                        wt["fourier.bias"], act=ACT_RELU)).reshape(h, half, 2 * SPECTRAL)
    updated = np.ascontiguousarray(spectral.copy())
    oracle.irfft2_add(filtered, updated)
    updated = f16(updated)
    out = oracle.multiply_rows(updated.reshape(h * w, SPECTRAL), wt["spectral_out.weight"], act=ACT_RELU,
                               out=cross.reshape(h * w, GLOBAL), accumulate=True)
    return f16(out).reshape(h, w, GLOBAL)


@pytest.mark.parametrize("h,w", SHAPES)
def test_spectral_matches_oracle(ctx, oracle, weights, h, w):
    import torch
    import ien

    print(f"spectral {h}x{w}", flush=True)
    rng = np.random.default_rng(h * 100 + w)
    x = f16(rng.standard_normal((h, w, CHANNELS)))
    base = f16(rng.standard_normal((h, w, CHANNELS)))
    m_in = ien.Matrix(ctx, weights["spectral_in.weight"], weights["spectral_in.bias"])
    m_f = ien.Matrix(ctx, weights["fourier.weight"], weights["fourier.bias"])
    m_out = ien.Matrix(ctx, weights["spectral_out.weight"])
    sp = ien.Spectral(ctx, h, w)
    d_x = torch.from_numpy(x).half().cuda()
    d_out = torch.from_numpy(base).half().cuda()
    d_spectral = torch.empty((h, w, SPECTRAL), dtype=torch.float16, device="cuda")
    work = torch.empty(sp.work_floats, dtype=torch.float32, device="cuda")
    sp.run(d_x[..., LOCAL:], CHANNELS, m_in, m_f, m_out, d_spectral, work, d_out[..., LOCAL:], CHANNELS)
    torch.cuda.synchronize()
    got = d_out.float().cpu().numpy()
    # The local channels are untouched.
    assert np.array_equal(got[..., :LOCAL], base[..., :LOCAL])
    want = oracle_chain(oracle, np.ascontiguousarray(x[..., LOCAL:]),
                        np.ascontiguousarray(base[..., LOCAL:]), weights)
    r, m = spread_errors(got[..., LOCAL:], want)
    print(f"  rms/std {r:.3g}, max/peak {m:.3g}", flush=True)
    assert r <= 2e-3 and m <= 1e-2, (r, m)
    # The spectral map the call leaves behind is the spectral_in product.
    from oracle.oracle import ACT_RELU
    s_want = f16(oracle.multiply_rows(np.ascontiguousarray(x[..., LOCAL:]).reshape(h * w, GLOBAL),
                                      weights["spectral_in.weight"], weights["spectral_in.bias"],
                                      act=ACT_RELU))
    s_got = d_spectral.float().cpu().numpy().reshape(h, SPECTRAL, w).transpose(0, 2, 1).reshape(h * w, SPECTRAL)
    assert float(np.abs(s_got - s_want).max()) <= 2e-3 * float(np.abs(s_want).max()) + 1e-3
    for o in (sp, m_in, m_f, m_out):
        o.free()


@pytest.mark.parametrize("h,w", [(64, 64), (12, 16), (9, 23)])
def test_spectral_matches_unfused_chain(ctx, weights, h, w):
    """The same outputs as the unfused GPU chain: products through
    ien_multiply and the Fourier units' four passes."""
    import torch
    import ien

    rng = np.random.default_rng(h + w)
    x = f16(rng.standard_normal((h, w, CHANNELS)))
    base = f16(rng.standard_normal((h, w, CHANNELS)))
    m_in = ien.Matrix(ctx, weights["spectral_in.weight"], weights["spectral_in.bias"])
    m_f = ien.Matrix(ctx, weights["fourier.weight"], weights["fourier.bias"])
    m_out = ien.Matrix(ctx, weights["spectral_out.weight"])
    d_x = torch.from_numpy(x).half().cuda()
    # Fused.
    sp = ien.Spectral(ctx, h, w)
    d_a = torch.from_numpy(base).half().cuda()
    d_spectral = torch.empty((h, w, SPECTRAL), dtype=torch.float16, device="cuda")
    work = torch.empty(sp.work_floats, dtype=torch.float32, device="cuda")
    sp.run(d_x[..., LOCAL:], CHANNELS, m_in, m_f, m_out, d_spectral, work, d_a[..., LOCAL:], CHANNELS)
    # Unfused.
    f = ien.Fourier(ctx, h, w)
    half = w // 2 + 1
    d_b = torch.from_numpy(base).half().cuda()
    spectral = torch.empty((h, w, SPECTRAL), dtype=torch.float16, device="cuda")
    spectrum = torch.empty((h, half, 2 * SPECTRAL), dtype=torch.float16, device="cuda")
    filtered = torch.empty_like(spectrum)
    work2 = torch.empty(h * half * 2 * SPECTRAL, dtype=torch.float32, device="cuda")
    ien.multiply(ctx, ien.rows_input(d_x[..., LOCAL:], CHANNELS), 0, h * w, m_in, spectral, SPECTRAL,
                 act=ien.ACT_RELU)
    f.forward(spectral, SPECTRAL, SPECTRAL, work2, spectrum)
    ien.multiply(ctx, ien.rows_input(spectrum, 2 * SPECTRAL), 0, h * half, m_f, filtered, 2 * SPECTRAL,
                 act=ien.ACT_RELU)
    f.inverse(filtered, SPECTRAL, work2, spectral, SPECTRAL)
    ien.multiply(ctx, ien.rows_input(spectral, SPECTRAL), 0, h * w, m_out, d_b[..., LOCAL:], CHANNELS,
                 act=ien.ACT_RELU, accumulate=True)
    torch.cuda.synchronize()
    a = d_a.float().cpu().numpy()
    b = d_b.float().cpu().numpy()
    r, m = spread_errors(a[..., LOCAL:], b[..., LOCAL:])
    print(f"fused vs unfused {h}x{w}: rms/std {r:.3g}, max/peak {m:.3g}", flush=True)
    assert r <= 2e-3 and m <= 1e-2, (r, m)
    for o in (sp, f, m_in, m_f, m_out):
        o.free()


def test_spectral_rejects_bad_arguments(ctx, weights):
    import torch
    import ien

    with pytest.raises(ien.IenError) as e:
        ien.Spectral(ctx, 65, 8)
    assert e.value.status == ien.ERR_INPUT
    with pytest.raises(ien.IenError):
        ien.Spectral(ctx, 8, 0)
    sp = ien.Spectral(ctx, 8, 8)
    m_in = ien.Matrix(ctx, weights["spectral_in.weight"], weights["spectral_in.bias"])
    m_f = ien.Matrix(ctx, weights["fourier.weight"], weights["fourier.bias"])
    m_out = ien.Matrix(ctx, weights["spectral_out.weight"])
    d_x = torch.zeros((8, 8, CHANNELS), dtype=torch.float16, device="cuda")
    d_s = torch.empty((8, 8, SPECTRAL), dtype=torch.float16, device="cuda")
    work = torch.empty(sp.work_floats, dtype=torch.float32, device="cuda")
    with pytest.raises(ien.IenError) as e:  # the matrices swapped
        sp.run(d_x, CHANNELS, m_f, m_in, m_out, d_s, work, d_x, CHANNELS)
    assert e.value.status == ien.ERR_INPUT
    with pytest.raises(ien.IenError):  # a pixel stride below the channels
        sp.run(d_x, 256, m_in, m_f, m_out, d_s, work, d_x[..., LOCAL:], CHANNELS)
    for o in (sp, m_in, m_f, m_out):
        o.free()
