"""GPU parity of the Fourier units (ien_fourier_*, crates/lama-native/src/
fourier.rs) against the oracle's transforms on the same f16 inputs: odd and
even sides, a channel slice of a wider map (the FFC's spectral map), channel
counts that leave a partial group, and sides up to 1024 that take every
channel-group size.  The GPU stores spectra and maps in f16: the bound is
2e-3 of the largest value plus 1e-3."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [
    (64, 64, 192, 512),   # the FFC's spectral map at 512 x 512, one slice of 512
    (9, 10, 8, 8),
    (5, 7, 3, 3),
    (1, 8, 4, 4),
    (72, 40, 36, 40),
    (256, 200, 20, 24),
    (1024, 16, 8, 8),
    (4, 1024, 8, 8),
]


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def close(got, want):
    bound = 2e-3 * float(np.abs(want).max()) + 1e-3
    err = float(np.abs(got - want).max())
    assert err <= bound, (err, bound)


@pytest.mark.parametrize("h,w,c,stride", SHAPES)
def test_forward_matches_oracle(ctx, oracle, h, w, c, stride):
    import torch
    import ien

    rng = np.random.default_rng(h * 1000 + w)
    x = f16(rng.standard_normal((h, w, stride)))
    f = ien.Fourier(ctx, h, w)
    half = w // 2 + 1
    assert f.half == half
    d_x = torch.from_numpy(x).half().cuda()
    work = torch.empty(h * half * 2 * c, dtype=torch.float32, device="cuda")
    spec = torch.zeros((h, half, 2 * c), dtype=torch.float16, device="cuda")
    f.forward(d_x, stride, c, work, spec)
    torch.cuda.synchronize()
    want = oracle.rfft2(np.ascontiguousarray(x[..., :c]))
    close(spec.float().cpu().numpy(), want)
    f.free()


@pytest.mark.parametrize("h,w,c,stride", SHAPES)
def test_inverse_adds_like_oracle(ctx, oracle, h, w, c, stride):
    import torch
    import ien

    rng = np.random.default_rng(h * 1000 + w + 1)
    half = w // 2 + 1
    # Not Hermitian: the edge columns' imaginary parts must be dropped after
    # the column transform, as the oracle (and irfftn) do.
    s = f16(rng.standard_normal((h, half, 2 * c)))
    base = f16(rng.standard_normal((h, w, stride)))
    f = ien.Fourier(ctx, h, w)
    d_s = torch.from_numpy(s).half().cuda()
    d_out = torch.from_numpy(base).half().cuda()
    work = torch.empty(h * half * 2 * c, dtype=torch.float32, device="cuda")
    f.inverse(d_s, c, work, d_out, stride)
    torch.cuda.synchronize()
    got = d_out.float().cpu().numpy()
    want = np.ascontiguousarray(base[..., :c])
    oracle.irfft2_add(s, want)
    close(got[..., :c], want)
    # Channels past `c` in the wider map are untouched.
    assert np.array_equal(got[..., c:], base[..., c:])
    f.free()


def test_round_trip_64(ctx):
    """forward then inverse onto zeros gives the map back."""
    import torch
    import ien

    h, w, c = 64, 64, 192
    x = f16(np.random.default_rng(9).standard_normal((h, w, c)))
    f = ien.Fourier(ctx, h, w)
    half = f.half
    d_x = torch.from_numpy(x).half().cuda()
    work = torch.empty(h * half * 2 * c, dtype=torch.float32, device="cuda")
    spec = torch.empty((h, half, 2 * c), dtype=torch.float16, device="cuda")
    back = torch.zeros_like(d_x)
    f.forward(d_x, c, c, work, spec)
    f.inverse(spec, c, work, back, c)
    torch.cuda.synchronize()
    assert float((back.float() - d_x.float()).abs().max()) < 1e-2
    f.free()


def test_rejects_bad_sizes(ctx):
    import ien

    with pytest.raises(ien.IenError):
        ien.Fourier(ctx, 0, 8)
    with pytest.raises(ien.IenError):
        ien.Fourier(ctx, 8, 1025)
