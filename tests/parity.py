"""Error bounds shared by the GPU parity tests.

The configuration's tolerance (max |error| <= 2e-2, PSNR >= 45 dB on [0, 1]
images) says little when an output's own spread is far below 1: SCUNet's
trunc-normal-0.02 network, for one, outputs values of about 0.1.  So every
model comparison also bounds the error by the output's spread: the error's
RMS against the reference output's standard deviation, and its maximum
against the reference output's largest magnitude.
"""

import numpy as np


def psnr(got, want, peak=1.0):
    mse = float(np.mean((np.asarray(got, np.float64) - np.asarray(want, np.float64)) ** 2))
    return 10 * np.log10(peak * peak / max(mse, 1e-30))


def spread_errors(got, want):
    """(rms error / std(want), max error / max |want|)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = got - want
    rms = float(np.sqrt(np.mean(err * err)))
    std = float(want.std())
    peak = float(np.abs(want).max())
    return rms / max(std, 1e-30), float(np.abs(err).max()) / max(peak, 1e-30)


def assert_spread(got, want, rms_frac=0.01, max_frac=0.05, what=""):
    """Error RMS <= rms_frac of std(want) and max error <= max_frac of
    max |want|."""
    r, m = spread_errors(got, want)
    assert r <= rms_frac and m <= max_frac, f"{what}: rms/std {r:.3g} (<= {rms_frac}), max/peak {m:.3g} (<= {max_frac})"
    return r, m


def assert_config_tolerance(got, want, peak=1.0, what=""):
    """The configuration's bar: max |error| <= 2e-2 * peak and PSNR >= 45 dB
    against `peak`."""
    err = float(np.abs(np.asarray(got, np.float64) - want).max())
    p = psnr(got, want, peak)
    assert err <= 2e-2 * peak and p >= 45.0, f"{what}: max err {err:.3g} (peak {peak}), PSNR {p:.1f} dB"
    return err, p
