"""GPU parity of the conv sweep exactly as bench.py times it: every shape
built by bench.SweepCase (synthetic.sweep_case's seeded N(0, 1) f16 input
and weights, NCHW in and out, through ien_multiply_ex / ien_depthwise), so
the kernel variants, chunk widths and split-K counts chosen for these grid
sizes are the ones checked.  The oracle is gemm::multiply's direct product
(gemm.rs:514-667) for every convolution, plus winograd::conv3
(winograd.rs:612-773, F(4x4) or F(2x2) by the reference's policy) for the
3x3 shapes, and the direct depthwise sum.

Bounds: f16 outputs of N(0, 1) data summed over K = 256 .. 4608 products
have a spread of sqrt(K); the GPU stores f16 (half an ulp is 2^-11
relative) of f32 sums taken in another order.  Error RMS <= 1e-3 of the
output's standard deviation, max error <= 2e-3 of its largest magnitude,
and elementwise <= 2e-3 |want| + 2e-3 std(want).
"""

import numpy as np
import pytest

import synthetic
from parity import assert_spread

pytestmark = pytest.mark.gpu

SHAPES = [e[0] for e in synthetic.SWEEP]


@pytest.mark.parametrize("name", SHAPES)
def test_sweep_shape_matches_oracle(ctx, oracle, name):
    import torch
    from bench import SweepCase

    case = SweepCase(ctx, name)
    print(f"sweep case {name}", flush=True)
    case.launch()
    torch.cuda.synchronize()
    got = case.out.float().cpu().numpy().T.reshape(case.h, case.w, -1)
    case.free()
    x = np.ascontiguousarray(case.x.transpose(1, 2, 0))
    threads = oracle.threads_default()
    if case.kind == "conv":
        want = oracle.multiply_conv(x, case.wt, case.bias, size=case.size, threads=threads)
    else:
        want = oracle.depthwise(x, case.wt, case.bias, threads=threads)
    assert np.isfinite(got).all()
    assert_spread(got, want, rms_frac=1e-3, max_frac=2e-3, what=name)
    assert (np.abs(got - want) <= 2e-3 * np.abs(want) + 2e-3 * want.std()).all(), name
    if case.kind == "conv" and case.size == 3:
        # The reference runs 3x3 stride-1 convolutions through conv3.
        wino = oracle.conv3(x, case.wt, case.bias, threads=threads)
        assert_spread(got, wino, rms_frac=1e-3, max_frac=2e-3, what=name + " vs conv3")
