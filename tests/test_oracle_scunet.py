"""Pin of the oracle's SCUNet U-Net (oracle/scunet.c, crates/scunet-native/
src/network.rs) against an independent torch restatement
(tests/scunet_torch.py): replicate padding and crop, the 28 Swin-Conv
blocks with shifted windows, the 2x2 halving and doubling convolutions,
skip adds and the head added before the tail."""

import numpy as np
import pytest

import synthetic
import scunet_torch


@pytest.mark.parametrize("init,h,w", [("fan", 64, 64), ("fan", 70, 90), ("trunc_normal", 64, 128)])
def test_scunet_matches_torch_restatement(oracle, init, h, w):
    t = synthetic.scunet_tensors(init=init)
    img = synthetic.scunet_image(h, w, seed=h + w)
    want = scunet_torch.run(t, img)
    got = oracle.scunet_run(t, synthetic.scunet_names(), img)
    assert got.shape == (h, w, 3)
    assert np.abs(got - want).max() < 1e-4 * max(1.0, float(np.abs(want).max()))
