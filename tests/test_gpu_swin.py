"""GPU parity of a whole Swin transformer block (ien_swin: scunet swin.rs
Transformer::attend + mlp, birefnet swin.rs Block) against the oracle's
or_swin_attend followed by or_swin_mlp, on f16-rounded maps; a second run
on a larger map reuses the block (scratch grown on demand).  Window 8 with
32, 64 or 128 channels runs the fused per-window attention (at 32 with the
MLP in the same pass); 32, 64 and 96 channels otherwise the fused MLP pass;
the other widths and windows run the gather, q k v and attention of a
window and head in one pass (window_attend.hip), then the projection."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def block_weights(rng, c, window):
    n, heads = window * window, c // 32
    r = lambda *s, scale=1.0: (scale * rng.standard_normal(s)).astype(np.float32)
    return dict(ln1_gamma=1 + r(c, scale=0.1), ln1_beta=r(c, scale=0.1),
                qkv_w=r(c, 3 * c, scale=1 / np.sqrt(c)), qkv_b=r(3 * c, scale=0.1),
                position=r(heads, n, n), proj_w=r(c, c, scale=1 / np.sqrt(c)), proj_b=r(c, scale=0.1),
                ln2_gamma=1 + r(c, scale=0.1), ln2_beta=r(c, scale=0.1),
                fc1_w=r(c, 4 * c, scale=1 / np.sqrt(c)), fc1_b=r(4 * c, scale=0.1),
                fc2_w=r(4 * c, c, scale=0.5 / np.sqrt(4 * c)), fc2_b=r(c, scale=0.1))


def oracle_block(oracle, x, window, shift, masked, wt):
    tables = oracle.bias_tables(wt["position"], window, shift, masked)
    y = oracle.swin_attend(x, window, shift, wt["ln1_gamma"], wt["ln1_beta"], wt["qkv_w"], wt["qkv_b"], tables,
                           wt["proj_w"], wt["proj_b"])
    return oracle.swin_mlp(y, wt["ln2_gamma"], wt["ln2_beta"], wt["fc1_w"], wt["fc1_b"], wt["fc2_w"], wt["fc2_b"])


@pytest.mark.parametrize("c,window,shift,masked,sizes", [
    (64, 8, 4, -np.inf, [(16, 24), (32, 40)]),    # SCUNet SW-MSA
    (64, 8, 0, -np.inf, [(16, 16)]),              # SCUNet W-MSA
    (96, 7, 3, -100.0, [(10, 10), (14, 21)]),     # the reference's BiRefNet window
    (32, 12, 6, -100.0, [(15, 13), (24, 24)]),    # the configuration's BiRefNet window
    (32, 8, 4, -np.inf, [(16, 24), (12, 20)]),    # SCUNet level 1; windows past the map's edge
    (32, 8, 0, -np.inf, [(8, 8), (24, 16)]),      # one window, then several
    (128, 8, 4, -np.inf, [(16, 24), (20, 12)]),   # SCUNet level 3
    (256, 8, 0, -np.inf, [(8, 16), (9, 13)]),     # SCUNet body; a ragged last row block
    (192, 12, 6, -100.0, [(12, 24)]),             # Swin-T stage 2
    (384, 12, 0, -100.0, [(12, 12)]),             # Swin-T stage 3 (MLP through the row products)
    (768, 12, 6, -100.0, [(16, 16)]),             # Swin-T stage 4 of a 512 image: rows read three times
    (384, 7, 3, -100.0, [(10, 9)]),               # the reference's stage 3 window, rows read three times
])
def test_swin_block(ctx, oracle, c, window, shift, masked, sizes):
    import torch
    import ien

    rng = np.random.default_rng(c + window)
    wt = block_weights(rng, c, window)
    blk = ien.Swin(ctx, c, window, shift, masked, wt)
    for h, w in sizes:
        x = rng.standard_normal((h, w, c)).astype(np.float16)
        stride = c + 32
        md = torch.zeros((h * w, stride), dtype=torch.float16, device="cuda")
        md[:, :c] = torch.from_numpy(x.reshape(h * w, c)).cuda()
        md[:, c:] = 3.0
        blk.run(md, stride, h, w)
        torch.cuda.synchronize()
        got = md.float().cpu().numpy()
        assert np.all(got[:, c:] == 3.0)  # channels past c untouched
        want = oracle_block(oracle, x.astype(np.float32), window, shift, masked, wt)
        err = np.abs(got[:, :c].reshape(h, w, c) - want)
        # The block's outputs reach 4-6 (unit-variance inputs plus the two
        # residual branches), where one f16 ulp is 2^-8 to 2^-7: the bound
        # is 2e-3 of the peak, about two ulps there (measured up to 3.5e-3
        # at peaks of 4-5.6, RMS under 5e-4).
        peak = max(1.0, float(np.abs(want).max()))
        assert err.max() < 2e-3 * peak, (h, w, err.max(), peak)
        assert np.sqrt(np.mean(err ** 2)) < 1e-3, (h, w)
    blk.free()


# Position biases gathered from a relative-position table, as both models'
# weights hold them (every entry of a cell's offset the same value), at
# windows 12, 7 and 8, shifted windows' region masks included.
@pytest.mark.parametrize("c,window,shift,masked,size", [
    (96, 12, 6, -100.0, (24, 30)),   # Swin-T stage 1 at window 12, shifted; windows past the edge
    (32, 12, 0, -100.0, (24, 24)),
    (96, 7, 3, -100.0, (14, 21)),
    (256, 8, 4, -np.inf, (16, 24)),  # SCUNet body, shifted
])
def test_swin_block_relative_bias(ctx, oracle, c, window, shift, masked, size):
    import torch
    import ien

    rng = np.random.default_rng(7 * c + window + shift)
    wt = block_weights(rng, c, window)
    heads, side = c // 32, 2 * window - 1
    rel = (0.5 * rng.standard_normal((side * side, heads))).astype(np.float32)
    wt["position"] = ien.position_bias(rel, heads, window, ien.POS_SWIN)
    blk = ien.Swin(ctx, c, window, shift, masked, wt)
    h, w = size
    x = rng.standard_normal((h, w, c)).astype(np.float16)
    md = torch.from_numpy(x.reshape(h * w, c)).cuda()
    blk.run(md, c, h, w)
    torch.cuda.synchronize()
    got = md.float().cpu().numpy().reshape(h, w, c)
    want = oracle_block(oracle, x.astype(np.float32), window, shift, masked, wt)
    err = np.abs(got - want)
    assert err.max() < 5e-2 and np.sqrt(np.mean(err ** 2)) < 6e-3, (err.max(), np.sqrt(np.mean(err ** 2)))
    blk.free()
