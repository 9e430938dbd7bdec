"""ien_swin_run_static, the Swin block entry point that allocates nothing
(its scratch is the library's static device array), against ien_swin_run
on the same blocks and maps: two calls in a row, the second on a smaller
map, bit-identical to the allocating entry point (the same kernels run);
the device's free memory unchanged across the static calls; a map whose
scratch exceeds the static array refused with IEN_ERR_INPUT and left
untouched."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from test_gpu_swin import block_weights

STATIC_BYTES = 32 << 20  # IEN_SWIN_STATIC_SCRATCH_BYTES


def map_of(rng, h, w, c, stride):
    import torch

    x = rng.standard_normal((h * w, c)).astype(np.float16)
    md = torch.zeros((h * w, stride), dtype=torch.float16, device="cuda")
    md[:, :c] = torch.from_numpy(x).cuda()
    md[:, c:] = 3.0
    return md


@pytest.mark.parametrize("c,window,shift,masked,sizes", [
    (96, 12, 6, -100.0, [(40, 52), (24, 24)]),   # unfused attention (window 12), fused MLP
    (192, 7, 3, -100.0, [(28, 35), (14, 9)]),    # both halves unfused
    (384, 12, 0, -100.0, [(24, 36), (12, 12)]),  # both halves unfused, wide rows
    (32, 8, 4, -np.inf, [(32, 48), (16, 24)]),   # one fused pass: no scratch touched
])
def test_static_scratch_block_matches_allocating_block(ctx, c, window, shift, masked, sizes):
    import torch
    import ien

    rng = np.random.default_rng(c * 7 + window)
    wt = block_weights(rng, c, window)
    static = ien.Swin(ctx, c, window, shift, masked, wt)
    alloc = ien.Swin(ctx, c, window, shift, masked, wt)
    stride = c + 32
    for call, (h, w) in enumerate(sizes):
        print(f"no-alloc block c={c} window={window} shift={shift} map {h}x{w} call {call}", flush=True)
        a = map_of(rng, h, w, c, stride)
        b = a.clone()
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        static.run_static(a, stride, h, w)
        torch.cuda.synchronize()
        free_after = torch.cuda.mem_get_info()[0]
        if call > 0:
            assert free_after == free_before, (free_before, free_after)
        alloc.run(b, stride, h, w)
        torch.cuda.synchronize()
        got, want = a.cpu().numpy(), b.cpu().numpy()
        assert np.all(got[:, c:] == 3.0)
        assert np.array_equal(got, want), (h, w, float(np.abs(got.astype(np.float32) - want).max()))
    static.free()
    alloc.free()


def test_static_scratch_refuses_maps_past_its_size(ctx):
    import torch
    import ien

    c, window = 192, 7
    rng = np.random.default_rng(5)
    wt = block_weights(rng, c, window)
    blk = ien.Swin(ctx, c, window, 3, -100.0, wt)
    h = w = 126  # 18 x 18 windows of 49 rows: 15876 rows x 6c halves > 32 MiB
    assert 15876 * 6 * c * 2 > STATIC_BYTES
    md = map_of(rng, h, w, c, c)
    before = md.clone()
    with pytest.raises(ien.IenError) as e:
        blk.run_static(md, c, h, w)
    assert e.value.status == ien.ERR_INPUT and "static scratch" in str(e.value)
    torch.cuda.synchronize()
    assert torch.equal(md, before)
    blk.free()
