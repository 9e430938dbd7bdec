"""GPU parity of the implicit-GEMM MFMA product (ien_multiply_ex,
ien_multiply, ien_conv3) against the oracle's gemm::multiply / conv3 on the
same seeded, f16-representable inputs.

The oracle sums in f32 in the reference's order; the GPU sums f16 products
in f32 on MFMA in another order and stores f16.  Bound: |gpu - oracle| <=
2e-3 |oracle| + 2e-3 for f16 outputs (half an f16 ulp is 2^-11 relative,
plus reordering), 1e-4 (1 + |oracle|) for f32 outputs.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def case(seed, h, w, c, n, taps):
    rng = np.random.default_rng(seed)
    x = f16(rng.standard_normal((h, w, c)))
    wt = f16(rng.standard_normal((taps * c, n)) / np.sqrt(taps * c))
    b = rng.standard_normal(n).astype(np.float32) * 0.1
    return x, wt, b


def run_gpu(ctx, x, wt, b, size=3, step=1, pad=0, offsets=None, act=0, slope=None, nchw_in=False,
            nchw_out=False, out_f32=False, init=None, row0=0, rows=None, stride_pad=0, out_pad=None):
    import torch
    import ien

    h, wd, c = x.shape
    n = wt.shape[1]
    if offsets is None:
        oh, ow = (h - 1) // step + 1, (wd - 1) // step + 1
    else:
        oh, ow = h, wd
    total = oh * ow
    rows = total - row0 if rows is None else rows
    if nchw_in:
        xt = torch.from_numpy(np.ascontiguousarray(x.transpose(2, 0, 1))).half().cuda()
        inp = ien.image_input(xt, h, wd, c, layout=ien.NCHW, size=size, step=step, pad=pad, offsets=offsets)
    else:
        xs = c + stride_pad
        xp = np.zeros((h, wd, xs), np.float32)
        xp[..., :c] = x
        xt = torch.from_numpy(xp).half().cuda()
        inp = ien.image_input(xt, h, wd, c, stride=xs, size=size, step=step, pad=pad, offsets=offsets)
    m = ien.Matrix(ctx, wt, b)
    dt = torch.float32 if out_f32 else torch.float16
    if nchw_out:
        out = torch.zeros((n, rows), dtype=dt, device="cuda")
        if init is not None:
            out.copy_(torch.from_numpy(init[row0:row0 + rows].T.copy()))
        ostride = rows
    else:
        ostride = n + (stride_pad if out_pad is None else out_pad)
        out = torch.zeros((rows, ostride), dtype=dt, device="cuda")
        if init is not None:
            out[:, :n].copy_(torch.from_numpy(init[row0:row0 + rows]))
    sl = None if slope is None else torch.from_numpy(slope).cuda()
    ien.multiply_ex(ctx, inp, row0, rows, m, out, ostride, layout=ien.NCHW if nchw_out else ien.NHWC,
                    out_f32=out_f32, act=act, slope=sl, accumulate=init is not None)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    got = got.T if nchw_out else got[:, :n]
    m.free()
    return got


def want_cpu(oracle, x, wt, b, size=3, step=1, pad=0, offsets=None, act=0, slope=None, init=None):
    import ien

    oact = {ien.ACT_NONE: oracle.ACT_NONE, ien.ACT_RELU: oracle.ACT_RELU, ien.ACT_GELU: oracle.ACT_GELU}
    y = oracle.multiply_conv(x, wt, b, size=size, step=step, pad=pad, offsets=offsets,
                             act=oact.get(act, oracle.ACT_NONE),
                             out=None if init is None else init, accumulate=init is not None)
    y = y.reshape(-1, wt.shape[1])
    if act == ien.ACT_PRELU:
        y = np.where(y < 0, y * slope[None, :], y)
    if act == ien.ACT_SIGMOID:
        y = oracle.sigmoid(y)
    return y


def close(got, want, f32=False):
    err = np.abs(got - want)
    bound = (1e-4 * (1 + np.abs(want))) if f32 else (2e-3 * np.abs(want) + 2e-3)
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} of {bad.size} off; max err {err.max():.3g}"


@pytest.mark.parametrize("h,w,c,n", [(8, 96, 64, 64), (12, 192, 64, 48), (7, 45, 64, 64), (9, 33, 32, 80),
                                     (5, 40, 128, 128), (4, 17, 48, 16)])
def test_conv3x3_nhwc(ctx, oracle, h, w, c, n):
    x, wt, b = case(1, h, w, c, n, 9)
    close(run_gpu(ctx, x, wt, b), want_cpu(oracle, x, wt, b))


# Launches that fill the CUs at most once stage their channel chunks
# double-buffered (the small cases above); a grid of 384 tiles takes the
# single-buffered kernel.
def test_conv3x3_large_grid(ctx, oracle):
    x, wt, b = case(12, 128, 192, 128, 128, 9)
    close(run_gpu(ctx, x, wt, b, pad=1), want_cpu(oracle, x, wt, b, pad=1))


# A small map with a deep reduction (LaMa's FFC local convolution: 64 x 64,
# 512 -> 128, reflect padding) runs in 4 splits of the channels whose
# partial sums each tile's last split adds (no finishing pass): against the
# oracle, plain and with ReLU onto an accumulated output, and bit for bit
# the same over repeated launches (the sums are added in split order,
# whichever split comes last).
@pytest.mark.parametrize("act,acc", [(0, False), (1, True)])
def test_split_k_counted_in(ctx, oracle, act, acc):
    x, wt, b = case(21, 64, 64, 512, 128, 9)
    init = (np.random.default_rng(22).standard_normal((64 * 64, 128)) * 0.5).astype(np.float16).astype(
        np.float32) if acc else None
    runs = [run_gpu(ctx, x, wt, b, pad=1, act=act, init=init) for _ in range(3)]
    close(runs[0], want_cpu(oracle, x, wt, b, pad=1, act=act, init=None if init is None else init.copy()))
    assert all(np.array_equal(r.view(np.uint32), runs[0].view(np.uint32)) for r in runs[1:])


@pytest.mark.parametrize("c", [3, 4, 8, 16])
def test_conv3x3_few_channels(ctx, oracle, c):
    x, wt, b = case(2, 11, 37, c, 64, 9)
    close(run_gpu(ctx, x, wt, b), want_cpu(oracle, x, wt, b))


@pytest.mark.parametrize("act", [1, 2, 3, 4])
def test_activations_and_accumulate(ctx, oracle, act):
    import ien

    x, wt, b = case(3, 6, 40, 64, 64, 9)
    slope = np.linspace(0.05, 0.5, 64).astype(np.float32)
    init = f16(np.random.default_rng(9).standard_normal((6 * 40, 64)))
    got = run_gpu(ctx, x, wt, b, act=act, slope=slope, init=init)
    want = want_cpu(oracle, x, wt, b, act=act, slope=slope, init=init)
    close(got, want)


# The resident kernel's accumulating path (old outputs staged one tile
# ahead for 16 and 32 input channels; element-wise stores at 64): ragged
# tiles, several tiles per CU, activations after the sum, a padded output
# stride.
@pytest.mark.parametrize("c,n,h,w,act,pad", [(32, 32, 7, 130, 0, 0), (32, 64, 33, 64, 1, 8),
                                            (16, 48, 20, 100, 3, 0), (32, 32, 320, 330, 0, 0),
                                            (16, 16, 65, 63, 2, 8), (64, 64, 7, 130, 0, 0),
                                            (64, 48, 33, 64, 1, 8), (64, 64, 200, 260, 2, 0)])
def test_resident_accumulate(ctx, oracle, c, n, h, w, act, pad):
    x, wt, b = case(11 + c + n, h, w, c, n, 9)
    slope = np.linspace(0.05, 0.5, n).astype(np.float32)
    init = f16(np.random.default_rng(h + w).standard_normal((h * w, n)))
    got = run_gpu(ctx, x, wt, b, act=act, slope=slope, init=init, stride_pad=pad)
    want = want_cpu(oracle, x, wt, b, act=act, slope=slope, init=init)
    close(got, want)


# The resident kernel's half mode (32 input channels, at most 32 outputs,
# not accumulating: every wave on the 32 channels, 4-row tiles): ragged
# tiles, fewer outputs, activations, padded strides, several tiles a CU.
@pytest.mark.parametrize("n,h,w,act,pad", [(32, 33, 70, 1, 0), (24, 9, 64, 3, 8), (16, 5, 130, 0, 0),
                                           (32, 200, 260, 1, 8)])
def test_resident_half(ctx, oracle, n, h, w, act, pad):
    x, wt, b = case(21 + n + h, h, w, 32, n, 9)
    slope = np.linspace(-0.2, 0.4, n).astype(np.float32)
    got = run_gpu(ctx, x, wt, b, act=act, slope=slope, stride_pad=pad)
    close(got, want_cpu(oracle, x, wt, b, act=act, slope=slope))


def test_nchw_in_and_out(ctx, oracle):
    import ien

    x, wt, b = case(4, 16, 96, 64, 64, 9)
    want = want_cpu(oracle, x, wt, b)
    close(run_gpu(ctx, x, wt, b, nchw_in=True, nchw_out=True), want)
    close(run_gpu(ctx, x, wt, b, nchw_in=True, nchw_out=True, out_f32=True), want, f32=False)


# NCHW 1 x 1 (the conv sweep's 256 -> 512): NCHW outputs through the
# register-transposing kernel, NHWC outputs through the general one.
def test_nchw_1x1(ctx, oracle):
    x, wt, b = case(13, 16, 64, 256, 512, 1)
    want = want_cpu(oracle, x, wt, b, size=1)
    close(run_gpu(ctx, x, wt, b, size=1, nchw_in=True, nchw_out=True), want)
    close(run_gpu(ctx, x, wt, b, size=1, nchw_in=True), want)


# The register-transposing NCHW 1 x 1 kernel (whole planes, NCHW f16 out,
# not accumulating): channel counts that leave a partial 128-channel chunk
# (48, 208), output counts that leave a partial 128-channel tile (40, 96,
# 200), pixel counts that leave a partial 64-pixel tile (104, 24), one
# chunk and four, every activation.
@pytest.mark.parametrize("h,w,c,n,act", [(8, 13, 48, 40, 0), (16, 64, 208, 96, 1), (4, 6, 16, 200, 2),
                                         (32, 32, 512, 128, 3), (64, 64, 256, 512, 4)])
def test_nchw_1x1_planes(ctx, oracle, h, w, c, n, act):
    x, wt, b = case(40 + c + n, h, w, c, n, 1)
    slope = np.linspace(-0.3, 0.3, n).astype(np.float32)
    want = want_cpu(oracle, x, wt, b, size=1, act=act, slope=slope)
    close(run_gpu(ctx, x, wt, b, size=1, act=act, slope=slope, nchw_in=True, nchw_out=True), want)


# NCHW 3 x 3 in and out over whole planes: odd heights, widths that leave a
# partial 32-pixel tile, output counts that leave a partial 64-channel
# tile, one tile and many, every activation.
@pytest.mark.parametrize("h,w,c,n,act", [(5, 40, 64, 64, 0), (9, 24, 32, 40, 1), (16, 96, 64, 200, 2),
                                         (64, 128, 32, 96, 3), (128, 192, 64, 64, 4), (1, 8, 64, 32, 0)])
def test_nchw_3x3_planes(ctx, oracle, h, w, c, n, act):
    x, wt, b = case(60 + h + c + n, h, w, c, n, 9)
    slope = np.linspace(-0.3, 0.3, n).astype(np.float32)
    want = want_cpu(oracle, x, wt, b, act=act, slope=slope)
    close(run_gpu(ctx, x, wt, b, act=act, slope=slope, nchw_in=True, nchw_out=True), want)


# The NCHW 3 x 3 64 -> 64 kernel (4 x 96 tiles, the layer's weights in
# LDS): heights that leave a partial 4-row tile, widths (multiples of 8)
# that leave a partial 96-pixel tile or fall short of one, every
# activation.
@pytest.mark.parametrize("h,w,act", [(4, 96, 0), (7, 200, 1), (13, 104, 3), (3, 8, 2), (10, 392, 4),
                                     (33, 16, 3)])
def test_nchw_3x3_64(ctx, oracle, h, w, act):
    x, wt, b = case(90 + h + w, h, w, 64, 64, 9)
    slope = np.linspace(-0.3, 0.3, 64).astype(np.float32)
    want = want_cpu(oracle, x, wt, b, act=act, slope=slope)
    close(run_gpu(ctx, x, wt, b, act=act, slope=slope, nchw_in=True, nchw_out=True), want)


# The NCHW 3 x 3 128 -> 128 kernel (2 x 96 tiles a channel half, K in four
# double-buffered quarters): heights that leave a partial 2-row tile, widths
# (multiples of 8) that leave a partial 96-pixel tile or fall short of one,
# every activation.
@pytest.mark.parametrize("h,w,act", [(2, 96, 0), (5, 200, 1), (9, 104, 3), (3, 8, 2), (6, 392, 4),
                                     (1, 16, 3)])
def test_nchw_3x3_128(ctx, oracle, h, w, act):
    x, wt, b = case(190 + h + w, h, w, 128, 128, 9)
    slope = np.linspace(-0.3, 0.3, 128).astype(np.float32)
    want = want_cpu(oracle, x, wt, b, act=act, slope=slope)
    close(run_gpu(ctx, x, wt, b, act=act, slope=slope, nchw_in=True, nchw_out=True), want)


# Where that kernel does not apply, the general one runs: a row range, an
# accumulating product, f32 outputs, pixel counts not a multiple of 8.
def test_nchw_1x1_other_forms(ctx, oracle):
    x, wt, b = case(77, 8, 16, 64, 96, 1)
    want = want_cpu(oracle, x, wt, b, size=1)
    close(run_gpu(ctx, x, wt, b, size=1, nchw_in=True, nchw_out=True, row0=8, rows=64), want[8:72])
    init = np.random.default_rng(3).standard_normal((8 * 16, 96)).astype(np.float16).astype(np.float32)
    want2 = want_cpu(oracle, x, wt, b, size=1, init=init)
    close(run_gpu(ctx, x, wt, b, size=1, nchw_in=True, nchw_out=True, init=init), want2)
    close(run_gpu(ctx, x, wt, b, size=1, nchw_in=True, nchw_out=True, out_f32=True), want, f32=False)
    x3, wt3, b3 = case(78, 3, 5, 32, 64, 1)
    close(run_gpu(ctx, x3, wt3, b3, size=1, nchw_in=True, nchw_out=True), want_cpu(oracle, x3, wt3, b3, size=1))


def test_f32_output_and_strides(ctx, oracle):
    x, wt, b = case(5, 9, 50, 32, 40, 9)
    want = want_cpu(oracle, x, wt, b)
    close(run_gpu(ctx, x, wt, b, out_f32=True, stride_pad=8), want, f32=True)


def test_row_range(ctx, oracle):
    x, wt, b = case(6, 10, 30, 64, 64, 9)
    want = want_cpu(oracle, x, wt, b)
    got = run_gpu(ctx, x, wt, b, row0=47, rows=133)
    close(got, want[47:180])


@pytest.mark.parametrize("pad", [0, 1])
def test_stride2(ctx, oracle, pad):
    x, wt, b = case(7, 13, 34, 64, 32, 9)
    close(run_gpu(ctx, x, wt, b, step=2, pad=pad), want_cpu(oracle, x, wt, b, step=2, pad=pad))


def test_reflect_3x3(ctx, oracle):
    x, wt, b = case(8, 9, 70, 64, 64, 9)
    close(run_gpu(ctx, x, wt, b, pad=1), want_cpu(oracle, x, wt, b, pad=1))


@pytest.mark.parametrize("c,pad", [(4, 1), (64, 1), (64, 0)])
def test_conv7x7(ctx, oracle, c, pad):
    x, wt, b = case(9, 12, 40, c, 64, 49)
    close(run_gpu(ctx, x, wt, b, size=7, pad=pad), want_cpu(oracle, x, wt, b, size=7, pad=pad))


# Four input channels (conv_narrow: K = taps x 4 dense on MFMA, the models'
# image inputs): 3x3, 5x5 and 7x7, zero and reflect padding, ragged 8 x 32
# tiles, two 64-channel output tiles, 48 outputs, a padded input stride
# (12 halves), activations after the old output.
@pytest.mark.parametrize("size,pad,h,w,n,act,acc,sp", [
    (7, 1, 37, 70, 64, "RELU", False, 0),    # LaMa's first conv
    (3, 0, 21, 45, 64, "NONE", True, 8),     # SCUNet's head, added a second time
    (5, 1, 9, 33, 128, "PRELU", False, 0),
    (3, 1, 64, 96, 48, "GELU", True, 0),
    (7, 0, 5, 7, 64, "SIGMOID", False, 8),   # smaller than one tile
])
def test_conv_four_channels(ctx, oracle, size, pad, h, w, n, act, acc, sp):
    import ien

    act = getattr(ien, "ACT_" + act)
    x, wt, b = case(40 + size + n, h, w, 4, n, size * size)
    slope = np.linspace(-0.3, 0.5, n).astype(np.float32)
    init = f16(np.random.default_rng(h * w).standard_normal((h * w, n))) if acc else None
    got = run_gpu(ctx, x, wt, b, size=size, pad=pad, act=act, slope=slope, init=init, stride_pad=sp)
    close(got, want_cpu(oracle, x, wt, b, size=size, pad=pad, act=act, slope=slope, init=init))


# Few outputs (conv_few: (output, kx) pairs as the MFMA rows, the kx sum read
# back from LDS; the models' last convolutions): 7x7 and 3x3, reflect and
# zero padding, 1 to 10 outputs, output strides of 3, 4 and 10 halves or f32,
# images narrower than one 58- or 62-column item and several items a row,
# and images of more items than the GPU has CUs (a workgroup then goes down
# its column tile reusing staged rows; the odd row-group counts put runs
# across tile boundaries).
@pytest.mark.parametrize("size,pad,h,w,n,act,acc,f32,op", [
    (7, 1, 500, 130, 3, "SIGMOID", False, False, 0),
    (3, 0, 402, 200, 3, "NONE", True, False, 1),
    (7, 1, 40, 130, 3, "SIGMOID", False, False, 0),  # LaMa's last conv
    (3, 0, 33, 70, 3, "NONE", False, False, 1),      # SCUNet's tail (output stride 4)
    (3, 1, 12, 61, 10, "RELU", True, False, 0),
    (7, 0, 9, 58, 4, "NONE", True, True, 0),
    (3, 0, 5, 5, 1, "GELU", False, True, 0),
    (7, 1, 17, 200, 2, "PRELU", False, False, 0),
])
def test_conv_few_outputs(ctx, oracle, size, pad, h, w, n, act, acc, f32, op):
    import ien

    act = getattr(ien, "ACT_" + act)
    x, wt, b = case(60 + size + n, h, w, 64, n, size * size)
    slope = np.linspace(-0.3, 0.5, n).astype(np.float32)
    init = f16(np.random.default_rng(h + w).standard_normal((h * w, n))) if acc else None
    got = run_gpu(ctx, x, wt, b, size=size, pad=pad, act=act, slope=slope, init=init, out_f32=f32,
                  out_pad=op)
    close(got, want_cpu(oracle, x, wt, b, size=size, pad=pad, act=act, slope=slope, init=init))


def test_1x1(ctx, oracle):
    x, wt, b = case(10, 16, 64, 256, 512, 1)
    close(run_gpu(ctx, x, wt, b, size=1), want_cpu(oracle, x, wt, b, size=1))


@pytest.mark.parametrize("offsets", [[(0, 0)], [(0, 0), (0, 1)], [(0, 0), (1, 0), (0, 1), (1, 1)]])
def test_offset_taps(ctx, oracle, offsets):
    x, wt, b = case(11, 9, 40, 64, 64, len(offsets))
    close(run_gpu(ctx, x, wt, b, offsets=offsets), want_cpu(oracle, x, wt, b, offsets=offsets))


@pytest.mark.parametrize("m,k,n", [(1, 16, 1), (100, 64, 96), (333, 256, 128), (64, 48, 96), (70, 40, 20)])
def test_rows(ctx, oracle, m, k, n):
    import torch
    import ien

    rng = np.random.default_rng(12)
    a = f16(rng.standard_normal((m, k)))
    wt = f16(rng.standard_normal((k, n)) / np.sqrt(k))
    b = rng.standard_normal(n).astype(np.float32)
    want = oracle.multiply_rows(a, wt, b, act=oracle.ACT_GELU)
    stride = k + (8 if k % 8 == 0 else 0)
    ap = np.zeros((m, stride), np.float32)
    ap[:, :k] = a
    at = torch.from_numpy(ap).half().cuda()
    mat = ien.Matrix(ctx, wt, b)
    out = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    ien.multiply(ctx, ien.rows_input(at, stride), 0, m, mat, out, n, act=ien.ACT_GELU)
    torch.cuda.synchronize()
    close(out.float().cpu().numpy(), want)


# A deep product with a small output (64 rows, 4096 deep, 64 wide): one tile
# in 8 splits of the reduction, whose finishing pass takes 8 lanes an item
# (strided splits, then a fixed group sum): against the oracle with ReLU
# onto an accumulated output, and bit for bit the same over repeats.
def test_deep_split_small_output(ctx, oracle):
    import torch
    import ien

    rng = np.random.default_rng(31)
    m, k, n = 64, 4096, 64
    a = f16(rng.standard_normal((m, k)))
    wt = f16(rng.standard_normal((k, n)) / np.sqrt(k))
    b = rng.standard_normal(n).astype(np.float32)
    init = f16(rng.standard_normal((m, n)))
    want = oracle.multiply_rows(a, wt, b, act=oracle.ACT_RELU, out=init.copy(), accumulate=True)
    at = torch.from_numpy(a).half().cuda()
    mat = ien.Matrix(ctx, wt, b)
    runs = []
    for _ in range(3):
        out = torch.from_numpy(init).half().cuda()
        ien.multiply(ctx, ien.rows_input(at, k), 0, m, mat, out, n, act=ien.ACT_RELU, accumulate=True)
        torch.cuda.synchronize()
        runs.append(out.float().cpu().numpy())
    mat.free()
    close(runs[0], want)
    assert all(np.array_equal(r, runs[0]) for r in runs[1:])


# Row products with enough tiles for the pipelined row kernel: 128 x 64
# tiles (N <= 64), 64 x 128 tiles (wider N) and, with K at least 512 deep
# and few tiles, split-K into the finishing pass (the last three), K a
# multiple of 64 or only of 32, ragged last tiles in M and N,
# accumulation, activations, padded strides and row ranges that start past
# row 0.
@pytest.mark.parametrize("m,k,n,act,acc,row0,pad", [
    (16500, 256, 128, 2, False, 0, 8), (33000, 64, 64, 0, True, 0, 0),
    (20000, 96, 96, 3, True, 0, 8), (17000, 160, 40, 1, False, 0, 0),
    (17000, 128, 256, 0, True, 1000, 8),
    (4096, 384, 192, 1, False, 0, 0), (4096, 192, 384, 1, True, 0, 8), (6100, 96, 256, 2, False, 37, 0),
    (1024, 768, 384, 0, False, 0, 0), (2000, 3072, 768, 2, True, 5, 8), (1000, 1536, 96, 3, True, 0, 0)])
def test_rows_tiles(ctx, oracle, m, k, n, act, acc, row0, pad):
    import torch
    import ien

    rng = np.random.default_rng(m + k + n)
    total = row0 + m
    a = f16(rng.standard_normal((total, k)))
    wt = f16(rng.standard_normal((k, n)) / np.sqrt(k))
    b = rng.standard_normal(n).astype(np.float32) * 0.1
    slope = np.linspace(0.05, 0.5, n).astype(np.float32)
    init = f16(rng.standard_normal((m, n))) if acc else None
    oact = {0: oracle.ACT_NONE, 1: oracle.ACT_RELU, 2: oracle.ACT_GELU, 3: oracle.ACT_NONE}[act]
    want = oracle.multiply_rows(a[row0:], wt, b, act=oact, out=None if init is None else init.copy(),
                                accumulate=acc, threads=8)
    if act == 3:
        want = np.where(want < 0, want * slope[None, :], want)
    xs, ys = k + pad, n + pad
    ap = np.zeros((total, xs), np.float32)
    ap[:, :k] = a
    at = torch.from_numpy(ap).half().cuda()
    mat = ien.Matrix(ctx, wt, b)
    out = torch.zeros((m, ys), dtype=torch.float16, device="cuda")
    if acc:
        out[:, :n].copy_(torch.from_numpy(init))
    sl = torch.from_numpy(slope).cuda()
    ien.multiply_ex(ctx, ien.rows_input(at, xs), row0, m, mat, out, ys, act=act, slope=sl if act == 3 else None,
                    accumulate=acc)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    mat.free()
    assert np.all(got[:, n:] == 0)  # padding columns untouched
    close(got[:, :n], want)


# Split-K: few output tiles and several channel chunks, so the reduction is
# spread over workgroups, summed by the finishing pass, then bias,
# accumulate and activation.
@pytest.mark.parametrize("act", [0, 1, 3])
def test_splitk_conv3_accumulate(ctx, oracle, act):
    x, wt, b = case(14, 6, 32, 512, 64, 9)
    slope = np.linspace(0.05, 0.5, 64).astype(np.float32)
    init = f16(np.random.default_rng(15).standard_normal((6 * 32, 64)))
    got = run_gpu(ctx, x, wt, b, act=act, slope=slope, init=init)
    close(got, want_cpu(oracle, x, wt, b, act=act, slope=slope, init=init))


def test_splitk_nchw_f32_reflect_rows(ctx, oracle):
    x, wt, b = case(16, 8, 32, 256, 96, 9)
    want = want_cpu(oracle, x, wt, b)
    close(run_gpu(ctx, x, wt, b, nchw_in=True, nchw_out=True), want)
    close(run_gpu(ctx, x, wt, b, out_f32=True, stride_pad=8), want, f32=True)
    close(run_gpu(ctx, x, wt, b, pad=1), want_cpu(oracle, x, wt, b, pad=1))
    close(run_gpu(ctx, x, wt, b, row0=37, rows=150), want[37:187])


# The NCHW finishing pass (32 pixels x 32 channels a workgroup, transposed
# through LDS): ragged pixel blocks and channel groups, accumulating, f16
# and f32 outputs.
@pytest.mark.parametrize("f32", [False, True])
def test_splitk_nchw_out_accumulate(ctx, oracle, f32):
    import ien

    x, wt, b = case(19, 7, 30, 512, 80, 9)
    slope = np.linspace(-0.2, 0.4, 80).astype(np.float32)
    init = f16(np.random.default_rng(20).standard_normal((7 * 30, 80)))
    got = run_gpu(ctx, x, wt, b, act=ien.ACT_PRELU, slope=slope, init=init, nchw_in=True,
                  nchw_out=True, out_f32=f32)
    close(got, want_cpu(oracle, x, wt, b, act=ien.ACT_PRELU, slope=slope, init=init))


def test_splitk_offsets_and_rows(ctx, oracle):
    import torch
    import ien

    offsets = [(0, 0), (1, 0), (0, 1), (1, 1)]
    x, wt, b = case(17, 8, 16, 512, 64, 4)
    close(run_gpu(ctx, x, wt, b, offsets=offsets), want_cpu(oracle, x, wt, b, offsets=offsets))
    rng = np.random.default_rng(18)
    m, k, n = 100, 1024, 96
    a = f16(rng.standard_normal((m, k)))
    wt = f16(rng.standard_normal((k, n)) / np.sqrt(k))
    bias = rng.standard_normal(n).astype(np.float32)
    init = f16(rng.standard_normal((m, n)))
    want = oracle.multiply_rows(a, wt, bias, out=init.copy(), accumulate=True)
    mat = ien.Matrix(ctx, wt, bias)
    out = torch.from_numpy(init).half().cuda()
    ien.multiply(ctx, ien.rows_input(torch.from_numpy(a).half().cuda(), k), 0, m, mat, out, n,
                 accumulate=True)
    torch.cuda.synchronize()
    close(out.float().cpu().numpy(), want)


def test_conv3_finish_prelu(ctx, oracle):
    import torch
    import ien

    x, wt, b = case(13, 8, 96, 64, 64, 9)
    slope = np.full(64, 0.25, np.float32)
    want = oracle.conv3(x, wt, b, finish=oracle.FINISH_PRELU, slope=slope).reshape(-1, 64)
    xt = torch.from_numpy(x).half().cuda()
    m = ien.Matrix(ctx, wt, b)
    out = torch.zeros((8 * 96, 64), dtype=torch.float16, device="cuda")
    ien.conv3(ctx, ien.image_input(xt, 8, 96, 64), m, out, 64, finish=ien.ACT_PRELU,
              slope=torch.from_numpy(slope).cuda())
    torch.cuda.synchronize()
    close(out.float().cpu().numpy(), want)


def test_errors(ctx):
    import torch
    import ien

    x = torch.zeros((4, 4, 64), dtype=torch.float16, device="cuda")
    m = ien.Matrix(ctx, np.zeros((9 * 32, 16), np.float32))
    out = torch.zeros((16, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(ien.IenError) as e:
        ien.multiply(ctx, ien.image_input(x, 4, 4, 64), 0, 16, m, out, 16)
    assert e.value.status == ien.ERR_INPUT and "does not match" in str(e.value)
    with pytest.raises(ien.IenError):
        ien.multiply(ctx, ien.image_input(x, 4, 4, 32), 10, 16, m, out, 16)
