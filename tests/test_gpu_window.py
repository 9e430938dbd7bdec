"""GPU parity of the Swin window path (crates/scunet-native/src/swin.rs,
crates/birefnet-native/src/swin.rs, native-engine attention.rs) against the
oracle, through the C ABI: the rolled, LayerNorm'd window gather; attention
over every window and head with the class bias tables; the residual
scatter; and the whole attention half of a block composed from them and the
row products.  Geometries: SCUNet 8/4 and 8/0, the reference's BiRefNet
7/3 and the configuration's 12/6 on maps that need padding."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEOMS = [(8, 4, 16, 24, 64), (8, 0, 16, 16, 64), (7, 3, 10, 10, 96), (12, 6, 15, 13, 32), (12, 0, 24, 24, 64)]


def masked_for(window):
    return -np.inf if window == 8 else -100.0


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def sources(oracle, window, shift, h, w, nwin):
    n = window * window
    return np.array([[oracle.window_source(k, i, window, shift, h, w) for i in range(n)] for k in range(nwin)])


@pytest.mark.parametrize("window,shift,h,w,c", GEOMS)
def test_window_gather(ctx, oracle, window, shift, h, w, c):
    import torch
    import ien

    rng = np.random.default_rng(window * 100 + shift)
    stride = c + 8
    x = f16(rng.standard_normal((h * w, stride)) * 2 + 0.3)
    g = (1 + 0.2 * rng.standard_normal(c)).astype(np.float32)
    b = (0.2 * rng.standard_normal(c)).astype(np.float32)
    win = ien.windows(window, shift, h, w)
    nwin, n = ien.window_count(win), window * window
    tok = torch.full((nwin * n, c), 7.0, dtype=torch.float16, device="cuda")
    ien.window_gather(ctx, win, torch.from_numpy(x).cuda(), stride, c, torch.from_numpy(g).cuda(),
                      torch.from_numpy(b).cuda(), tok)
    torch.cuda.synchronize()
    got = tok.float().cpu().numpy()
    src = sources(oracle, window, shift, h, w, nwin).reshape(-1)
    want = np.zeros((nwin * n, c), np.float32)
    valid = src >= 0
    want[valid] = oracle.layer_norm(x[src[valid], :c].astype(np.float32), g, b)
    assert np.all(got[~valid] == 0)
    err = np.abs(got - want)
    assert (err <= 2e-3 * np.abs(want) + 2e-3).all(), err.max()


def attention_want(oracle, qkv, tables, c, window, shift, h, w, nwin):
    n, heads = window * window, c // 32
    want = np.zeros((nwin * n, c), np.float32)
    q32 = qkv.astype(np.float32)
    for k in range(nwin):
        cls = oracle.window_class(k, window, shift, h, w)
        for hd in range(heads):
            want[k * n:(k + 1) * n] += oracle.attention(q32[k * n:(k + 1) * n], c, hd, tables[cls, hd])
    return want


@pytest.mark.parametrize("window,shift,h,w,c", GEOMS)
def test_window_attention(ctx, oracle, window, shift, h, w, c):
    import torch
    import ien

    rng = np.random.default_rng(window * 10 + shift + c)
    win = ien.windows(window, shift, h, w)
    nwin, n, heads = ien.window_count(win), window * window, c // 32
    qkv = f16(rng.standard_normal((nwin * n, 3 * c)))
    pos = rng.standard_normal((heads, n, n)).astype(np.float32)
    tables = ien.bias_tables(pos, window, shift, masked_for(window))
    out = torch.zeros((nwin * n, c), dtype=torch.float16, device="cuda")
    ien.window_attention(ctx, win, torch.from_numpy(qkv).cuda(), c, torch.from_numpy(tables).cuda(), out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = attention_want(oracle, qkv, tables, c, window, shift, h, w, nwin)
    err = np.abs(got - want)
    # f16 probabilities and output: a few units of 2^-11 of the values.
    assert (err <= 4e-3 * np.abs(want) + 4e-3).all(), err.max()


def test_window_attention_many_windows(ctx, oracle):
    """A SCUNet-level map (64 x 96, 96 windows) with 4 heads: every window's
    class and every head's table."""
    import torch
    import ien

    window, shift, h, w, c = 8, 4, 64, 96, 128
    rng = np.random.default_rng(11)
    win = ien.windows(window, shift, h, w)
    nwin, n, heads = ien.window_count(win), 64, 4
    qkv = f16(rng.standard_normal((nwin * n, 3 * c)))
    tables = ien.bias_tables(rng.standard_normal((heads, n, n)).astype(np.float32), window, shift, -np.inf)
    out = torch.zeros((nwin * n, c), dtype=torch.float16, device="cuda")
    ien.window_attention(ctx, win, torch.from_numpy(qkv).cuda(), c, torch.from_numpy(tables).cuda(), out)
    torch.cuda.synchronize()
    want = attention_want(oracle, qkv, tables, c, window, shift, h, w, nwin)
    err = np.abs(out.float().cpu().numpy() - want)
    assert (err <= 4e-3 * np.abs(want) + 4e-3).all(), err.max()


@pytest.mark.parametrize("window,shift,h,w,c", GEOMS)
def test_window_scatter_add(ctx, oracle, window, shift, h, w, c):
    import torch
    import ien

    rng = np.random.default_rng(3)
    stride = c + 16
    win = ien.windows(window, shift, h, w)
    nwin, n = ien.window_count(win), window * window
    m = f16(rng.standard_normal((h * w, stride)))
    rows = f16(rng.standard_normal((nwin * n, c)))
    md = torch.from_numpy(m).cuda()
    ien.window_scatter_add(ctx, win, torch.from_numpy(rows).cuda(), c, md, stride)
    torch.cuda.synchronize()
    got = md.cpu().numpy()
    want = m.copy()
    src = sources(oracle, window, shift, h, w, nwin).reshape(-1)
    valid = src >= 0
    want[src[valid], :c] = (m[src[valid], :c].astype(np.float32) + rows[valid].astype(np.float32)).astype(np.float16)
    assert np.array_equal(got, want)  # one f32 add, one rounding: exact


@pytest.mark.parametrize("window,shift,h,w,c", GEOMS)
def test_swin_attend_composed(ctx, oracle, window, shift, h, w, c):
    """The attention half of a Swin block from the ABI's pieces (gather,
    qkv product, attention, projection, scatter-add) against
    or_swin_attend on the same f16-rounded map and weights."""
    import torch
    import ien

    rng = np.random.default_rng(window + 7 * shift)
    n, heads = window * window, c // 32
    x = f16(rng.standard_normal((h, w, c)))
    g = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    b = (0.1 * rng.standard_normal(c)).astype(np.float32)
    wqkv = (rng.standard_normal((c, 3 * c)) / np.sqrt(c)).astype(np.float32)
    bqkv = (0.1 * rng.standard_normal(3 * c)).astype(np.float32)
    wproj = (rng.standard_normal((c, c)) / np.sqrt(c)).astype(np.float32)
    bproj = (0.1 * rng.standard_normal(c)).astype(np.float32)
    tables = ien.bias_tables(rng.standard_normal((heads, n, n)).astype(np.float32), window, shift,
                             masked_for(window))
    want = oracle.swin_attend(x.astype(np.float32), window, shift, g, b, wqkv, bqkv, tables, wproj, bproj)

    win = ien.windows(window, shift, h, w)
    rows = ien.window_count(win) * n
    md = torch.from_numpy(x.reshape(h * w, c)).cuda()
    tok = torch.empty((rows, c), dtype=torch.float16, device="cuda")
    qkv = torch.empty((rows, 3 * c), dtype=torch.float16, device="cuda")
    att = torch.empty((rows, c), dtype=torch.float16, device="cuda")
    mq, mp = ien.Matrix(ctx, wqkv, bqkv), ien.Matrix(ctx, wproj, bproj)
    ien.window_gather(ctx, win, md, c, c, torch.from_numpy(g).cuda(), torch.from_numpy(b).cuda(), tok)
    ien.multiply_ex(ctx, ien.rows_input(tok, c), 0, rows, mq, qkv, 3 * c)
    ien.window_attention(ctx, win, qkv, c, torch.from_numpy(tables).cuda(), att)
    ien.multiply_ex(ctx, ien.rows_input(att, c), 0, rows, mp, tok, c)
    ien.window_scatter_add(ctx, win, tok, c, md, c)
    torch.cuda.synchronize()
    got = md.float().cpu().numpy().reshape(h, w, c)
    err = np.abs(got - want)
    assert err.max() < 3e-2, err.max()
    assert np.sqrt(np.mean(err ** 2)) < 4e-3
    mq.free()
    mp.free()
