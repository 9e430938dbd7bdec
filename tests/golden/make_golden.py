#!/usr/bin/env python3
"""Write golden.npz: small input/output vectors computed with torch's
functional operators in float64, in this container, for pinning the oracle.

    python tests/golden/make_golden.py

The reference (a Rust workspace) cannot be built or run here and commits no
golden files of its own; its tests check each op against textbook
definitions.  These vectors pin the same ops by an independent route:
torch.nn.functional.conv2d / conv_transpose2d / layer_norm / gelu /
scaled_dot_product_attention / pixel_shuffle / interpolate, all in float64.
Conventions follow the reference's layouts: images NHWC, convolution
weights as (kh, kw, cin) rows by cout columns (tools/realesrgan/
export_weights.py:48-56).  Inputs are seeded (numpy PCG64) and stored with
the outputs.  The Real-ESRGAN vector runs SRVGGNetCompact (conv3x3 + PReLU
x33, conv3x3 to 48, pixel shuffle x4, plus the nearest-upsampled input) on
the random-init weights of image-engine-native_amd/synthetic.py.
"""

import pathlib
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "image-engine-native_amd"))
import synthetic  # noqa: E402

torch.set_default_dtype(torch.float64)


def to_oihw(w, size, cin, cout):
    """(kh, kw, cin) x cout rows -> torch's [cout, cin, kh, kw]."""
    return torch.from_numpy(w.reshape(size, size, cin, cout).transpose(3, 2, 0, 1).copy())


def conv_nhwc(x, w, b, size, step=1, pad="zero"):
    h, wd, cin = x.shape
    cout = w.shape[1]
    t = torch.from_numpy(x.transpose(2, 0, 1)[None].copy())
    p = size // 2
    if pad == "reflect":
        t = F.pad(t, (p, p, p, p), mode="reflect")
        p = 0
    y = F.conv2d(t, to_oihw(w, size, cin, cout), torch.from_numpy(b), stride=step, padding=p)
    return y[0].numpy().transpose(1, 2, 0)


def swin_attend_torch(x, window, shift, masked, gamma, beta, wqkv, bqkv, pos, wproj, bproj):
    """The attention half of a Swin block in the standard formulation:
    LayerNorm, zero-pad to whole windows, roll by -shift, window partition,
    multi-head attention with the position bias and the region mask of the
    shifted map (img_mask slices, as in timm / SCUNet), reverse partition,
    roll back, crop, residual.  x: [H, W, c] float64."""
    h, wd, c = x.shape
    heads, n = c // 32, window * window
    xn = F.layer_norm(x, (c,), gamma, beta, eps=1e-5)
    ph, pw = -(-h // window) * window, -(-wd // window) * window
    xp = F.pad(xn, (0, 0, 0, pw - wd, 0, ph - h))
    if shift:
        xp = torch.roll(xp, shifts=(-shift, -shift), dims=(0, 1))

    def part(t):
        return t.reshape(ph // window, window, pw // window, window, -1).permute(0, 2, 1, 3, 4).reshape(-1, n, t.shape[-1])

    win = part(xp)
    nw = win.shape[0]
    qkv = win @ wqkv + bqkv
    q, k, v = qkv.split(c, dim=-1)
    q = q.reshape(nw, n, heads, 32).transpose(1, 2)
    k = k.reshape(nw, n, heads, 32).transpose(1, 2)
    v = v.reshape(nw, n, heads, 32).transpose(1, 2)
    attn = (q * 32 ** -0.5) @ k.transpose(-2, -1) + pos[None]
    if shift:
        img = torch.zeros(ph, pw, 1, dtype=torch.float64)
        cnt = 0
        for hs in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
            for ws in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
                img[hs, ws] = cnt
                cnt += 1
        mw = part(img)[..., 0]
        am = mw[:, None, :] - mw[:, :, None]
        am = torch.where(am != 0, torch.tensor(masked, dtype=torch.float64), torch.tensor(0.0, dtype=torch.float64))
        attn = attn + am[:, None]
    attn = torch.softmax(attn, dim=-1)
    o = (attn @ v).transpose(1, 2).reshape(nw, n, c) @ wproj + bproj
    y = o.reshape(ph // window, pw // window, window, window, c).permute(0, 2, 1, 3, 4).reshape(ph, pw, c)
    if shift:
        y = torch.roll(y, shifts=(shift, shift), dims=(0, 1))
    return x + y[:h, :wd]


def swin_mlp_torch(x, gamma, beta, w1, b1, w2, b2):
    c = x.shape[-1]
    hdn = F.gelu(F.layer_norm(x, (c,), gamma, beta, eps=1e-5) @ w1 + b1, approximate="none")
    return x + hdn @ w2 + b2


def main():
    rng = np.random.default_rng(20261201)
    out = {}

    def f32(a):
        return np.asarray(a, np.float32)

    # gemm.rs Input::Image taps: zero padding, several sizes and strides.
    for name, (h, w, c, n, size, step, pad) in {
        "conv_3x3_zero": (5, 7, 3, 20, 3, 1, "zero"),
        "conv_7x7_zero": (6, 9, 8, 16, 7, 1, "zero"),
        "conv_1x1": (4, 6, 24, 10, 1, 1, "zero"),
        "conv_3x3_reflect": (6, 5, 16, 12, 3, 1, "reflect"),
        "conv_3x3_s2_reflect": (9, 8, 16, 24, 3, 2, "reflect"),
        "conv_7x7_reflect": (8, 10, 4, 8, 7, 1, "reflect"),
    }.items():
        x = f32(rng.standard_normal((h, w, c)))
        wt = f32(rng.standard_normal((size * size * c, n)) / np.sqrt(size * size * c))
        b = f32(rng.standard_normal(n))
        out[name + "_x"], out[name + "_w"], out[name + "_b"] = x, wt, b
        out[name + "_y"] = conv_nhwc(x.astype(np.float64), wt.astype(np.float64), b.astype(np.float64),
                                     size, step, pad)

    # A stride-2, padding-1, output-padding-1 3x3 transposed convolution
    # (LaMa's upsampling), for the offset-tap phases.
    x = f32(rng.standard_normal((5, 6, 8)))
    wt = f32(rng.standard_normal((8, 6, 3, 3)) / 6)  # torch layout [cin, cout, kh, kw]
    b = f32(rng.standard_normal(6))
    y = F.conv_transpose2d(torch.from_numpy(x.astype(np.float64).transpose(2, 0, 1)[None].copy()),
                           torch.from_numpy(wt.astype(np.float64)), torch.from_numpy(b.astype(np.float64)),
                           stride=2, padding=1, output_padding=1)
    out["convT_x"], out["convT_w"], out["convT_b"] = x, wt, b
    out["convT_y"] = y[0].numpy().transpose(1, 2, 0)

    # Depthwise 7x7 (groups = channels), NHWC, weights (tap, channel).
    x = f32(rng.standard_normal((11, 13, 6)))
    wt = f32(rng.standard_normal((49, 6)) / 7)
    b = f32(rng.standard_normal(6))
    k = torch.from_numpy(wt.astype(np.float64).T.reshape(6, 1, 7, 7).copy())
    y = F.conv2d(torch.from_numpy(x.astype(np.float64).transpose(2, 0, 1)[None].copy()), k,
                 torch.from_numpy(b.astype(np.float64)), padding=3, groups=6)
    out["dw_x"], out["dw_w"], out["dw_b"], out["dw_y"] = x, wt, b, y[0].numpy().transpose(1, 2, 0)

    # math.rs: LayerNorm (eps 1e-5), exact GELU, logistic.
    x = f32(rng.standard_normal((7, 96)) * 3 + 0.5)
    g = f32(1 + 0.2 * rng.standard_normal(96))
    bb = f32(0.2 * rng.standard_normal(96))
    out["ln_x"], out["ln_g"], out["ln_b"] = x, g, bb
    out["ln_y"] = F.layer_norm(torch.from_numpy(x.astype(np.float64)), (96,), torch.from_numpy(g.astype(np.float64)),
                               torch.from_numpy(bb.astype(np.float64)), eps=1e-5).numpy()
    x = f32(np.linspace(-9, 9, 3001))
    out["act_x"] = x
    out["gelu_y"] = F.gelu(torch.from_numpy(x.astype(np.float64)), approximate="none").numpy()
    out["sigmoid_y"] = torch.sigmoid(torch.from_numpy(x.astype(np.float64))).numpy()

    # attention.rs: one head of a window, softmax(q k^T / sqrt(32) + bias) v,
    # with masked (-100 and -inf) biases; N = 49, 64 and 144.
    for tokens in (49, 64, 144):
        c = 64
        qkv = f32(rng.standard_normal((tokens, 3 * c)))
        bias = f32(rng.standard_normal((tokens, tokens)))
        bias[rng.random((tokens, tokens)) < 0.2] = -100.0
        if tokens == 64:
            bias[:, 60:] = -np.inf  # whole masked key columns, as SCUNet's shift mask
        head = 1
        q = torch.from_numpy(qkv[:, head * 32:head * 32 + 32].astype(np.float64))[None, None]
        kk = torch.from_numpy(qkv[:, c + head * 32:c + head * 32 + 32].astype(np.float64))[None, None]
        v = torch.from_numpy(qkv[:, 2 * c + head * 32:2 * c + head * 32 + 32].astype(np.float64))[None, None]
        y = F.scaled_dot_product_attention(q, kk, v, attn_mask=torch.from_numpy(bias.astype(np.float64))[None, None])
        out[f"attn{tokens}_qkv"], out[f"attn{tokens}_bias"], out[f"attn{tokens}_y"] = qkv, bias, y[0, 0].numpy()

    # Swin window attention blocks (scunet swin.rs, birefnet swin.rs) on small
    # maps: SCUNet's window 8 / shift 4 with a -inf mask, the configuration's
    # BiRefNet window 12 / shift 6 with -100 on a map that needs padding, and
    # unshifted blocks.  For these (window = 2 shift) the standard three-slice
    # region mask is the reference's two-region one.
    for name, (h, wd, c, window, shift, masked) in {
        "swin_w8s4": (16, 24, 64, 8, 4, float("-inf")),
        "swin_w8s0": (16, 16, 64, 8, 0, float("-inf")),
        "swin_w12s6": (15, 13, 32, 12, 6, -100.0),
    }.items():
        heads, n = c // 32, window * window
        x = f32(rng.standard_normal((h, wd, c)))
        g = f32(1 + 0.1 * rng.standard_normal(c))
        bt = f32(0.1 * rng.standard_normal(c))
        wqkv = f32(rng.standard_normal((c, 3 * c)) / np.sqrt(c))
        bqkv = f32(0.1 * rng.standard_normal(3 * c))
        pos = f32(rng.standard_normal((heads, n, n)))
        wproj = f32(rng.standard_normal((c, c)) / np.sqrt(c))
        bproj = f32(0.1 * rng.standard_normal(c))
        t = lambda a: torch.from_numpy(a.astype(np.float64))
        y = swin_attend_torch(t(x), window, shift, masked, t(g), t(bt), t(wqkv), t(bqkv), t(pos), t(wproj), t(bproj))
        for k, v in dict(x=x, g=g, b=bt, wqkv=wqkv, bqkv=bqkv, pos=pos, wproj=wproj, bproj=bproj).items():
            out[f"{name}_{k}"] = v
        out[f"{name}_y"] = y.numpy()
    x = f32(rng.standard_normal((37, 64)))
    g = f32(1 + 0.1 * rng.standard_normal(64))
    bt = f32(0.1 * rng.standard_normal(64))
    w1 = f32(rng.standard_normal((64, 256)) / 8)
    b1 = f32(0.1 * rng.standard_normal(256))
    w2 = f32(rng.standard_normal((256, 64)) / 16)
    b2 = f32(0.1 * rng.standard_normal(64))
    t = lambda a: torch.from_numpy(a.astype(np.float64))
    out.update(mlp_x=x, mlp_g=g, mlp_b=bt, mlp_w1=w1, mlp_b1=b1, mlp_w2=w2, mlp_b2=b2)
    out["mlp_y"] = swin_mlp_torch(t(x), t(g), t(bt), t(w1), t(b1), t(w2), t(b2)).numpy()

    # realesrgan network.rs:115-141: pixel shuffle x4 of 48 channels plus
    # the input repeated, against pixel_shuffle + nearest interpolate.
    last = f32(rng.standard_normal((3, 5, 48)))
    img = f32(rng.random((3, 5, 3)))
    ps = F.pixel_shuffle(torch.from_numpy(last.astype(np.float64).transpose(2, 0, 1)[None].copy()), 4)
    up = F.interpolate(torch.from_numpy(img.astype(np.float64).transpose(2, 0, 1)[None].copy()),
                       scale_factor=4, mode="nearest")
    out["shuffle_last"], out["shuffle_img"] = last, img
    out["shuffle_y"] = (ps + up)[0].numpy().transpose(1, 2, 0)

    # Real-ESRGAN SRVGGNetCompact on the synthetic random-init weights.
    tensors = synthetic.esrgan_tensors()
    img = synthetic.esrgan_image(12, 16, seed=7)
    t = torch.from_numpy(img.astype(np.float64).transpose(2, 0, 1)[None].copy())
    x = t
    for i in range(synthetic.ESRGAN_STEPS):
        cin = 3 if i == 0 else 64
        w = tensors[f"body.{2 * i}.weight"].astype(np.float64)
        cout = w.shape[1]
        x = F.conv2d(x, to_oihw(w, 3, cin, cout), torch.from_numpy(tensors[f"body.{2 * i}.bias"].astype(np.float64)),
                     padding=1)
        if i != synthetic.ESRGAN_STEPS - 1:
            x = F.prelu(x, torch.from_numpy(tensors[f"body.{2 * i + 1}.weight"].astype(np.float64)))
    x = F.pixel_shuffle(x, 4) + F.interpolate(t, scale_factor=4, mode="nearest")
    out["esrgan_img"] = img
    out["esrgan_y"] = x[0].numpy().transpose(1, 2, 0)

    # lama-native fourier.rs: rfftn / irfftn over the two spatial axes with
    # "ortho" scale; spectra as [re | im] per pixel.  The inverse inputs are
    # not Hermitian: irfftn reads only the real parts of column 0 and (even
    # widths) of the last column.
    x = f32(rng.standard_normal((12, 10, 3)))
    z = torch.fft.rfftn(torch.from_numpy(x.astype(np.float64)), dim=(0, 1), norm="ortho")
    out["rfft_x"] = x
    out["rfft_y"] = torch.cat([z.real, z.imag], dim=-1).numpy()
    for name, (h, w) in (("irfft_odd", (9, 7)), ("irfft_even", (8, 6))):
        s = f32(rng.standard_normal((h, w // 2 + 1, 4)))
        zc = torch.complex(torch.from_numpy(s[..., :2].astype(np.float64)),
                           torch.from_numpy(s[..., 2:].astype(np.float64)))
        out[f"{name}_s"] = s
        out[f"{name}_y"] = torch.fft.irfftn(zc, s=(h, w), dim=(0, 1), norm="ortho").numpy()

    # lama-native network.rs:271-335: a stride-2 transposed 3x3 convolution
    # (padding 1, output padding 1) and ReLU, the layer the four phase
    # products restate; kernel in torch's [in, out, ky, kx] layout.
    x = f32(rng.standard_normal((5, 6, 8)))
    wt = f32(rng.standard_normal((8, 4, 3, 3)) / 6)
    bt = f32(0.1 * rng.standard_normal(4))
    y = F.conv_transpose2d(torch.from_numpy(x.astype(np.float64).transpose(2, 0, 1)[None].copy()),
                           torch.from_numpy(wt.astype(np.float64)), torch.from_numpy(bt.astype(np.float64)),
                           stride=2, padding=1, output_padding=1)
    out.update(up_x=x, up_w=wt, up_b=bt)
    out["up_y"] = F.relu(y)[0].numpy().transpose(1, 2, 0)

    packed = {k: (v.astype(np.float32) if v.dtype == np.float64 else v) for k, v in out.items()}
    np.savez_compressed(HERE / "golden.npz", **packed)
    print(f"wrote {len(packed)} arrays, {sum(v.nbytes for v in packed.values())} bytes")


if __name__ == "__main__":
    main()
