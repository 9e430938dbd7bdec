"""BiRefNet-lite written directly in torch (CPU, f32), from the layer
description of crates/birefnet-native/src/swin.rs:1-11 and decoder.rs:1-14
and the Swin Transformer definitions: timm-style windows (LayerNorm, zero
padding to whole windows, torch.roll, the shift mask built from the three
slices of the padded grid, -100 between regions), patch merging by strided
slices, F.conv2d with zero padding, F.interpolate(bilinear,
align_corners=True), deformable sampling through F.grid_sample (zeros
outside, bilinear), and the full-resolution branch as its two convolutions.
It shares no code with the oracle and pins its composition.  Weights come
as the weights file's matrices and are turned back into torch kernels
here."""

import math

import numpy as np
import torch
import torch.nn.functional as F

STAGES = ((96, 2), (192, 2), (384, 6), (768, 2))
LEVELS = ((1728, 768), (960, 384), (480, 192), (240, 96))
SIZES = (1, 1, 3, 7)


def T(a):
    return torch.as_tensor(np.asarray(a, np.float32))


def kernel(m, k):
    """[(ky, kx, cin), cout] -> [cout, cin, ky, kx]."""
    m = T(m)
    cin = m.shape[0] // (k * k)
    return m.reshape(k, k, cin, -1).permute(3, 2, 0, 1).contiguous()


def conv(x, m, b, k):
    """x [1, C, H, W], zero padding."""
    return F.conv2d(x, kernel(m, k), None if b is None else T(b), padding=k // 2)


def ln(x, g, b):
    return F.layer_norm(x, (x.shape[-1],), T(g), T(b), eps=1e-5)


def resize(x, size):
    """[1, C, h, w] -> [1, C, size, size]."""
    return F.interpolate(x, size=(size, size), mode="bilinear", align_corners=True)


def swin_block(x, t, p, window, shift):
    """x [H, W, C]."""
    H, W, C = x.shape
    heads = C // 32
    n = window * window
    ph, pw = -(-H // window) * window, -(-W // window) * window
    y = ln(x, t[p + "norm1.weight"], t[p + "norm1.bias"])
    y = F.pad(y, (0, 0, 0, pw - W, 0, ph - H))
    if shift:
        y = torch.roll(y, shifts=(-shift, -shift), dims=(0, 1))
    win = y.reshape(ph // window, window, pw // window, window, C).permute(0, 2, 1, 3, 4).reshape(-1, n, C)
    qkv = win @ T(t[p + "qkv.weight"]) + T(t[p + "qkv.bias"])
    q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    split = lambda z: z.reshape(-1, n, heads, 32).permute(0, 2, 1, 3)
    q, k, v = split(q), split(k), split(v)
    attn = (q @ k.transpose(-1, -2)) / math.sqrt(32) + T(t[p + "position_bias"])[None]
    if shift:
        img = torch.zeros(ph, pw)
        cnt = 0
        for hs in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
            for ws in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
                img[hs, ws] = cnt
                cnt += 1
        mw = img.reshape(ph // window, window, pw // window, window).permute(0, 2, 1, 3).reshape(-1, n)
        mask = (mw[:, None, :] != mw[:, :, None]).float() * -100.0
        attn = attn + mask[:, None]
    o = (attn.softmax(-1) @ v).permute(0, 2, 1, 3).reshape(-1, n, C)
    o = o @ T(t[p + "proj.weight"]) + T(t[p + "proj.bias"])
    o = o.reshape(ph // window, pw // window, window, window, C).permute(0, 2, 1, 3, 4).reshape(ph, pw, C)
    if shift:
        o = torch.roll(o, shifts=(shift, shift), dims=(0, 1))
    x = x + o[:H, :W]
    h = F.gelu(ln(x, t[p + "norm2.weight"], t[p + "norm2.bias"]) @ T(t[p + "fc1.weight"]) + T(t[p + "fc1.bias"]))
    return x + h @ T(t[p + "fc2.weight"]) + T(t[p + "fc2.bias"])


def backbone(t, image, window):
    """image [side, side, 3] -> four normalised stage maps [g, g, c]."""
    x = F.conv2d(image.permute(2, 0, 1)[None], kernel(t["patch_embed.weight"], 4), T(t["patch_embed.bias"]),
                 stride=4)[0].permute(1, 2, 0)
    x = ln(x, t["patch_embed.norm.weight"], t["patch_embed.norm.bias"])
    feats = []
    for s, (c, depth) in enumerate(STAGES):
        for b in range(depth):
            x = swin_block(x, t, f"stage{s}.block{b}.", window, window // 2 if b % 2 else 0)
        feats.append(ln(x, t[f"stage{s}.norm.weight"], t[f"stage{s}.norm.bias"]))
        if s < 3:
            x = torch.cat([x[0::2, 0::2], x[1::2, 0::2], x[0::2, 1::2], x[1::2, 1::2]], dim=-1)
            x = ln(x, t[f"stage{s}.merge.norm.weight"], t[f"stage{s}.merge.norm.bias"]) @ T(t[f"stage{s}.merge.weight"])
    return feats


def deform_branch(tm, t, q, i, k):
    """One ASPP branch: offsets conv, modulators through the sigmoid, taps
    bilinearly sampled (zeros outside) times twice the modulator, then the
    branch matrix and ReLU.  tm [1, 64, H, W]."""
    _, _, H, W = tm.shape
    taps = k * k
    off = conv(tm, t[f"{q}.aspp.branch{i}.offset.weight"], t[f"{q}.aspp.branch{i}.offset.bias"], k)[0]
    ys = torch.arange(H, dtype=torch.float32)[:, None].expand(H, W)
    xs = torch.arange(W, dtype=torch.float32)[None, :].expand(H, W)
    cols = []
    for tap in range(taps):
        py = ys - k // 2 + tap // k + off[2 * tap]
        px = xs - k // 2 + tap % k + off[2 * tap + 1]
        m = 2.0 * torch.sigmoid(off[2 * taps + tap])
        grid = torch.stack([(2 * px + 1) / W - 1, (2 * py + 1) / H - 1], dim=-1)[None]
        s = F.grid_sample(tm, grid, mode="bilinear", padding_mode="zeros", align_corners=False)[0]
        cols.append(s * m)
    rows = torch.stack(cols).permute(2, 3, 0, 1).reshape(H * W, taps * 64)
    out = rows @ T(t[f"{q}.aspp.branch{i}.weight"]) + T(t[f"{q}.aspp.branch{i}.bias"])
    return F.relu(out)


def dblock(x, t, q, gate):
    """x [1, cin, H, W] -> [1, cout, H, W]."""
    _, _, H, W = x.shape
    tm = F.relu(conv(x, t[f"{q}.conv_in.weight"], t[f"{q}.conv_in.bias"], 3))
    mean = tm.double().mean(dim=(2, 3))[0].float()
    pooled = F.relu(mean @ T(t[f"{q}.aspp.pool.weight"]) + T(t[f"{q}.aspp.pool.bias"]))
    w1 = T(t[f"{q}.aspp.conv1.weight"])
    bias = T(t[f"{q}.aspp.conv1.bias"]) + pooled @ w1[1024:]
    cat = torch.cat([deform_branch(tm, t, q, i, k) for i, k in enumerate(SIZES)], dim=1)
    a = F.relu(cat @ w1[:1024] + bias).reshape(H, W, 64).permute(2, 0, 1)[None]
    out = conv(a, t[f"{q}.conv_out.weight"], t[f"{q}.conv_out.bias"], 3)
    if gate:
        g = F.relu(conv(out, t[f"{q}.gdt.weight"], t[f"{q}.gdt.bias"], 3))
        s = torch.sigmoid(torch.einsum("bchw,c->bhw", g, T(t[f"{q}.gdt_attn.weight"])[:, 0])
                          + T(t[f"{q}.gdt_attn.bias"])[0])
        out = out * s[:, None]
    return out


def patches(t, n, image, size):
    """image2patches (channel (c grid + gy) grid + gx), then both convs."""
    side = image.shape[0]
    grid = side // size
    x = image.permute(2, 0, 1).reshape(3, grid, size, grid, size).permute(0, 1, 3, 2, 4).reshape(1, 3 * grid * grid, size, size)
    mid = conv(x, t[f"patches{n}.conv1.weight"], t[f"patches{n}.conv1.bias"], 3)
    return conv(mid, t[f"patches{n}.conv_out.weight"], t[f"patches{n}.conv_out.bias"], 3)


def run(t, image, window):
    """image [side, side, 3] normalised -> logits [side, side]."""
    with torch.no_grad():
        img = T(image).double().float()
        side = img.shape[0]
        half = resize(img.permute(2, 0, 1)[None], side // 2)[0].permute(1, 2, 0)
        full_f, half_f = backbone(t, img, window), backbone(t, half, window)
        levels = []
        for i in range(4):
            g = side >> (i + 2)
            f = full_f[i].permute(2, 0, 1)[None]
            h = resize(half_f[i].permute(2, 0, 1)[None], g)
            levels.append(torch.cat([f, h], dim=1))
        g4 = side >> 5
        x4 = torch.cat([resize(levels[i], g4) for i in range(3)] + [levels[3]], dim=1)
        prev = dblock(x4, t, "squeeze", False)
        for i in range(4):
            level = 3 - i
            g = side >> (level + 2)
            if i == 0:
                main = prev
            else:
                lat = levels[level][0].permute(1, 2, 0) @ T(t[f"lateral{5 - i}.weight"]) + T(t[f"lateral{5 - i}.bias"])
                main = lat.permute(2, 0, 1)[None] + resize(prev, g)
            x = torch.cat([main, patches(t, 5 - i, img, g)], dim=1)
            prev = dblock(x, t, f"block{4 - i}", i < 3)
        low = torch.einsum("bchw,c->bhw", prev, T(t["head.weight"])[:, 0])[:, None]
        logits = T(t["head.bias"])[0] + resize(low, side)[0, 0]
        fr = conv(conv(img.permute(2, 0, 1)[None], t["patches1.conv1.weight"], t["patches1.conv1.bias"], 3),
                  t["patches1.conv_out.weight"], t["patches1.conv_out.bias"], 3)[0, 0]
        return (logits + fr).numpy()
