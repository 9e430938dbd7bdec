"""SCUNet written directly in torch (CPU, f32), from the layer description
of crates/scunet-native/src/network.rs:1-16 and the Swin-Conv block:
replicate padding to multiples of 64 (F.pad mode="replicate"), the 3x3 head
and tail as F.conv2d, 2x2 stride-2 halving as F.conv2d and doubling as
F.conv_transpose2d, skip adds, and per block a 1x1 split, the convolution
half (3x3, ReLU, 3x3, residual), the Swin half (timm-style windows of 8
rolled by 4 in odd blocks, the three-slice mask at -inf, multi-head
attention with the gathered position bias, the LayerNorm-GELU MLP) and a
1x1 join added back.  It shares no code with the oracle and pins its
composition; weights come as the weights file's matrices."""

import math

import numpy as np
import torch
import torch.nn.functional as F

WINDOW = 8


def T(a):
    return torch.as_tensor(np.asarray(a, np.float32))


def kernel(m, k):
    """[(ky, kx, cin), cout] -> [cout, cin, ky, kx]."""
    m = T(m)
    cin = m.shape[0] // (k * k)
    return m.reshape(k, k, cin, -1).permute(3, 2, 0, 1).contiguous()


def ln(x, g, b):
    return F.layer_norm(x, (x.shape[-1],), T(g), T(b), eps=1e-5)


def swin(x, t, p, shift):
    """x [H, W, C] (H, W multiples of 8): x + attn(LN1 x), then + MLP."""
    H, W, C = x.shape
    heads, n = C // 32, WINDOW * WINDOW
    y = ln(x, t[p + "ln1.weight"], t[p + "ln1.bias"])
    if shift:
        y = torch.roll(y, shifts=(-shift, -shift), dims=(0, 1))
    win = y.reshape(H // WINDOW, WINDOW, W // WINDOW, WINDOW, C).permute(0, 2, 1, 3, 4).reshape(-1, n, C)
    qkv = win @ T(t[p + "msa.embedding_layer.weight"]) + T(t[p + "msa.embedding_layer.bias"])
    split = lambda z: z.reshape(-1, n, heads, 32).permute(0, 2, 1, 3)
    q, k, v = split(qkv[..., :C]), split(qkv[..., C:2 * C]), split(qkv[..., 2 * C:])
    attn = (q @ k.transpose(-1, -2)) / math.sqrt(32) + T(t[p + "msa.position_bias"])[None]
    if shift:
        img = torch.zeros(H, W)
        cnt = 0
        for hs in (slice(0, -WINDOW), slice(-WINDOW, -shift), slice(-shift, None)):
            for ws in (slice(0, -WINDOW), slice(-WINDOW, -shift), slice(-shift, None)):
                img[hs, ws] = cnt
                cnt += 1
        mw = img.reshape(H // WINDOW, WINDOW, W // WINDOW, WINDOW).permute(0, 2, 1, 3).reshape(-1, n)
        attn = attn.masked_fill((mw[:, None, :] != mw[:, :, None])[:, None], float("-inf"))
    o = (attn.softmax(-1) @ v).permute(0, 2, 1, 3).reshape(-1, n, C)
    o = o @ T(t[p + "msa.linear.weight"]) + T(t[p + "msa.linear.bias"])
    o = o.reshape(H // WINDOW, W // WINDOW, WINDOW, WINDOW, C).permute(0, 2, 1, 3, 4).reshape(H, W, C)
    if shift:
        o = torch.roll(o, shifts=(shift, shift), dims=(0, 1))
    x = x + o
    h = F.gelu(ln(x, t[p + "ln2.weight"], t[p + "ln2.bias"]) @ T(t[p + "mlp.0.weight"]) + T(t[p + "mlp.0.bias"]))
    return x + h @ T(t[p + "mlp.2.weight"]) + T(t[p + "mlp.2.bias"])


def block(x, t, p, shift):
    """x [1, C, H, W] -> the block's output."""
    c = x.shape[1]
    h = c // 2
    y = F.conv2d(x, kernel(t[p + "conv1_1.weight"], 1), T(t[p + "conv1_1.bias"]))
    conv, tr = y[:, :h], y[:, h:]
    r = F.relu(F.conv2d(conv, kernel(t[p + "conv_block.0.weight"], 3), padding=1))
    conv = conv + F.conv2d(r, kernel(t[p + "conv_block.2.weight"], 3), padding=1)
    tr = swin(tr[0].permute(1, 2, 0), t, p + "trans_block.", shift).permute(2, 0, 1)[None]
    y = torch.cat([conv, tr], dim=1)
    return x + F.conv2d(y, kernel(t[p + "conv1_2.weight"], 1), T(t[p + "conv1_2.bias"]))


def level(x, t, name, first):
    for b in range(4):
        x = block(x, t, f"{name}.{first + b}.", WINDOW // 2 if b % 2 else 0)
    return x


def run(t, image):
    """image (H, W, 3) in 0..1 -> (H, W, 3)."""
    with torch.no_grad():
        h, w, _ = image.shape
        ph, pw = -(-h // 64) * 64, -(-w // 64) * 64
        img = F.pad(T(image).permute(2, 0, 1)[None], (0, pw - w, 0, ph - h), mode="replicate")
        head = F.conv2d(img, kernel(t["m_head.0.weight"], 3), padding=1)
        x = head
        skips = []
        for i, c in ((1, 64), (2, 128), (3, 256)):
            x = level(x, t, f"m_down{i}", 0)
            x = F.conv2d(x, kernel(t[f"m_down{i}.4.weight"], 2), stride=2)
            skips.append(x)
        x = level(x, t, "m_body", 0)
        for i, c in ((3, 256), (2, 128), (1, 64)):
            x = x + skips.pop()
            m = T(t[f"m_up{i}.0.weight"])  # [2c][4 c]: columns (2 dy + dx) c
            wt = m.reshape(2 * c, 2, 2, c).permute(0, 3, 1, 2).contiguous()
            x = F.conv_transpose2d(x, wt, stride=2)
            x = level(x, t, f"m_up{i}", 1)
        x = x + head
        out = F.conv2d(x, kernel(t["m_tail.0.weight"], 3), padding=1)
        return out[0].permute(1, 2, 0).numpy()[:h, :w]
