"""Big LaMa's generator written directly in torch (CPU, f32), from the
layer description in crates/lama-native/src/network.rs:1-20 and LaMa's
FFC definitions: reflect-padded F.conv2d, torch.fft.rfftn / irfftn with
norm="ortho", F.conv_transpose2d(stride 2, padding 1, output_padding 1).
It shares no code with the oracle and pins its composition: the spectrum
layout, the phase split of the transposed convolutions, the padding and
the crop.  Weights come as the weights file's matrices
(tools/lama/export_weights.py layouts) and are turned back into torch
kernels here."""

import numpy as np
import torch
import torch.nn.functional as F

LOCAL, GLOBAL, BLOCKS = 128, 384, 18
SPECTRAL = GLOBAL // 2
# network.rs:271: (input offset, kernel tap) per output phase along an axis.
PHASE_TAPS = [[(0, 1)], [(0, 2), (1, 0)]]


def kernel(m, k):
    """[(ky, kx, cin), cout] matrix -> torch [cout, cin, ky, kx]."""
    m = torch.as_tensor(m, dtype=torch.float32)
    cin = m.shape[0] // (k * k)
    return m.reshape(k, k, cin, -1).permute(3, 2, 0, 1).contiguous()


def conv(x, m, b, k, step=1, reflect=True):
    """x [1, C, H, W]."""
    if reflect and k > 1:
        x = F.pad(x, (k // 2,) * 4, mode="reflect")
    bias = None if b is None else torch.as_tensor(b, dtype=torch.float32)
    return F.conv2d(x, kernel(m, k), bias, stride=step)


def transposed_kernel(phases, cin):
    """The [cin, cout, 3, 3] kernel whose four output phases are `phases`."""
    cout = phases[0].shape[1]
    w = torch.zeros(cin, cout, 3, 3)
    for p in range(4):
        ys, xs = PHASE_TAPS[p // 2], PHASE_TAPS[p % 2]
        m = torch.as_tensor(phases[p], dtype=torch.float32)
        i = 0
        for _, ky in ys:
            for _, kx in xs:
                w[:, :, ky, kx] = m[i * cin:(i + 1) * cin]
                i += 1
    return w


def ffc(x, t, n):
    local = F.relu(conv(x, t[f"{n}.local.weight"], t[f"{n}.local.bias"], 3))
    cross = conv(x[:, :LOCAL], t[f"{n}.cross.weight"], t[f"{n}.cross.bias"], 3)
    spectral = F.relu(conv(x[:, LOCAL:], t[f"{n}.spectral_in.weight"], t[f"{n}.spectral_in.bias"], 1))
    h, w = spectral.shape[-2:]
    z = torch.fft.rfftn(spectral, dim=(-2, -1), norm="ortho")
    z = torch.cat([z.real, z.imag], dim=1)
    z = F.relu(conv(z, t[f"{n}.fourier.weight"], t[f"{n}.fourier.bias"], 1))
    back = torch.fft.irfftn(torch.complex(z[:, :SPECTRAL], z[:, SPECTRAL:]), s=(h, w), dim=(-2, -1),
                            norm="ortho")
    glob = F.relu(cross + conv(spectral + back, t[f"{n}.spectral_out.weight"], None, 1))
    return torch.cat([local, glob], dim=1)


def run(t, image, mask, trace=None):
    """image (H, W, 3), mask (H, W) -> (H, W, 3); `trace` collects the RMS
    of every stage when a list."""
    h, w = mask.shape
    ph, pw = -(-h // 8) * 8, -(-w // 8) * 8
    sy = [y if y < h else 2 * h - 1 - y for y in range(ph)]
    sx = [x if x < w else 2 * w - 1 - x for x in range(pw)]
    img = np.asarray(image, np.float32)[np.ix_(sy, sx)]
    m = np.asarray(mask, np.float32)[np.ix_(sy, sx)]
    x = np.concatenate([img * (1 - m)[..., None], m[..., None]], axis=-1)
    note = (lambda name, v: trace.append((name, float(v.pow(2).mean().sqrt())))) if trace is not None \
        else (lambda name, v: None)
    with torch.no_grad():
        a = torch.from_numpy(np.ascontiguousarray(x.transpose(2, 0, 1)))[None]
        a = F.relu(conv(a, t["first.weight"], t["first.bias"], 7))
        note("first", a)
        for i in range(3):
            a = F.relu(conv(a, t[f"down{i}.weight"], t[f"down{i}.bias"], 3, step=2))
            note(f"down{i}", a)
        for b in range(BLOCKS):
            mid = ffc(a, t, f"block{b}.ffc0")
            a = a + ffc(mid, t, f"block{b}.ffc1")
            note(f"block{b}", a)
        for i in range(3):
            phases = [t[f"up{i}.phase{p}.weight"] for p in range(4)]
            wt = transposed_kernel(phases, a.shape[1])
            bias = torch.as_tensor(t[f"up{i}.phase0.bias"], dtype=torch.float32)
            a = F.relu(F.conv_transpose2d(a, wt, bias, stride=2, padding=1, output_padding=1))
            note(f"up{i}", a)
        rgb = conv(a, t["last.weight"], t["last.bias"], 7)
        note("last", rgb)
        rgb = torch.sigmoid(rgb)
    return rgb[0].permute(1, 2, 0).numpy()[:h, :w]
