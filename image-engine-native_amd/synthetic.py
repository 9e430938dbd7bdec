"""Synthetic workloads of the benchmark configurations: seeded inputs and
random-init weights, the same on every machine (numpy's PCG64 generator,
`numpy.random.default_rng(seed)`; seed 0 for inputs, seed 1 for weights).

Real-ESRGAN general x4v3 (SRVGGNetCompact, crates/realesrgan-native/src/
network.rs): weights Kaiming-normal (std sqrt(2 / fan_in), fan_in = 9 cin,
as torch.nn.init.kaiming_normal_), biases uniform in +-1/sqrt(fan_in)
(torch's Conv2d default), PReLU slopes 0.25 (torch's PReLU default); the
weights file layout of tools/realesrgan/export_weights.py:48-56 (conv
[o, i, kh, kw] -> [(kh, kw, i), o]).
"""

import numpy as np

INPUT_SEED, WEIGHT_SEED = 0, 1
ESRGAN_STEPS, ESRGAN_FEATURES, ESRGAN_SCALE = 34, 64, 4


def esrgan_tensors(seed=WEIGHT_SEED, features=ESRGAN_FEATURES):
    """name -> array, as a realesrgan-native weights file holds them."""
    rng = np.random.default_rng(seed)
    tensors = {}
    for i in range(ESRGAN_STEPS):
        cin = 3 if i == 0 else features
        cout = 3 * ESRGAN_SCALE ** 2 if i == ESRGAN_STEPS - 1 else features
        fan = 9 * cin
        w = (rng.standard_normal((9 * cin, cout)) * np.sqrt(2.0 / fan)).astype(np.float32)
        b = rng.uniform(-1 / np.sqrt(fan), 1 / np.sqrt(fan), cout).astype(np.float32)
        tensors[f"body.{2 * i}.weight"] = w
        tensors[f"body.{2 * i}.bias"] = b
        if i != ESRGAN_STEPS - 1:
            tensors[f"body.{2 * i + 1}.weight"] = np.full(features, 0.25, np.float32)
    return tensors


def esrgan_layers(tensors):
    """The 34 (weight, bias, slope) triples of a tensor dict, in order."""
    out = []
    for i in range(ESRGAN_STEPS):
        slope = tensors.get(f"body.{2 * i + 1}.weight") if i != ESRGAN_STEPS - 1 else None
        out.append((tensors[f"body.{2 * i}.weight"], tensors[f"body.{2 * i}.bias"], slope))
    return out


def esrgan_image(height=256, width=384, seed=INPUT_SEED):
    """H x W x 3 RGB, uniform [0, 1)."""
    return np.random.default_rng(seed).random((height, width, 3), dtype=np.float32)


# Conv sweep: the models' layer shapes, NCHW, f16 storage, N(0, 1) values.
# (name, kind, cin, cout, size, height, width)
SWEEP = (
    ("conv3x3_64_64_256x384", "conv", 64, 64, 3, 256, 384),
    ("conv3x3_128_128_128x192", "conv", 128, 128, 3, 128, 192),
    ("conv1x1_256_512_64x64", "conv", 256, 512, 1, 64, 64),
    ("conv3x3_512_512_32x32", "conv", 512, 512, 3, 32, 32),
    ("depthwise7x7_192_128x128", "depthwise", 192, 192, 7, 128, 128),
)


def sweep_case(name, seed=INPUT_SEED):
    """x (C x H x W, f16-rounded f32), w ((size*size*cin) x cout or (size*size) x C), bias."""
    entry = next(e for e in SWEEP if e[0] == name)
    _, kind, cin, cout, size, h, w = entry
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((cin, h, w)).astype(np.float16).astype(np.float32)
    wrng = np.random.default_rng(WEIGHT_SEED)
    if kind == "conv":
        wt = wrng.standard_normal((size * size * cin, cout)).astype(np.float16).astype(np.float32)
    else:
        wt = wrng.standard_normal((size * size, cin)).astype(np.float16).astype(np.float32)
    bias = wrng.standard_normal(cout).astype(np.float32)
    return entry, x, wt, bias
