"""Synthetic workloads of the benchmark configurations: seeded inputs and
random-init weights, the same on every machine (numpy's PCG64 generator,
`numpy.random.default_rng(seed)`; seed 0 for inputs, seed 1 for weights).

Real-ESRGAN general x4v3 (SRVGGNetCompact, crates/realesrgan-native/src/
network.rs): weights Kaiming-normal (std sqrt(2 / fan_in), fan_in = 9 cin,
as torch.nn.init.kaiming_normal_), biases uniform in +-1/sqrt(fan_in)
(torch's Conv2d default), PReLU slopes 0.25 (torch's PReLU default); the
weights file layout of tools/realesrgan/export_weights.py:48-56 (conv
[o, i, kh, kw] -> [(kh, kw, i), o]).

SCUNet (crates/scunet-native/src/network.rs, swin.rs): the tensor names and
[k, n] layouts of tools/scunet/export_weights.py (convolutions [(kh, kw, i),
o], position biases gathered to [heads, 64, 64]).  The configuration's init
is trunc-normal with std 0.02 for every weight and position table (at that
std the +-2 cut is never reached: plain N(0, 0.02^2)), zero biases,
LayerNorm gamma 1 and beta 0.  Parity tests use a fan-in-scaled init instead
(N(0, 1 / fan_in) weights, small random biases and norms) so that
activations do not vanish through the network.
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


# ---- SCUNet ------------------------------------------------------------------
SCUNET_DIM, SCUNET_BLOCKS, SCUNET_WINDOW = 64, 4, 8
RESIDUAL_GAIN = 0.2
LAMA_RESIDUAL_GAIN = 0.05


def _scunet_block(name, c):
    h = c // 2
    t = f"{name}.trans_block"
    return [(f"{name}.conv1_1.weight", (c, c)), (f"{name}.conv1_1.bias", (c,)),
            (f"{name}.conv_block.0.weight", (9 * h, h)), (f"{name}.conv_block.2.weight", (9 * h, h)),
            (f"{t}.ln1.weight", (h,)), (f"{t}.ln1.bias", (h,)),
            (f"{t}.msa.embedding_layer.weight", (h, 3 * h)), (f"{t}.msa.embedding_layer.bias", (3 * h,)),
            (f"{t}.msa.position_bias", (h // 32, 64, 64)),
            (f"{t}.msa.linear.weight", (h, h)), (f"{t}.msa.linear.bias", (h,)),
            (f"{t}.ln2.weight", (h,)), (f"{t}.ln2.bias", (h,)),
            (f"{t}.mlp.0.weight", (h, 4 * h)), (f"{t}.mlp.0.bias", (4 * h,)),
            (f"{t}.mlp.2.weight", (4 * h, h)), (f"{t}.mlp.2.bias", (h,)),
            (f"{name}.conv1_2.weight", (c, c)), (f"{name}.conv1_2.bias", (c,))]


def scunet_names():
    """(name, shape) of the 540 tensors, in the order the network consumes
    them (the oracle's or_scunet_run order)."""
    out = [("m_head.0.weight", (27, SCUNET_DIM))]
    for i, c in ((1, 64), (2, 128), (3, 256)):
        for b in range(SCUNET_BLOCKS):
            out += _scunet_block(f"m_down{i}.{b}", c)
        out.append((f"m_down{i}.{SCUNET_BLOCKS}.weight", (4 * c, 2 * c)))
    for b in range(SCUNET_BLOCKS):
        out += _scunet_block(f"m_body.{b}", 512)
    for i, c in ((3, 256), (2, 128), (1, 64)):
        out.append((f"m_up{i}.0.weight", (2 * c, 4 * c)))
        for b in range(SCUNET_BLOCKS):
            out += _scunet_block(f"m_up{i}.{b + 1}", c)
    out.append(("m_tail.0.weight", (9 * SCUNET_DIM, 3)))
    return out


def gathered_position_bias(rel, window, swin_layout):
    """[heads][N][N] position bias gathered from a relative-position table,
    the way both models' attention builds it: `rel` is [(2W - 1)^2][heads]
    (Swin: birefnet-native swin.rs) or [heads][2W - 1][2W - 1] (scunet-native
    swin.rs); entry (i, j) takes cell (yi - yj + W - 1, xi - xj + W - 1)."""
    side, n = 2 * window - 1, window * window
    i = np.arange(n)
    y, x = i // window, i % window
    cell = (y[:, None] - y[None, :] + window - 1) * side + (x[:, None] - x[None, :] + window - 1)
    table = rel.T if swin_layout else rel.reshape(rel.shape[0], side * side)
    return np.stack([table[h][cell] for h in range(table.shape[0])])


def scunet_tensors(seed=WEIGHT_SEED, init="trunc_normal"):
    """name -> array for every SCUNet tensor.  init: "trunc_normal" (the
    configuration's std 0.02) or "fan" (N(0, 1/fan_in) weights, for parity
    tests)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in scunet_names():
        last = name.rsplit(".", 1)[-1]
        is_norm = ".ln1." in name or ".ln2." in name
        if last == "position_bias":
            # A relative-position table [heads][15][15], gathered per window.
            side = 2 * SCUNET_WINDOW - 1
            rel = rng.standard_normal((shape[0], side, side)) * (0.02 if init == "trunc_normal" else 1.0)
            v = gathered_position_bias(rel, SCUNET_WINDOW, swin_layout=False)
        elif init == "trunc_normal":
            if is_norm:
                v = np.ones(shape) if last == "weight" else np.zeros(shape)
            elif last == "bias":
                v = np.zeros(shape)
            else:
                v = 0.02 * rng.standard_normal(shape)
        else:
            if is_norm:
                v = (1 + 0.1 * rng.standard_normal(shape)) if last == "weight" else 0.1 * rng.standard_normal(shape)
            elif last == "bias":
                v = 0.05 * rng.standard_normal(shape)
            elif last == "position_bias":
                v = rng.standard_normal(shape)
            else:
                v = rng.standard_normal(shape) / np.sqrt(shape[0])
                # Matrices whose output is added onto a residual stream get a
                # small gain, so the 28 residual blocks keep activations O(1).
                if any(k in name for k in ("conv_block.2", "msa.linear", "mlp.2", "conv1_2")):
                    v *= RESIDUAL_GAIN
        out[name] = np.asarray(v, np.float32)
    return out


def scunet_image(height=512, width=768, seed=INPUT_SEED):
    """H x W x 3 RGB, uniform [0, 1)."""
    return np.random.default_rng(seed).random((height, width, 3), dtype=np.float32)


# Big LaMa (crates/lama-native/src/network.rs): 4 -> 64 -> 128 -> 256 -> 512
# channels, 18 blocks of two fast Fourier convolutions at an eighth of the
# size, three transposed upsamplings, 7x7 to RGB.
LAMA_LOCAL, LAMA_GLOBAL, LAMA_BLOCKS = 128, 384, 18


def lama_names():
    """(name, shape) of every LaMa tensor in the weights file's order
    (tools/lama/export_weights.py export)."""
    c = LAMA_LOCAL + LAMA_GLOBAL
    spectral = LAMA_GLOBAL // 2
    names = [("first.weight", (49 * 4, 64)), ("first.bias", (64,))]
    for i, (cin, cout) in enumerate(((64, 128), (128, 256), (256, c))):
        names += [(f"down{i}.weight", (9 * cin, cout)), (f"down{i}.bias", (cout,))]
    for b in range(LAMA_BLOCKS):
        for f in range(2):
            n = f"block{b}.ffc{f}"
            names += [
                (f"{n}.local.weight", (9 * c, LAMA_LOCAL)), (f"{n}.local.bias", (LAMA_LOCAL,)),
                (f"{n}.cross.weight", (9 * LAMA_LOCAL, LAMA_GLOBAL)), (f"{n}.cross.bias", (LAMA_GLOBAL,)),
                (f"{n}.spectral_in.weight", (LAMA_GLOBAL, spectral)), (f"{n}.spectral_in.bias", (spectral,)),
                (f"{n}.fourier.weight", (2 * spectral, 2 * spectral)), (f"{n}.fourier.bias", (2 * spectral,)),
                (f"{n}.spectral_out.weight", (spectral, LAMA_GLOBAL)),
            ]
    for i, (cin, cout) in enumerate(((c, 256), (256, 128), (128, 64))):
        for p in range(4):
            taps = (1, 2, 2, 4)[p]
            names += [(f"up{i}.phase{p}.weight", (taps * cin, cout)), (f"up{i}.phase{p}.bias", (cout,))]
    names += [("last.weight", (49 * 64, 3)), ("last.bias", (3,))]
    return names


def lama_tensors(seed=WEIGHT_SEED):
    """name -> array for every LaMa tensor: He-normal matrices (N(0, 2 /
    fan_in), the ReLU networks' init with every batch norm folded as the
    identity), small biases; the second FFC of each block, whose output is
    added onto the residual stream, scaled by LAMA_RESIDUAL_GAIN so 18
    blocks keep activations O(1) and the sigmoid out of saturation."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in lama_names():
        if ".phase" in name and name.endswith(".bias") and ".phase0." not in name:
            # One transposed convolution's bias, shared by its four phases
            # (export_weights.py puts the same bias on each).
            out[name] = out[name.split(".phase")[0] + ".phase0.bias"]
            continue
        if name.endswith(".bias"):
            v = 0.02 * rng.standard_normal(shape)
        else:
            v = rng.standard_normal(shape) * np.sqrt(2.0 / shape[0])
            if ".ffc1." in name and not name.endswith(("spectral_in.weight", "fourier.weight")):
                v *= LAMA_RESIDUAL_GAIN
        out[name] = np.asarray(v, np.float32)
    return out


def lama_image(height=512, width=512, seed=INPUT_SEED):
    """H x W x 3 RGB, uniform [0, 1)."""
    return np.random.default_rng(seed).random((height, width, 3), dtype=np.float32)


def lama_mask(height=512, width=512, seed=INPUT_SEED + 1, cover=0.25):
    """H x W binary mask (1 = fill) of random rectangles, added until about
    `cover` of the pixels are set."""
    rng = np.random.default_rng(seed)
    m = np.zeros((height, width), np.float32)
    while m.mean() < cover:
        rh = int(rng.integers(max(1, height // 16), max(2, height // 3)))
        rw = int(rng.integers(max(1, width // 16), max(2, width // 3)))
        y = int(rng.integers(0, height - rh + 1))
        x = int(rng.integers(0, width - rw + 1))
        m[y:y + rh, x:x + rw] = 1.0
    return m


# BiRefNet-lite (crates/birefnet-native/src/swin.rs, decoder.rs): Swin-T
# backbone (96..768 channels, depths 2/2/6/2, head dim 32) and the decoder;
# the configured network uses windows of 12 (shift 6) and a deformable-free
# ASPP (all-zero offset and modulator convolutions).
BIREFNET_STAGES = ((96, 2), (192, 2), (384, 6), (768, 2))
BIREFNET_WINDOW = 12
BIREFNET_LEVELS = ((1728, 768), (960, 384), (480, 192), (240, 96))  # decoder.rs:776
BIREFNET_ASPP_SIZES = (1, 1, 3, 7)


def birefnet_names(window=BIREFNET_WINDOW):
    """(name, shape) of every BiRefNet tensor in the reference's load order
    (swin.rs Backbone::load, then decoder.rs Decoder::load)."""
    n = window * window
    names = [("patch_embed.weight", (48, 96)), ("patch_embed.bias", (96,)),
             ("patch_embed.norm.weight", (96,)), ("patch_embed.norm.bias", (96,))]
    for s, (c, depth) in enumerate(BIREFNET_STAGES):
        for b in range(depth):
            p = f"stage{s}.block{b}."
            names += [(p + "norm1.weight", (c,)), (p + "norm1.bias", (c,)),
                      (p + "qkv.weight", (c, 3 * c)), (p + "qkv.bias", (3 * c,)),
                      (p + "position_bias", (c // 32, n, n)),
                      (p + "proj.weight", (c, c)), (p + "proj.bias", (c,)),
                      (p + "norm2.weight", (c,)), (p + "norm2.bias", (c,)),
                      (p + "fc1.weight", (c, 4 * c)), (p + "fc1.bias", (4 * c,)),
                      (p + "fc2.weight", (4 * c, c)), (p + "fc2.bias", (c,))]
        if s < 3:
            names += [(f"stage{s}.merge.norm.weight", (4 * c,)), (f"stage{s}.merge.norm.bias", (4 * c,)),
                      (f"stage{s}.merge.weight", (4 * c, 2 * c))]
        names += [(f"stage{s}.norm.weight", (c,)), (f"stage{s}.norm.bias", (c,))]
    blocks = [("squeeze", 2880, 1536, False)] + [
        (f"block{4 - i}", cin, cout, i < 3) for i, (cin, cout) in enumerate(BIREFNET_LEVELS)]
    for q, cin, cout, gate in blocks:
        names += [(f"{q}.conv_in.weight", (9 * cin, 64)), (f"{q}.conv_in.bias", (64,)),
                  (f"{q}.conv_out.weight", (9 * 64, cout)), (f"{q}.conv_out.bias", (cout,))]
        if gate:
            names += [(f"{q}.gdt.weight", (9 * cout, 16)), (f"{q}.gdt.bias", (16,)),
                      (f"{q}.gdt_attn.weight", (16, 1)), (f"{q}.gdt_attn.bias", (1,))]
        for i, k in enumerate(BIREFNET_ASPP_SIZES):
            taps = k * k
            names += [(f"{q}.aspp.branch{i}.offset.weight", (taps * 64, 3 * taps)),
                      (f"{q}.aspp.branch{i}.offset.bias", (3 * taps,)),
                      (f"{q}.aspp.branch{i}.weight", (taps * 64, 256)),
                      (f"{q}.aspp.branch{i}.bias", (256,))]
        names += [(f"{q}.aspp.pool.weight", (64, 256)), (f"{q}.aspp.pool.bias", (256,)),
                  (f"{q}.aspp.conv1.weight", (1280, 64)), (f"{q}.aspp.conv1.bias", (64,))]
    for nn_, c in ((4, 768), (3, 384), (2, 192)):
        names += [(f"lateral{nn_}.weight", (c, c)), (f"lateral{nn_}.bias", (c,))]
    for nn_, cin, cout in ((5, 3072, 192), (4, 768, 192), (3, 192, 96), (2, 48, 48)):
        names += [(f"patches{nn_}.conv1.weight", (9 * cin, 64)), (f"patches{nn_}.conv1.bias", (64,)),
                  (f"patches{nn_}.conv_out.weight", (9 * 64, cout)), (f"patches{nn_}.conv_out.bias", (cout,))]
    names += [("head.weight", (96, 1)), ("head.bias", (1,)),
              ("patches1.conv1.weight", (27, 64)), ("patches1.conv1.bias", (64,)),
              ("patches1.conv_out.weight", (576, 1)), ("patches1.conv_out.bias", (1,))]
    return names


def _relu_followed(name):
    """Matrices whose output goes through a ReLU (He gain)."""
    return any(k in name for k in (".conv_in.", ".aspp.branch", ".aspp.pool.", ".aspp.conv1.", ".gdt."))


def birefnet_tensors(seed=WEIGHT_SEED, window=BIREFNET_WINDOW, init="trunc_normal", offsets=0.0):
    """name -> array for every BiRefNet tensor.  The Swin backbone: "trunc_normal"
    (timm's std 0.02, LayerNorms 1 / 0, zero biases: the configuration's
    random init) or "fan" (N(0, 1 / fan_in), residual writers scaled by
    RESIDUAL_GAIN, position biases N(0, 1): attention far from uniform, for
    parity tests).  The decoder: N(0, g^2 / fan_in) matrices (g = sqrt 2
    before a ReLU), small biases.  The ASPP's offset and modulator
    convolutions are zero (the deformable-free network) unless `offsets`
    sets their standard deviation."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in birefnet_names(window):
        last = name.rsplit(".", 1)[-1]
        is_norm = ".norm" in name and not name.endswith("merge.weight")
        if name.startswith("stage") or name.startswith("patch_embed"):
            if is_norm and last in ("weight", "bias") and name.split(".")[-2].startswith("norm"):
                if init == "trunc_normal":
                    v = np.ones(shape) if last == "weight" else np.zeros(shape)
                else:
                    v = (1 + 0.1 * rng.standard_normal(shape)) if last == "weight" else 0.1 * rng.standard_normal(shape)
            elif name.endswith("position_bias"):
                # A relative-position table [(2W - 1)^2][heads], gathered per window.
                rel_shape = ((2 * window - 1) ** 2, shape[0])
                rel = (np.clip(rng.standard_normal(rel_shape), -2, 2) * 0.02 if init == "trunc_normal"
                       else rng.standard_normal(rel_shape))
                v = gathered_position_bias(rel, window, swin_layout=True)
            elif last == "bias":
                v = np.zeros(shape) if init == "trunc_normal" else 0.05 * rng.standard_normal(shape)
            elif init == "trunc_normal" and not name.startswith("patch_embed"):
                v = np.clip(rng.standard_normal(shape), -2, 2) * 0.02
            else:
                v = rng.standard_normal(shape) / np.sqrt(shape[0])
                if init == "fan" and (name.endswith("proj.weight") or name.endswith("fc2.weight")):
                    v *= RESIDUAL_GAIN
        elif ".offset." in name:
            v = offsets * rng.standard_normal(shape) if offsets else np.zeros(shape)
        elif last == "bias":
            v = 0.02 * rng.standard_normal(shape)
        else:
            gain = np.sqrt(2.0) if _relu_followed(name) else 1.0
            v = gain * rng.standard_normal(shape) / np.sqrt(shape[0])
        out[name] = np.asarray(v, np.float32)
    return out


def birefnet_image(side=1024, seed=INPUT_SEED):
    """side x side x 3, N(0, 1): an image already normalised with ImageNet's
    statistics (the reference's run_normalized input)."""
    return np.random.default_rng(seed).standard_normal((side, side, 3)).astype(np.float32)
