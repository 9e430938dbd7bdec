"""Weights files and the export layouts of image-engine-native.

A weights file (crates/native-engine/src/weight_file.rs) is, little-endian:
8 magic bytes naming the model, u32 version 1, u32 tensor count, then per
tensor a u16 name length, the UTF-8 name, a u8 type (0 f32, 1 f16), a u8
rank, u32 dimensions and the values.  ien_model_load reads these files
unchanged; `write` produces them (as tools/*/export_weights.py write them)
and `read` parses them with the reference's checks.

The export functions turn a model's upstream tensors into the layouts the
reference's networks (and this backend's model drivers) read, following
tools/realesrgan/export_weights.py, tools/scunet/export_weights.py and
tools/lama/export_weights.py: convolutions as [(ky, kx, cin), cout]
matrices, transposed convolutions as [cin, (ky, kx, cout)], linear layers as
[in, out], batch norms folded into the convolution before them, LaMa's
Fourier channels made planar and its stride-2 transposed convolutions split
into four output phases.  BiRefNet's exporter reads an ONNX graph whose
decoder tensors are unnamed (tools/birefnet/export_weights.py:44-92); its
folds -- batch norm into the deformable convolutions, the offset and
modulator convolutions as one, the head split around the final upsampling --
are given here as functions of the named tensors.
"""

import struct

import numpy as np

MAGIC_REALESRGAN = b"REALESRG"
MAGIC_SCUNET = b"SCUNET\0\0"
MAGIC_LAMA = b"LAMA\0\0\0\0"
MAGIC_BIREFNET = b"BIREFNET"
VERSION = 1
BN_EPS = 1e-5


class WeightsError(ValueError):
    """A malformed weights file (the reference's Error::Weights)."""


# ---- the file format (weight_file.rs:15-146) --------------------------------
def write(path, magic, tensors, half=lambda name, array: False):
    """Write `tensors` (name -> array, in order) with `magic`; tensors for
    which half(name, array) holds are stored as IEEE half floats."""
    assert len(magic) == 8
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<II", VERSION, len(tensors)))
        for name, array in tensors.items():
            array = np.asarray(array, dtype=np.float32)
            encoded = name.encode()
            as_half = bool(half(name, array))
            f.write(struct.pack("<H", len(encoded)))
            f.write(encoded)
            f.write(struct.pack("<BB", int(as_half), array.ndim))
            f.write(struct.pack(f"<{array.ndim}I", *array.shape))
            f.write(np.ascontiguousarray(array).astype("<f2" if as_half else "<f4").tobytes())


def matrices_half(name, array):
    """The export tools' --half rule: weight matrices in f16, biases,
    normalisations and position biases in f32."""
    return array.ndim == 2 and name.endswith(".weight")


def read(path, magic):
    """Parse a weights file as weight_file.rs:40-117 does: every length is
    checked against what is left before it is used.  Returns name ->
    (shape, f32 values); raises WeightsError."""
    with open(path, "rb") as f:
        data = f.read()
    at = 0

    def take(n):
        nonlocal at
        if n > len(data) - at:
            raise WeightsError("weights file is truncated")
        out = data[at:at + n]
        at += n
        return out

    if take(8) != magic:
        kind = magic.rstrip(b"\0").decode()
        raise WeightsError(f"not a {kind} weights file")
    version, count = struct.unpack("<II", take(4) + take(4))
    if version != VERSION:
        raise WeightsError(f"weights file version {version}, expected {VERSION}")
    tensors = {}
    for _ in range(count):
        (name_len,) = struct.unpack("<H", take(2))
        try:
            name = take(name_len).decode("utf-8")
        except UnicodeDecodeError:
            raise WeightsError("tensor name is not UTF-8") from None
        dtype, rank = take(2)
        if dtype not in (0, 1):
            raise WeightsError(f"{name}: unknown type {dtype}")
        width = 4 if dtype == 0 else 2
        shape = struct.unpack(f"<{rank}I", take(4 * rank))
        count_ = 1
        for d in shape:
            count_ *= d
            if count_ > (1 << 64) - 1:
                raise WeightsError(f"{name}: too large")
        raw = take(count_ * width)
        values = np.frombuffer(raw, "<f4" if width == 4 else "<f2").astype(np.float32)
        if name in tensors:
            raise WeightsError(f"{name}: stored twice")
        tensors[name] = (tuple(shape), values.reshape(shape))
    if at != len(data):
        raise WeightsError("trailing bytes after the last tensor")
    return tensors


# ---- layouts shared by the exporters ----------------------------------------
def conv_matrix(w):
    """Convolution [out, in, kh, kw] -> [(kh, kw, in), out] (in w's type)."""
    o, i, kh, kw = w.shape
    return np.asarray(w).transpose(2, 3, 1, 0).reshape(kh * kw * i, o)


def transposed_matrix(w):
    """Transposed convolution [in, out, kh, kw] -> [in, (kh, kw, out)]."""
    i, o, kh, kw = w.shape
    return np.asarray(w, np.float32).transpose(0, 2, 3, 1).reshape(i, kh * kw * o)


def bn_scale_shift(weight, bias, mean, var, eps=BN_EPS, dtype=np.float32):
    """A batch norm in evaluation as scale and shift, computed in `dtype`
    (f32 for LaMa, whose exporter loads f32 tensors; f64 for BiRefNet's)."""
    weight, bias, mean, var = (np.asarray(a, dtype) for a in (weight, bias, mean, var))
    scale = weight / np.sqrt(var + dtype(eps))
    return scale, bias - mean * scale


# ---- Real-ESRGAN (tools/realesrgan/export_weights.py:48-56) -----------------
def realesrgan_export(state):
    """SRVGGNetCompact's state dict (body.{2i}.weight [o, i, 3, 3], biases,
    PReLU weights) -> the weights file's tensors."""
    out = {}
    for name, value in state.items():
        value = np.asarray(value, np.float32)
        out[name] = conv_matrix(value) if value.ndim == 4 else value
    return out


# ---- SCUNet (tools/scunet/export_weights.py:51-88) ---------------------------
SCUNET_WINDOW = 8


def scunet_position_bias(params, window=SCUNET_WINDOW):
    """[heads, 2W-1, 2W-1] relative position parameters -> the whole
    [heads, W^2, W^2] bias: tokens (y1, x1), (y2, x2) of a window read
    params[:, y1 - y2 + W - 1, x1 - x2 + W - 1]."""
    cells = np.array([(y, x) for y in range(window) for x in range(window)])
    d = cells[:, None, :] - cells[None, :, :] + window - 1
    return np.asarray(params, np.float32)[:, d[..., 0], d[..., 1]]


def scunet_export(state):
    """SCUNet's state dict (KAIR names) -> the weights file's tensors."""
    out = {}
    for name, value in state.items():
        value = np.asarray(value, np.float32)
        if name.endswith(".relative_position_params"):
            out[name[: -len("relative_position_params")] + "position_bias"] = scunet_position_bias(value)
        elif name.startswith("m_up") and name.split(".")[1:] == ["0", "weight"]:
            out[name] = transposed_matrix(value)
        elif value.ndim == 4:
            out[name] = conv_matrix(value)
        elif value.ndim == 2:
            out[name] = value.T.copy()
        else:
            out[name] = value
    return out


# ---- Big LaMa (tools/lama/export_weights.py:51-143) --------------------------
LAMA_LOCAL, LAMA_GLOBAL, LAMA_BLOCKS = 128, 384, 18
LAMA_SPECTRAL = LAMA_GLOBAL // 2
# (input offset, kernel tap) per output phase along one axis: an even output
# 2m reads input m through tap 1, an odd one 2m + 1 reads m through tap 2
# and m + 1 through tap 0 (crates/lama-native/src/network.rs:268-271).
LAMA_PHASE_TAPS = [[(0, 1)], [(0, 2), (1, 0)]]


def lama_phases(weight):
    """A stride-2 transposed convolution [in, out, 3, 3] as its four output
    phases (even/odd row, even/odd column): the stacked [in, out] blocks of
    the kernel taps each phase reads, in offset order."""
    weight = np.asarray(weight)
    phases = []
    for phase in range(4):
        ys, xs = LAMA_PHASE_TAPS[phase // 2], LAMA_PHASE_TAPS[phase % 2]
        phases.append(np.concatenate([weight[:, :, ky, kx] for _, ky in ys for _, kx in xs]))
    return phases


def lama_planar(channels=LAMA_SPECTRAL):
    """The permutation from LaMa's interleaved spectrum channels (real and
    imaginary parts alternating) to all real parts, then all imaginary."""
    return np.array([2 * c + j for j in range(2) for c in range(channels)])


def lama_export(state):
    """Big LaMa generator tensors (names relative to generator.model., batch
    norms with running statistics) -> the weights file's tensors.  Raises
    KeyError for a missing tensor and ValueError for unused ones."""
    used = set()

    def get(name):
        used.add(name)
        return np.asarray(state[name], np.float32)

    def bn(name):
        return bn_scale_shift(get(f"{name}.weight"), get(f"{name}.bias"), get(f"{name}.running_mean"),
                              get(f"{name}.running_var"))

    out = {}

    def put(name, matrix, bias=None):
        out[f"{name}.weight"] = np.asarray(matrix, np.float32)
        if bias is not None:
            out[f"{name}.bias"] = np.asarray(bias, np.float32)

    scale, shift = bn("1.bn_l")
    put("first", conv_matrix(get("1.ffc.convl2l.weight")) * scale, shift)
    for i, layer in enumerate((2, 3)):
        scale, shift = bn(f"{layer}.bn_l")
        put(f"down{i}", conv_matrix(get(f"{layer}.ffc.convl2l.weight")) * scale, shift)
    weight = np.concatenate([get("4.ffc.convl2l.weight"), get("4.ffc.convl2g.weight")])
    (sl, hl), (sg, hg) = bn("4.bn_l"), bn("4.bn_g")
    put("down2", conv_matrix(weight) * np.concatenate([sl, sg]), np.concatenate([hl, hg]))
    planar = lama_planar()
    for b in range(LAMA_BLOCKS):
        for f, half in enumerate(("conv1", "conv2")):
            p, name = f"{5 + b}.{half}", f"block{b}.ffc{f}"
            (sl, hl), (sg, hg) = bn(f"{p}.bn_l"), bn(f"{p}.bn_g")
            local = np.concatenate([get(f"{p}.ffc.convl2l.weight"), get(f"{p}.ffc.convg2l.weight")], axis=1)
            put(f"{name}.local", conv_matrix(local) * sl, hl)
            put(f"{name}.cross", conv_matrix(get(f"{p}.ffc.convl2g.weight")) * sg, hg)
            g = f"{p}.ffc.convg2g"
            scale, shift = bn(f"{g}.conv1.1")
            put(f"{name}.spectral_in", conv_matrix(get(f"{g}.conv1.0.weight")) * scale, shift)
            scale, shift = bn(f"{g}.fu.bn")
            fourier = conv_matrix(get(f"{g}.fu.conv_layer.weight")) * scale
            put(f"{name}.fourier", fourier[planar][:, planar], shift[planar])
            put(f"{name}.spectral_out", conv_matrix(get(f"{g}.conv2.weight")) * sg)
    for i, (layer, norm) in enumerate(((24, 25), (27, 28), (30, 31))):
        scale, shift = bn(str(norm))
        bias = get(f"{layer}.bias") * scale + shift
        for phase, taps in enumerate(lama_phases(get(f"{layer}.weight"))):
            put(f"up{i}.phase{phase}", taps * scale, bias)
    put("last", conv_matrix(get("34.weight")), get("34.bias"))
    unused = sorted(set(state) - used - {k for k in state if k.endswith("num_batches_tracked")})
    if unused:
        raise ValueError(f"generator tensors not exported: {unused[:5]}")
    return out


# ---- BiRefNet folds (tools/birefnet/export_weights.py:170-247) ---------------
def birefnet_deformable(offset_w, offset_b, modulator_w, modulator_b):
    """A deformable convolution's offset [2 k^2, 64, k, k] and modulator
    [k^2, 64, k, k] convolutions, which read the same input with the same
    kernel, as one matrix [(k, k, 64), 3 k^2] and its bias."""
    w = np.concatenate([np.asarray(offset_w, np.float64), np.asarray(modulator_w, np.float64)])
    return conv_matrix(w), np.concatenate([offset_b, modulator_b]).astype(np.float32)


def birefnet_branch(weight, gamma, beta, mean, var):
    """A deformable branch's regular convolution [256, 64, k, k] with the
    batch norm after it folded in: matrix and bias."""
    scale, shift = bn_scale_shift(gamma, beta, mean, var, dtype=np.float64)
    return conv_matrix(np.asarray(weight, np.float64) * scale[:, None, None, None]), shift.astype(np.float32)


def birefnet_head(head_w, head_b, patch_w, patch_b):
    """The last 1x1 convolution [1, 120, 1, 1] split: its 96 decoder
    channels (before the final upsampling, with which it commutes) as
    head.weight [96, 1] and head.bias, and its 24 image-patch channels
    folded into the 3x3 convolution that makes them ([24, 64, 3, 3] and
    bias [24]) as patches1.conv_out's one output channel."""
    head = np.asarray(head_w, np.float64)[0, :, 0, 0]
    patch_w = np.asarray(patch_w, np.float64)
    folded = np.einsum("k,kcij->cij", head[96:], patch_w)[None]
    return {"head.weight": head[:96].reshape(96, 1).astype(np.float32),
            "head.bias": np.asarray(head_b, np.float32),
            "patches1.conv_out.weight": conv_matrix(folded),
            "patches1.conv_out.bias": np.array([head[96:] @ np.asarray(patch_b, np.float64)], np.float32)}
