"""ctypes face of the oracle (liboracle.so), for tests, smoke() and the CPU
baseline of bench.py.

TEST INFRASTRUCTURE ONLY: the oracle is the CPU restatement of the
reference's f32 path (crates/native-engine, crates/realesrgan-native) that
the HIP backend is checked against and timed beside.  The product never
imports this module.
"""

import ctypes
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

INPUT_ROWS, INPUT_IMAGE = 0, 1
TAPS_CONV, TAPS_OFFSETS = 0, 1
PAD_ZERO, PAD_REFLECT = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2
FINISH_NONE, FINISH_PRELU, FINISH_RELU = 0, 1, 2


class _Input(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("data", ctypes.c_void_p),
        ("height", ctypes.c_size_t),
        ("width", ctypes.c_size_t),
        ("channels", ctypes.c_size_t),
        ("stride", ctypes.c_size_t),
        ("taps", ctypes.c_int),
        ("size", ctypes.c_size_t),
        ("step", ctypes.c_size_t),
        ("pad", ctypes.c_int),
        ("offsets", (ctypes.c_size_t * 2) * 4),
        ("count", ctypes.c_size_t),
    ]


_lib = None


def build():
    """Compile liboracle.so with its Makefile (gcc only)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, sz, f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
        L.or_f32_to_half.restype = ctypes.c_uint16
        L.or_f32_to_half.argtypes = [f]
        L.or_half_to_f32.restype = f
        L.or_half_to_f32.argtypes = [ctypes.c_uint16]
        L.or_floats_to_halves.argtypes = [vp, vp, sz]
        L.or_halves_to_f32.argtypes = [vp, vp, sz]
        L.or_exp_neg.restype = f
        L.or_exp_neg.argtypes = [f]
        L.or_sigmoid.argtypes = [vp, sz]
        L.or_gelu.argtypes = [vp, sz]
        L.or_layer_norm.argtypes = [vp, sz, vp, vp, sz]
        L.or_softmax.argtypes = [vp, sz]
        L.or_multiply.argtypes = [vp, sz, sz, vp, sz, sz, vp, vp, sz, ctypes.c_int, ctypes.c_int]
        L.or_multiply_mt.argtypes = [ctypes.c_int, vp, sz, vp, sz, sz, vp, vp, sz, ctypes.c_int, ctypes.c_int]
        L.or_conv3.argtypes = [ctypes.c_int, vp, vp, sz, vp, vp, sz, ctypes.c_int, ctypes.c_int, vp]
        L.or_conv3_form.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, sz, vp, vp, sz, ctypes.c_int, ctypes.c_int, vp]
        L.or_attention.argtypes = [vp, sz, sz, sz, vp, vp]
        L.or_position_bias.argtypes = [vp, sz, sz, ctypes.c_int, vp]
        L.or_bias_tables.restype = sz
        L.or_bias_tables.argtypes = [vp, sz, sz, sz, f, vp]
        L.or_window_source.restype = ctypes.c_long
        L.or_window_source.argtypes = [sz, sz, sz, sz, sz, sz]
        L.or_window_class.restype = sz
        L.or_window_class.argtypes = [sz, sz, sz, sz, sz]
        L.or_swin_attend.argtypes = [ctypes.c_int, vp, sz, sz, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp, vp]
        L.or_swin_mlp.argtypes = [ctypes.c_int, vp, sz, sz, sz, vp, vp, vp, vp, vp, vp]
        L.or_scunet_run.restype = ctypes.c_int
        L.or_scunet_run.argtypes = [ctypes.c_int, vp, vp, sz, sz, vp]
        L.or_realesrgan_run.restype = ctypes.c_int
        L.or_realesrgan_run.argtypes = [ctypes.c_int, vp, vp, vp, vp, sz, sz, vp]
        L.or_pixel_shuffle_add.argtypes = [vp, vp, sz, sz, vp]
        L.or_depthwise.argtypes = [ctypes.c_int, vp, sz, sz, sz, vp, sz, vp, vp]
        L.or_resize.argtypes = [vp, sz, sz, sz, vp, sz, sz, sz, ctypes.c_int]
        L.or_pad_replicate.argtypes = [vp, sz, sz, sz, vp]
        L.or_masked_rows.argtypes = [vp, vp, sz, sz, sz, vp]
        L.or_rfft2.argtypes = [vp, sz, sz, sz, vp]
        L.or_irfft2_add.argtypes = [vp, sz, sz, sz, vp]
        L.or_lama_run.argtypes = [ctypes.c_int, vp, vp, vp, sz, sz, vp]
        L.or_lama_run.restype = ctypes.c_int
        L.or_lama_up.argtypes = [ctypes.c_int, vp, vp, vp, sz, sz, sz, sz, vp]
        L.or_birefnet_run.argtypes = [ctypes.c_int, vp, sz, vp, sz, vp]
        L.or_birefnet_run.restype = ctypes.c_int
        L.or_to_float.restype = f
        L.or_to_float.argtypes = [ctypes.c_uint8]
        L.or_to_byte.restype = ctypes.c_uint8
        L.or_to_byte.argtypes = [f]
        L.or_bytes_to_floats.argtypes = [vp, vp, sz]
        L.or_floats_to_bytes.argtypes = [vp, vp, sz]
        L.or_normalize_bytes.argtypes = [vp, sz, vp]
        L.or_mask_bytes.argtypes = [vp, vp, sz]
        L.or_composite_bytes.argtypes = [vp, vp, vp, sz, vp]
        L.or_tile_regions.restype = sz
        L.or_tile_regions.argtypes = [sz, sz, sz, sz, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def threads_default():
    return os.cpu_count() or 1


# ---- 8-bit image I/O and tiling (io.c) --------------------------------------
def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def bytes_to_floats(b):
    """realesrgan-native lib.rs:292-295 to_float over an array of bytes."""
    b = _u8(b)
    out = np.empty(b.shape, np.float32)
    lib().or_bytes_to_floats(_p(b), _p(out), b.size)
    return out


def floats_to_bytes(x):
    """realesrgan-native lib.rs:297-300 to_byte over an array of floats."""
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().or_floats_to_bytes(_p(x), _p(out), x.size)
    return out


def normalize_bytes(rgb):
    """birefnet-native lib.rs:111-116: interleaved RGB bytes (..., 3) to the
    ImageNet-normalised floats."""
    rgb = _u8(rgb)
    out = np.empty(rgb.shape, np.float32)
    lib().or_normalize_bytes(_p(rgb), rgb.size // 3, _p(out))
    return out


def mask_bytes(mask):
    mask = _u8(mask)
    out = np.empty(mask.shape, np.float32)
    lib().or_mask_bytes(_p(mask), _p(out), mask.size)
    return out


def composite_bytes(rgb, mask, pred):
    """lama-native lib.rs:147-155 over H x W x 3 bytes, an H x W byte mask
    and H x W x 3 predicted floats."""
    rgb, mask, pred = _u8(rgb), _u8(mask), _f32(pred)
    out = np.empty(rgb.shape, np.uint8)
    lib().or_composite_bytes(_p(rgb), _p(mask), _p(pred), mask.size, _p(out))
    return out


def tile_regions(width, height, tile, margin):
    """realesrgan-native lib.rs:251-265: rows of (x0, x1, y0, y1, rx0, rx1,
    ry0, ry1), one per tile in row-major order."""
    if tile == 0:
        return np.zeros((0, 8), np.uint64)
    n = -(-width // tile) * -(-height // tile)
    out = np.zeros((n, 8), np.uint64)
    k = lib().or_tile_regions(width, height, tile, margin, _p(out))
    return out[:k].astype(np.int64)


# ---- half.rs ---------------------------------------------------------------
def f32_to_half(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_floats_to_halves(_p(x), _p(out), x.size)
    return out


def half_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_halves_to_f32(_p(h), _p(out), h.size)
    return out


# ---- math.rs ---------------------------------------------------------------
def exp_neg(z):
    return np.array([lib().or_exp_neg(float(v)) for v in np.ravel(z)], np.float32).reshape(np.shape(z))


def sigmoid(x):
    x = _f32(x).copy()
    lib().or_sigmoid(_p(x), x.size)
    return x


def gelu(x):
    x = _f32(x).copy()
    lib().or_gelu(_p(x), x.size)
    return x


def layer_norm(x, gamma, beta):
    x = _f32(x).copy()
    gamma, beta = _f32(gamma), _f32(beta)
    lib().or_layer_norm(_p(x), x.size, _p(gamma), _p(beta), gamma.size)
    return x


def softmax(x):
    x = _f32(x).copy()
    lib().or_softmax(_p(x), x.size)
    return x


# ---- gemm.rs ---------------------------------------------------------------
def _image_input(data, height, width, channels, stride, size=3, step=1, pad=PAD_ZERO, offsets=None):
    s = _Input()
    s.kind = INPUT_IMAGE
    s.data = data.ctypes.data
    s.height, s.width, s.channels, s.stride = height, width, channels, stride
    if offsets is None:
        s.taps = TAPS_CONV
        s.size, s.step, s.pad = size, step, pad
    else:
        s.taps = TAPS_OFFSETS
        s.count = len(offsets)
        for i, (dy, dx) in enumerate(offsets):
            s.offsets[i][0], s.offsets[i][1] = dy, dx
    return s


def _rows_input(data, stride):
    s = _Input()
    s.kind = INPUT_ROWS
    s.data = data.ctypes.data
    s.stride = stride
    return s


def multiply_rows(a, w, bias=None, act=ACT_NONE, out=None, accumulate=False, threads=1):
    """gemm::multiply on Input::Rows: a is m x k, w k x n."""
    a, w = _f32(a), _f32(w)
    m, k = a.shape
    n = w.shape[1]
    bias = None if bias is None else _f32(bias)
    res = np.zeros((m, n), np.float32) if out is None else _f32(out).copy()
    inp = _rows_input(a, k)
    lib().or_multiply_mt(threads, ctypes.byref(inp), m, _p(w), k, n, _p(bias), _p(res), n, act, int(accumulate))
    return res


def multiply_conv(x, w, bias=None, size=3, step=1, pad=PAD_ZERO, act=ACT_NONE, offsets=None,
                  out=None, accumulate=False, threads=1):
    """gemm::multiply on Input::Image: x is H x W x C (NHWC), w (taps*C) x n."""
    x, w = _f32(x), _f32(w)
    h, wd, c = x.shape
    n = w.shape[1]
    inp = _image_input(x, h, wd, c, c, size, step, pad, offsets)
    if offsets is None:
        oh, ow = (h - 1) // step + 1, (wd - 1) // step + 1
    else:
        oh, ow = h, wd
    bias = None if bias is None else _f32(bias)
    res = np.zeros((oh * ow, n), np.float32) if out is None else _f32(out).reshape(oh * ow, n).copy()
    lib().or_multiply_mt(threads, ctypes.byref(inp), oh * ow, _p(w), w.shape[0], n, _p(bias), _p(res), n, act,
                         int(accumulate))
    return res.reshape(oh, ow, n)


def conv3(x, w, bias=None, pad=PAD_ZERO, finish=FINISH_NONE, slope=None, out=None, accumulate=False,
          threads=1, form=None):
    """winograd::conv3 on an H x W x C image; form None = the reference policy."""
    x, w = _f32(x), _f32(w)
    h, wd, c = x.shape
    n = w.shape[1]
    inp = _image_input(x, h, wd, c, c, 3, 1, pad)
    bias = None if bias is None else _f32(bias)
    slope = None if slope is None else _f32(slope)
    res = np.zeros((h * wd, n), np.float32) if out is None else _f32(out).reshape(h * wd, n).copy()
    if form is None:
        lib().or_conv3(threads, ctypes.byref(inp), _p(w), n, _p(bias), _p(res), n, int(accumulate), finish,
                       _p(slope))
    else:
        lib().or_conv3_form(threads, form, ctypes.byref(inp), _p(w), n, _p(bias), _p(res), n, int(accumulate),
                            finish, _p(slope))
    return res.reshape(h, wd, n)


# ---- attention.rs ----------------------------------------------------------
def attention(qkv, c, head, bias):
    qkv, bias = _f32(qkv), _f32(bias)
    tokens = qkv.shape[0]
    out = np.zeros((tokens, c), np.float32)
    lib().or_attention(_p(qkv), tokens, c, head, _p(bias), _p(out))
    return out


# ---- Swin window attention -------------------------------------------------
POS_SCUNET, POS_SWIN = 0, 1


def position_bias(table, heads, window, layout):
    """[heads, N, N] relative-position bias of a window from its table."""
    n = window * window
    out = np.zeros((heads, n, n), np.float32)
    lib().or_position_bias(_p(_f32(table)), heads, window, layout, _p(out))
    return out


def bias_tables(position, window, shift, masked):
    """[classes, heads, N, N]: 1 class unshifted, 4 shifted."""
    position = _f32(position)
    heads, n = position.shape[0], window * window
    out = np.zeros((4, heads, n, n), np.float32)
    k = lib().or_bias_tables(_p(position), heads, window, shift, masked, _p(out))
    return out[:k]


def window_source(w, i, window, shift, height, width):
    return lib().or_window_source(w, i, window, shift, height, width)


def window_class(w, window, shift, height, width):
    return lib().or_window_class(w, window, shift, height, width)


def swin_attend(x, window, shift, gamma, beta, wqkv, bqkv, tables, wproj, bproj, threads=None):
    """The attention half of a Swin block on an H x W x c map (returns a copy)."""
    x = _f32(x).copy()
    h, wd, c = x.shape
    lib().or_swin_attend(threads or threads_default(), _p(x), c, h, wd, c, window, shift, _p(_f32(gamma)),
                         _p(_f32(beta)), _p(_f32(wqkv)), _p(_f32(bqkv)), _p(_f32(tables)), _p(_f32(wproj)),
                         _p(_f32(bproj)))
    return x


def swin_mlp(x, gamma, beta, w1, b1, w2, b2, threads=None):
    """The MLP half on rows of c values (returns a copy)."""
    x = _f32(x).copy()
    c = x.shape[-1]
    rows = x.size // c
    lib().or_swin_mlp(threads or threads_default(), _p(x), c, rows, c, _p(_f32(gamma)), _p(_f32(beta)),
                      _p(_f32(w1)), _p(_f32(b1)), _p(_f32(w2)), _p(_f32(b2)))
    return x


# ---- realesrgan-native -----------------------------------------------------
def realesrgan_run(layers, image, threads=None):
    """layers: list of 34 (w[9cin x cout], b[cout], slope[64] or None); image H x W x 3."""
    image = _f32(image)
    h, w, _ = image.shape
    ws = [_f32(l[0]) for l in layers]
    bs = [_f32(l[1]) for l in layers]
    ss = [_f32(l[2]) if l[2] is not None else _f32(np.zeros(64)) for l in layers]
    arr = ctypes.c_void_p * len(layers)
    wp = arr(*[a.ctypes.data for a in ws])
    bp = arr(*[a.ctypes.data for a in bs])
    sp = arr(*[a.ctypes.data for a in ss])
    out = np.zeros((h * 4, w * 4, 3), np.float32)
    rc = lib().or_realesrgan_run(threads or threads_default(), ctypes.cast(wp, ctypes.c_void_p),
                                 ctypes.cast(bp, ctypes.c_void_p), ctypes.cast(sp, ctypes.c_void_p),
                                 _p(image), w, h, _p(out))
    if rc != 0:
        raise MemoryError("oracle realesrgan: allocation failed")
    return out


def pixel_shuffle_add(last, image):
    last, image = _f32(last), _f32(image)
    h, w, _ = image.shape
    out = np.zeros((h * 4, w * 4, 3), np.float32)
    lib().or_pixel_shuffle_add(_p(last), _p(image), w, h, _p(out))
    return out


def depthwise(x, w, bias=None, threads=1):
    """x H x W x C, w (size*size) x C -> H x W x C (zero pad, stride 1)."""
    x, w = _f32(x), _f32(w)
    h, wd, c = x.shape
    size = int(round(np.sqrt(w.shape[0])))
    bias = None if bias is None else _f32(bias)
    y = np.zeros_like(x)
    lib().or_depthwise(threads, _p(x), h, wd, c, _p(w), size, _p(bias), _p(y))
    return y


# ---- resize and padding helpers -------------------------------------------
def resize(src, dh, dw, out=None, add=False):
    """src [sh, sw, c] -> [dh, dw, c] (into a copy of `out` when adding)."""
    src = _f32(src)
    sh, sw, c = src.shape
    dst = np.zeros((dh, dw, c), np.float32) if out is None else _f32(out).copy()
    lib().or_resize(_p(src), sh, sw, c, _p(dst), dh, dw, c, int(add))
    return dst


def pad_replicate(image, multiple):
    image = _f32(image)
    h, w, _ = image.shape
    ph, pw = -(-h // multiple) * multiple, -(-w // multiple) * multiple
    out = np.zeros((ph, pw, 3), np.float32)
    lib().or_pad_replicate(_p(image), w, h, multiple, _p(out))
    return out


def masked_rows(image, mask, multiple):
    image, mask = _f32(image), _f32(mask)
    h, w, _ = image.shape
    ph, pw = -(-h // multiple) * multiple, -(-w // multiple) * multiple
    out = np.zeros((ph, pw, 4), np.float32)
    lib().or_masked_rows(_p(image), _p(mask), w, h, multiple, _p(out))
    return out


# ---- scunet-native -----------------------------------------------------------
def scunet_run(tensors, names, image, threads=None):
    """tensors: name -> array; names: the canonical order (synthetic.scunet_names)."""
    image = _f32(image)
    h, w, _ = image.shape
    arrs = [_f32(tensors[n]) for n, _ in names]
    ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    out = np.zeros((h, w, 3), np.float32)
    rc = lib().or_scunet_run(threads or threads_default(), ctypes.cast(ptrs, ctypes.c_void_p), _p(image), w, h,
                             _p(out))
    if rc != 0:
        raise RuntimeError(f"or_scunet_run: {rc}")
    return out


def rfft2(x):
    """fourier.rs forward: x (h, w, c) -> spectrum (h, w // 2 + 1, 2c) as [re | im]."""
    x = _f32(x)
    h, w, c = x.shape
    out = np.zeros((h, w // 2 + 1, 2 * c), np.float32)
    lib().or_rfft2(_p(x), h, w, c, _p(out))
    return out


def irfft2_add(spectrum, out):
    """fourier.rs inverse: out (h, w, c) += irfftn(spectrum), in place; returns out."""
    s = _f32(spectrum)
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    h, w, c = out.shape
    assert s.shape == (h, w // 2 + 1, 2 * c)
    lib().or_irfft2_add(_p(s), h, w, c, _p(out))
    return out


def lama_run(tensors, names, image, mask, threads=None):
    """tensors: name -> array; names: the weights file's order (synthetic.lama_names)."""
    image = _f32(image)
    mask = _f32(mask)
    h, w, _ = image.shape
    assert mask.shape == (h, w)
    arrs = [_f32(tensors[n]) for n, _ in names]
    ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    out = np.zeros((h, w, 3), np.float32)
    rc = lib().or_lama_run(threads or threads_default(), ctypes.cast(ptrs, ctypes.c_void_p), _p(image),
                           _p(mask), w, h, _p(out))
    if rc != 0:
        raise RuntimeError(f"or_lama_run: {rc}")
    return out


def lama_up(phase_w, phase_b, x, threads=1):
    """network.rs Up::run: x (h, w, cin) -> (2h, 2w, cout), ReLU."""
    x = _f32(x)
    h, w, cin = x.shape
    ws = [_f32(m) for m in phase_w]
    bs = [_f32(b) for b in phase_b]
    cout = ws[0].shape[1]
    pw = (ctypes.c_void_p * 4)(*[m.ctypes.data for m in ws])
    pb = (ctypes.c_void_p * 4)(*[b.ctypes.data for b in bs])
    out = np.zeros((2 * h, 2 * w, cout), np.float32)
    lib().or_lama_up(threads, ctypes.cast(pw, ctypes.c_void_p), ctypes.cast(pb, ctypes.c_void_p), _p(x), h, w,
                     cin, cout, _p(out))
    return out


def birefnet_run(tensors, names, image, window, threads=None):
    """tensors: name -> array; names: the load order (synthetic.birefnet_names).
    image: (side, side, 3) normalised; returns (side, side) logits."""
    image = _f32(image)
    side = image.shape[0]
    arrs = [_f32(tensors[n]) for n, _ in names]
    ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    out = np.zeros((side, side), np.float32)
    rc = lib().or_birefnet_run(threads or threads_default(), ctypes.cast(ptrs, ctypes.c_void_p), window,
                               _p(image), side, _p(out))
    if rc != 0:
        raise RuntimeError(f"or_birefnet_run: {rc}")
    return out
