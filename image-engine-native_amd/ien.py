"""ctypes binding of libien_hip.so, the MI355X backend's C ABI
(include/ien_hip.h), for the tests and the benchmark.

Device buffers are torch tensors on the GPU (plumbing only: the kernels are
the library's); the library runs on torch's current stream, so torch events
and synchronisation order with it.  Nothing here falls back to the CPU: a
missing or unloadable library raises.
"""

import ctypes
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libien_hip.so"

OK, ERR_IO, ERR_WEIGHTS, ERR_INPUT, ERR_CANCELLED, ERR_GPU = range(6)
W_F32, W_F16 = 0, 1
PAD_ZERO, PAD_REFLECT = 0, 1
TAPS_CONV, TAPS_OFFSETS = 0, 1
INPUT_ROWS, INPUT_IMAGE = 0, 1
NHWC, NCHW = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU, ACT_PRELU, ACT_SIGMOID = range(5)
OUT_F16, OUT_F32 = 0, 1
MODEL_REALESRGAN, MODEL_SCUNET, MODEL_LAMA, MODEL_BIREFNET = 0, 1, 2, 3

# Every symbol include/ien_hip.h declares.
EXPORTS = (
    "ien_last_error", "ien_open", "ien_close", "ien_device_name", "ien_stream", "ien_set_stream",
    "ien_alloc", "ien_free", "ien_upload", "ien_download", "ien_sync",
    "ien_floats_to_halves", "ien_halves_to_floats",
    "ien_matrix_new", "ien_matrix_free", "ien_multiply", "ien_multiply_ex", "ien_conv3",
    "ien_conv3_pair", "ien_conv3_chain", "ien_conv3_chain_status", "ien_measure_mfma",
    "ien_layer_norm", "ien_gelu", "ien_sigmoid", "ien_pixel_shuffle_add", "ien_depthwise",
    "ien_model_load", "ien_model_from_tensors", "ien_model_free", "ien_model_run",
    "ien_model_run_device", "ien_model_status", "ien_model_set_graph", "ien_model_run_tiled", "ien_model_run_u8",
    "ien_bytes_to_floats", "ien_floats_to_bytes", "ien_mask_bytes", "ien_normalize_bytes",
    "ien_composite_bytes",
    "ien_window_count", "ien_position_bias", "ien_bias_tables", "ien_window_gather",
    "ien_window_attention", "ien_window_scatter_add", "ien_swin_new", "ien_swin_free", "ien_swin_run",
    "ien_swin_run_static",
    "ien_resize", "ien_pad_image", "ien_crop", "ien_gather_2x2", "ien_scatter_2x2", "ien_add",
    "ien_fourier_new", "ien_fourier_free", "ien_fourier_half", "ien_fourier_forward",
    "ien_fourier_inverse", "ien_spectral_new", "ien_spectral_free", "ien_spectral_work",
    "ien_spectral_run",
)


class Windows(ctypes.Structure):
    """ien_windows: a Swin block's windows over a height x width token map."""
    _fields_ = [("window", ctypes.c_int), ("shift", ctypes.c_int), ("height", ctypes.c_int),
                ("width", ctypes.c_int)]


POS_SCUNET, POS_SWIN = 0, 1
PAD_REPLICATE, PAD_SYMMETRIC_MASKED = 0, 1
ORDER_ROW_MAJOR, ORDER_COLUMN_MAJOR = 0, 1


class SwinWeights(ctypes.Structure):
    """ien_swin_weights (host f32 pointers)."""
    _fields_ = [("c", ctypes.c_int), ("window", ctypes.c_int), ("shift", ctypes.c_int),
                ("masked", ctypes.c_float)] + [
        (name, ctypes.c_void_p) for name in (
            "ln1_gamma", "ln1_beta", "qkv_w", "qkv_b", "position", "proj_w", "proj_b", "ln2_gamma",
            "ln2_beta", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class IenError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


class Input(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("data", ctypes.c_void_p),
        ("height", ctypes.c_size_t),
        ("width", ctypes.c_size_t),
        ("channels", ctypes.c_size_t),
        ("stride", ctypes.c_size_t),
        ("layout", ctypes.c_int),
        ("taps", ctypes.c_int),
        ("size", ctypes.c_size_t),
        ("step", ctypes.c_size_t),
        ("pad", ctypes.c_int),
        ("offsets", (ctypes.c_size_t * 2) * 4),
        ("count", ctypes.c_size_t),
    ]


class Output(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride", ctypes.c_size_t),
        ("layout", ctypes.c_int),
        ("type", ctypes.c_int),
    ]


class Tensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("rank", ctypes.c_size_t),
        ("dims", ctypes.c_size_t * 4),
        ("values", ctypes.c_void_p),
    ]


PROGRESS = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_float, ctypes.c_void_p)

_lib = None


def load():
    """The library, loaded once; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, sz, st, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int
        L.ien_last_error.restype = ctypes.c_char_p
        L.ien_open.argtypes = [i, ctypes.POINTER(vp)]
        L.ien_close.argtypes = [vp]
        L.ien_close.restype = None
        L.ien_device_name.argtypes = [vp]
        L.ien_device_name.restype = ctypes.c_char_p
        L.ien_stream.argtypes = [vp]
        L.ien_stream.restype = vp
        L.ien_set_stream.argtypes = [vp, vp]
        L.ien_alloc.argtypes = [vp, sz, ctypes.POINTER(vp)]
        L.ien_free.argtypes = [vp, vp]
        L.ien_upload.argtypes = [vp, vp, vp, sz]
        L.ien_download.argtypes = [vp, vp, vp, sz]
        L.ien_sync.argtypes = [vp]
        L.ien_floats_to_halves.argtypes = [vp, vp, vp, sz]
        L.ien_halves_to_floats.argtypes = [vp, vp, vp, sz]
        L.ien_matrix_new.argtypes = [vp, vp, i, sz, sz, vp, ctypes.POINTER(vp)]
        L.ien_matrix_free.argtypes = [vp]
        L.ien_matrix_free.restype = None
        L.ien_multiply.argtypes = [vp, ctypes.POINTER(Input), sz, sz, vp, vp, sz, i, i]
        L.ien_multiply_ex.argtypes = [vp, ctypes.POINTER(Input), sz, sz, vp, ctypes.POINTER(Output), i, vp, i]
        L.ien_conv3.argtypes = [vp, ctypes.POINTER(Input), vp, vp, sz, i, i, vp]
        L.ien_conv3_pair.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp, vp]
        L.ien_conv3_chain.argtypes = [vp, vp, vp, sz, sz, sz, ctypes.POINTER(vp), ctypes.POINTER(vp),
                                      ctypes.POINTER(vp)]
        L.ien_conv3_chain_status.argtypes = [vp]
        L.ien_measure_mfma.argtypes = [vp, i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        L.ien_layer_norm.argtypes = [vp, vp, sz, sz, sz, vp, vp]
        L.ien_gelu.argtypes = [vp, vp, sz]
        L.ien_sigmoid.argtypes = [vp, vp, sz]
        L.ien_pixel_shuffle_add.argtypes = [vp, vp, sz, vp, sz, sz, vp]
        L.ien_depthwise.argtypes = [vp, vp, sz, sz, sz, i, vp, sz, vp, vp]
        L.ien_model_load.argtypes = [vp, i, ctypes.c_char_p, ctypes.POINTER(vp)]
        L.ien_model_from_tensors.argtypes = [vp, i, ctypes.POINTER(Tensor), sz, ctypes.POINTER(vp)]
        L.ien_model_free.argtypes = [vp]
        L.ien_model_free.restype = None
        L.ien_model_run.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp]
        L.ien_model_run_tiled.argtypes = [vp, vp, sz, sz, sz, sz, vp, vp, vp]
        L.ien_model_run_u8.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp]
        L.ien_bytes_to_floats.argtypes = [vp, vp, vp, sz]
        L.ien_floats_to_bytes.argtypes = [vp, vp, vp, sz]
        L.ien_mask_bytes.argtypes = [vp, vp, vp, sz]
        L.ien_normalize_bytes.argtypes = [vp, vp, sz, vp, vp, vp]
        L.ien_composite_bytes.argtypes = [vp, vp, vp, vp, sz, vp]
        L.ien_model_run_device.argtypes = [vp, vp, vp, sz, sz, vp]
        L.ien_model_status.argtypes = [vp]
        L.ien_model_set_graph.argtypes = [vp, i]
        wp = ctypes.POINTER(Windows)
        L.ien_window_count.argtypes = [wp]
        L.ien_window_count.restype = ctypes.c_long
        L.ien_position_bias.argtypes = [vp, i, i, i, vp]
        L.ien_bias_tables.argtypes = [vp, i, i, i, ctypes.c_float, vp]
        L.ien_bias_tables.restype = i
        L.ien_window_gather.argtypes = [vp, wp, vp, sz, i, vp, vp, vp]
        L.ien_window_attention.argtypes = [vp, wp, vp, i, vp, vp]
        L.ien_window_scatter_add.argtypes = [vp, wp, vp, i, vp, sz]
        L.ien_swin_new.argtypes = [vp, ctypes.POINTER(SwinWeights), ctypes.POINTER(vp)]
        L.ien_swin_free.argtypes = [vp]
        L.ien_swin_free.restype = None
        L.ien_swin_run.argtypes = [vp, vp, sz, i, i]
        L.ien_swin_run_static.argtypes = [vp, vp, sz, i, i]
        L.ien_resize.argtypes = [vp, vp, sz, sz, sz, sz, vp, sz, sz, sz, i, i]
        L.ien_pad_image.argtypes = [vp, i, vp, vp, sz, sz, sz, vp, sz]
        L.ien_crop.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp]
        L.ien_gather_2x2.argtypes = [vp, vp, sz, sz, sz, sz, i, vp]
        L.ien_scatter_2x2.argtypes = [vp, vp, sz, sz, sz, sz, vp, sz]
        L.ien_add.argtypes = [vp, vp, vp, sz]
        L.ien_fourier_new.argtypes = [vp, sz, sz, ctypes.POINTER(vp)]
        L.ien_fourier_free.argtypes = [vp]
        L.ien_fourier_free.restype = None
        L.ien_fourier_half.argtypes = [vp]
        L.ien_fourier_half.restype = sz
        L.ien_fourier_forward.argtypes = [vp, vp, sz, sz, vp, vp]
        L.ien_fourier_inverse.argtypes = [vp, vp, sz, vp, vp, sz]
        L.ien_spectral_new.argtypes = [vp, sz, sz, ctypes.POINTER(vp)]
        L.ien_spectral_free.argtypes = [vp]
        L.ien_spectral_free.restype = None
        L.ien_spectral_work.argtypes = [vp]
        L.ien_spectral_work.restype = sz
        L.ien_spectral_run.argtypes = [vp, vp, sz, vp, vp, vp, vp, vp, vp, sz]
        for name in EXPORTS:
            getattr(L, name)
        _lib = L
    return _lib


def check(status):
    if status != OK:
        raise IenError(status, load().ien_last_error().decode(errors="replace"))


def _ptr(t):
    """Device pointer of a torch tensor, or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Context:
    """ien_ctx on one device.  The context's own (non-blocking) HIP stream
    becomes torch's current stream, so torch's copies, fills and events are
    ordered with the library's launches."""

    def __init__(self, device=0):
        import torch

        L = load()
        h = ctypes.c_void_p()
        check(L.ien_open(device, ctypes.byref(h)))
        self.h = h
        self.device = device
        self.stream = torch.cuda.ExternalStream(L.ien_stream(h), device=torch.device("cuda", device))
        torch.cuda.set_stream(self.stream)

    @property
    def name(self):
        return load().ien_device_name(self.h).decode()

    def close(self):
        if self.h:
            import torch

            torch.cuda.synchronize(self.device)
            torch.cuda.set_stream(torch.cuda.default_stream(self.device))
            load().ien_close(self.h)
            self.h = None

    def sync(self):
        check(load().ien_sync(self.h))


class Matrix:
    """gemm.rs Matrix::new: host weights k x n (numpy f32 or f16) + bias."""

    def __init__(self, ctx, w, bias=None):
        import numpy as np

        w = np.ascontiguousarray(w)
        wtype = W_F16 if w.dtype == np.float16 else W_F32
        if wtype == W_F32:
            w = np.ascontiguousarray(w, dtype=np.float32)
        k, n = w.shape
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        h = ctypes.c_void_p()
        check(load().ien_matrix_new(ctx.h, w.ctypes.data_as(ctypes.c_void_p), wtype, k, n,
                                    None if b is None else b.ctypes.data_as(ctypes.c_void_p),
                                    ctypes.byref(h)))
        self.h, self.k, self.n, self.ctx = h, k, n, ctx

    def free(self):
        if self.h:
            load().ien_matrix_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def image_input(x, height, width, channels, stride=None, layout=NHWC, size=3, step=1, pad=PAD_ZERO,
                offsets=None):
    s = Input()
    s.kind = INPUT_IMAGE
    s.data = x.data_ptr()
    s._tensor = x  # the descriptor holds a raw pointer: keep its storage alive
    s.height, s.width, s.channels = height, width, channels
    s.stride = stride if stride is not None else (channels if layout == NHWC else height * width)
    s.layout = layout
    if offsets is None:
        s.taps, s.size, s.step, s.pad = TAPS_CONV, size, step, pad
    else:
        s.taps, s.count = TAPS_OFFSETS, len(offsets)
        for j, (dy, dx) in enumerate(offsets):
            s.offsets[j][0], s.offsets[j][1] = dy, dx
    return s


def rows_input(x, stride):
    s = Input()
    s.kind = INPUT_ROWS
    s.data = x.data_ptr()
    s._tensor = x  # the descriptor holds a raw pointer: keep its storage alive
    s.stride = stride
    return s


def multiply_ex(ctx, inp, row0, rows, matrix, out, out_stride, layout=NHWC, out_f32=False, act=ACT_NONE,
                slope=None, accumulate=False):
    o = Output()
    o.data = out.data_ptr()
    o.stride = out_stride
    o.layout = layout
    o.type = OUT_F32 if out_f32 else OUT_F16
    check(load().ien_multiply_ex(ctx.h, ctypes.byref(inp), row0, rows, matrix.h, ctypes.byref(o), act,
                                 _ptr(slope), int(accumulate)))


def multiply(ctx, inp, row0, rows, matrix, out, stride, act=ACT_NONE, accumulate=False):
    check(load().ien_multiply(ctx.h, ctypes.byref(inp), row0, rows, matrix.h, _ptr(out), stride, act,
                              int(accumulate)))


def conv3(ctx, inp, matrix, out, stride, accumulate=False, finish=ACT_NONE, slope=None):
    check(load().ien_conv3(ctx.h, ctypes.byref(inp), matrix.h, _ptr(out), stride, int(accumulate), finish,
                           _ptr(slope)))


def conv3_pair(ctx, x, y, height, width, m1, slope1, m2, slope2):
    """Two 3x3 64->64 PReLU layers in one launch, x -> y (H x W x 64 f16)."""
    check(load().ien_conv3_pair(ctx.h, _ptr(x), _ptr(y), height, width, m1.h, _ptr(slope1), m2.h,
                                _ptr(slope2)))


def conv3_chain(ctx, a, b, height, width, matrices, slopes):
    """len(matrices) / 2 pairs of 3x3 64->64 PReLU layers in one launch; the
    input in a, b a second map; returns the tensor (a or b) holding the
    output."""
    n = len(matrices)
    w = (ctypes.c_void_p * n)(*[m.h for m in matrices])
    s = (ctypes.c_void_p * n)(*[_ptr(x) for x in slopes])
    out = ctypes.c_void_p()
    check(load().ien_conv3_chain(ctx.h, _ptr(a), _ptr(b), height, width, n // 2, w, s, ctypes.byref(out)))
    return a if out.value == a.data_ptr() else b


def conv3_chain_status(ctx):
    check(load().ien_conv3_chain_status(ctx.h))


def measure_mfma(ctx, iters):
    """(sustained f16 MFMA TFLOP/s, ms) of a register-only MFMA loop on every SIMD."""
    tf, ms = ctypes.c_double(), ctypes.c_double()
    check(load().ien_measure_mfma(ctx.h, iters, ctypes.byref(tf), ctypes.byref(ms)))
    return tf.value, ms.value


def floats_to_halves(ctx, src, dst):
    check(load().ien_floats_to_halves(ctx.h, _ptr(src), _ptr(dst), src.numel()))


def halves_to_floats(ctx, src, dst):
    check(load().ien_halves_to_floats(ctx.h, _ptr(src), _ptr(dst), src.numel()))


def layer_norm(ctx, x, rows, c, stride, gamma, beta):
    check(load().ien_layer_norm(ctx.h, _ptr(x), rows, c, stride, _ptr(gamma), _ptr(beta)))


def gelu(ctx, x):
    check(load().ien_gelu(ctx.h, _ptr(x), x.numel()))


def sigmoid(ctx, x):
    check(load().ien_sigmoid(ctx.h, _ptr(x), x.numel()))


def pixel_shuffle_add(ctx, last, last_stride, image, width, height, out):
    check(load().ien_pixel_shuffle_add(ctx.h, _ptr(last), last_stride, _ptr(image), width, height, _ptr(out)))


def depthwise(ctx, x, height, width, channels, layout, w, size, bias, y):
    check(load().ien_depthwise(ctx.h, _ptr(x), height, width, channels, layout, _ptr(w), size, _ptr(bias),
                               _ptr(y)))


def windows(window, shift, height, width):
    return Windows(window, shift, height, width)


def window_count(w):
    n = load().ien_window_count(ctypes.byref(w))
    if n < 0:
        check(ERR_INPUT)
    return n


def _np_ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def position_bias(table, heads, window, layout):
    """[heads, N, N] from a SCUNet [heads, 2W-1, 2W-1] or Swin [(2W-1)^2, heads] table (host)."""
    import numpy as np

    table = np.ascontiguousarray(table, dtype=np.float32)
    out = np.zeros((heads, window * window, window * window), np.float32)
    check(load().ien_position_bias(_np_ptr(table), heads, window, layout, _np_ptr(out)))
    return out


def bias_tables(position, window, shift, masked):
    """[classes, heads, N, N] (host): swin.rs bias_tables."""
    import numpy as np

    position = np.ascontiguousarray(position, dtype=np.float32)
    heads, n = position.shape[0], window * window
    out = np.zeros((4, heads, n, n), np.float32)
    k = load().ien_bias_tables(_np_ptr(position), heads, window, shift, masked, _np_ptr(out))
    if k < 0:
        check(ERR_INPUT)
    return out[:k]


def window_gather(ctx, w, map_, stride, c, gamma, beta, tokens):
    check(load().ien_window_gather(ctx.h, ctypes.byref(w), _ptr(map_), stride, c, _ptr(gamma), _ptr(beta),
                                   _ptr(tokens)))


def window_attention(ctx, w, qkv, c, tables, out):
    check(load().ien_window_attention(ctx.h, ctypes.byref(w), _ptr(qkv), c, _ptr(tables), _ptr(out)))


def window_scatter_add(ctx, w, rows, c, map_, stride):
    check(load().ien_window_scatter_add(ctx.h, ctypes.byref(w), _ptr(rows), c, _ptr(map_), stride))


def resize(ctx, src, sh, sw, src_stride, c, dst, dh, dw, dst_stride, out_f32=False, add=False):
    check(load().ien_resize(ctx.h, _ptr(src), sh, sw, src_stride, c, _ptr(dst), dh, dw, dst_stride,
                            OUT_F32 if out_f32 else OUT_F16, int(add)))


def pad_image(ctx, mode, image, mask, width, height, multiple, out, stride):
    check(load().ien_pad_image(ctx.h, mode, _ptr(image), _ptr(mask), width, height, multiple, _ptr(out),
                               stride))


def crop(ctx, map_, map_width, stride, width, height, channels, out):
    check(load().ien_crop(ctx.h, _ptr(map_), map_width, stride, width, height, channels, _ptr(out)))


def gather_2x2(ctx, map_, height, width, c, stride, order, rows):
    check(load().ien_gather_2x2(ctx.h, _ptr(map_), height, width, c, stride, order, _ptr(rows)))


def scatter_2x2(ctx, rows, row_stride, height, width, c, map_, stride):
    check(load().ien_scatter_2x2(ctx.h, _ptr(rows), row_stride, height, width, c, _ptr(map_), stride))


def add(ctx, x, y):
    check(load().ien_add(ctx.h, _ptr(x), _ptr(y), x.numel()))


class Fourier:
    """ien_fourier: the 2-D real transforms of height x width maps."""

    def __init__(self, ctx, height, width):
        h = ctypes.c_void_p()
        check(load().ien_fourier_new(ctx.h, height, width, ctypes.byref(h)))
        self.h, self.height, self.width = h, height, width
        self.half = load().ien_fourier_half(h)

    def forward(self, x, stride, channels, work, spectrum):
        check(load().ien_fourier_forward(self.h, _ptr(x), stride, channels, _ptr(work), _ptr(spectrum)))

    def inverse(self, spectrum, channels, work, out, stride):
        check(load().ien_fourier_inverse(self.h, _ptr(spectrum), channels, _ptr(work), _ptr(out), stride))

    def free(self):
        if self.h:
            load().ien_fourier_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Spectral:
    """ien_spectral: LaMa's FFC spectral branch (spectral_in product, rfftn,
    fourier product, irfftn added, spectral_out product accumulated with
    ReLU) for height x width maps of sides up to 64."""

    def __init__(self, ctx, height, width):
        h = ctypes.c_void_p()
        check(load().ien_spectral_new(ctx.h, height, width, ctypes.byref(h)))
        self.h, self.height, self.width = h, height, width
        self.work_floats = load().ien_spectral_work(h)

    def run(self, x, stride, spectral_in, fourier, spectral_out, spectral, work, out, out_stride):
        check(load().ien_spectral_run(self.h, _ptr(x), stride, spectral_in.h, fourier.h,
                                      spectral_out.h, _ptr(spectral), _ptr(work), _ptr(out),
                                      out_stride))

    def free(self):
        if self.h:
            load().ien_spectral_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Swin:
    """ien_swin: one Swin transformer block (attend then MLP, in place).
    `weights`: dict of host arrays ln1_gamma, ln1_beta, qkv_w (c x 3c),
    qkv_b, position ([heads, N, N]), proj_w, proj_b, ln2_gamma, ln2_beta,
    fc1_w (c x 4c), fc1_b, fc2_w (4c x c), fc2_b."""

    def __init__(self, ctx, c, window, shift, masked, weights):
        import numpy as np

        keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        sw = SwinWeights(c, window, shift, masked)
        for name, _ in SwinWeights._fields_[4:]:
            setattr(sw, name, keep[name].ctypes.data)
        h = ctypes.c_void_p()
        check(load().ien_swin_new(ctx.h, ctypes.byref(sw), ctypes.byref(h)))
        self.h = h

    def run(self, map_, stride, height, width):
        check(load().ien_swin_run(self.h, _ptr(map_), stride, height, width))

    def run_static(self, map_, stride, height, width):
        """ien_swin_run_static: the same block with the library's static
        scratch (allocates nothing)."""
        check(load().ien_swin_run_static(self.h, _ptr(map_), stride, height, width))

    def free(self):
        if self.h:
            load().ien_swin_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def bytes_to_floats(ctx, src, dst):
    """to_float on device: uint8 tensor to float32 tensor of the same size."""
    check(load().ien_bytes_to_floats(ctx.h, _ptr(src), _ptr(dst), src.numel()))


def floats_to_bytes(ctx, src, dst):
    """to_byte on device: float32 tensor to uint8 tensor of the same size."""
    check(load().ien_floats_to_bytes(ctx.h, _ptr(src), _ptr(dst), src.numel()))


def mask_bytes(ctx, mask, dst):
    check(load().ien_mask_bytes(ctx.h, _ptr(mask), _ptr(dst), mask.numel()))


def normalize_bytes(ctx, rgb, mean, std, dst):
    """rgb: uint8 tensor of pixels x 3 values; mean, std: three floats."""
    m = (ctypes.c_float * 3)(*mean)
    d = (ctypes.c_float * 3)(*std)
    check(load().ien_normalize_bytes(ctx.h, _ptr(rgb), rgb.numel() // 3, m, d, _ptr(dst)))


def composite_bytes(ctx, rgb, mask, pred, out):
    check(load().ien_composite_bytes(ctx.h, _ptr(rgb), _ptr(mask), _ptr(pred), mask.numel(), _ptr(out)))


class Model:
    """ien_model: the reference's Model with the HIP engine."""

    def __init__(self, ctx, kind, tensors=None, path=None):
        import numpy as np

        self.kind = kind
        L = load()
        h = ctypes.c_void_p()
        if path is not None:
            check(L.ien_model_load(ctx.h, kind, str(path).encode(), ctypes.byref(h)))
        else:
            arr = (Tensor * len(tensors))()
            keep = []
            for j, (name, value) in enumerate(tensors.items()):
                v = np.ascontiguousarray(value, dtype=np.float32)
                keep.append(v)
                arr[j].name = name.encode()
                arr[j].rank = v.ndim
                for d, s in enumerate(v.shape):
                    arr[j].dims[d] = s
                arr[j].values = v.ctypes.data
            check(L.ien_model_from_tensors(ctx.h, kind, arr, len(tensors), ctypes.byref(h)))
        self.h, self.ctx = h, ctx

    def free(self):
        if self.h:
            load().ien_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def set_graph(self, enabled):
        check(load().ien_model_set_graph(self.h, int(enabled)))

    def run(self, image, progress=None, mask=None):
        """Host f32 H x W x 3 in, host f32 out (Model::run_float): 4H x 4W x 3
        for Real-ESRGAN, H x W x 3 for SCUNet and LaMa (which takes the
        H x W mask, 1 = fill), H x W logits for BiRefNet (whose input is
        already normalised)."""
        import numpy as np

        image = np.ascontiguousarray(image, dtype=np.float32)
        h, w, _ = image.shape
        s = 4 if self.kind == MODEL_REALESRGAN else 1
        shape = (h, w) if self.kind == MODEL_BIREFNET else (s * h, s * w, 3)
        out = np.empty(shape, np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
        cb = PROGRESS(progress) if progress else None
        check(load().ien_model_run(self.h, image.ctypes.data_as(ctypes.c_void_p),
                                   None if m is None else m.ctypes.data_as(ctypes.c_void_p), w, h,
                                   out.ctypes.data_as(ctypes.c_void_p),
                                   ctypes.cast(cb, ctypes.c_void_p) if cb else None, None))
        return out

    def run_tiled(self, image, tile, margin, progress=None):
        """Model::run_float_tiled (Real-ESRGAN, SCUNet): host f32 H x W x 3
        in, the run's output shape out."""
        import numpy as np

        image = np.ascontiguousarray(image, dtype=np.float32)
        h, w, _ = image.shape
        s = 4 if self.kind == MODEL_REALESRGAN else 1
        out = np.empty((s * h, s * w, 3), np.float32)
        cb = PROGRESS(progress) if progress else None
        check(load().ien_model_run_tiled(self.h, image.ctypes.data_as(ctypes.c_void_p), w, h, tile, margin,
                                         out.ctypes.data_as(ctypes.c_void_p),
                                         ctypes.cast(cb, ctypes.c_void_p) if cb else None, None))
        return out

    def run_u8(self, rgb, mask=None, progress=None):
        """Model::run on 8-bit RGB H x W x 3 (uint8): bytes out (4H x 4W x 3
        for Real-ESRGAN, H x W x 3 for SCUNet and LaMa, which takes the
        H x W byte mask), H x W f32 logits for BiRefNet."""
        import numpy as np

        rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
        h, w, _ = rgb.shape
        if self.kind == MODEL_BIREFNET:
            out = np.empty((h, w), np.float32)
        else:
            s = 4 if self.kind == MODEL_REALESRGAN else 1
            out = np.empty((s * h, s * w, 3), np.uint8)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        cb = PROGRESS(progress) if progress else None
        check(load().ien_model_run_u8(self.h, rgb.ctypes.data_as(ctypes.c_void_p),
                                      None if m is None else m.ctypes.data_as(ctypes.c_void_p), w, h,
                                      out.ctypes.data_as(ctypes.c_void_p),
                                      ctypes.cast(cb, ctypes.c_void_p) if cb else None, None))
        return out

    def run_device(self, d_image, width, height, d_out, d_mask=None):
        check(load().ien_model_run_device(self.h, _ptr(d_image), None if d_mask is None else _ptr(d_mask),
                                          width, height, _ptr(d_out)))

    def status(self):
        """Waits for the model's stream; raises IenError (ERR_GPU) when a chain
        launched by run_device since the last report gave up."""
        check(load().ien_model_status(self.h))
