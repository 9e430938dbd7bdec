/*
 * ien_hip.h -- C ABI of the MI355X (gfx950) backend for image-engine-native.
 *
 * The library (libien_hip.so) sits beside the reference's Vulkan backend
 * (crates/native-vulkan) behind the same model interface: each model crate's
 * `Engine` enum (crates/realesrgan-native/src/lib.rs:48-79) would gain a
 * `Hip` variant whose `load`/`run` call the ien_model_* entry points below,
 * and the native-engine op interface (crates/native-engine/src/lib.rs:51-57:
 * gemm::{Matrix, multiply, Input, Taps, Pad, Act}, winograd::conv3,
 * attention::attention, math::*, half::*) maps onto the ien_* op entry points.
 *
 * Conventions
 *  - Every entry point returns an ien_status; on failure ien_last_error()
 *    (thread-local) holds the message, as the reference's Error's Display
 *    (crates/native-engine/src/lib.rs:61-85).  IEN_ERR_GPU means "this GPU
 *    cannot run it; fall back to the CPU" (realesrgan-native lib.rs:134).
 *  - A context owns one HIP stream on one device.  It is Send but not Sync,
 *    like native-vulkan's Gpu (native-vulkan/src/lib.rs:140-143): calls on
 *    one context must not overlap.  Ops are asynchronous on the context's
 *    stream; ien_sync waits.
 *  - Device activations are IEEE half floats (f16), NHWC with a pixel
 *    stride in halves (the reference's layout, gemm.rs:3-7), or NCHW with a
 *    channel-plane stride; products accumulate in f32 on f16 MFMA.
 *  - Pointers named `d_*` or documented as device pointers are device
 *    memory from ien_alloc (or any hipMalloc'd memory of the same device).
 */
#ifndef IEN_HIP_H
#define IEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* crates/native-engine/src/lib.rs:61-71 Error {Io, Weights, Input,
 * Cancelled, Gpu} */
typedef enum {
  IEN_OK = 0,
  IEN_ERR_IO = 1,
  IEN_ERR_WEIGHTS = 2,
  IEN_ERR_INPUT = 3,
  IEN_ERR_CANCELLED = 4,
  IEN_ERR_GPU = 5
} ien_status;

typedef struct ien_ctx ien_ctx;
typedef struct ien_matrix ien_matrix;
typedef struct ien_model ien_model;

/* Message of the last failure on this thread (lib.rs:73-83 Display). */
const char *ien_last_error(void);

/* ---- device context: native-vulkan/src/lib.rs:168 Gpu::open, name ----- */
ien_status ien_open(int device, ien_ctx **out);
void ien_close(ien_ctx *ctx);
/* The GPU's name (native-vulkan lib.rs Gpu::name). */
const char *ien_device_name(const ien_ctx *ctx);
/* The context's hipStream_t, for callers that order their own work on it. */
void *ien_stream(ien_ctx *ctx);
/* Run this context's work on the caller's hipStream_t instead (NULL: the
 * context's own stream).  The caller keeps the stream alive. */
ien_status ien_set_stream(ien_ctx *ctx, void *stream);

/* ---- memory: native-vulkan lib.rs buffer/upload/Buffer::bytes ---------- */
ien_status ien_alloc(ien_ctx *ctx, size_t bytes, void **d_out);
ien_status ien_free(ien_ctx *ctx, void *d_ptr);
ien_status ien_upload(ien_ctx *ctx, void *d_dst, const void *src, size_t bytes);
ien_status ien_download(ien_ctx *ctx, void *dst, const void *d_src, size_t bytes);
ien_status ien_sync(ien_ctx *ctx);

/* ---- half floats: crates/native-engine/src/half.rs:50-79 --------------- */
/* floats_to_halves / halves_to_f32 on the device, round to nearest even. */
ien_status ien_floats_to_halves(ien_ctx *ctx, const float *d_src, uint16_t *d_dst, size_t n);
ien_status ien_halves_to_floats(ien_ctx *ctx, const uint16_t *d_src, float *d_dst, size_t n);

/* ---- products: crates/native-engine/src/gemm.rs ------------------------ */
typedef enum { IEN_W_F32 = 0, IEN_W_F16 = 1 } ien_wtype;

/* gemm.rs:109-147 Matrix::new: row-major k x n host weights (f32, or f16
 * bits), k = taps * channels with channels fastest, plus an optional
 * length-n host bias.  Packed once onto the device in MFMA fragment order. */
ien_status ien_matrix_new(ien_ctx *ctx, const void *w, ien_wtype wtype, size_t k, size_t n,
                          const float *bias, ien_matrix **out);
void ien_matrix_free(ien_matrix *m);

/* gemm.rs:264-270 Pad */
typedef enum { IEN_PAD_ZERO = 0, IEN_PAD_REFLECT = 1 } ien_pad;
/* gemm.rs:273-286 Taps */
typedef enum { IEN_TAPS_CONV = 0, IEN_TAPS_OFFSETS = 1 } ien_taps;
/* gemm.rs:289-304 Input */
typedef enum { IEN_INPUT_ROWS = 0, IEN_INPUT_IMAGE = 1 } ien_input_kind;
typedef enum { IEN_LAYOUT_NHWC = 0, IEN_LAYOUT_NCHW = 1 } ien_layout;
/* gemm.rs:486-491 Act, plus the per-pixel `finish` closures the callers
 * pass to winograd::conv3 (PReLU: realesrgan network.rs:31-41) and the
 * logistic output of LaMa/BiRefNet (math.rs:145-152). */
typedef enum {
  IEN_ACT_NONE = 0,
  IEN_ACT_RELU = 1,
  IEN_ACT_GELU = 2,
  IEN_ACT_PRELU = 3,
  IEN_ACT_SIGMOID = 4
} ien_act;

/* The left operand of a product (gemm.rs:289-304).  `data` is device f16.
 * ROWS: row r is data[r * stride ..][..k].
 * IMAGE: a height x width image of `channels` channels; NHWC pixels are
 * `stride` halves apart, NCHW channel planes are `stride` halves apart.
 * Taps CONV: centred size x size every `step` pixels with `pad`;
 * OFFSETS: output pixel (y, x) reads (y + dy, x + dx) for `count` offsets,
 * zeros past the edge. */
typedef struct {
  ien_input_kind kind;
  const void *data;
  size_t height, width, channels, stride;
  ien_layout layout;
  ien_taps taps;
  size_t size, step;
  ien_pad pad;
  size_t offsets[4][2];
  size_t count;
} ien_input;

/* Where a product's results go: device memory, f16 or f32, NHWC rows
 * `stride` elements apart (row = output pixel) or NCHW planes `stride`
 * apart. */
typedef enum { IEN_OUT_F16 = 0, IEN_OUT_F32 = 1 } ien_out_type;
typedef struct {
  void *data;
  size_t stride;
  ien_layout layout;
  ien_out_type type;
} ien_output;

/* gemm.rs:514-667 multiply: out[r] = act((accumulate ? out[r] : 0) +
 * input[r] . w + bias) for rows row0 .. row0 + rows of the input's output
 * grid (row-major pixels), into f16 NHWC rows `stride` halves apart
 * starting at d_out (row row0 at d_out). */
ien_status ien_multiply(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                        const ien_matrix *w, void *d_out, size_t stride, ien_act act,
                        int accumulate);

/* The general form of ien_multiply: any output layout/type, PReLU slopes
 * (device f32, length n) for IEN_ACT_PRELU. */
ien_status ien_multiply_ex(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                           const ien_matrix *w, const ien_output *out, ien_act act,
                           const float *d_slope, int accumulate);

/* winograd.rs:612-672 conv3: the 3x3 stride-1 convolution of an IMAGE
 * input with w (9 cin x n), bias, stored to or (accumulate) added to the
 * f16 NHWC pixels of d_out `stride` halves apart, then `finish` (NONE,
 * RELU or PRELU with d_slope) on each pixel.  Computed as an implicit GEMM
 * on MFMA, not by Winograd's transforms (which lose accuracy in f16). */
ien_status ien_conv3(ien_ctx *ctx, const ien_input *input, const ien_matrix *w, void *d_out,
                     size_t stride, int accumulate, ien_act finish, const float *d_slope);

/* realesrgan-native network.rs:96-109, two consecutive body steps in one
 * launch: y = prelu(conv3(prelu(conv3(x, w1), s1), w2), s2) on an
 * H x W x 64 f16 NHWC map (pixels 64 halves apart, zero padding), both
 * layers 3x3 64->64 with their bias and PReLU slopes (device f32, 64
 * each).  The first layer's results stay on chip as f16, so y is bit for
 * bit what two ien_multiply_ex launches of the layers give.  x and y are
 * 16-byte aligned and do not overlap. */
ien_status ien_conv3_pair(ien_ctx *ctx, const uint16_t *d_x, uint16_t *d_y, size_t height,
                          size_t width, const ien_matrix *w1, const float *d_slope1,
                          const ien_matrix *w2, const float *d_slope2);

/* realesrgan-native network.rs:96-109, 2 pairs consecutive body steps in
 * one launch (pairs <= 16; layer i: w[i], slopes d_slopes[i], each 3x3
 * 64->64 with bias and PReLU), bit for bit what `pairs` ien_conv3_pair
 * launches give.  The input is in d_a; d_b and d_a also carry the 2-pixel
 * borders that the 16 x 24 tiles exchange, and *d_out is set to the map
 * that holds the output (d_a for an even count).  Every tile's workgroup
 * must be resident at once (at most one per CU: 256 tiles on MI355X);
 * larger maps are refused.  The tiles wait for their neighbours with a
 * bounded wait; ien_conv3_chain_status (after the stream's work) reports
 * whether any chain since the last report gave up waiting, and clears
 * that report. */
ien_status ien_conv3_chain(ien_ctx *ctx, uint16_t *d_a, uint16_t *d_b, size_t height,
                           size_t width, size_t pairs, const ien_matrix *const *w,
                           const float *const *d_slopes, uint16_t **d_out);
ien_status ien_conv3_chain_status(ien_ctx *ctx);

/* ---- elementwise: crates/native-engine/src/math.rs --------------------- */
/* math.rs:154-170 layer_norm over rows of c values (f16 in place, f32
 * statistics, epsilon 1e-5); gamma/beta device f32. */
ien_status ien_layer_norm(ien_ctx *ctx, uint16_t *d_x, size_t rows, size_t c, size_t stride,
                          const float *d_gamma, const float *d_beta);
/* math.rs:136-152 gelu / sigmoid in place on n f16 values. */
ien_status ien_gelu(ien_ctx *ctx, uint16_t *d_x, size_t n);
ien_status ien_sigmoid(ien_ctx *ctx, uint16_t *d_x, size_t n);

/* realesrgan-native network.rs:115-141 shuffled: out (f32, (4h) x (4w) x 3
 * NHWC) = pixel shuffle x4 of `last` (f16 NHWC, 48 channels used of
 * `last_stride`) plus the f32 RGB image repeated 4 x 4. */
ien_status ien_pixel_shuffle_add(ien_ctx *ctx, const uint16_t *d_last, size_t last_stride,
                                 const float *d_image, size_t width, size_t height,
                                 float *d_out);

/* Depthwise size x size convolution, zero padding, stride 1 (no reference
 * implementation; the reference op interface expresses it as `channels`
 * one-channel products, gemm.rs:288-304).  f16 in and out, NHWC or NCHW,
 * weights (size*size) x channels and bias as device f32. */
ien_status ien_depthwise(ien_ctx *ctx, const uint16_t *d_x, size_t height, size_t width,
                         size_t channels, ien_layout layout, const float *d_w, size_t size,
                         const float *d_bias, uint16_t *d_y);

/* ---- 8-bit images: the models' Model::run byte I/O -------------------- */
/* realesrgan-native lib.rs:292-295 to_float: n bytes to f32 v / 255. */
ien_status ien_bytes_to_floats(ien_ctx *ctx, const uint8_t *d_src, float *d_dst, size_t n);
/* realesrgan-native lib.rs:297-300 to_byte: n floats to bytes,
 * round(clamp(v, 0, 1) * 255) with halves away from zero (NaN to 0). */
ien_status ien_floats_to_bytes(ien_ctx *ctx, const float *d_src, uint8_t *d_dst, size_t n);
/* lama-native lib.rs:142: a byte mask as f32 holes, 1 where the byte is
 * not 0, else 0. */
ien_status ien_mask_bytes(ien_ctx *ctx, const uint8_t *d_mask, float *d_dst, size_t n);
/* birefnet-native lib.rs:111-116: interleaved 8-bit RGB (pixels x 3) to
 * f32 (v / 255 - mean[c]) / deviation[c] (host mean and deviation). */
ien_status ien_normalize_bytes(ien_ctx *ctx, const uint8_t *d_rgb, size_t pixels,
                               const float mean[3], const float deviation[3], float *d_dst);
/* lama-native lib.rs:147-155: out = the RGB bytes where the mask byte is 0,
 * to_byte(prediction) where it is not (pixels x 3 values, one mask byte a
 * pixel). */
ien_status ien_composite_bytes(ien_ctx *ctx, const uint8_t *d_rgb, const uint8_t *d_mask,
                               const float *d_pred, size_t pixels, uint8_t *d_out);

/* ---- resampling and padding ------------------------------------------- */

/* birefnet-native decoder.rs:436-522 resize: bilinear with aligned corners
 * as ONNX Runtime computes it (source position out (in - 1) / (out - 1);
 * when both taps are the same pixel, weights 0.5 and 0.5): the sh x sw map
 * (f16 NHWC, `c` channels, pixel stride src_stride) into columns 0..c of
 * the dh x dw map at d_dst (pixel stride dst_stride, f16 or f32 by
 * out_type), added to what is there when `add`. */
ien_status ien_resize(ien_ctx *ctx, const uint16_t *d_src, size_t sh, size_t sw, size_t src_stride,
                      size_t c, void *d_dst, size_t dh, size_t dw, size_t dst_stride,
                      ien_out_type out_type, int add);

/* A model's input padded to whole multiples of `multiple` (device f32 RGB
 * image, height x width x 3, in; f16 NHWC out with pixel stride `stride`):
 * IEN_PAD_REPLICATE repeats the last row and column (scunet-native
 * network.rs:356-379, 3 channels); IEN_PAD_SYMMETRIC_MASKED mirrors past the
 * bottom and right edges (2n - 1 - i) and writes image * (1 - mask), then the
 * mask (lama-native network.rs:336-370, 4 channels; d_mask height x width). */
typedef enum { IEN_PAD_REPLICATE = 0, IEN_PAD_SYMMETRIC_MASKED = 1 } ien_pad_mode;
ien_status ien_pad_image(ien_ctx *ctx, ien_pad_mode mode, const float *d_image,
                         const float *d_mask, size_t width, size_t height, size_t multiple,
                         uint16_t *d_out, size_t stride);

/* The crop back (scunet-native network.rs:347-351): the top-left width x
 * height pixels of an f16 NHWC map `map_width` pixels wide (pixel stride
 * `stride`), `channels` values each, to f32 height x width x channels. */
ien_status ien_crop(ien_ctx *ctx, const uint16_t *d_map, size_t map_width, size_t stride,
                    size_t width, size_t height, size_t channels, float *d_out);

/* 2 x 2 space-to-depth: row (y, x) of `d_rows` (row stride 4c) holds the
 * 2 x 2 input pixels of output pixel (y, x) of the (height / 2) x
 * (width / 2) grid, c channels each, in IEN_ORDER_ROW_MAJOR ((0,0), (0,1),
 * (1,0), (1,1) by (dy, dx): scunet-native network.rs:403-437 halved) or
 * IEN_ORDER_COLUMN_MAJOR ((0,0), (1,0), (0,1), (1,1): birefnet-native
 * swin.rs:372-392 merge).  The map is f16 NHWC, pixel stride `stride`;
 * height and width even, c a multiple of 8. */
typedef enum { IEN_ORDER_ROW_MAJOR = 0, IEN_ORDER_COLUMN_MAJOR = 1 } ien_order;
ien_status ien_gather_2x2(ien_ctx *ctx, const uint16_t *d_map, size_t height, size_t width,
                          size_t c, size_t stride, ien_order order, uint16_t *d_rows);

/* Its inverse for a transposed 2 x 2 stride-2 convolution (scunet-native
 * network.rs:439-478 doubled): input pixel (y, x) of the height x width grid
 * gives output pixels (2y + dy, 2x + dx) of the map, channels = columns
 * (2 dy + dx) c .. of its row in d_rows (row stride `row_stride`); the map
 * is f16 NHWC, (2 height) x (2 width), pixel stride `stride`. */
ien_status ien_scatter_2x2(ien_ctx *ctx, const uint16_t *d_rows, size_t row_stride,
                           size_t height, size_t width, size_t c, uint16_t *d_map,
                           size_t stride);

/* x += y over n f16 values (scunet-native network.rs:380-391 add). */
ien_status ien_add(ien_ctx *ctx, uint16_t *d_x, const uint16_t *d_y, size_t n);

/* ---- Swin window attention: scunet-native/src/swin.rs,
 *      birefnet-native/src/swin.rs, native-engine attention.rs ---------- */

/* The windows of a Swin block over a height x width map of tokens: window x
 * window tokens each (N = window^2 <= 256), over the map padded to whole
 * windows and rolled by `shift` (0 for W-MSA, window / 2 for SW-MSA; SCUNet
 * swin.rs:153-158, BiRefNet swin.rs:240-247).  Window w covers rows
 * w / ceil(width / window) and columns w % ceil(width / window). */
typedef struct {
  int window;
  int shift;
  int height, width;
} ien_windows;

/* ceil(height / window) * ceil(width / window), or -1 if `w` is invalid. */
long ien_window_count(const ien_windows *w);

/* Relative-position bias [heads][N][N] of a window from its learned table
 * (host memory): IEN_POS_SCUNET [heads][2W-1][2W-1] as
 * tools/scunet/export_weights.py:61-67 gathers it, IEN_POS_SWIN
 * [(2W-1)^2][heads] indexed (dy + W - 1)(2W - 1) + (dx + W - 1). */
typedef enum { IEN_POS_SCUNET = 0, IEN_POS_SWIN = 1 } ien_position_layout;
ien_status ien_position_bias(const float *table, int heads, int window,
                             ien_position_layout layout, float *out);

/* swin.rs bias_tables (scunet :26-50, birefnet :31-51), host memory: out
 * receives [classes][heads][N][N]: the bias itself when shift is 0 (1
 * class), else 4 classes (1: window last in its row, 2: last in its column)
 * with `masked` (-inf for SCUNet, -100 for BiRefNet) between tokens of
 * different regions.  Returns the class count, or -1. */
int ien_bias_tables(const float *position, int heads, int window, int shift, float masked,
                    float *out);

/* The gather of swin.rs attend (scunet :147-161, birefnet :238-254): token
 * rows [windows * N][c] (f16) from the map (f16, token t at d_map + t *
 * stride), each LayerNorm'd with gamma, beta (device f32, eps 1e-5,
 * math.rs:95-116); rows past the map's edge are zero (the padding follows
 * the normalisation).  c a multiple of 8, at most 1024; gamma and beta
 * 16-byte aligned. */
ien_status ien_window_gather(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_map,
                             size_t stride, int c, const float *d_gamma, const float *d_beta,
                             uint16_t *d_tokens);

/* attention.rs:25-111 attention for every window and head at once: qkv
 * rows [windows * N][3c] (f16; queries, keys, values), tables the device
 * copy (f32) of ien_bias_tables' output for the block, window w using
 * class (shift ? [last column] + 2 [last row] : 0) as swin.rs:171-176
 * picks it; out rows [windows * N][c] (f16).  c a multiple of 32 (heads of
 * 32 channels), N <= 256. */
ien_status ien_window_attention(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_qkv, int c,
                                const float *d_tables, uint16_t *d_out);

/* The residual of swin.rs attend (scunet :218-230, birefnet :291-303): each
 * window row is added onto its source token of the map (f16; rows past the
 * edge are dropped).  c a multiple of 8. */
ien_status ien_window_scatter_add(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_rows,
                                  int c, uint16_t *d_map, size_t stride);

/* A Swin transformer block (scunet swin.rs:85-276 Transformer, birefnet
 * swin.rs:87-347 Block): weights as host f32, row-major k x n matrices in
 * the order the weights files hold them. */
typedef struct {
  int c;          /* channels: heads of 32 */
  int window;     /* 8 (SCUNet), 7 or 12 (BiRefNet) */
  int shift;      /* 0, or window / 2 for a shifted block */
  float masked;   /* -inf (SCUNet) or -100 (BiRefNet) */
  const float *ln1_gamma, *ln1_beta;  /* c */
  const float *qkv_w, *qkv_b;         /* c x 3c, 3c */
  const float *position;              /* [heads][N][N] relative-position bias */
  const float *proj_w, *proj_b;       /* c x c, c */
  const float *ln2_gamma, *ln2_beta;  /* c */
  const float *fc1_w, *fc1_b;         /* c x 4c, 4c (GELU) */
  const float *fc2_w, *fc2_b;         /* 4c x c, c */
} ien_swin_weights;
typedef struct ien_swin ien_swin;

/* Transformer::load: upload the products, the norms and the class tables
 * (ien_bias_tables) once. */
ien_status ien_swin_new(ien_ctx *ctx, const ien_swin_weights *weights, ien_swin **out);
void ien_swin_free(ien_swin *block);
/* Transformer::attend then Transformer::mlp, in place on the height x width
 * token map (f16, token t at d_map + t * stride): windows gathered, rolled
 * and normalised, attention, projection added back; then LayerNorm, fc1 +
 * GELU, fc2 added back.  Scratch is the block's own, grown on demand. */
ien_status ien_swin_run(ien_swin *block, uint16_t *d_map, size_t stride, int height, int width);

/* No counterpart in the reference: ien_swin_run for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  The same kernels and results as ien_swin_run, but the
 * unfused path's scratch (window rows of 6c halves, at least height x width
 * of them) lives in a static device array of IEN_SWIN_STATIC_SCRATCH_BYTES
 * per GPU, held until the process ends; this call allocates and frees
 * nothing.  A map whose scratch would not fit is refused with
 * IEN_ERR_INPUT.  Every call on one GPU shares that GPU's array (its
 * contents are overwritten before they are read), so calls that overlap on
 * one GPU, from any context or stream, race. */
#define IEN_SWIN_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
ien_status ien_swin_run_static(ien_swin *block, uint16_t *d_map, size_t stride, int height,
                               int width);

/* ---- Fourier units: crates/lama-native/src/fourier.rs ----------------- */
/* fourier.rs:262-288 Fourier::new: the transforms of height x width maps
 * (sides 1 .. 1024); a spectrum has half = width / 2 + 1 columns. */
typedef struct ien_fourier ien_fourier;
ien_status ien_fourier_new(ien_ctx *ctx, size_t height, size_t width, ien_fourier **out);
void ien_fourier_free(ien_fourier *f);
size_t ien_fourier_half(const ien_fourier *f);
/* fourier.rs:291-344 forward: the spectrum of the map d_x (f16 NHWC, pixel
 * stride `stride`, `channels` values), rfftn over both axes with "ortho"
 * scale, into d_spectrum (f16, height x half pixels of 2 channels values:
 * the real parts, then the imaginary parts).  d_work: height x half x 2
 * channels f32 of scratch. */
ien_status ien_fourier_forward(const ien_fourier *f, const uint16_t *d_x, size_t stride,
                               size_t channels, float *d_work, uint16_t *d_spectrum);
/* fourier.rs:347-403 inverse: the map whose spectrum is d_spectrum (irfftn,
 * "ortho": the complex transform down the columns, then each row's real
 * transform, which drops the imaginary parts of column 0 and, for an even
 * width, of column width / 2), ADDED to d_out (f16 NHWC, pixel stride
 * `stride`).  d_work as for the forward transform. */
ien_status ien_fourier_inverse(const ien_fourier *f, const uint16_t *d_spectrum, size_t channels,
                               float *d_work, uint16_t *d_out, size_t stride);

/* crates/lama-native/src/network.rs:205-245 (Ffc::run's spectral path):
 * spectral = ReLU(x spectral_in + b); spectrum = fourier.forward(spectral);
 * filtered = ReLU(spectrum fourier + b) over spectrum pixels; spectral +=
 * fourier.inverse(filtered); out = ReLU(out + spectral spectral_out), in
 * three launches for height x width maps of sides 1 .. 64.  A plan holds the
 * transform tables for one size. */
typedef struct ien_spectral ien_spectral;
ien_status ien_spectral_new(ien_ctx *ctx, size_t height, size_t width, ien_spectral **out);
void ien_spectral_free(ien_spectral *s);
/* Floats of d_work that ien_spectral_run needs. */
size_t ien_spectral_work(const ien_spectral *s);
/* d_x: the 384 global channels (f16 NHWC, pixel stride `stride`, a multiple
 * of 8, 16-byte aligned); spectral_in 384 x 192 and fourier 384 x 384 with
 * bias, spectral_out 192 x 384; d_spectral: height x 192 x width f16 of
 * scratch (the spectral map, channel-major per row); d_work:
 * ien_spectral_work floats; d_out: the 384 global output channels (pixel
 * stride `out_stride`, a multiple of 8, 16-byte aligned), holding the cross
 * convolution's output, which the call accumulates onto. */
ien_status ien_spectral_run(const ien_spectral *s, const uint16_t *d_x, size_t stride,
                            const ien_matrix *spectral_in, const ien_matrix *fourier,
                            const ien_matrix *spectral_out, uint16_t *d_spectral, float *d_work,
                            uint16_t *d_out, size_t out_stride);

/* ---- models: crates/<model>-native/src/lib.rs Model ------------------- */
typedef enum {
  IEN_MODEL_REALESRGAN = 0,
  IEN_MODEL_SCUNET = 1,
  IEN_MODEL_LAMA = 2,
  IEN_MODEL_BIREFNET = 3
} ien_model_kind;

/* Model::load (realesrgan-native lib.rs:120-137, scunet-native
 * lib.rs:79-111, lama-native lib.rs:75-108, birefnet-native lib.rs:63-96,
 * with the GPU engine): read the weights file (weight_file.rs format, magic
 * b"REALESRG", b"SCUNET\0\0", b"LAMA\0\0\0\0" or b"BIREFNET"), check every
 * tensor, upload once.  BiRefNet's window (7 as exported, 12 in the
 * configured network) follows from its position-bias tensors; an ASPP
 * branch with all-zero offset convolutions runs as a plain convolution,
 * any other as the deformable convolution (decoder.rs:176-313). */
ien_status ien_model_load(ien_ctx *ctx, ien_model_kind kind, const char *weights_path,
                          ien_model **out);
/* The same from weights already in memory: `tensors` name/shape/value
 * triples as a weights file holds them (for synthetic random-init weights). */
typedef struct {
  const char *name;
  size_t rank;
  size_t dims[4];
  const float *values; /* host f32 */
} ien_tensor;
ien_status ien_model_from_tensors(ien_ctx *ctx, ien_model_kind kind, const ien_tensor *tensors,
                                  size_t count, ien_model **out);
void ien_model_free(ien_model *model);

/* Progress callback: share done in 0..1, after each layer (Real-ESRGAN, 34),
 * block (SCUNet, 28) or step (LaMa, 26: lama-native lib.rs:128-157; BiRefNet,
 * 14: the 2 x 4 backbone stages, the five decoder blocks and the head, which
 * the reference does not report); nonzero return cancels the run with
 * IEN_ERR_CANCELLED (realesrgan lib.rs:168-188, scunet lib.rs:205-215). */
typedef int (*ien_progress)(float done, void *user);

/* Model::run_float (realesrgan-native lib.rs:194-214, scunet-native
 * lib.rs:151-171, lama-native lib.rs:159-178) and BiRefNet's run_normalized
 * (birefnet-native lib.rs:144-171): host f32 NHWC image of width x height x
 * 3 (in [0, 1]; for BiRefNet already normalised with ImageNet's mean and
 * deviation, square, sides a multiple of 64), host f32 output (Real-ESRGAN
 * 4h x 4w x 3, SCUNet and LaMa h x w x 3, BiRefNet h x w logits).  `mask`
 * (height x width, 1 = fill) for LaMa, whose sides are at least 9; NULL for
 * the others. */
ien_status ien_model_run(ien_model *model, const float *image, const float *mask, size_t width,
                         size_t height, float *out, ien_progress progress, void *user);

/* Model::run_float_tiled (realesrgan-native lib.rs:216-229, scunet-native
 * lib.rs:172-185), Real-ESRGAN and SCUNet: the image cut into a grid of
 * equal tiles at most `tile` pixels on a side, each run with up to `margin`
 * pixels of its surroundings on every side, only the tile's own output
 * kept.  Real-ESRGAN with a margin of at least 34 (the 34 layers' reach)
 * gives the whole image's result bit for bit.  Progress counts the steps
 * of every tile; a cancel stops issuing work and returns
 * IEN_ERR_CANCELLED. */
ien_status ien_model_run_tiled(ien_model *model, const float *image, size_t width,
                               size_t height, size_t tile, size_t margin, float *out,
                               ien_progress progress, void *user);

/* Model::run / run_with_progress on 8-bit RGB (host, width x height x 3):
 * Real-ESRGAN (realesrgan-native lib.rs:161-189: tiles of 768 with margin
 * 34, out 4h x 4w x 3 bytes) and SCUNet (scunet-native lib.rs:120-148:
 * tiles of 896 with margin 64, out h x w x 3 bytes) take to_float in and
 * to_byte out; LaMa (lama-native lib.rs:114-156) takes `mask` (width x
 * height bytes, not 0 = fill) and returns the image with only the holes
 * replaced (h x w x 3 bytes); BiRefNet (birefnet-native lib.rs:107-141,
 * square sides a multiple of 64) normalises with ImageNet's statistics and
 * returns f32 logits (h x w floats) in `out`. */
ien_status ien_model_run_u8(ien_model *model, const uint8_t *rgb, const uint8_t *mask,
                            size_t width, size_t height, void *out, ien_progress progress,
                            void *user);

/* The same on device buffers (f32 NHWC in and out), no host copies and no
 * synchronisation: the hot path a serving loop or a benchmark times.
 * Real-ESRGAN runs as one chain launch whose tiles wait for their
 * neighbours; that needs every tile's workgroup resident at once (one per
 * CU), so another stream or process holding CUs for longer than the wait's
 * limit (1 s) makes the chain give up and leave its output incomplete.  The
 * call cannot see that when it returns: ien_model_status does. */
ien_status ien_model_run_device(ien_model *model, const float *d_image, const float *d_mask,
                                size_t width, size_t height, float *d_out);

/* No counterpart in the reference (its runs are synchronous): waits for the
 * model's stream and returns IEN_ERR_GPU ("body chain: ...", the reference's
 * Error::Gpu, lib.rs:130-136: fall back) when a chain launched by
 * ien_model_run_device since the last report gave up, or when the stream
 * failed; each failure is reported once.  The host-buffer runs
 * (ien_model_run, _tiled, _u8) check their own chains and repeat a run
 * whose chain gave up through two-layer launches (the same bits), so they
 * never need this call. */
ien_status ien_model_status(ien_model *model);

/* Launch-free replay: capture ien_model_run_device at this size into a HIP
 * graph once, then replay it (0 = eager launches).  A run that is a single
 * launch (Real-ESRGAN with its whole network in one chain) is launched
 * directly instead: a graph saves it no host work and adds a few
 * microseconds a replay. */
ien_status ien_model_set_graph(ien_model *model, int enabled);

/* No counterpart in the reference: a measurement of this device for
 * reports.  Back-to-back v_mfma_f32_32x32x16_f16 on register operands on
 * every SIMD (one workgroup of 8 waves per CU, 4 accumulator chains a
 * wave, `iters` rounds), timed with HIP events on the context's stream:
 * the sustained f16 dense rate in *tflops, the launch in *ms. */
ien_status ien_measure_mfma(ien_ctx *ctx, int iters, double *tflops, double *ms);

#ifdef __cplusplus
}
#endif
#endif
