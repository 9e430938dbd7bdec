/*
 * oracle.h -- CPU restatement of image-engine-native's f32 CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend and the timed CPU baseline: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  The product (libien_hip.so)
 * never links, loads or calls it.
 *
 * Each function restates the reference's algorithm, including its order of
 * sums, from the Rust sources it cites (paths relative to the reference
 * root).  The multiply-adds are unfused (the reference's SSE/AVX tiers 0-1;
 * tier 2 fuses them, which moves results by rounding only).
 *
 * Pins (tests/test_oracle_*.py): f64 definitions, brute force on small
 * shapes, the reference's own known answers (half.rs tests) and torch
 * functional fixtures under tests/golden/.  Every function below has at least
 * one pin; none is "parity unpinned".
 */
#ifndef IEN_ORACLE_H
#define IEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- half.rs ---------------------------------------------------------- */
uint16_t or_f32_to_half(float v);              /* half.rs:7-40 */
float or_half_to_f32(uint16_t h);              /* half.rs:125-140 */
void or_floats_to_halves(const float *src, uint16_t *dst, size_t n);
void or_halves_to_f32(const uint16_t *src, float *dst, size_t n);

/* ---- 8-bit image I/O and tiling (io.c) -------------------------------- */
float or_to_float(uint8_t v);                  /* realesrgan lib.rs:292-295 */
uint8_t or_to_byte(float v);                   /* realesrgan lib.rs:297-300 */
void or_bytes_to_floats(const uint8_t *src, float *dst, size_t n);
void or_floats_to_bytes(const float *src, uint8_t *dst, size_t n);
void or_normalize_bytes(const uint8_t *rgb, size_t pixels, float *dst); /* birefnet lib.rs:111-116 */
void or_mask_bytes(const uint8_t *mask, float *dst, size_t n);         /* lama lib.rs:142 */
void or_composite_bytes(const uint8_t *rgb, const uint8_t *mask, const float *pred,
                        size_t pixels, uint8_t *out);                   /* lama lib.rs:147-155 */
size_t or_tile_regions(size_t width, size_t height, size_t tile, size_t margin,
                       size_t *out);                                    /* realesrgan lib.rs:251-265 */

/* ---- math.rs ---------------------------------------------------------- */
float or_exp_neg(float z);                     /* math.rs:21-31 */
void or_sigmoid(float *x, size_t n);           /* math.rs:33-39,145-152 */
void or_gelu(float *x, size_t n);              /* math.rs:41-75,136-143 */
void or_layer_norm(float *x, size_t len, const float *gamma,
                   const float *beta, size_t c); /* math.rs:95-116,154-170 */
void or_softmax(float *x, size_t n);           /* math.rs:118-134 */

/* ---- gemm.rs ---------------------------------------------------------- */
enum { OR_INPUT_ROWS = 0, OR_INPUT_IMAGE = 1 };
enum { OR_TAPS_CONV = 0, OR_TAPS_OFFSETS = 1 };
enum { OR_PAD_ZERO = 0, OR_PAD_REFLECT = 1 };
enum { OR_ACT_NONE = 0, OR_ACT_RELU = 1, OR_ACT_GELU = 2 };

/* gemm.rs:272-304: Input::{Rows, Image} with Taps::{Conv, Offsets}. */
typedef struct {
  int kind;             /* OR_INPUT_* */
  const float *data;
  size_t height, width, channels, stride;
  int taps;             /* OR_TAPS_* */
  size_t size, step;    /* Conv */
  int pad;              /* OR_PAD_* */
  size_t offsets[4][2]; /* Offsets: (dy, dx) */
  size_t count;
} or_input;

/* gemm.rs:514-667 multiply: out[r] = act((acc ? out[r] : 0) + bias +
 * sum_k in(r,k) w[k][n]), rows row0..row0+rows, weights row-major k x n
 * (the reference packs them into panels, which changes no sum). */
void or_multiply(const or_input *in, size_t row0, size_t rows, const float *w,
                 size_t k, size_t n, const float *bias, float *out,
                 size_t stride, int act, int accumulate);
/* The same, split over `threads` threads by rows (pool.rs: a task never
 * splits one output's reduction, so results do not depend on threads). */
void or_multiply_mt(int threads, const or_input *in, size_t rows,
                    const float *w, size_t k, size_t n, const float *bias,
                    float *out, size_t stride, int act, int accumulate);

/* ---- winograd.rs ------------------------------------------------------ */
enum { OR_FINISH_NONE = 0, OR_FINISH_PRELU = 1, OR_FINISH_RELU = 2 };
/* winograd.rs:612-773 conv3: 3x3 stride-1 conv, F(4x4,3x3) when
 * cin + cout <= 576, F(2x2,3x3) above, direct product when cin < 16; then
 * `finish` on each output pixel (PReLU slopes or ReLU). */
void or_conv3(int threads, const or_input *in, const float *w, size_t n,
              const float *bias, float *out, size_t stride, int accumulate,
              int finish, const float *slope);
/* Force a form (2 or 4), for tests of both transforms. */
void or_conv3_form(int threads, int form, const or_input *in, const float *w,
                   size_t n, const float *bias, float *out, size_t stride,
                   int accumulate, int finish, const float *slope);

/* ---- attention.rs ----------------------------------------------------- */
/* attention.rs:25-111: one head of one window of `tokens` tokens; qkv rows of
 * 3c (q | k | v), head dim 32, bias tokens x tokens (mask included). */
void or_attention(const float *qkv, size_t tokens, size_t c, size_t head,
                  const float *bias, float *out);

/* ---- Swin window attention (scunet swin.rs, birefnet swin.rs) -------- */
enum { OR_POS_SCUNET = 0, OR_POS_SWIN = 1 };
/* The relative-position bias [heads][N][N] of a W x W window from its table:
 * OR_POS_SCUNET [heads][2W-1][2W-1] (tools/scunet/export_weights.py:61-67),
 * OR_POS_SWIN [(2W-1)^2][heads] indexed (dy+W-1)(2W-1)+(dx+W-1). */
void or_position_bias(const float *table, size_t heads, size_t window, int layout,
                      float *out);
/* swin.rs bias_tables (scunet :26-50, birefnet :31-51): returns the number of
 * classes written to out ([classes][heads][N][N]): 1 unshifted, 4 shifted. */
size_t or_bias_tables(const float *position, size_t heads, size_t window, size_t shift,
                      float masked, float *out);
/* Source token of window token i of window w (-1: padding past the edge). */
long or_window_source(size_t w, size_t i, size_t window, size_t shift, size_t height,
                      size_t width);
/* Class of window w in a block rolled by `shift` (0 when unshifted). */
size_t or_window_class(size_t w, size_t window, size_t shift, size_t height, size_t width);
/* The attention half of a Swin block, in place (scunet swin.rs:131-232,
 * birefnet swin.rs:219-306); weights row-major k x n. */
void or_swin_attend(int threads, float *map, size_t stride, size_t height, size_t width,
                    size_t c, size_t window, size_t shift, const float *gamma,
                    const float *beta, const float *wqkv, const float *bqkv,
                    const float *tables, const float *wproj, const float *bproj);
/* The MLP half (scunet swin.rs:236-275, birefnet swin.rs:308-347), in place. */
void or_swin_mlp(int threads, float *map, size_t stride, size_t rows, size_t c,
                 const float *gamma, const float *beta, const float *w1, const float *b1,
                 const float *w2, const float *b2);

/* ---- scunet-native network.rs ----------------------------------------- */
/* network.rs:262-354 run: the RGB image (height x width x 3, values 0..1)
 * through the U-Net, out height x width x 3.  `t` holds 540 tensors in
 * this order: head [27][64]; per level down (64, 128, 256 channels) four
 * blocks then the halving matrix [4c][2c]; the body's four blocks (512);
 * per level up (256, 128, 64) the doubling matrix [2c][4c] then four blocks;
 * the tail [576][3].  A block of c channels (h = c / 2): split [c][c], [c];
 * conv1 [9h][h]; conv2 [9h][h]; ln1 [h], [h]; qkv [h][3h], [3h]; position
 * bias [h/32][64][64]; proj [h][h], [h]; ln2 [h], [h]; fc1 [h][4h], [4h];
 * fc2 [4h][h], [h]; join [c][c], [c]. */
int or_scunet_run(int threads, const float *const *t, const float *image, size_t width,
                  size_t height, float *out);

/* ---- lama-native fourier.rs and network.rs ---------------------------- */
/* fourier.rs:291-344 forward: the "ortho" rfftn of x (h x w x c, NHWC) into
 * out (h x (w/2+1) pixels of [re x c | im x c]). */
void or_rfft2(const float *x, size_t h, size_t w, size_t c, float *out);
/* fourier.rs:347-403 inverse: the "ortho" irfftn of s ADDED to out. */
void or_irfft2_add(const float *s, size_t h, size_t w, size_t c, float *out);
/* network.rs:271-335 Up::run: a stride-2 transposed 3x3 convolution as four
 * output-phase products (PHASE_TAPS), through a ReLU: x (h x w x cin) to out
 * (2h x 2w x cout); phase_w[p] [(taps) cin][cout] row-major, phase_b[p]. */
void or_lama_up(int threads, const float *const *phase_w, const float *const *phase_b,
                const float *x, size_t h, size_t w, size_t cin, size_t cout, float *out);
/* network.rs:415-489 run: image (height x width x 3 in 0..1) and mask
 * (height x width, 1 = fill) through Big LaMa's generator; out height x
 * width x 3.  `t` holds the 358 tensors in the weights file's order
 * (lama.c). */
int or_lama_run(int threads, const float *const *t, const float *image, const float *mask,
                size_t width, size_t height, float *out);

/* ---- birefnet-native swin.rs and decoder.rs --------------------------- */
/* lib.rs:144-171 run_normalized: logits (side x side) of a normalised RGB
 * image (side x side x 3, side a multiple of 64) through the Swin-T backbone
 * (windows of `window`, shift window / 2, at the full and the half size) and
 * the decoder.  `t` holds the tensors in the reference's load order
 * (Backbone::load then Decoder::load: birefnet.c). */
int or_birefnet_run(int threads, const float *const *t, size_t window, const float *image,
                    size_t side, float *logits);

/* ---- realesrgan-native network.rs ------------------------------------- */
/* network.rs:80-141: 34 conv3 layers (PReLU on all but the last), then the
 * x4 pixel shuffle plus the input repeated.  w[i] is 9cin x cout row-major
 * ((ky,kx,cin) rows), b[i] cout, slope[i] 64 (ignored for the last). */
int or_realesrgan_run(int threads, const float *const *w,
                      const float *const *b, const float *const *slope,
                      const float *image, size_t width, size_t height,
                      float *out);
/* network.rs:115-141 alone: last is pixels x 48, image pixels x 3. */
void or_pixel_shuffle_add(const float *last, const float *image, size_t width,
                          size_t height, float *out);

/* ---- resize and padding helpers ---------------------------------------- */
/* birefnet-native decoder.rs:436-522: bilinear, aligned corners, ONNX
 * Runtime weights (i0 == i1: 0.5, 0.5); NHWC in, columns 0..c of rows
 * `stride` apart out, added when `add`. */
void or_resize(const float *src, size_t sh, size_t sw, size_t c, float *dst, size_t dh,
               size_t dw, size_t stride, int add);
/* scunet-native network.rs:356-379: replicate-pad RGB to multiples of `multiple`. */
void or_pad_replicate(const float *image, size_t width, size_t height, size_t multiple,
                      float *out);
/* lama-native network.rs:336-370: symmetric pad of image * (1 - m) | m. */
void or_masked_rows(const float *image, const float *mask, size_t width, size_t height,
                    size_t multiple, float *out);

/* ---- depthwise (no reference implementation) -------------------------- */
/* y[p][c] = bias[c] + sum_{ky,kx} w[(ky*size+kx)][c] * x[p + tap][c], NHWC,
 * zero padding, stride 1: the 192 single-channel products of the reference
 * op interface (gemm.rs:288-304 with channels 1, stride C), in tap order. */
void or_depthwise(int threads, const float *x, size_t height, size_t width,
                  size_t channels, const float *w, size_t size,
                  const float *bias, float *y);

#ifdef __cplusplus
}
#endif
#endif
