/*
 * models.c -- oracle restatement of native-engine's attention.rs, of
 * realesrgan-native's network.rs, and a textbook depthwise convolution.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Pins: tests/test_oracle_attention.py (f64 softmax-attention definition and
 * torch scaled_dot_product_attention fixtures, N = 49, 64, 144, masked
 * biases), tests/test_oracle_realesrgan.py (an independent torch
 * composition of SRVGGNetCompact -- conv2d, PReLU, pixel_shuffle, nearest
 * interpolate -- on seeded weights, fixture under tests/golden/),
 * tests/test_oracle_depthwise.py (torch conv2d(groups=C) fixture, f64 brute
 * force).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "pool.h"

#define HEAD_DIM 32

/* attention.rs:66-111 attention_portable: scores = (q * 1/sqrt(32)) . k
 * accumulated over d with the scale applied to q first, + bias, softmax,
 * then the weighted sum of values in key order. */
void or_attention(const float *qkv, size_t tokens, size_t c, size_t head,
                  const float *bias, float *out) {
  const size_t D = HEAD_DIM;
  const float scale = 1.0f / sqrtf((float)D);
  size_t q0 = head * D, k0 = c + head * D, v0 = 2 * c + head * D;
  float *s = (float *)malloc(sizeof(float) * tokens);
  for (size_t i = 0; i < tokens; i++) {
    for (size_t j = 0; j < tokens; j++) s[j] = 0.0f;
    for (size_t d = 0; d < D; d++) {
      float q = qkv[i * 3 * c + q0 + d] * scale;
      for (size_t j = 0; j < tokens; j++) s[j] += q * qkv[j * 3 * c + k0 + d];
    }
    for (size_t j = 0; j < tokens; j++) s[j] += bias[i * tokens + j];
    or_softmax(s, tokens);
    float sum[HEAD_DIM];
    for (size_t d = 0; d < D; d++) sum[d] = 0.0f;
    for (size_t j = 0; j < tokens; j++) {
      const float *v = qkv + j * 3 * c + v0;
      for (size_t d = 0; d < D; d++) sum[d] += s[j] * v[d];
    }
    memcpy(out + i * c + head * D, sum, sizeof(float) * D);
  }
  free(s);
}

/* realesrgan-native network.rs:115-141 -- output pixel (4y+i, 4x+j) channel
 * c = last(y, x, 16c + 4i + j) + image(y, x, c). */
void or_pixel_shuffle_add(const float *last, const float *image, size_t width,
                          size_t height, float *out) {
  const size_t S = 4, row = width * S * 3;
  for (size_t y = 0; y < height; y++)
    for (size_t x = 0; x < width; x++) {
      size_t p = y * width + x;
      for (size_t i = 0; i < S; i++)
        for (size_t j = 0; j < S; j++) {
          size_t o = (y * S + i) * row + (x * S + j) * 3;
          for (size_t ch = 0; ch < 3; ch++)
            out[o + ch] = last[p * 3 * S * S + ch * S * S + i * S + j] + image[p * 3 + ch];
        }
    }
}

/* realesrgan-native network.rs:80-113 -- 34 layers on two 64-channel maps
 * taking turns; layer 0 (3 channels) runs the direct product, the others
 * F(4x4, 3x3) (winograd.rs:647-671), each followed by its PReLU. */
int or_realesrgan_run(int threads, const float *const *w,
                      const float *const *b, const float *const *slope,
                      const float *image, size_t width, size_t height,
                      float *out) {
  const size_t FEATURES = 64, STEPS = 34;
  size_t pixels = width * height;
  float *a = (float *)calloc(pixels * FEATURES, sizeof(float));
  float *bb = (float *)calloc(pixels * FEATURES, sizeof(float));
  if (!a || !bb) {
    free(a);
    free(bb);
    return -1;
  }
  size_t channels = 3;
  for (size_t i = 0; i < STEPS; i++) {
    int last = i == STEPS - 1;
    size_t n = last ? 48 : FEATURES;
    or_input in = {0};
    in.kind = OR_INPUT_IMAGE;
    in.data = i == 0 ? image : a;
    in.height = height;
    in.width = width;
    in.channels = channels;
    in.stride = channels;
    in.taps = OR_TAPS_CONV;
    in.size = 3;
    in.step = 1;
    in.pad = OR_PAD_ZERO;
    or_conv3(threads, &in, w[i], n, b[i], bb, n, 0,
             last ? OR_FINISH_NONE : OR_FINISH_PRELU, last ? NULL : slope[i]);
    float *t = a;
    a = bb;
    bb = t;
    channels = n;
  }
  or_pixel_shuffle_add(a, image, width, height, out);
  free(a);
  free(bb);
  return 0;
}

typedef struct {
  const float *x, *w, *bias;
  float *y;
  size_t h, wd, c, size;
} dw_job;

static void dw_task(void *ctx, size_t start, size_t end) {
  const dw_job *j = (const dw_job *)ctx;
  ptrdiff_t half = (ptrdiff_t)(j->size / 2);
  for (size_t p = start; p < end; p++) {
    ptrdiff_t oy = (ptrdiff_t)(p / j->wd), ox = (ptrdiff_t)(p % j->wd);
    for (size_t ch = 0; ch < j->c; ch++) {
      float acc = j->bias ? j->bias[ch] : 0.0f;
      for (size_t t = 0; t < j->size * j->size; t++) {
        ptrdiff_t yy = oy + (ptrdiff_t)(t / j->size) - half;
        ptrdiff_t xx = ox + (ptrdiff_t)(t % j->size) - half;
        float v = 0.0f;
        if (yy >= 0 && yy < (ptrdiff_t)j->h && xx >= 0 && xx < (ptrdiff_t)j->wd)
          v = j->x[((size_t)yy * j->wd + (size_t)xx) * j->c + ch];
        acc += v * j->w[t * j->c + ch];
      }
      j->y[p * j->c + ch] = acc;
    }
  }
}

void or_depthwise(int threads, const float *x, size_t height, size_t width,
                  size_t channels, const float *w, size_t size,
                  const float *bias, float *y) {
  dw_job j = {x, w, bias, y, height, width, channels, size};
  or_parallel(threads, height * width, 1, 256, dw_task, &j);
}

/* birefnet-native decoder.rs:467-488 axis: source pixels and weights of
 * output coordinate `out` for aligned corners, as ONNX Runtime computes
 * them (i0 == i1: 0.5 and 0.5). */
static void resize_axis(size_t out, size_t len_in, size_t len_out, size_t *i0, size_t *i1,
                        float *d1, float *d2) {
  float pos = len_out == 1 ? 0.0f : (float)out * (float)(len_in - 1) / (float)(len_out - 1);
  if (pos < 0.0f) pos = 0.0f;
  if (pos > (float)(len_in - 1)) pos = (float)(len_in - 1);
  *i0 = (size_t)pos;
  *i1 = *i0 + 1 < len_in ? *i0 + 1 : len_in - 1;
  if (*i0 == *i1) {
    *d1 = 0.5f;
    *d2 = 0.5f;
  } else {
    *d1 = fabsf(pos - (float)*i0);
    *d2 = fabsf(pos - (float)*i1);
  }
}

/* decoder.rs:436-522 resize: the sh x sw x c map (NHWC) bilinearly to
 * dh x dw, into columns 0..c of rows `stride` apart, added when `add`. */
void or_resize(const float *src, size_t sh, size_t sw, size_t c, float *dst, size_t dh,
               size_t dw, size_t stride, int add) {
  for (size_t y = 0; y < dh; y++) {
    size_t y1, y2;
    float dy1, dy2;
    resize_axis(y, sh, dh, &y1, &y2, &dy1, &dy2);
    for (size_t x = 0; x < dw; x++) {
      size_t x1, x2;
      float dx1, dx2;
      resize_axis(x, sw, dw, &x1, &x2, &dx1, &dx2);
      const float *p11 = src + (y1 * sw + x1) * c, *p21 = src + (y1 * sw + x2) * c;
      const float *p12 = src + (y2 * sw + x1) * c, *p22 = src + (y2 * sw + x2) * c;
      float *d = dst + (y * dw + x) * stride;
      for (size_t j = 0; j < c; j++) {
        const float v = dx2 * dy2 * p11[j] + dx1 * dy2 * p21[j] + dx2 * dy1 * p12[j] +
                        dx1 * dy1 * p22[j];
        d[j] = add ? d[j] + v : v;
      }
    }
  }
}

/* scunet-native network.rs:356-379 pad: the RGB image to the next multiples
 * of `multiple`, the last row and column repeated; out ph x pw x 3. */
void or_pad_replicate(const float *image, size_t width, size_t height, size_t multiple,
                      float *out) {
  const size_t ph = (height + multiple - 1) / multiple * multiple;
  const size_t pw = (width + multiple - 1) / multiple * multiple;
  for (size_t y = 0; y < ph; y++) {
    const size_t sy = y < height ? y : height - 1;
    for (size_t x = 0; x < pw; x++) {
      const size_t sx = x < width ? x : width - 1;
      for (size_t ch = 0; ch < 3; ch++) out[(y * pw + x) * 3 + ch] = image[(sy * width + sx) * 3 + ch];
    }
  }
}

/* lama-native network.rs:336-370 masked_rows: image * (1 - mask) and the
 * mask, mirrored past the bottom and right edges (2n - 1 - i), padded to the
 * next multiples of `multiple`; out ph x pw x 4. */
void or_masked_rows(const float *image, const float *mask, size_t width, size_t height,
                    size_t multiple, float *out) {
  const size_t ph = (height + multiple - 1) / multiple * multiple;
  const size_t pw = (width + multiple - 1) / multiple * multiple;
  for (size_t y = 0; y < ph; y++) {
    const size_t sy = y < height ? y : 2 * height - 1 - y;
    for (size_t x = 0; x < pw; x++) {
      const size_t sx = x < width ? x : 2 * width - 1 - x;
      const size_t p = sy * width + sx;
      const float m = mask[p];
      float *o = out + (y * pw + x) * 4;
      for (size_t ch = 0; ch < 3; ch++) o[ch] = image[p * 3 + ch] * (1.0f - m);
      o[3] = m;
    }
  }
}
