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
