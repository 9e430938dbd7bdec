/*
 * gemm.c -- oracle restatement of native-engine's gemm.rs (indirect
 * convolution product) and pool.rs's row splitting.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Order of sums (gemm/kernel.rs:68-110 kernel_portable, driven by
 * gemm.rs:514-667): each output starts from its loaded value (accumulate) or
 * 0, adds the bias, then every product in reduction order, taps then
 * channels; ReLU at the last store, GELU after the whole product.  The KC
 * blocking stores and reloads partial sums in f32, which changes no value,
 * so it is not restated.  Rows are computed in groups of six and columns in
 * panels of sixteen, as the micro-kernel does, so gcc vectorises across the
 * sixteen columns without reordering any one output's sum.
 *
 * Pins: tests/test_oracle_gemm.py (f64 brute force over dense rows, partial
 * groups and panels, accumulate, zero/reflect padded convolutions, transposed
 * phase offsets, plus torch conv2d fixtures).
 */
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "pool.h"

#define MR 6
#define NR 16

static const float ZEROS[4096];

/* gemm.rs:306-311 */
static size_t reflect_index(ptrdiff_t i, size_t n) {
  ptrdiff_t last = (ptrdiff_t)n - 1;
  ptrdiff_t a = i < 0 ? -i : i;
  ptrdiff_t b = 2 * last - i;
  return (size_t)(a < b ? a : b);
}

/* gemm.rs:343-359 */
static void out_size(const or_input *in, size_t *oh, size_t *ow) {
  if (in->taps == OR_TAPS_CONV) {
    *oh = (in->height - 1) / in->step + 1;
    *ow = (in->width - 1) / in->step + 1;
  } else {
    *oh = in->height;
    *ow = in->width;
  }
}

static size_t tap_count(const or_input *in) {
  if (in->kind == OR_INPUT_ROWS) return 1;
  return in->taps == OR_TAPS_CONV ? in->size * in->size : in->count;
}

/* gemm.rs:406-441 Input::at -- pointer to channel 0 of tap `t` of row `r`,
 * or to zeros. */
static const float *tap_at(const or_input *in, size_t r, size_t t) {
  if (in->kind == OR_INPUT_ROWS) return in->data + r * in->stride;
  size_t oh, ow;
  out_size(in, &oh, &ow);
  size_t oy = r / ow, ox = r % ow;
  (void)oh;
  if (in->taps == OR_TAPS_CONV) {
    ptrdiff_t half = (ptrdiff_t)(in->size / 2);
    ptrdiff_t y = (ptrdiff_t)(oy * in->step + t / in->size) - half;
    ptrdiff_t x = (ptrdiff_t)(ox * in->step + t % in->size) - half;
    int inside = y >= 0 && y < (ptrdiff_t)in->height && x >= 0 &&
                 x < (ptrdiff_t)in->width;
    if (!inside) {
      if (in->pad == OR_PAD_ZERO) return ZEROS;
      y = (ptrdiff_t)reflect_index(y, in->height);
      x = (ptrdiff_t)reflect_index(x, in->width);
    }
    return in->data + ((size_t)y * in->width + (size_t)x) * in->stride;
  }
  size_t y = oy + in->offsets[t][0], x = ox + in->offsets[t][1];
  if (y < in->height && x < in->width)
    return in->data + (y * in->width + x) * in->stride;
  return ZEROS;
}

void or_multiply(const or_input *in, size_t row0, size_t rows, const float *w,
                 size_t k, size_t n, const float *bias, float *out,
                 size_t stride, int act, int accumulate) {
  if (rows == 0) return;
  size_t taps = tap_count(in);
  size_t channels = in->kind == OR_INPUT_ROWS ? k : in->channels;
  const float *ptrs[MR * 64];
  for (size_t g = 0; g < rows; g += MR) {
    size_t mr = rows - g < MR ? rows - g : MR;
    for (size_t t = 0; t < taps; t++)
      for (size_t i = 0; i < mr; i++) ptrs[t * MR + i] = tap_at(in, row0 + g + i, t);
    for (size_t p = 0; p < n; p += NR) {
      size_t cols = n - p < NR ? n - p : NR;
      float acc[MR][NR];
      for (size_t i = 0; i < MR; i++)
        for (size_t j = 0; j < NR; j++) {
          float v = 0.0f;
          if (i < mr && j < cols && accumulate) v = out[(g + i) * stride + p + j];
          acc[i][j] = v + ((j < cols && bias) ? bias[p + j] : 0.0f);
        }
      float wrow[NR];
      for (size_t t = 0; t < taps; t++) {
        for (size_t c = 0; c < channels; c++) {
          const float *src = w + (t * channels + c) * n + p;
          for (size_t j = 0; j < NR; j++) wrow[j] = j < cols ? src[j] : 0.0f;
          for (size_t i = 0; i < MR; i++) {
            float a = i < mr ? ptrs[t * MR + i][c] : 0.0f;
            for (size_t j = 0; j < NR; j++) acc[i][j] += a * wrow[j];
          }
        }
      }
      for (size_t i = 0; i < mr; i++)
        for (size_t j = 0; j < cols; j++) {
          float v = acc[i][j];
          if (act == OR_ACT_RELU) v = v > 0.0f ? v : 0.0f;
          out[(g + i) * stride + p + j] = v;
        }
    }
  }
  if (act == OR_ACT_GELU)
    for (size_t r = 0; r < rows; r++) or_gelu(out + r * stride, n);
}

typedef struct {
  const or_input *in;
  const float *w;
  size_t k, n;
  const float *bias;
  float *out;
  size_t stride;
  int act, accumulate;
} mul_job;

static void mul_task(void *ctx, size_t start, size_t end) {
  mul_job *j = (mul_job *)ctx;
  or_multiply(j->in, start, end - start, j->w, j->k, j->n, j->bias,
              j->out + start * j->stride, j->stride, j->act, j->accumulate);
}

void or_multiply_mt(int threads, const or_input *in, size_t rows,
                    const float *w, size_t k, size_t n, const float *bias,
                    float *out, size_t stride, int act, int accumulate) {
  mul_job j = {in, w, k, n, bias, out, stride, act, accumulate};
  or_parallel(threads, rows, MR, 96, mul_task, &j);
}
