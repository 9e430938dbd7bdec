/*
 * winograd.c -- oracle restatement of native-engine's winograd.rs: 3x3
 * stride-1 convolution by F(2x2,3x3) and F(4x4,3x3) (Lavin and Gray 2016),
 * with the reference's transforms in its order of operations.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Pins: tests/test_oracle_winograd.py (both forms against f64 direct
 * convolution and the oracle's direct product, zero and reflect padding,
 * accumulate, odd sizes, the policy thresholds).
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "pool.h"

#define MIN_CHANNELS 16  /* winograd.rs:53 */
#define F4_CHANNELS 576  /* winograd.rs:56 */
#define TASK_FLOATS (1u << 16) /* winograd.rs:58 */

/* ---- F(2x2, 3x3): winograd.rs:179-352 -------------------------------- */
static void f2_weight(const float g[9], float v[16]) {
  float t[4][3];
  for (int x = 0; x < 3; x++) {
    float g0 = g[x], g1 = g[3 + x], g2 = g[6 + x];
    t[0][x] = g0;
    t[1][x] = 0.5f * (g0 + g1 + g2);
    t[2][x] = 0.5f * (g0 - g1 + g2);
    t[3][x] = g2;
  }
  for (int y = 0; y < 4; y++) {
    float t0 = t[y][0], t1 = t[y][1], t2 = t[y][2];
    v[4 * y] = t0;
    v[4 * y + 1] = 0.5f * (t0 + t1 + t2);
    v[4 * y + 2] = 0.5f * (t0 - t1 + t2);
    v[4 * y + 3] = t2;
  }
}

static void f2_input(const float *const d[16], float *u, size_t cin) {
  for (size_t c = 0; c < cin; c++) {
    float q[4][4];
    for (int a = 0; a < 4; a++) {
      float v0 = d[4 * a][c], v1 = d[4 * a + 1][c], v2 = d[4 * a + 2][c],
            v3 = d[4 * a + 3][c];
      q[a][0] = v0 - v2;
      q[a][1] = v1 + v2;
      q[a][2] = v2 - v1;
      q[a][3] = v1 - v3;
    }
    for (int x = 0; x < 4; x++) {
      u[x * cin + c] = q[0][x] - q[2][x];
      u[(4 + x) * cin + c] = q[1][x] + q[2][x];
      u[(8 + x) * cin + c] = q[2][x] - q[1][x];
      u[(12 + x) * cin + c] = q[1][x] - q[3][x];
    }
  }
}

static void f2_output(const float *m, const float *bias, float *y, size_t cout) {
  for (size_t c = 0; c < cout; c++) {
    float s[4][2];
    for (int i = 0; i < 4; i++) {
      float v0 = m[(4 * i) * cout + c], v1 = m[(4 * i + 1) * cout + c],
            v2 = m[(4 * i + 2) * cout + c], v3 = m[(4 * i + 3) * cout + c];
      s[i][0] = v0 + v1 + v2;
      s[i][1] = v1 - v2 - v3;
    }
    for (int x = 0; x < 2; x++) {
      y[x * cout + c] = s[0][x] + s[1][x] + s[2][x] + bias[c];
      y[(2 + x) * cout + c] = s[1][x] - s[2][x] - s[3][x] + bias[c];
    }
  }
}

/* ---- F(4x4, 3x3): winograd.rs:354-604 -------------------------------- */
static void g_column(float a, float b, float c, float out[6]) {
  out[0] = a / 4.0f;
  out[1] = -(a + b + c) / 6.0f;
  out[2] = -(a - b + c) / 6.0f;
  out[3] = a / 24.0f + b / 12.0f + c / 6.0f;
  out[4] = a / 24.0f - b / 12.0f + c / 6.0f;
  out[5] = c;
}

static void f4_weight(const float g[9], float v[36]) {
  float t[6][3];
  for (int x = 0; x < 3; x++) {
    float col[6];
    g_column(g[x], g[3 + x], g[6 + x], col);
    for (int r = 0; r < 6; r++) t[r][x] = col[r];
  }
  for (int y = 0; y < 6; y++) {
    float row[6];
    g_column(t[y][0], t[y][1], t[y][2], row);
    for (int x = 0; x < 6; x++) v[6 * y + x] = row[x];
  }
}

static void b_t(const float v[6], float o[6]) {
  float a = v[4] - 4.0f * v[2];
  float b = v[3] - 4.0f * v[1];
  float c = v[4] - v[2];
  float e = 2.0f * (v[3] - v[1]);
  o[0] = 4.0f * v[0] - 5.0f * v[2] + v[4];
  o[1] = a + b;
  o[2] = a - b;
  o[3] = c + e;
  o[4] = c - e;
  o[5] = 4.0f * v[1] - 5.0f * v[3] + v[5];
}

static void a_t(const float v[6], float bias, float o[4]) {
  float s = v[1] + v[2];
  float d = v[1] - v[2];
  float s2 = v[3] + v[4];
  float d2 = v[3] - v[4];
  o[0] = v[0] + s + s2 + bias;
  o[1] = d + 2.0f * d2 + bias;
  o[2] = s + 4.0f * s2 + bias;
  o[3] = d + 8.0f * d2 + v[5] + bias;
}

static void f4_input(const float *const d[36], float *u, size_t cin) {
  for (size_t c = 0; c < cin; c++) {
    float rows[6][6];
    for (int y = 0; y < 6; y++) {
      float v[6];
      for (int x = 0; x < 6; x++) v[x] = d[6 * y + x][c];
      b_t(v, rows[y]);
    }
    for (int x = 0; x < 6; x++) {
      float v[6], col[6];
      for (int y = 0; y < 6; y++) v[y] = rows[y][x];
      b_t(v, col);
      for (int y = 0; y < 6; y++) u[(6 * y + x) * cin + c] = col[y];
    }
  }
}

static void f4_output(const float *m, const float *bias, float *y, size_t cout) {
  for (size_t c = 0; c < cout; c++) {
    float rows[6][4];
    for (int i = 0; i < 6; i++) {
      float v[6];
      for (int x = 0; x < 6; x++) v[x] = m[(6 * i + x) * cout + c];
      a_t(v, 0.0f, rows[i]);
    }
    for (int x = 0; x < 4; x++) {
      float v[6], col[4];
      for (int i = 0; i < 6; i++) v[i] = rows[i][x];
      a_t(v, bias[c], col);
      for (int i = 0; i < 4; i++) y[(4 * i + x) * cout + c] = col[i];
    }
  }
}

/* ---- conv3: winograd.rs:606-773 -------------------------------------- */
typedef struct {
  int form; /* 2 or 4 */
  const or_input *in;
  size_t cin, cout;
  const float *points; /* points x cin x cout transformed weights */
  const float *bias;   /* cout */
  float *out;
  size_t stride;
  int accumulate, finish;
  const float *slope;
  size_t blocks_x;
  const float *zeros;
} wino_job;

static void finish_pixel(const wino_job *j, float *pixel) {
  if (j->finish == OR_FINISH_PRELU) {
    /* realesrgan-native network.rs:31-41 */
    for (size_t c = 0; c < j->cout; c++)
      pixel[c] = pixel[c] < 0.0f ? pixel[c] * j->slope[c] : pixel[c];
  } else if (j->finish == OR_FINISH_RELU) {
    for (size_t c = 0; c < j->cout; c++) pixel[c] = pixel[c] > 0.0f ? pixel[c] : 0.0f;
  }
}

static int near_edge(ptrdiff_t i, size_t n) { return i >= -1 && i <= (ptrdiff_t)n; }
static int inside(ptrdiff_t i, size_t n) { return i >= 0 && i < (ptrdiff_t)n; }
static size_t reflect_i(ptrdiff_t i, size_t n) {
  ptrdiff_t last = (ptrdiff_t)n - 1, a = i < 0 ? -i : i, b = 2 * last - i;
  return (size_t)(a < b ? a : b);
}

static void wino_task(void *ctx, size_t start, size_t end) {
  const wino_job *j = (const wino_job *)ctx;
  const or_input *in = j->in;
  size_t size = (size_t)j->form, side = size + 2, np = side * side;
  size_t cin = j->cin, cout = j->cout, nb = end - start;
  float *u = (float *)malloc(sizeof(float) * nb * np * cin);
  float *m = (float *)malloc(sizeof(float) * nb * np * cout);
  float *y = (float *)malloc(sizeof(float) * size * size * cout);
  const float *d[36];
  for (size_t b = start; b < end; b++) {
    size_t by = b / j->blocks_x, bx = b % j->blocks_x;
    for (size_t k = 0; k < np; k++) {
      ptrdiff_t py = (ptrdiff_t)(size * by + k / side) - 1;
      ptrdiff_t px = (ptrdiff_t)(size * bx + k % side) - 1;
      size_t yy, xx;
      if (in->pad == OR_PAD_REFLECT && near_edge(py, in->height) &&
          near_edge(px, in->width)) {
        yy = reflect_i(py, in->height);
        xx = reflect_i(px, in->width);
      } else if (inside(py, in->height) && inside(px, in->width)) {
        yy = (size_t)py;
        xx = (size_t)px;
      } else {
        d[k] = j->zeros;
        continue;
      }
      d[k] = in->data + (yy * in->width + xx) * in->stride;
    }
    if (j->form == 4)
      f4_input(d, u + (b - start) * np * cin, cin);
    else
      f2_input(d, u + (b - start) * np * cin, cin);
  }
  /* One product per point: blocks x cin by cin x cout, no bias
   * (winograd.rs:737-751). */
  for (size_t p = 0; p < np; p++) {
    or_input rows = {0};
    rows.kind = OR_INPUT_ROWS;
    rows.data = u + p * cin;
    rows.stride = np * cin;
    or_multiply(&rows, 0, nb, j->points + p * cin * cout, cin, cout, NULL,
                m + p * cout, np * cout, OR_ACT_NONE, 0);
  }
  for (size_t b = start; b < end; b++) {
    size_t by = b / j->blocks_x, bx = b % j->blocks_x;
    const float *mb = m + (b - start) * np * cout;
    if (j->form == 4)
      f4_output(mb, j->bias, y, cout);
    else
      f2_output(mb, j->bias, y, cout);
    for (size_t corner = 0; corner < size * size; corner++) {
      size_t py = size * by + corner / size, px = size * bx + corner % size;
      if (py >= in->height || px >= in->width) continue;
      float *pixel = j->out + (py * in->width + px) * j->stride;
      const float *v = y + corner * cout;
      if (j->accumulate)
        for (size_t c = 0; c < cout; c++) pixel[c] += v[c];
      else
        memcpy(pixel, v, sizeof(float) * cout);
      finish_pixel(j, pixel);
    }
  }
  free(u);
  free(m);
  free(y);
}

typedef struct {
  const or_input *in;
  const float *w, *bias;
  size_t n;
  float *out;
  size_t stride;
  int accumulate, finish;
  const float *slope;
} direct_job;

static void direct_task(void *ctx, size_t start, size_t end) {
  const direct_job *j = (const direct_job *)ctx;
  or_multiply(j->in, start, end - start, j->w, 9 * j->in->channels, j->n,
              j->bias, j->out + start * j->stride, j->stride, OR_ACT_NONE,
              j->accumulate);
  wino_job f = {0};
  f.cout = j->n;
  f.finish = j->finish;
  f.slope = j->slope;
  for (size_t p = start; p < end; p++) finish_pixel(&f, j->out + p * j->stride);
}

void or_conv3_form(int threads, int form, const or_input *in, const float *w,
                   size_t n, const float *bias, float *out, size_t stride,
                   int accumulate, int finish, const float *slope) {
  size_t cin = in->channels, cout = n;
  if (form == 0) {
    direct_job dj = {in, w, bias, n, out, stride, accumulate, finish, slope};
    or_parallel(threads, in->height * in->width, 6, 96, direct_task, &dj);
    return;
  }
  size_t size = (size_t)form, side = size + 2, np = side * side;
  /* transform_weights (winograd.rs:107-146): G g G^T per channel pair. */
  float *points = (float *)malloc(sizeof(float) * np * cin * cout);
  for (size_t c = 0; c < cin; c++)
    for (size_t o = 0; o < cout; o++) {
      float g[9], v[36];
      for (int t = 0; t < 9; t++) g[t] = w[((size_t)t * cin + c) * cout + o];
      if (form == 4)
        f4_weight(g, v);
      else
        f2_weight(g, v);
      for (size_t p = 0; p < np; p++) points[(p * cin + c) * cout + o] = v[p];
    }
  float *zero_bias = NULL;
  if (!bias) {
    zero_bias = (float *)calloc(cout, sizeof(float));
    bias = zero_bias;
  }
  float *zeros = (float *)calloc(cin, sizeof(float));
  size_t blocks_y = (in->height + size - 1) / size;
  size_t blocks_x = (in->width + size - 1) / size;
  size_t per_block = np * (cin + cout);
  size_t max = TASK_FLOATS / per_block;
  if (max < 6) max = 6;
  wino_job j = {form, in, cin, cout, points, bias, out, stride, accumulate,
                finish, slope, blocks_x, zeros};
  or_parallel(threads, blocks_y * blocks_x, 6, max, wino_task, &j);
  free(points);
  free(zeros);
  free(zero_bias);
}

void or_conv3(int threads, const or_input *in, const float *w, size_t n,
              const float *bias, float *out, size_t stride, int accumulate,
              int finish, const float *slope) {
  int form;
  if (in->channels < MIN_CHANNELS)
    form = 0;
  else if (in->channels + n <= F4_CHANNELS)
    form = 4;
  else
    form = 2;
  or_conv3_form(threads, form, in, w, n, bias, out, stride, accumulate, finish,
                slope);
}
