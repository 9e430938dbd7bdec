/*
 * scunet.c -- the SCUNet U-Net of image-engine-native's CPU path, restated
 * (TEST INFRASTRUCTURE ONLY: see oracle.h), crates/scunet-native/src/
 * network.rs:113-354 over the pinned products, Winograd convolutions and
 * Swin halves of this library.
 *
 * Tensors come in one canonical order (or_scunet_run in oracle.h): the head;
 * per level down its four blocks then the halving matrix; the body's four
 * blocks; per level up the doubling matrix then its four blocks; the tail.
 * A block is 19 tensors: split w, b; conv1 w; conv2 w; ln1 g, b; qkv w, b;
 * position bias [heads][64][64]; proj w, b; ln2 g, b; fc1 w, b; fc2 w, b;
 * join w, b.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define DIM 64
#define WIN 8

typedef struct {
  const float *split_w, *split_b, *conv1, *conv2, *ln1_g, *ln1_b, *qkv_w, *qkv_b, *pos, *proj_w,
      *proj_b, *ln2_g, *ln2_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b, *join_w, *join_b;
} block_t;

static block_t take_block(const float *const **t) {
  block_t b;
  const float **f = (const float **)&b;
  for (int i = 0; i < 19; i++) f[i] = *(*t)++;
  return b;
}

static or_input rows_input(const float *data, size_t stride) {
  or_input in;
  memset(&in, 0, sizeof in);
  in.kind = OR_INPUT_ROWS;
  in.data = data;
  in.stride = stride;
  return in;
}

static or_input conv3_input(const float *data, size_t h, size_t w, size_t c, size_t stride) {
  or_input in;
  memset(&in, 0, sizeof in);
  in.kind = OR_INPUT_IMAGE;
  in.data = data;
  in.height = h;
  in.width = w;
  in.channels = c;
  in.stride = stride;
  in.taps = OR_TAPS_CONV;
  in.size = 3;
  in.step = 1;
  in.pad = OR_PAD_ZERO;
  return in;
}

/* network.rs:158-208 run_level: y = split(x); per block the convolution
 * half (winograd conv3 + ReLU, conv3 accumulated: :135-153), the
 * transformer's attention and MLP on the second half (swin.rs), the join
 * added onto x, and the next block's split. */
static void run_level(int threads, const block_t *blocks, float *x, size_t h, size_t w,
                      size_t c) {
  const size_t half = c / 2, pixels = h * w;
  float *y = (float *)malloc(sizeof(float) * pixels * c);
  float *t = (float *)malloc(sizeof(float) * pixels * half);
  float *tables = (float *)malloc(sizeof(float) * 4 * (half / 32) * 64 * 64);
  or_input in = rows_input(x, c);
  or_multiply_mt(threads, &in, pixels, blocks[0].split_w, c, c, blocks[0].split_b, y, c,
                 OR_ACT_NONE, 0);
  for (int b = 0; b < 4; b++) {
    const block_t *B = &blocks[b];
    or_input ci = conv3_input(y, h, w, half, c);
    or_conv3(threads, &ci, B->conv1, half, NULL, t, half, 0, OR_FINISH_RELU, NULL);
    or_input ct = conv3_input(t, h, w, half, half);
    or_conv3(threads, &ct, B->conv2, half, NULL, y, c, 1, OR_FINISH_NONE, NULL);
    const size_t shift = b % 2 == 1 ? WIN / 2 : 0;
    or_bias_tables(B->pos, half / 32, WIN, shift, -INFINITY, tables);
    or_swin_attend(threads, y + half, c, h, w, half, WIN, shift, B->ln1_g, B->ln1_b, B->qkv_w,
                   B->qkv_b, tables, B->proj_w, B->proj_b);
    or_swin_mlp(threads, y + half, c, pixels, half, B->ln2_g, B->ln2_b, B->fc1_w, B->fc1_b,
                B->fc2_w, B->fc2_b);
    or_input yi = rows_input(y, c);
    or_multiply_mt(threads, &yi, pixels, B->join_w, c, c, B->join_b, x, c, OR_ACT_NONE, 1);
    if (b < 3) {
      or_input xi = rows_input(x, c);
      or_multiply_mt(threads, &xi, pixels, blocks[b + 1].split_w, c, c, blocks[b + 1].split_b, y,
                     c, OR_ACT_NONE, 0);
    }
  }
  free(y);
  free(t);
  free(tables);
}

/* network.rs:403-437 halved: 2x2 input pixels in row-major order,
 * channels within each, times the halving matrix (no bias). */
static float *halved(int threads, const float *x, size_t h, size_t w, size_t c, const float *m) {
  const size_t h2 = h / 2, w2 = w / 2;
  float *rows = (float *)malloc(sizeof(float) * h2 * w2 * 4 * c);
  for (size_t r = 0; r < h2 * w2; r++) {
    const size_t yy = 2 * (r / w2), xx = 2 * (r % w2);
    for (size_t q = 0; q < 4; q++)
      memcpy(rows + (r * 4 + q) * c, x + ((yy + q / 2) * w + xx + q % 2) * c, sizeof(float) * c);
  }
  float *out = (float *)malloc(sizeof(float) * h2 * w2 * 2 * c);
  or_input in = rows_input(rows, 4 * c);
  or_multiply_mt(threads, &in, h2 * w2, m, 4 * c, 2 * c, NULL, out, 2 * c, OR_ACT_NONE, 0);
  free(rows);
  return out;
}

/* network.rs:439-478 doubled: input pixel (y, x) gives output pixels
 * (2y + dy, 2x + dx), channels = columns (2 dy + dx) cout.. of its product. */
static float *doubled(int threads, const float *x, size_t h, size_t w, size_t cin,
                      const float *m) {
  const size_t cout = cin / 2;
  float *buf = (float *)malloc(sizeof(float) * h * w * 4 * cout);
  or_input in = rows_input(x, cin);
  or_multiply_mt(threads, &in, h * w, m, cin, 4 * cout, NULL, buf, 4 * cout, OR_ACT_NONE, 0);
  float *out = (float *)malloc(sizeof(float) * 4 * h * w * cout);
  for (size_t r = 0; r < h * w; r++) {
    const size_t yy = r / w, xx = r % w;
    for (size_t q = 0; q < 4; q++)
      memcpy(out + ((2 * yy + q / 2) * 2 * w + 2 * xx + q % 2) * cout, buf + (r * 4 + q) * cout,
             sizeof(float) * cout);
  }
  free(buf);
  return out;
}

/* network.rs:262-354 run (padding and crop: :356-379, :347-351). */
int or_scunet_run(int threads, const float *const *t, const float *image, size_t width,
                  size_t height, float *out) {
  const size_t ph = (height + 63) / 64 * 64, pw = (width + 63) / 64 * 64;
  float *padded = (float *)malloc(sizeof(float) * ph * pw * 3);
  or_pad_replicate(image, width, height, 64, padded);
  const float *head = *t++;
  block_t down[3][4], body[4], up[3][4];
  const float *halve[3], *dbl[3];
  for (int l = 0; l < 3; l++) {
    for (int b = 0; b < 4; b++) down[l][b] = take_block(&t);
    halve[l] = *t++;
  }
  for (int b = 0; b < 4; b++) body[b] = take_block(&t);
  for (int l = 0; l < 3; l++) {
    dbl[l] = *t++;
    for (int b = 0; b < 4; b++) up[l][b] = take_block(&t);
  }
  const float *tail = *t++;

  size_t h = ph, w = pw, c = DIM;
  float *x = (float *)malloc(sizeof(float) * h * w * DIM);
  or_input hin = conv3_input(padded, ph, pw, 3, 3);
  or_multiply_mt(threads, &hin, ph * pw, head, 27, DIM, NULL, x, DIM, OR_ACT_NONE, 0);
  float *skips[3];
  for (int l = 0; l < 3; l++) {
    run_level(threads, down[l], x, h, w, c);
    skips[l] = halved(threads, x, h, w, c, halve[l]);
    free(x);
    h /= 2;
    w /= 2;
    c *= 2;
    x = (float *)malloc(sizeof(float) * h * w * c);
    memcpy(x, skips[l], sizeof(float) * h * w * c);
  }
  run_level(threads, body, x, h, w, c);
  for (int l = 0; l < 3; l++) {
    const float *skip = skips[2 - l];
    for (size_t i = 0; i < h * w * c; i++) x[i] += skip[i];
    float *nx = doubled(threads, x, h, w, c, dbl[l]);
    free(x);
    x = nx;
    h *= 2;
    w *= 2;
    c /= 2;
    run_level(threads, up[l], x, h, w, c);
  }
  or_multiply_mt(threads, &hin, ph * pw, head, 27, DIM, NULL, x, DIM, OR_ACT_NONE, 1);
  float *full = (float *)malloc(sizeof(float) * ph * pw * 3);
  or_input tin = conv3_input(x, ph, pw, DIM, DIM);
  or_multiply_mt(threads, &tin, ph * pw, tail, 9 * DIM, 3, NULL, full, 3, OR_ACT_NONE, 0);
  for (size_t yy = 0; yy < height; yy++)
    memcpy(out + yy * width * 3, full + yy * pw * 3, sizeof(float) * width * 3);
  for (int l = 0; l < 3; l++) free(skips[l]);
  free(x);
  free(full);
  free(padded);
  return 0;
}
