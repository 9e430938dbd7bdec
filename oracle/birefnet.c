/*
 * birefnet.c -- BiRefNet-lite of image-engine-native's CPU path, restated
 * (TEST INFRASTRUCTURE ONLY: see oracle.h): the Swin-T backbone of
 * crates/birefnet-native/src/swin.rs and the decoder of decoder.rs, over the
 * pinned products, Winograd convolutions, Swin halves and resize of this
 * library.  The window is a parameter (the reference fixes 7, shift 3;
 * the configured network uses 12, shift 6), and the deformable ASPP
 * branches sample as decoder.rs:239-313 (with all-zero offsets and
 * modulator logits they read exactly the integer taps).
 *
 * Tensors come in the reference's load order (or_birefnet_run in oracle.h).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define INTER 64
#define BRANCH 256

static const size_t STAGE_C[4] = {96, 192, 384, 768};
static const size_t STAGE_DEPTH[4] = {2, 2, 6, 2};
static const size_t ASPP_SIZES[4] = {1, 1, 3, 7};

typedef struct {
  const float *n1g, *n1b, *qkv_w, *qkv_b, *pos, *proj_w, *proj_b, *n2g, *n2b, *fc1_w, *fc1_b,
      *fc2_w, *fc2_b;
} sblock_t;

typedef struct {
  const float *offset_w[4], *offset_b[4], *weight[4], *bias[4];
  const float *pool_w, *pool_b, *conv1_w, *conv1_b;
} aspp_t;

typedef struct {
  const float *conv_in_w, *conv_in_b, *conv_out_w, *conv_out_b;
  const float *gdt_w, *gdt_b, *gdt_attn_w, *gdt_attn_b; /* NULL without a gate */
  aspp_t aspp;
  size_t cin, cout;
} dblock_t;

static or_input rows_in(const float *data, size_t stride) {
  or_input in;
  memset(&in, 0, sizeof in);
  in.kind = OR_INPUT_ROWS;
  in.data = data;
  in.stride = stride;
  return in;
}

static or_input conv_in(const float *data, size_t h, size_t w, size_t c, size_t stride,
                        size_t size) {
  or_input in;
  memset(&in, 0, sizeof in);
  in.kind = OR_INPUT_IMAGE;
  in.data = data;
  in.height = h;
  in.width = w;
  in.channels = c;
  in.stride = stride;
  in.taps = OR_TAPS_CONV;
  in.size = size;
  in.step = 1;
  in.pad = OR_PAD_ZERO;
  return in;
}

/* ---- swin.rs ---------------------------------------------------------- */

/* swin.rs:182-215 embed: 4x4 patches, rows (ky, kx, c), times the matrix,
 * then the LayerNorm. */
static float *embed(int threads, const float *w, const float *b, const float *ng,
                    const float *nb, const float *image, size_t side) {
  const size_t grid = side / 4, tokens = grid * grid;
  float *patches = (float *)malloc(sizeof(float) * tokens * 48);
  for (size_t r = 0; r < tokens; r++) {
    const size_t ty = r / grid, tx = r % grid;
    for (size_t ky = 0; ky < 4; ky++)
      memcpy(patches + r * 48 + ky * 12, image + ((ty * 4 + ky) * side + tx * 4) * 3,
             sizeof(float) * 12);
  }
  float *x = (float *)malloc(sizeof(float) * tokens * 96);
  or_input in = rows_in(patches, 48);
  or_multiply_mt(threads, &in, tokens, w, 48, 96, b, x, 96, OR_ACT_NONE, 0);
  or_layer_norm(x, tokens * 96, ng, nb, 96);
  free(patches);
  return x;
}

/* swin.rs:377-405 merge: 2x2 groups in the order (0,0), (1,0), (0,1), (1,1)
 * by (row, column), LayerNorm over 4c, then 4c -> 2c. */
static float *merge(int threads, const float *x, size_t grid, size_t c, const float *ng,
                    const float *nb, const float *w) {
  const size_t half = grid / 2, tokens = half * half;
  static const size_t dy[4] = {0, 1, 0, 1}, dx[4] = {0, 0, 1, 1};
  float *rows = (float *)malloc(sizeof(float) * tokens * 4 * c);
  for (size_t r = 0; r < tokens; r++) {
    const size_t y = 2 * (r / half), xx = 2 * (r % half);
    for (size_t q = 0; q < 4; q++)
      memcpy(rows + (r * 4 + q) * c, x + ((y + dy[q]) * grid + xx + dx[q]) * c,
             sizeof(float) * c);
  }
  or_layer_norm(rows, tokens * 4 * c, ng, nb, 4 * c);
  float *out = (float *)malloc(sizeof(float) * tokens * 2 * c);
  or_input in = rows_in(rows, 4 * c);
  or_multiply_mt(threads, &in, tokens, w, 4 * c, 2 * c, NULL, out, 2 * c, OR_ACT_NONE, 0);
  free(rows);
  return out;
}

typedef struct {
  const float *embed_w, *embed_b, *embed_g, *embed_nb;
  sblock_t blocks[4][6];
  const float *merge_g[3], *merge_b[3], *merge_w[3];
  const float *norm_g[4], *norm_b[4];
} backbone_t;

/* swin.rs:171-180 run: the four normalised stage outputs. */
static void backbone_run(int threads, const backbone_t *B, const float *image, size_t side,
                         size_t window, float **features) {
  size_t grid = side / 4;
  float *x = embed(threads, B->embed_w, B->embed_b, B->embed_g, B->embed_nb, image, side);
  const size_t n = window * window;
  for (int s = 0; s < 4; s++) {
    const size_t c = STAGE_C[s], heads = c / 32;
    float *tables = (float *)malloc(sizeof(float) * 4 * heads * n * n);
    for (size_t b = 0; b < STAGE_DEPTH[s]; b++) {
      const sblock_t *K = &B->blocks[s][b];
      const size_t shift = b % 2 == 1 ? window / 2 : 0;
      or_bias_tables(K->pos, heads, window, shift, -100.0f, tables);
      or_swin_attend(threads, x, c, grid, grid, c, window, shift, K->n1g, K->n1b, K->qkv_w,
                     K->qkv_b, tables, K->proj_w, K->proj_b);
      or_swin_mlp(threads, x, c, grid * grid, c, K->n2g, K->n2b, K->fc1_w, K->fc1_b, K->fc2_w,
                  K->fc2_b);
    }
    free(tables);
    float *f = (float *)malloc(sizeof(float) * grid * grid * c);
    memcpy(f, x, sizeof(float) * grid * grid * c);
    or_layer_norm(f, grid * grid * c, B->norm_g[s], B->norm_b[s], c);
    features[s] = f;
    if (s < 3) {
      float *nx = merge(threads, x, grid, c, B->merge_g[s], B->merge_b[s], B->merge_w[s]);
      free(x);
      x = nx;
      grid /= 2;
    }
  }
  free(x);
}

/* ---- decoder.rs ------------------------------------------------------- */

/* decoder.rs:254-313 sample: pixel (y, x)'s deformable input, every tap's 64
 * channels bilinearly sampled at the tap moved by its offset, times twice
 * its modulator (already through the sigmoid); points more than a pixel
 * outside read zero, corners outside count as zero. */
static void sample(const float *t, size_t height, size_t width, size_t y, size_t x, size_t size,
                   const float *offsets, float *out) {
  const size_t taps = size * size;
  const float half = (float)(size / 2), h = (float)height, w = (float)width;
  for (size_t tap = 0; tap < taps; tap++) {
    float *dst = out + tap * INTER;
    const float py = ((float)y - half + (float)(tap / size)) + offsets[2 * tap];
    const float px = ((float)x - half + (float)(tap % size)) + offsets[2 * tap + 1];
    const float m = 2.0f * offsets[2 * taps + tap];
    memset(dst, 0, sizeof(float) * INTER);
    if (py <= -1.0f || py >= h || px <= -1.0f || px >= w) continue;
    const float y0f = floorf(py), x0f = floorf(px);
    const float ly = py - y0f, lx = px - x0f, hy = 1.0f - ly, hx = 1.0f - lx;
    const long y0 = (long)y0f, x0 = (long)x0f;
    const long cy[4] = {y0, y0, y0 + 1, y0 + 1}, cx[4] = {x0, x0 + 1, x0, x0 + 1};
    const float cw[4] = {hy * hx, hy * lx, ly * hx, ly * lx};
    for (int k = 0; k < 4; k++) {
      if (cy[k] < 0 || cx[k] < 0 || cy[k] >= (long)height || cx[k] >= (long)width) continue;
      const float *v = t + ((size_t)cy[k] * width + (size_t)cx[k]) * INTER;
      for (size_t d = 0; d < INTER; d++) dst[d] += cw[k] * v[d];
    }
    for (size_t d = 0; d < INTER; d++) dst[d] *= m;
  }
}

/* decoder.rs:138-236 Aspp::run on an h x w x 64 map. */
static float *aspp_run(int threads, const aspp_t *A, const float *t, size_t h, size_t w) {
  const size_t pixels = h * w;
  double mean[INTER];
  for (size_t c = 0; c < INTER; c++) mean[c] = 0.0;
  for (size_t p = 0; p < pixels; p++)
    for (size_t c = 0; c < INTER; c++) mean[c] += (double)t[p * INTER + c];
  float pooled[BRANCH];
  memcpy(pooled, A->pool_b, sizeof pooled);
  for (size_t c = 0; c < INTER; c++) {
    const float m = (float)(mean[c] / (double)pixels);
    for (size_t j = 0; j < BRANCH; j++) pooled[j] += m * A->pool_w[c * BRANCH + j];
  }
  float bias[INTER];
  memcpy(bias, A->conv1_b, sizeof bias);
  for (size_t j = 0; j < BRANCH; j++) {
    const float p = pooled[j] > 0.0f ? pooled[j] : 0.0f;
    for (size_t k = 0; k < INTER; k++) bias[k] += p * A->conv1_w[(4 * BRANCH + j) * INTER + k];
  }
  float *cat = (float *)malloc(sizeof(float) * pixels * 4 * BRANCH);
  for (int i = 0; i < 4; i++) {
    const size_t size = ASPP_SIZES[i], taps = size * size;
    float *offsets = (float *)malloc(sizeof(float) * pixels * 3 * taps);
    or_input in = conv_in(t, h, w, INTER, INTER, size);
    or_multiply_mt(threads, &in, pixels, A->offset_w[i], taps * INTER, 3 * taps, A->offset_b[i],
                   offsets, 3 * taps, OR_ACT_NONE, 0);
    float *samples = (float *)malloc(sizeof(float) * pixels * taps * INTER);
    for (size_t p = 0; p < pixels; p++) {
      float *o = offsets + p * 3 * taps;
      or_sigmoid(o + 2 * taps, taps);
      sample(t, h, w, p / w, p % w, size, o, samples + p * taps * INTER);
    }
    or_input sin = rows_in(samples, taps * INTER);
    or_multiply_mt(threads, &sin, pixels, A->weight[i], taps * INTER, BRANCH, A->bias[i],
                   cat + i * BRANCH, 4 * BRANCH, OR_ACT_RELU, 0);
    free(offsets);
    free(samples);
  }
  float *out = (float *)malloc(sizeof(float) * pixels * INTER);
  or_input cin = rows_in(cat, 4 * BRANCH);
  /* conv1's rows for the four branches (the first 4 x 256 of 5 x 256). */
  or_multiply_mt(threads, &cin, pixels, A->conv1_w, 4 * BRANCH, INTER, NULL, out, INTER,
                 OR_ACT_NONE, 0);
  for (size_t p = 0; p < pixels; p++)
    for (size_t k = 0; k < INTER; k++) {
      const float v = out[p * INTER + k] + bias[k];
      out[p * INTER + k] = v > 0.0f ? v : 0.0f;
    }
  free(cat);
  return out;
}

/* decoder.rs:346-413 Block::run; takes x (h x w x cin) and frees it. */
static float *dblock_run(int threads, const dblock_t *D, float *x, size_t h, size_t w) {
  const size_t pixels = h * w, cout = D->cout;
  float *t = (float *)malloc(sizeof(float) * pixels * INTER);
  or_input in = conv_in(x, h, w, D->cin, D->cin, 3);
  or_conv3(threads, &in, D->conv_in_w, INTER, D->conv_in_b, t, INTER, 0, OR_FINISH_RELU, NULL);
  free(x);
  float *a = aspp_run(threads, &D->aspp, t, h, w);
  free(t);
  float *out = (float *)malloc(sizeof(float) * pixels * cout);
  or_input ain = conv_in(a, h, w, INTER, INTER, 3);
  or_conv3(threads, &ain, D->conv_out_w, cout, D->conv_out_b, out, cout, 0, OR_FINISH_NONE,
           NULL);
  free(a);
  if (D->gdt_w) {
    float *g = (float *)malloc(sizeof(float) * pixels * 16);
    or_input gin = conv_in(out, h, w, cout, cout, 3);
    or_multiply_mt(threads, &gin, pixels, D->gdt_w, 9 * cout, 16, D->gdt_b, g, 16, OR_ACT_RELU,
                   0);
    for (size_t p = 0; p < pixels; p++) {
      float s = D->gdt_attn_b[0];
      for (size_t k = 0; k < 16; k++) s = s + g[p * 16 + k] * D->gdt_attn_w[k];
      or_sigmoid(&s, 1);
      for (size_t k = 0; k < cout; k++) out[p * cout + k] *= s;
    }
    free(g);
  }
  return out;
}

/* decoder.rs:535-591 Patches::run: the image cut into grid x grid patches of
 * size x size pixels (patch (gy, gx) of colour c -> channel
 * (c grid + gy) grid + gx), through both 3x3 convolutions into out. */
static void patches_run(int threads, const float *conv1_w, const float *conv1_b,
                        const float *out_w, const float *out_b, size_t cout, const float *image,
                        size_t side, size_t size, float *out, size_t stride) {
  const size_t grid = side / size, channels = 3 * grid * grid;
  float *stacked = (float *)malloc(sizeof(float) * size * size * channels);
  for (size_t p = 0; p < size * size; p++) {
    const size_t y = p / size, x = p % size;
    float *row = stacked + p * channels;
    size_t k = 0;
    for (size_t c = 0; c < 3; c++)
      for (size_t gy = 0; gy < grid; gy++)
        for (size_t gx = 0; gx < grid; gx++)
          row[k++] = image[((gy * size + y) * side + gx * size + x) * 3 + c];
  }
  float *mid = (float *)malloc(sizeof(float) * size * size * INTER);
  or_input in = conv_in(stacked, size, size, channels, channels, 3);
  or_conv3(threads, &in, conv1_w, INTER, conv1_b, mid, INTER, 0, OR_FINISH_NONE, NULL);
  or_input min = conv_in(mid, size, size, INTER, INTER, 3);
  or_conv3(threads, &min, out_w, cout, out_b, out, stride, 0, OR_FINISH_NONE, NULL);
  free(stacked);
  free(mid);
}

/* decoder.rs:594-757 FullResolution::add: conv_out(conv1(image)) added to
 * out, the two 3x3 convolutions composed into one 5x5 (weights summed in
 * f64) for interior pixels and taken one after the other on the edge ring,
 * where the intermediate map's zero padding is reached. */
static void full_resolution_add(const float *conv1, const float *bias1, const float *conv_out,
                                float bias_out, const float *image, size_t side, float *out) {
  double composed[75];
  for (int i = 0; i < 75; i++) composed[i] = 0.0;
  double cb = (double)bias_out;
  for (int d = 0; d < 9; d++)
    for (int k = 0; k < INTER; k++) {
      const double w2 = (double)conv_out[d * INTER + k];
      cb += w2 * (double)bias1[k];
      for (int e = 0; e < 9; e++) {
        const int ey = d / 3 + e / 3, ex = d % 3 + e % 3;
        for (int c = 0; c < 3; c++)
          composed[(ey * 5 + ex) * 3 + c] += w2 * (double)conv1[(e * 3 + c) * INTER + k];
      }
    }
  float cw[75];
  for (int i = 0; i < 75; i++) cw[i] = (float)composed[i];
  const float cbias = (float)cb;
  const long S = (long)side;
  for (long y = 0; y < S; y++)
    for (long x = 0; x < S; x++) {
      float v;
      if (y == 0 || x == 0 || y == S - 1 || x == S - 1) {
        /* exact: decoder.rs:700-734 */
        float s = bias_out;
        for (int d = 0; d < 9; d++) {
          const long qy = y + d / 3 - 1, qx = x + d % 3 - 1;
          if (qy < 0 || qx < 0 || qy >= S || qx >= S) continue;
          float mid[INTER];
          memcpy(mid, bias1, sizeof mid);
          for (int e = 0; e < 9; e++) {
            const long py = qy + e / 3 - 1, px = qx + e % 3 - 1;
            if (py < 0 || px < 0 || py >= S || px >= S) continue;
            const float *p = image + (py * S + px) * 3;
            for (int c = 0; c < 3; c++)
              for (int k = 0; k < INTER; k++) mid[k] += p[c] * conv1[(e * 3 + c) * INTER + k];
          }
          float dot = 0.0f;
          for (int k = 0; k < INTER; k++) dot += mid[k] * conv_out[d * INTER + k];
          s += dot;
        }
        v = s;
      } else {
        /* composed: decoder.rs:737-757, per pixel the bias then each tap's
         * three products in order, zero outside the image */
        float s = cbias;
        for (int e = 0; e < 25; e++) {
          const long py = y + e / 5 - 2, px = x + e % 5 - 2;
          float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f;
          if (py >= 0 && px >= 0 && py < S && px < S) {
            const float *p = image + (py * S + px) * 3;
            p0 = p[0];
            p1 = p[1];
            p2 = p[2];
          }
          s += cw[e * 3] * p0 + cw[e * 3 + 1] * p1 + cw[e * 3 + 2] * p2;
        }
        v = s;
      }
      out[y * S + x] += v;
    }
}

/* Copy a pixels x c map into columns offset.. of rows `stride` apart. */
static void place(const float *src, size_t pixels, size_t c, float *dst, size_t stride,
                  size_t offset) {
  for (size_t p = 0; p < pixels; p++)
    memcpy(dst + p * stride + offset, src + p * c, sizeof(float) * c);
}

static const size_t LEVEL_CIN[4] = {1728, 960, 480, 240};
static const size_t LEVEL_COUT[4] = {768, 384, 192, 96};

int or_birefnet_run(int threads, const float *const *t, size_t window, const float *image,
                    size_t side, float *logits) {
  if (side == 0 || side % 64 != 0 || window < 2) return -1;
  backbone_t B;
  B.embed_w = *t++;
  B.embed_b = *t++;
  B.embed_g = *t++;
  B.embed_nb = *t++;
  for (int s = 0; s < 4; s++) {
    for (size_t b = 0; b < STAGE_DEPTH[s]; b++) {
      sblock_t *K = &B.blocks[s][b];
      const float **f = (const float **)K;
      for (int i = 0; i < 13; i++) f[i] = *t++;
    }
    if (s < 3) {
      B.merge_g[s] = *t++;
      B.merge_b[s] = *t++;
      B.merge_w[s] = *t++;
    }
    B.norm_g[s] = *t++;
    B.norm_b[s] = *t++;
  }
  dblock_t D[5];
  for (int i = 0; i < 5; i++) {
    dblock_t *K = &D[i];
    K->cin = i == 0 ? 2880 : LEVEL_CIN[i - 1];
    K->cout = i == 0 ? 1536 : LEVEL_COUT[i - 1];
    K->conv_in_w = *t++;
    K->conv_in_b = *t++;
    K->conv_out_w = *t++;
    K->conv_out_b = *t++;
    if (i >= 1 && i <= 3) {
      K->gdt_w = *t++;
      K->gdt_b = *t++;
      K->gdt_attn_w = *t++;
      K->gdt_attn_b = *t++;
    } else {
      K->gdt_w = K->gdt_b = K->gdt_attn_w = K->gdt_attn_b = NULL;
    }
    for (int j = 0; j < 4; j++) {
      K->aspp.offset_w[j] = *t++;
      K->aspp.offset_b[j] = *t++;
      K->aspp.weight[j] = *t++;
      K->aspp.bias[j] = *t++;
    }
    K->aspp.pool_w = *t++;
    K->aspp.pool_b = *t++;
    K->aspp.conv1_w = *t++;
    K->aspp.conv1_b = *t++;
  }
  const float *lat_w[3], *lat_b[3];
  for (int i = 0; i < 3; i++) {
    lat_w[i] = *t++;
    lat_b[i] = *t++;
  }
  const float *pc1_w[4], *pc1_b[4], *pco_w[4], *pco_b[4];
  for (int i = 0; i < 4; i++) {
    pc1_w[i] = *t++;
    pc1_b[i] = *t++;
    pco_w[i] = *t++;
    pco_b[i] = *t++;
  }
  const float *head_w = *t++, *head_b = *t++;
  const float *fr_c1 = *t++, *fr_b1 = *t++, *fr_co = *t++, *fr_bo = *t++;

  /* lib.rs:144-171 run_normalized: the half-size copy, both backbone runs. */
  const size_t hs = side / 2;
  float *half = (float *)malloc(sizeof(float) * hs * hs * 3);
  or_resize(image, side, side, 3, half, hs, hs, 3, 0);
  float *full_f[4], *half_f[4];
  backbone_run(threads, &B, image, side, window, full_f);
  backbone_run(threads, &B, half, hs, window, half_f);
  free(half);

  /* decoder.rs:796-926 Decoder::run */
  float *levels[4];
  size_t lgrid[4], lc[4];
  for (int i = 0; i < 4; i++) {
    const size_t grid = side >> (i + 2), c = STAGE_C[i];
    float *x = (float *)malloc(sizeof(float) * grid * grid * 2 * c);
    place(full_f[i], grid * grid, c, x, 2 * c, 0);
    or_resize(half_f[i], grid / 2, grid / 2, c, x + c, grid, grid, 2 * c, 0);
    free(full_f[i]);
    free(half_f[i]);
    levels[i] = x;
    lgrid[i] = grid;
    lc[i] = 2 * c;
  }
  const size_t g4 = side >> 5;
  float *x4 = (float *)malloc(sizeof(float) * g4 * g4 * 2880);
  size_t offset = 0;
  for (int i = 0; i < 3; i++) {
    or_resize(levels[i], lgrid[i], lgrid[i], lc[i], x4 + offset, g4, g4, 2880, 0);
    offset += lc[i];
  }
  place(levels[3], g4 * g4, lc[3], x4, 2880, offset);
  free(levels[3]);
  levels[3] = NULL;
  float *previous = dblock_run(threads, &D[0], x4, g4, g4);
  size_t previous_grid = g4;
  static const size_t patch_cout[4] = {192, 192, 96, 48};
  for (int i = 0; i < 4; i++) {
    const int level = 3 - i;
    const size_t cin = LEVEL_CIN[i], grid = side >> (level + 2);
    const size_t main_c = i == 0 ? 1536 : LEVEL_COUT[i - 1];
    float *input = (float *)calloc(grid * grid * cin, sizeof(float));
    if (i == 0) {
      place(previous, grid * grid, main_c, input, cin, 0);
    } else {
      float *x = levels[level];
      or_input lin = rows_in(x, lc[level]);
      or_multiply_mt(threads, &lin, grid * grid, lat_w[i - 1], lc[level], lc[level],
                     lat_b[i - 1], input, cin, OR_ACT_NONE, 0);
      free(x);
      levels[level] = NULL;
      or_resize(previous, previous_grid, previous_grid, main_c, input, grid, grid, cin, 1);
    }
    patches_run(threads, pc1_w[i], pc1_b[i], pco_w[i], pco_b[i], patch_cout[i], image, side,
                grid, input + main_c, cin);
    free(previous);
    previous = dblock_run(threads, &D[i + 1], input, grid, grid);
    previous_grid = grid;
  }
  const size_t pixels = previous_grid * previous_grid;
  float *low = (float *)malloc(sizeof(float) * pixels);
  or_input hin = rows_in(previous, 96);
  or_multiply_mt(threads, &hin, pixels, head_w, 96, 1, NULL, low, 1, OR_ACT_NONE, 0);
  for (size_t i = 0; i < side * side; i++) logits[i] = head_b[0];
  or_resize(low, previous_grid, previous_grid, 1, logits, side, side, 1, 1);
  full_resolution_add(fr_c1, fr_b1, fr_co, fr_bo[0], image, side, logits);
  free(low);
  free(previous);
  for (int i = 0; i < 3; i++) free(levels[i]);
  return 0;
}
