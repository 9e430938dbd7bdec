/*
 * swin.c -- the Swin window-attention block of image-engine-native's CPU
 * path, restated (TEST INFRASTRUCTURE ONLY: see oracle.h).
 *
 * One routine covers SCUNet's and BiRefNet's blocks: windows of W x W
 * tokens over an H x Wd map padded to whole windows (no padding for SCUNet,
 * whose maps are multiples of 8), rolled by `shift` in shifted blocks, with
 * the mask value of the model (-inf for SCUNet, -100 for BiRefNet).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* tools/scunet/export_weights.py:61-67 position_bias (OR_POS_SCUNET: a
 * [heads][2W-1][2W-1] table; the bias between tokens (y1, x1) and (y2, x2)
 * is table[h][y1 - y2 + W - 1][x1 - x2 + W - 1]) and the Swin layout of
 * random-init BiRefNet (OR_POS_SWIN: a [(2W-1)^2][heads] table indexed by
 * (dy + W - 1)(2W - 1) + (dx + W - 1)).  out: [heads][N][N], N = W * W. */
void or_position_bias(const float *table, size_t heads, size_t window, int layout,
                      float *out) {
  const size_t n = window * window, side = 2 * window - 1;
  for (size_t h = 0; h < heads; h++)
    for (size_t i = 0; i < n; i++)
      for (size_t j = 0; j < n; j++) {
        const size_t dy = i / window + window - 1 - j / window;
        const size_t dx = i % window + window - 1 - j % window;
        const size_t cell = dy * side + dx;
        out[(h * n + i) * n + j] =
            layout == OR_POS_SCUNET ? table[h * side * side + cell] : table[cell * heads + h];
      }
}

/* scunet swin.rs:26-50 and birefnet swin.rs:31-51 bias_tables: unshifted,
 * the position bias itself; shifted, four copies (class = last window in
 * its row + 2 * last in its column) each plus the mask: tokens of different
 * regions (region = 2 [row >= W - shift, in a last row] + [col >= W - shift,
 * in a last column]) get `masked` added. */
size_t or_bias_tables(const float *position, size_t heads, size_t window, size_t shift,
                      float masked, float *out) {
  const size_t n = window * window;
  if (shift == 0) {
    memcpy(out, position, sizeof(float) * heads * n * n);
    return 1;
  }
  for (size_t cls = 0; cls < 4; cls++) {
    const int last_col = (cls & 1) != 0, last_row = (cls & 2) != 0;
    for (size_t h = 0; h < heads; h++)
      for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) {
          const size_t ri = 2 * (last_row && i / window >= window - shift) +
                            (last_col && i % window >= window - shift);
          const size_t rj = 2 * (last_row && j / window >= window - shift) +
                            (last_col && j % window >= window - shift);
          const float mask = ri == rj ? 0.0f : masked;
          out[((cls * heads + h) * n + i) * n + j] = position[(h * n + i) * n + j] + mask;
        }
  }
  return 4;
}

/* The source token of window token i of window w, or -1 past the map's
 * edge (scunet swin.rs:153-158, birefnet swin.rs:240-254). */
static long window_source(size_t w, size_t i, size_t window, size_t shift, size_t height,
                          size_t width) {
  const size_t ph = (height + window - 1) / window * window;
  const size_t pw = (width + window - 1) / window * window;
  const size_t wx_count = pw / window;
  const size_t wy = w / wx_count, wx = w % wx_count;
  const size_t y = (wy * window + i / window + shift) % ph;
  const size_t x = (wx * window + i % window + shift) % pw;
  if (y >= height || x >= width) return -1;
  return (long)(y * width + x);
}

long or_window_source(size_t w, size_t i, size_t window, size_t shift, size_t height,
                      size_t width) {
  return window_source(w, i, window, shift, height, width);
}

/* scunet swin.rs:171-176, birefnet swin.rs:273-279: a shifted block's window
 * class (1: last in its row of windows, 2: last in its column). */
size_t or_window_class(size_t w, size_t window, size_t shift, size_t height, size_t width) {
  if (shift == 0) return 0;
  const size_t wxs = (width + window - 1) / window, wys = (height + window - 1) / window;
  return (size_t)(w % wxs == wxs - 1) + 2 * (size_t)(w / wxs == wys - 1);
}

/* The attention half of a block (scunet swin.rs:131-232, birefnet
 * swin.rs:219-306), in place on the map whose token t starts at
 * map[t * stride]: gather each window (rolled, zero rows past the edge),
 * LayerNorm, qkv product, per-head attention with the window's class table,
 * projection, and the projected rows added back onto their tokens. */
void or_swin_attend(int threads, float *map, size_t stride, size_t height, size_t width,
                    size_t c, size_t window, size_t shift, const float *gamma,
                    const float *beta, const float *wqkv, const float *bqkv,
                    const float *tables, const float *wproj, const float *bproj) {
  const size_t n = window * window, heads = c / 32;
  const size_t wins = ((height + window - 1) / window) * ((width + window - 1) / window);
  const size_t rows = wins * n;
  float *tokens = (float *)calloc(rows * c, sizeof(float));
  float *qkv = (float *)malloc(sizeof(float) * rows * 3 * c);
  float *heads_out = (float *)malloc(sizeof(float) * rows * c);
  for (size_t w = 0; w < wins; w++)
    for (size_t i = 0; i < n; i++) {
      const long src = window_source(w, i, window, shift, height, width);
      float *row = tokens + (w * n + i) * c;
      if (src < 0) continue; /* stays zero: padding after the normalisation */
      memcpy(row, map + (size_t)src * stride, sizeof(float) * c);
      or_layer_norm(row, c, gamma, beta, c);
    }
  or_input in = {OR_INPUT_ROWS, tokens, 0, 0, 0, c, 0, 0, 0, 0, {{0}}, 0};
  or_multiply_mt(threads, &in, rows, wqkv, c, 3 * c, bqkv, qkv, 3 * c, OR_ACT_NONE, 0);
  for (size_t w = 0; w < wins; w++) {
    const size_t cls = or_window_class(w, window, shift, height, width);
    for (size_t h = 0; h < heads; h++)
      or_attention(qkv + w * n * 3 * c, n, c, h, tables + (cls * heads + h) * n * n,
                   heads_out + w * n * c);
  }
  or_input in2 = {OR_INPUT_ROWS, heads_out, 0, 0, 0, c, 0, 0, 0, 0, {{0}}, 0};
  or_multiply_mt(threads, &in2, rows, wproj, c, c, bproj, tokens, c, OR_ACT_NONE, 0);
  for (size_t w = 0; w < wins; w++)
    for (size_t i = 0; i < n; i++) {
      const long src = window_source(w, i, window, shift, height, width);
      if (src < 0) continue;
      float *dst = map + (size_t)src * stride;
      const float *v = tokens + (w * n + i) * c;
      for (size_t d = 0; d < c; d++) dst[d] += v[d];
    }
  free(tokens);
  free(qkv);
  free(heads_out);
}

/* The MLP half (scunet swin.rs:236-275, birefnet swin.rs:308-347) on `rows`
 * tokens map[r * stride]: LayerNorm, fc1 (c -> 4c) with GELU, fc2 (4c -> c)
 * added onto the tokens. */
void or_swin_mlp(int threads, float *map, size_t stride, size_t rows, size_t c,
                 const float *gamma, const float *beta, const float *w1, const float *b1,
                 const float *w2, const float *b2) {
  float *normed = (float *)malloc(sizeof(float) * rows * c);
  float *hidden = (float *)malloc(sizeof(float) * rows * 4 * c);
  for (size_t r = 0; r < rows; r++) memcpy(normed + r * c, map + r * stride, sizeof(float) * c);
  or_layer_norm(normed, rows * c, gamma, beta, c);
  or_input in = {OR_INPUT_ROWS, normed, 0, 0, 0, c, 0, 0, 0, 0, {{0}}, 0};
  or_multiply_mt(threads, &in, rows, w1, c, 4 * c, b1, hidden, 4 * c, OR_ACT_GELU, 0);
  or_input in2 = {OR_INPUT_ROWS, hidden, 0, 0, 0, 4 * c, 0, 0, 0, 0, {{0}}, 0};
  or_multiply_mt(threads, &in2, rows, w2, 4 * c, c, b2, map, stride, OR_ACT_NONE, 1);
  free(normed);
  free(hidden);
}
