/*
 * io.c -- oracle restatement of the models' 8-bit image I/O and tiling.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Pins: tests/test_oracle_io.py (every byte through to_float against f32
 * division; to_byte's known answers -- ties away from zero, saturation, NaN
 * to 0 -- and random floats against the f64 definition; the normalisation
 * against an f64 ImageNet normalisation to within one f32 rounding of each
 * step; compositing against a per-pixel brute force; tile regions as an
 * exact partition of the image, each inside its region with the margin
 * clipped at the edges).
 */
#include <math.h>

#include "oracle.h"

/* realesrgan-native lib.rs:292-295 to_float: f32::from(v) / 255.0. */
float or_to_float(uint8_t v) { return (float)v / 255.0f; }

/* realesrgan-native lib.rs:297-300 to_byte: (v.clamp(0.0, 1.0) * 255.0)
 * .round() as u8.  f32::clamp keeps a NaN, round() takes ties away from
 * zero, and `as u8` saturates with NaN to 0. */
uint8_t or_to_byte(float v) {
  if (isnan(v)) return 0;
  float c = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
  float r = roundf(c * 255.0f);
  if (r <= 0.0f) return 0;
  if (r >= 255.0f) return 255;
  return (uint8_t)r;
}

void or_bytes_to_floats(const uint8_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_to_float(src[i]);
}

void or_floats_to_bytes(const float *src, uint8_t *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_to_byte(src[i]);
}

/* birefnet-native lib.rs:36-37 MEAN, STD and lib.rs:111-116: the table of
 * each colour's 256 values, (f32::from(v) / 255.0 - MEAN[c]) / STD[c] in
 * f32, then each value of interleaved RGB looked up. */
void or_normalize_bytes(const uint8_t *rgb, size_t pixels, float *dst) {
  static const float mean[3] = {0.485f, 0.456f, 0.406f}, std[3] = {0.229f, 0.224f, 0.225f};
  float table[256][3];
  for (int v = 0; v < 256; v++)
    for (int c = 0; c < 3; c++) table[v][c] = ((float)v / 255.0f - mean[c]) / std[c];
  for (size_t p = 0; p < pixels; p++)
    for (int c = 0; c < 3; c++) dst[p * 3 + c] = table[rgb[p * 3 + c]][c];
}

/* lama-native lib.rs:142: the holes, f32::from(u8::from(m != 0)). */
void or_mask_bytes(const uint8_t *mask, float *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = mask[i] != 0 ? 1.0f : 0.0f;
}

/* lama-native lib.rs:147-155: the bytes of the image where the mask is 0,
 * the prediction as bytes where it is not. */
void or_composite_bytes(const uint8_t *rgb, const uint8_t *mask, const float *pred,
                        size_t pixels, uint8_t *out) {
  for (size_t p = 0; p < pixels; p++)
    for (int c = 0; c < 3; c++)
      out[p * 3 + c] = mask[p] != 0 ? or_to_byte(pred[p * 3 + c]) : rgb[p * 3 + c];
}

/* realesrgan-native lib.rs:251-265 (scunet-native lib.rs:212-226): tile
 * (j, i) of a rows x cols grid, cols = ceil(width / tile), rows =
 * ceil(height / tile): its own pixels [x0, x1) x [y0, y1) and its region
 * [rx0, rx1) x [ry0, ry1) with up to `margin` pixels around it.  Writes
 * tiles x 8 values (x0, x1, y0, y1, rx0, rx1, ry0, ry1) in row-major tile
 * order; returns the tile count. */
size_t or_tile_regions(size_t width, size_t height, size_t tile, size_t margin, size_t *out) {
  if (tile == 0) return 0;
  const size_t cols = (width + tile - 1) / tile, rows = (height + tile - 1) / tile;
  size_t k = 0;
  for (size_t j = 0; j < rows; j++) {
    const size_t y0 = j * height / rows, y1 = (j + 1) * height / rows;
    for (size_t i = 0; i < cols; i++) {
      const size_t x0 = i * width / cols, x1 = (i + 1) * width / cols;
      const size_t rx0 = x0 > margin ? x0 - margin : 0, ry0 = y0 > margin ? y0 - margin : 0;
      const size_t rx1 = x1 + margin < width ? x1 + margin : width;
      const size_t ry1 = y1 + margin < height ? y1 + margin : height;
      size_t *r = out + 8 * k++;
      r[0] = x0, r[1] = x1, r[2] = y0, r[3] = y1, r[4] = rx0, r[5] = rx1, r[6] = ry0, r[7] = ry1;
    }
  }
  return k;
}
