/*
 * lama.c -- LaMa's generator of image-engine-native's CPU path, restated
 * (TEST INFRASTRUCTURE ONLY: see oracle.h): the 2-D real Fourier transforms
 * of crates/lama-native/src/fourier.rs and the network of
 * crates/lama-native/src/network.rs over the pinned products and Winograd
 * convolutions of this library.
 *
 * The transforms: rfftn / irfftn over the two spatial axes, "ortho" scale,
 * spectrum pixels [re x C | im x C] over width / 2 + 1 columns
 * (fourier.rs:1-14).  Each line goes through a mixed-radix
 * decimation-in-time FFT (radix 4 while it divides, then 2, then each odd
 * prime by its direct sum: fourier.rs:17-61) with f32 arithmetic and
 * twiddles computed in double (fourier.rs:50-58).  Real rows go in one at a
 * time with zero imaginary parts (the reference packs two rows into one
 * complex transform, fourier.rs:291-344: the same sums up to rounding).
 *
 * Tensors come in the weights file's order (tools/lama/export_weights.py
 * export): first w, b; down0..2 w, b; per block b and FFC f: local w, b;
 * cross w, b; spectral_in w, b; fourier w, b; spectral_out w; up0..2 per
 * phase 0..3 w, b; last w, b: 358 tensors.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define LOCAL 128
#define GLOBAL 384
#define CHANNELS 512
#define SPECTRAL 192
#define BLOCKS 18

/* ---- fourier.rs ------------------------------------------------------- */

typedef struct {
  size_t n, nr;
  size_t radices[40];
  float *cos_t, *sin_t; /* exp(2 pi i j / n), j < n */
} fft_t;

static void fft_init(fft_t *f, size_t n) {
  f->n = n;
  f->nr = 0;
  size_t left = n;
  for (size_t p = 4; p >= 2; p -= 2)
    while (left % p == 0) {
      f->radices[f->nr++] = p;
      left /= p;
    }
  for (size_t p = 3; left > 1; p += 2)
    while (left % p == 0) {
      f->radices[f->nr++] = p;
      left /= p;
    }
  f->cos_t = (float *)malloc(sizeof(float) * n);
  f->sin_t = (float *)malloc(sizeof(float) * n);
  for (size_t j = 0; j < n; j++) {
    const double a = 6.283185307179586476925 * (double)j / (double)n;
    f->cos_t[j] = (float)cos(a);
    f->sin_t[j] = (float)sin(a);
  }
}

static void fft_free(fft_t *f) {
  free(f->cos_t);
  free(f->sin_t);
}

/* fourier.rs:78-139 step: the transform of points x[j * stride] for j <
 * n_here, radices rad[0..nr). */
static void fft_step(const fft_t *f, const float *xr, const float *xi, size_t stride,
                     const size_t *rad, size_t nr, float sign, size_t n_here, float *outr,
                     float *outi) {
  if (nr == 0) {
    outr[0] = xr[0];
    outi[0] = xi[0];
    return;
  }
  const size_t p = rad[0], m = n_here / p, turn = f->n / n_here;
  for (size_t q = 0; q < p; q++)
    fft_step(f, xr + q * stride, xi + q * stride, stride * p, rad + 1, nr - 1, sign, m,
             outr + q * m, outi + q * m);
  float ir[p], ii[p], orr[p], oi[p];
  for (size_t k = 0; k < m; k++) {
    for (size_t q = 0; q < p; q++) {
      const size_t j = q * k * turn % f->n;
      const float c = f->cos_t[j], s = sign * f->sin_t[j];
      const float r = outr[q * m + k], i = outi[q * m + k];
      ir[q] = r * c - i * s;
      ii[q] = r * s + i * c;
    }
    if (p == 2) {
      orr[0] = ir[0] + ir[1];
      oi[0] = ii[0] + ii[1];
      orr[1] = ir[0] - ir[1];
      oi[1] = ii[0] - ii[1];
    } else if (p == 4) {
      const float b0r = ir[0] + ir[2], b0i = ii[0] + ii[2];
      const float b1r = ir[0] - ir[2], b1i = ii[0] - ii[2];
      const float b2r = ir[1] + ir[3], b2i = ii[1] + ii[3];
      const float b3r = ir[1] - ir[3], b3i = ii[1] - ii[3];
      orr[0] = b0r + b2r;
      oi[0] = b0i + b2i;
      orr[2] = b0r - b2r;
      oi[2] = b0i - b2i;
      orr[1] = b1r - sign * b3i;
      oi[1] = b1i + sign * b3r;
      orr[3] = b1r + sign * b3i;
      oi[3] = b1i - sign * b3r;
    } else {
      for (size_t t = 0; t < p; t++) {
        float ar = 0.0f, ai = 0.0f;
        for (size_t q = 0; q < p; q++) {
          const size_t j = (q * t % p) * (f->n / p);
          const float c = f->cos_t[j], s = sign * f->sin_t[j];
          ar += ir[q] * c - ii[q] * s;
          ai += ir[q] * s + ii[q] * c;
        }
        orr[t] = ar;
        oi[t] = ai;
      }
    }
    for (size_t t = 0; t < p; t++) {
      outr[k + t * m] = orr[t];
      outi[k + t * m] = oi[t];
    }
  }
}

static void fft_run(const fft_t *f, const float *xr, const float *xi, float sign, float *outr,
                    float *outi) {
  fft_step(f, xr, xi, 1, f->radices, f->nr, sign, f->n, outr, outi);
}

/* fourier.rs:291-344 forward: spectrum of x (h x w x c) into out (h x half x 2c). */
void or_rfft2(const float *x, size_t h, size_t w, size_t c, float *out) {
  const size_t half = w / 2 + 1;
  fft_t rows, cols;
  fft_init(&rows, w);
  fft_init(&cols, h);
  const size_t nmax = h > w ? h : w;
  float *lr = (float *)malloc(sizeof(float) * nmax), *li = (float *)malloc(sizeof(float) * nmax);
  float *tr = (float *)malloc(sizeof(float) * nmax), *ti = (float *)malloc(sizeof(float) * nmax);
  float *work = (float *)malloc(sizeof(float) * h * half * 2 * c);
  for (size_t y = 0; y < h; y++)
    for (size_t ch = 0; ch < c; ch++) {
      for (size_t xx = 0; xx < w; xx++) {
        lr[xx] = x[(y * w + xx) * c + ch];
        li[xx] = 0.0f;
      }
      fft_run(&rows, lr, li, -1.0f, tr, ti);
      for (size_t k = 0; k < half; k++) {
        work[(y * half + k) * 2 * c + ch] = tr[k];
        work[(y * half + k) * 2 * c + c + ch] = ti[k];
      }
    }
  /* fourier.rs:406-436 columns: the forward direction applies the scale. */
  const float scale = 1.0f / sqrtf((float)(h * w));
  for (size_t k = 0; k < half; k++)
    for (size_t ch = 0; ch < c; ch++) {
      for (size_t y = 0; y < h; y++) {
        lr[y] = work[(y * half + k) * 2 * c + ch];
        li[y] = work[(y * half + k) * 2 * c + c + ch];
      }
      fft_run(&cols, lr, li, -1.0f, tr, ti);
      for (size_t ky = 0; ky < h; ky++) {
        out[(ky * half + k) * 2 * c + ch] = tr[ky] * scale;
        out[(ky * half + k) * 2 * c + c + ch] = ti[ky] * scale;
      }
    }
  free(work);
  free(lr);
  free(li);
  free(tr);
  free(ti);
  fft_free(&rows);
  fft_free(&cols);
}

/* fourier.rs:347-403 inverse: the map of spectrum s ADDED to out (h x w x c):
 * columns with exp(+), then each row's full spectrum from its half (mirrored
 * points conjugated, imaginary parts of column 0 and, for even w, column
 * w / 2 read as zero: :370-380) through the complex transform, real part
 * times 1 / sqrt(h w). */
void or_irfft2_add(const float *s, size_t h, size_t w, size_t c, float *out) {
  const size_t half = w / 2 + 1;
  fft_t rows, cols;
  fft_init(&rows, w);
  fft_init(&cols, h);
  const size_t nmax = h > w ? h : w;
  float *lr = (float *)malloc(sizeof(float) * nmax), *li = (float *)malloc(sizeof(float) * nmax);
  float *tr = (float *)malloc(sizeof(float) * nmax), *ti = (float *)malloc(sizeof(float) * nmax);
  float *work = (float *)malloc(sizeof(float) * h * half * 2 * c);
  for (size_t k = 0; k < half; k++)
    for (size_t ch = 0; ch < c; ch++) {
      for (size_t y = 0; y < h; y++) {
        lr[y] = s[(y * half + k) * 2 * c + ch];
        li[y] = s[(y * half + k) * 2 * c + c + ch];
      }
      fft_run(&cols, lr, li, 1.0f, tr, ti);
      for (size_t y = 0; y < h; y++) {
        work[(y * half + k) * 2 * c + ch] = tr[y];
        work[(y * half + k) * 2 * c + c + ch] = ti[y];
      }
    }
  const float scale = 1.0f / sqrtf((float)(h * w));
  for (size_t y = 0; y < h; y++)
    for (size_t ch = 0; ch < c; ch++) {
      for (size_t k = 0; k < w; k++) {
        const int mirror = k >= half;
        const size_t j = mirror ? w - k : k;
        const int real = j == 0 || 2 * j == w;
        const float re = work[(y * half + j) * 2 * c + ch];
        const float im = real ? 0.0f : work[(y * half + j) * 2 * c + c + ch];
        lr[k] = re;
        li[k] = mirror ? -im : im;
      }
      fft_run(&rows, lr, li, 1.0f, tr, ti);
      for (size_t xx = 0; xx < w; xx++) out[(y * w + xx) * c + ch] += scale * tr[xx];
    }
  free(work);
  free(lr);
  free(li);
  free(tr);
  free(ti);
  fft_free(&rows);
  fft_free(&cols);
}

/* ---- network.rs ------------------------------------------------------- */

static or_input image_input(const float *data, size_t h, size_t w, size_t c, size_t stride,
                            size_t size, size_t step, int pad) {
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
  in.step = step;
  in.pad = pad;
  return in;
}

static or_input rows_input(const float *data, size_t stride) {
  or_input in;
  memset(&in, 0, sizeof in);
  in.kind = OR_INPUT_ROWS;
  in.data = data;
  in.stride = stride;
  return in;
}

typedef struct {
  const float *local_w, *local_b, *cross_w, *cross_b, *in_w, *in_b, *four_w, *four_b, *out_w;
} ffc_t;

static ffc_t take_ffc(const float *const **t) {
  ffc_t f;
  const float **p = (const float **)&f;
  for (int i = 0; i < 9; i++) p[i] = *(*t)++;
  return f;
}

/* network.rs:174-249 Ffc::run: out = ffc(x) on an h x w map of 512. */
static void ffc_run(int threads, const ffc_t *f, const float *x, float *out, size_t h, size_t w) {
  const size_t pixels = h * w, half = w / 2 + 1, spix = h * half;
  or_input local = image_input(x, h, w, CHANNELS, CHANNELS, 3, 1, OR_PAD_REFLECT);
  or_conv3(threads, &local, f->local_w, LOCAL, f->local_b, out, CHANNELS, 0, OR_FINISH_RELU,
           NULL);
  or_input cross = image_input(x, h, w, LOCAL, CHANNELS, 3, 1, OR_PAD_REFLECT);
  or_conv3(threads, &cross, f->cross_w, GLOBAL, f->cross_b, out + LOCAL, CHANNELS, 0,
           OR_FINISH_NONE, NULL);
  float *spectral = (float *)malloc(sizeof(float) * pixels * SPECTRAL);
  or_input gin = image_input(x + LOCAL, h, w, GLOBAL, CHANNELS, 1, 1, OR_PAD_ZERO);
  or_multiply_mt(threads, &gin, pixels, f->in_w, GLOBAL, SPECTRAL, f->in_b, spectral, SPECTRAL,
                 OR_ACT_RELU, 0);
  float *spectrum = (float *)malloc(sizeof(float) * spix * 2 * SPECTRAL);
  or_rfft2(spectral, h, w, SPECTRAL, spectrum);
  float *filtered = (float *)malloc(sizeof(float) * spix * 2 * SPECTRAL);
  or_input sin = rows_input(spectrum, 2 * SPECTRAL);
  or_multiply_mt(threads, &sin, spix, f->four_w, 2 * SPECTRAL, 2 * SPECTRAL, f->four_b, filtered,
                 2 * SPECTRAL, OR_ACT_RELU, 0);
  or_irfft2_add(filtered, h, w, SPECTRAL, spectral);
  or_input oin = rows_input(spectral, SPECTRAL);
  or_multiply_mt(threads, &oin, pixels, f->out_w, SPECTRAL, GLOBAL, NULL, out + LOCAL, CHANNELS,
                 OR_ACT_RELU, 1);
  free(spectral);
  free(spectrum);
  free(filtered);
}

/* network.rs:271 PHASE_TAPS and :279-335 Up: output phase p = 2 py + px
 * reads input offsets (dy, dx) over PHASE_TAPS[py] x PHASE_TAPS[px]; the
 * doubled map through a ReLU. */
void or_lama_up(int threads, const float *const *phase_w, const float *const *phase_b,
                const float *x, size_t h, size_t w, size_t cin, size_t cout, float *out) {
  static const size_t counts[2] = {1, 2};
  static const size_t offs[2][2] = {{0, 0}, {0, 1}};
  float *buf = (float *)malloc(sizeof(float) * h * w * cout);
  for (size_t p = 0; p < 4; p++) {
    const size_t py = p / 2, px = p % 2;
    or_input in;
    memset(&in, 0, sizeof in);
    in.kind = OR_INPUT_IMAGE;
    in.data = x;
    in.height = h;
    in.width = w;
    in.channels = cin;
    in.stride = cin;
    in.taps = OR_TAPS_OFFSETS;
    in.count = 0;
    for (size_t a = 0; a < counts[py]; a++)
      for (size_t b = 0; b < counts[px]; b++) {
        in.offsets[in.count][0] = offs[py][a];
        in.offsets[in.count][1] = offs[px][b];
        in.count++;
      }
    or_multiply_mt(threads, &in, h * w, phase_w[p], in.count * cin, cout, phase_b[p], buf, cout,
                   OR_ACT_RELU, 0);
    for (size_t y = 0; y < h; y++)
      for (size_t xx = 0; xx < w; xx++)
        memcpy(out + ((2 * y + py) * 2 * w + 2 * xx + px) * cout, buf + (y * w + xx) * cout,
               sizeof(float) * cout);
  }
  free(buf);
}

/* network.rs:415-489 run: padded masked input, first 7x7, three stride-2
 * downs, 18 blocks (x += ffc1(ffc0(x))), three transposed ups, the last 7x7
 * through a sigmoid, cropped. */
int or_lama_run(int threads, const float *const *t, const float *image, const float *mask,
                size_t width, size_t height, float *out) {
  size_t h = (height + 7) / 8 * 8, w = (width + 7) / 8 * 8;
  const size_t ph = h, pw = w;
  float *x = (float *)malloc(sizeof(float) * h * w * 4);
  or_masked_rows(image, mask, width, height, 8, x);
  const float *first_w = *t++, *first_b = *t++;
  const float *down_w[3], *down_b[3];
  for (int i = 0; i < 3; i++) {
    down_w[i] = *t++;
    down_b[i] = *t++;
  }
  ffc_t blocks[BLOCKS][2];
  for (int b = 0; b < BLOCKS; b++) {
    blocks[b][0] = take_ffc(&t);
    blocks[b][1] = take_ffc(&t);
  }
  const float *up_w[3][4], *up_b[3][4];
  for (int i = 0; i < 3; i++)
    for (int p = 0; p < 4; p++) {
      up_w[i][p] = *t++;
      up_b[i][p] = *t++;
    }
  const float *last_w = *t++, *last_b = *t++;

  float *a = (float *)malloc(sizeof(float) * h * w * 64);
  or_input fin = image_input(x, h, w, 4, 4, 7, 1, OR_PAD_REFLECT);
  or_multiply_mt(threads, &fin, h * w, first_w, 49 * 4, 64, first_b, a, 64, OR_ACT_RELU, 0);
  free(x);
  size_t c = 64;
  static const size_t douts[3] = {128, 256, CHANNELS};
  for (int i = 0; i < 3; i++) {
    or_input din = image_input(a, h, w, c, c, 3, 2, OR_PAD_REFLECT);
    const size_t nh = (h - 1) / 2 + 1, nw = (w - 1) / 2 + 1;
    float *next = (float *)malloc(sizeof(float) * nh * nw * douts[i]);
    or_multiply_mt(threads, &din, nh * nw, down_w[i], 9 * c, douts[i], down_b[i], next, douts[i],
                   OR_ACT_RELU, 0);
    free(a);
    a = next;
    h = nh;
    w = nw;
    c = douts[i];
  }
  float *mid = (float *)malloc(sizeof(float) * h * w * CHANNELS);
  float *o = (float *)malloc(sizeof(float) * h * w * CHANNELS);
  for (int b = 0; b < BLOCKS; b++) {
    ffc_run(threads, &blocks[b][0], a, mid, h, w);
    ffc_run(threads, &blocks[b][1], mid, o, h, w);
    for (size_t i = 0; i < h * w * CHANNELS; i++) a[i] += o[i];
  }
  free(mid);
  free(o);
  static const size_t ucouts[3] = {256, 128, 64};
  for (int i = 0; i < 3; i++) {
    float *next = (float *)malloc(sizeof(float) * 4 * h * w * ucouts[i]);
    or_lama_up(threads, up_w[i], up_b[i], a, h, w, c, ucouts[i], next);
    free(a);
    a = next;
    h *= 2;
    w *= 2;
    c = ucouts[i];
  }
  float *rgb = (float *)malloc(sizeof(float) * h * w * 3);
  or_input lin = image_input(a, h, w, 64, 64, 7, 1, OR_PAD_REFLECT);
  or_multiply_mt(threads, &lin, h * w, last_w, 49 * 64, 3, last_b, rgb, 3, OR_ACT_NONE, 0);
  free(a);
  or_sigmoid(rgb, h * w * 3);
  for (size_t y = 0; y < height; y++)
    memcpy(out + y * width * 3, rgb + y * pw * 3, sizeof(float) * width * 3);
  (void)ph;
  free(rgb);
  return 0;
}
