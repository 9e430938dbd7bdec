// fourier.hip -- the 2-D real Fourier transforms of LaMa's spectral units on
// gfx950 (crates/lama-native/src/fourier.rs): rfftn / irfftn over the two
// spatial axes with "ortho" scaling, on NHWC maps, spectra of width / 2 + 1
// columns whose pixels hold every channel's real part, then every
// imaginary part (fourier.rs:1-14).
//
// Each pass transforms whole lines (a row or a column of one map) for a
// group of channels, the line staged in LDS in f32 and the twiddles
// exp(2 pi i j / n) read from a table computed in double precision (as
// fourier.rs:50-58), by the direct sum over the line's points: a lane owns
// one channel and a strided set of outputs, so LDS reads of one step are
// consecutive channels of one point (no bank conflicts) and the twiddle is a
// broadcast.  Four passes:
//   forward  rows    f16 map -> f32 work (columns 0 .. w / 2, e^-)
//   forward  columns f32 work -> f16 spectrum (e^-, times 1 / sqrt(h w))
//   inverse  columns f16 spectrum -> f32 work (e^+)
//   inverse  rows    f32 work -> f16 map, added, times 1 / sqrt(h w); the
//            imaginary parts of column 0 and (even w) column w / 2 of the
//            column-transformed spectrum are read as zero, as irfftn's real
//            transform does (fourier.rs:376-379).
// The sums run in f32 over at most 1024 points; the reference's mixed-radix
// FFT (fourier.rs:17-160) computes the same transform with a different
// rounding order.

#include <cmath>
#include <vector>

#include "conv_common.h"

struct ien_fourier {
  ien_ctx *ctx = nullptr;
  int height = 0, width = 0, half = 0;
  float2 *d_tw_rows = nullptr;  // exp(2 pi i j / width), j < width
  float2 *d_tw_cols = nullptr;  // exp(2 pi i j / height), j < height
};

namespace ien {
namespace {

constexpr int THREADS = 256;
constexpr int MAX_SIDE = 1024;

// Channels per workgroup (32, 16, 8 or 4): the line of `n` points times
// that many channels (complex where `complex_line`) within 48 KiB of LDS,
// which leaves room for the twiddles under 64 KiB.
int group_channels(int n, bool complex_line) {
  const int bytes = complex_line ? 8 : 4;
  int cg = 32;
  while (cg > 4 && n * cg * bytes > 48 * 1024) cg /= 2;
  return cg;
}

// kernel<CG, ...> launched for the runtime group size `cg`.
#define IEN_BY_CG(cg, KERNEL, ...)                                           \
  switch (cg) {                                                            \
    case 32: hipLaunchKernelGGL(KERNEL(32), __VA_ARGS__); break;           \
    case 16: hipLaunchKernelGGL(KERNEL(16), __VA_ARGS__); break;           \
    case 8: hipLaunchKernelGGL(KERNEL(8), __VA_ARGS__); break;             \
    default: hipLaunchKernelGGL(KERNEL(4), __VA_ARGS__); break;            \
  }

// Forward rows: R[y][k][c] = sum_x x[y][x][c] exp(-2 pi i k x / w), k <= w / 2.
template <int CG>
__global__ __launch_bounds__(THREADS) void k_rows_forward(const uint16_t *__restrict__ map,
                                                          long stride, int channels, int w,
                                                          int half, const float2 *__restrict__ tw,
                                                          float *__restrict__ work) {
  extern __shared__ float lds[];
  float *line = lds;                        // [w][CG]
  float2 *twl = (float2 *)(lds + w * CG);   // [w]
  const int y = blockIdx.x, c0 = blockIdx.y * CG, tid = threadIdx.x;
  for (int i = tid; i < w * CG; i += THREADS) {
    const int x = i / CG, c = i % CG;
    line[i] = c0 + c < channels ? h2f(map[((long)y * w + x) * stride + c0 + c]) : 0.0f;
  }
  for (int i = tid; i < w; i += THREADS) twl[i] = tw[i];
  __syncthreads();
  const int c = tid % CG;
  if (c0 + c >= channels) return;
  float *out = work + (long)y * half * 2 * channels;
  for (int k = tid / CG; k < half; k += THREADS / CG) {
    float re = 0.0f, im = 0.0f;
    int j = 0;
    for (int x = 0; x < w; x++) {
      const float v = line[x * CG + c];
      const float2 t = twl[j];
      re = fmaf(v, t.x, re);
      im = fmaf(-v, t.y, im);
      j += k;
      if (j >= w) j -= w;
    }
    out[(long)k * 2 * channels + c0 + c] = re;
    out[(long)k * 2 * channels + channels + c0 + c] = im;
  }
}

// Columns: out[ky][k][c] = scale sum_y in[y][k][c] exp(sign 2 pi i ky y / h).
template <int CG, bool IN_F16, bool OUT_F16>
__global__ __launch_bounds__(THREADS) void k_columns(const void *__restrict__ src, int channels,
                                                     int h, int half, float sign, float scale,
                                                     const float2 *__restrict__ tw,
                                                     void *__restrict__ dst) {
  extern __shared__ float lds[];
  float2 *line = (float2 *)lds;     // [h][CG]
  float2 *twl = line + h * CG;      // [h]
  const int k = blockIdx.x, c0 = blockIdx.y * CG, tid = threadIdx.x;
  const long pitch = 2L * channels;  // values per spectrum pixel
  for (int i = tid; i < h * CG; i += THREADS) {
    const int y = i / CG, c = i % CG;
    float2 z = {0.0f, 0.0f};
    if (c0 + c < channels) {
      const long at = ((long)y * half + k) * pitch + c0 + c;
      if (IN_F16) {
        const uint16_t *s = (const uint16_t *)src;
        z = {h2f(s[at]), h2f(s[at + channels])};
      } else {
        const float *s = (const float *)src;
        z = {s[at], s[at + channels]};
      }
    }
    line[i] = z;
  }
  for (int i = tid; i < h; i += THREADS) twl[i] = tw[i];
  __syncthreads();
  const int c = tid % CG;
  if (c0 + c >= channels) return;
  for (int ky = tid / CG; ky < h; ky += THREADS / CG) {
    float re = 0.0f, im = 0.0f;
    int j = 0;
    for (int y = 0; y < h; y++) {
      const float2 z = line[y * CG + c];
      const float2 t = twl[j];
      const float s = sign * t.y;
      re = fmaf(z.x, t.x, fmaf(-z.y, s, re));
      im = fmaf(z.x, s, fmaf(z.y, t.x, im));
      j += ky;
      if (j >= h) j -= h;
    }
    const long at = ((long)ky * half + k) * pitch + c0 + c;
    if (OUT_F16) {
      uint16_t *d = (uint16_t *)dst;
      d[at] = f2h(re * scale);
      d[at + channels] = f2h(im * scale);
    } else {
      float *d = (float *)dst;
      d[at] = re * scale;
      d[at + channels] = im * scale;
    }
  }
}

// Inverse rows, added to the map: x[y][x][c] += scale (Re U0 + sum over
// 0 < k < w / 2 of 2 Re(U_k e^{+i theta}) + [w even] Re U_{w/2} (-1)^x).
template <int CG>
__global__ __launch_bounds__(THREADS) void k_rows_inverse(const float *__restrict__ work,
                                                          int channels, int w, int half,
                                                          float scale,
                                                          const float2 *__restrict__ tw,
                                                          uint16_t *__restrict__ map,
                                                          long stride) {
  extern __shared__ float lds[];
  float2 *line = (float2 *)lds;   // [half][CG]
  float2 *twl = line + half * CG;  // [w]
  const int y = blockIdx.x, c0 = blockIdx.y * CG, tid = threadIdx.x;
  const float *in = work + (long)y * half * 2 * channels;
  for (int i = tid; i < half * CG; i += THREADS) {
    const int k = i / CG, c = i % CG;
    float2 z = {0.0f, 0.0f};
    if (c0 + c < channels) {
      z.x = in[(long)k * 2 * channels + c0 + c];
      // Column 0 and, for an even width, column w / 2 hold real values.
      const bool real = k == 0 || 2 * k == w;
      z.y = real ? 0.0f : in[(long)k * 2 * channels + channels + c0 + c];
    }
    line[i] = z;
  }
  for (int i = tid; i < w; i += THREADS) twl[i] = tw[i];
  __syncthreads();
  const int c = tid % CG;
  if (c0 + c >= channels) return;
  for (int x = tid / CG; x < w; x += THREADS / CG) {
    float sum = line[c].x;
    int j = 0;
    for (int k = 1; k < half; k++) {
      j += x;
      if (j >= w) j -= w;
      const float2 z = line[k * CG + c];
      const float2 t = twl[j];
      const float term = fmaf(z.x, t.x, -z.y * t.y);
      sum = fmaf(2 * k == w ? 1.0f : 2.0f, term, sum);
    }
    uint16_t *o = map + ((long)y * w + x) * stride + c0 + c;
    *o = f2h(h2f(*o) + sum * scale);
  }
}

std::vector<float2> twiddles(int n) {
  std::vector<float2> t(n);
  for (int j = 0; j < n; j++) {
    const double a = 6.283185307179586476925 * j / n;
    t[j] = {(float)std::cos(a), (float)std::sin(a)};
  }
  return t;
}

}  // namespace
}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_fourier_new(ien_ctx *ctx, size_t height, size_t width, ien_fourier **out) {
  IEN_CHECK(ctx && out, IEN_ERR_INPUT, "null argument");
  *out = nullptr;
  IEN_CHECK(height >= 1 && width >= 1 && height <= MAX_SIDE && width <= MAX_SIDE, IEN_ERR_INPUT,
            "%zu x %zu map (sides 1 .. %d)", width, height, MAX_SIDE);
  IEN_HIP(hipSetDevice(ctx->device));
  ien_fourier *f = new ien_fourier;
  f->ctx = ctx;
  f->height = (int)height;
  f->width = (int)width;
  f->half = (int)width / 2 + 1;
  const std::vector<float2> tr = twiddles((int)width), tc = twiddles((int)height);
  hipError_t e = hipMalloc((void **)&f->d_tw_rows, width * sizeof(float2));
  if (e == hipSuccess) e = hipMalloc((void **)&f->d_tw_cols, height * sizeof(float2));
  if (e == hipSuccess)
    e = hipMemcpy(f->d_tw_rows, tr.data(), width * sizeof(float2), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(f->d_tw_cols, tc.data(), height * sizeof(float2), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    ien_fourier_free(f);
    return fail(IEN_ERR_GPU, "fourier tables: %s", hipGetErrorString(e));
  }
  *out = f;
  return IEN_OK;
}

void ien_fourier_free(ien_fourier *f) {
  if (!f) return;
  (void)hipFree(f->d_tw_rows);
  (void)hipFree(f->d_tw_cols);
  delete f;
}

size_t ien_fourier_half(const ien_fourier *f) { return f ? (size_t)f->half : 0; }

ien_status ien_fourier_forward(const ien_fourier *f, const uint16_t *d_x, size_t stride,
                               size_t channels, float *d_work, uint16_t *d_spectrum) {
  IEN_CHECK(f && d_x && d_work && d_spectrum, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(channels >= 1 && channels <= 4096 && stride >= channels, IEN_ERR_INPUT,
            "%zu channels, pixel stride %zu", channels, stride);
  const int h = f->height, w = f->width, half = f->half, ch = (int)channels;
  hipStream_t s = f->ctx->stream;
  {
    const int cg = group_channels(w, false);
    const dim3 grid((unsigned)h, (unsigned)((ch + cg - 1) / cg));
    const size_t lds = (size_t)w * cg * 4 + (size_t)w * 8;
#define K(CG) k_rows_forward<CG>
    IEN_BY_CG(cg, K, grid, dim3(THREADS), lds, s, d_x, (long)stride, ch, w, half, f->d_tw_rows,
              d_work)
#undef K
    IEN_HIP(hipGetLastError());
  }
  {
    const int cg = group_channels(h, true);
    const dim3 grid((unsigned)half, (unsigned)((ch + cg - 1) / cg));
    const size_t lds = (size_t)h * cg * 8 + (size_t)h * 8;
    const float scale = (float)(1.0 / std::sqrt((double)h * w));
#define K(CG) k_columns<CG, false, true>
    IEN_BY_CG(cg, K, grid, dim3(THREADS), lds, s, (const void *)d_work, ch, h, half, -1.0f,
              scale, f->d_tw_cols, (void *)d_spectrum)
#undef K
    IEN_HIP(hipGetLastError());
  }
  return IEN_OK;
}

ien_status ien_fourier_inverse(const ien_fourier *f, const uint16_t *d_spectrum, size_t channels,
                               float *d_work, uint16_t *d_out, size_t stride) {
  IEN_CHECK(f && d_spectrum && d_work && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(channels >= 1 && channels <= 4096 && stride >= channels, IEN_ERR_INPUT,
            "%zu channels, pixel stride %zu", channels, stride);
  const int h = f->height, w = f->width, half = f->half, ch = (int)channels;
  hipStream_t s = f->ctx->stream;
  {
    const int cg = group_channels(h, true);
    const dim3 grid((unsigned)half, (unsigned)((ch + cg - 1) / cg));
    const size_t lds = (size_t)h * cg * 8 + (size_t)h * 8;
#define K(CG) k_columns<CG, true, false>
    IEN_BY_CG(cg, K, grid, dim3(THREADS), lds, s, (const void *)d_spectrum, ch, h, half, 1.0f,
              1.0f, f->d_tw_cols, (void *)d_work)
#undef K
    IEN_HIP(hipGetLastError());
  }
  {
    const int cg = group_channels(w, true);
    const dim3 grid((unsigned)h, (unsigned)((ch + cg - 1) / cg));
    const size_t lds = (size_t)half * cg * 8 + (size_t)w * 8;
    const float scale = (float)(1.0 / std::sqrt((double)h * w));
#define K(CG) k_rows_inverse<CG>
    IEN_BY_CG(cg, K, grid, dim3(THREADS), lds, s, (const float *)d_work, ch, w, half, scale,
              f->d_tw_rows, d_out, (long)stride)
#undef K
    IEN_HIP(hipGetLastError());
  }
  return IEN_OK;
}

}  // extern "C"
