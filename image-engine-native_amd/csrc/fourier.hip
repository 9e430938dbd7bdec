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
// rounding order.  Lines of at most 256 points (maps up to 128 x 255) take
// the same four passes as real matrix products on f32 MFMA instead
// (k_line_mfma): the DFT matrices, scales and edge-column rules folded into
// tables built in double.

#include <cmath>
#include <vector>

#include "conv_common.h"

struct ien_fourier {
  ien_ctx *ctx = nullptr;
  int height = 0, width = 0, half = 0;
  float2 *d_tw_rows = nullptr;  // exp(2 pi i j / width), j < width
  float2 *d_tw_cols = nullptr;  // exp(2 pi i j / height), j < height
  // The four passes as real matrices (transposed: [k][m], m padded to a
  // multiple of 32), for lines of at most MFMA_MAX_K points: forward rows
  // (2 half x w), forward columns (2h x 2h, 1 / sqrt(h w) folded in),
  // inverse columns (2h x 2h), inverse rows (w x 2 half, 1 / sqrt(h w) and
  // the edge-column rules folded in).  Null above that size.
  float *d_fr = nullptr, *d_fc = nullptr, *d_ic = nullptr, *d_ir = nullptr;
  int mp_fr = 0, mp_fc = 0, mp_ir = 0;
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

// ---- the passes on f32 MFMA: out_line = A in_line, a line at a time -------
//
// A line is K real values per channel (a row of the map, or the re / im
// halves of a spectrum row or column); the pass writes M real values per
// channel.  Element k of a line sits at line * in_line + (k % K1) in_k +
// (k / K1) in_part (K1 points per part: real parts, then imaginary ones);
// output element m likewise with M1, out_k, out_part.  A workgroup stages
// one line of 32 channels in LDS as f32; wave w computes 32-row blocks
// w, w + 4, ... of A x line on v_mfma_f32_32x32x2_f32 (A from the
// transposed table, k-major, so the 32 lanes of a fragment read 128
// consecutive bytes); each lane then holds 16 outputs of one channel.
constexpr int MFMA_MAX_K = 256;

struct LinePass {
  const void *in;
  void *out;
  int C, K, KP, K1, M, M1, MP;  // KP: K rounded up to even (zero rows); MP: the table's padded M
  long in_line, in_k, in_part, out_line, out_k, out_part;
  const float *at;  // [K][MP]
};

template <bool IN_F16, bool OUT_F16, bool ADD>
__global__ __launch_bounds__(THREADS) void k_line_mfma(LinePass p) {
  __shared__ float line[MFMA_MAX_K * 32];
  const int ln = blockIdx.x, c0 = blockIdx.y * 32, tid = threadIdx.x;
  // 8 unconditional loads in flight per thread (from clamped, valid
  // addresses; what lies outside the line is zeroed after the load), so one
  // memory latency covers the batch.
  for (int i0 = tid; i0 < p.KP * 32; i0 += 8 * THREADS) {
    float v[8];
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const int i = i0 + b * THREADS;
      const int k = min(i >> 5, p.K - 1), c = min(c0 + (i & 31), p.C - 1);
      const int part = k >= p.K1;  // k < 2 K1
      const long at = ln * p.in_line + (k - part * p.K1) * p.in_k + part * p.in_part + c;
      v[b] = IN_F16 ? h2f(((const uint16_t *)p.in)[at]) : ((const float *)p.in)[at];
    }
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const int i = i0 + b * THREADS;
      const bool ok = (i >> 5) < p.K && c0 + (i & 31) < p.C;
      if (i < p.KP * 32) line[i] = ok ? v[b] : 0.0f;
    }
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63;
  const int cc = lane & 31;
  for (int mb = wave; mb * 32 < p.M; mb += 4) {
    // Two accumulator chains (even and odd steps), so consecutive MFMAs do
    // not wait on each other's results.
    floatx16 acc, acc2;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = acc2[r] = 0.0f;
    const float *a = p.at + mb * 32 + cc;
    // 32 k at a time: the 16 table loads of a lane are issued together, and
    // those of the next 32 k before this batch's MFMAs, so their latency
    // overlaps the products.  Lane halves take k of either parity; KP is
    // even, so a step is valid for both or neither.
    // A[m = 32 mb + lane % 32][k]; steps past KP are never used (clamped to
    // a valid row so the load needs no branch).
    auto table = [&](int k0, float *av) {
#pragma unroll
      for (int i = 0; i < 16; i++) av[i] = a[(long)min(k0 + 2 * i + (lane >> 5), p.KP - 1) * p.MP];
    };
    float nx[16];
    table(0, nx);
    for (int k0 = 0; k0 < p.KP; k0 += 32) {
      float av[16];
#pragma unroll
      for (int i = 0; i < 16; i++) av[i] = nx[i];
      if (k0 + 32 < p.KP) table(k0 + 32, nx);
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        if (k0 + 2 * i >= p.KP) break;
        const int k = k0 + 2 * i + (lane >> 5);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], line[k * 32 + cc], acc, 0, 0, 0);
        if (k0 + 2 * i + 2 >= p.KP) break;
        acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i + 1], line[(k + 2) * 32 + cc], acc2, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] += acc2[r];
    if (c0 + cc >= p.C) continue;
    auto out_at = [&](int r) {
      const int m = min(mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), p.M - 1);
      const int part = m >= p.M1;  // m < 2 M1
      return ln * p.out_line + (m - part * p.M1) * p.out_k + part * p.out_part + c0 + cc;
    };
    // When adding, the 16 old values are loaded together first (from
    // clamped, valid positions), so one latency covers them.
    float old[16];
#pragma unroll
    for (int r = 0; r < 16; r++)
      old[r] = !ADD ? 0.0f
               : OUT_F16 ? h2f(((const uint16_t *)p.out)[out_at(r)])
                         : ((const float *)p.out)[out_at(r)];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int m = mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (m >= p.M) continue;
      const long at = out_at(r);
      if (OUT_F16)
        ((uint16_t *)p.out)[at] = f2h(ADD ? old[r] + acc[r] : acc[r]);
      else
        ((float *)p.out)[at] = ADD ? old[r] + acc[r] : acc[r];
    }
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

// The four pass matrices of an h x w map (see ien_fourier), transposed and
// padded, computed in double.
struct Tables {
  int mp_fr, mp_fc, mp_ir;
  std::vector<float> fr, fc, ic, ir;
};

Tables pass_tables(int h, int w) {
  const int half = w / 2 + 1;
  const double tau = 6.283185307179586476925, s = 1.0 / std::sqrt((double)h * w);
  auto pad = [](int m) { return (m + 31) / 32 * 32; };
  Tables t;
  t.mp_fr = pad(2 * half);
  t.mp_fc = pad(2 * h);
  t.mp_ir = pad(w);
  t.fr.assign((size_t)(w + (w & 1)) * t.mp_fr, 0.0f);  // an even number of (zero-padded) rows
  for (int x = 0; x < w; x++)
    for (int k = 0; k < half; k++) {
      const double a = tau * (double)((long)k * x % w) / w;
      t.fr[(size_t)x * t.mp_fr + k] = (float)std::cos(a);
      t.fr[(size_t)x * t.mp_fr + half + k] = (float)-std::sin(a);
    }
  // Columns: (a + i b) e^{-+i theta}; input k < h real parts, k >= h imaginary.
  t.fc.assign((size_t)2 * h * t.mp_fc, 0.0f);
  t.ic.assign((size_t)2 * h * t.mp_fc, 0.0f);
  for (int y = 0; y < h; y++)
    for (int ky = 0; ky < h; ky++) {
      const double a = tau * (double)((long)ky * y % h) / h, c = std::cos(a), sn = std::sin(a);
      // forward: input y, output ky
      t.fc[(size_t)y * t.mp_fc + ky] = (float)(c * s);
      t.fc[(size_t)(h + y) * t.mp_fc + ky] = (float)(sn * s);
      t.fc[(size_t)y * t.mp_fc + h + ky] = (float)(-sn * s);
      t.fc[(size_t)(h + y) * t.mp_fc + h + ky] = (float)(c * s);
      // inverse: input ky, output y
      t.ic[(size_t)ky * t.mp_fc + y] = (float)c;
      t.ic[(size_t)(h + ky) * t.mp_fc + y] = (float)-sn;
      t.ic[(size_t)ky * t.mp_fc + h + y] = (float)sn;
      t.ic[(size_t)(h + ky) * t.mp_fc + h + y] = (float)c;
    }
  // Inverse rows: x = sum_k w_k (re_k cos - im_k sin), w_k = 1 at k = 0 and
  // (even w) k = w / 2, whose imaginary parts are not read; 2 elsewhere.
  t.ir.assign((size_t)2 * half * t.mp_ir, 0.0f);
  for (int k = 0; k < half; k++) {
    const bool edge = k == 0 || 2 * k == w;
    const double wk = edge ? 1.0 : 2.0;
    for (int x = 0; x < w; x++) {
      const double a = tau * (double)((long)k * x % w) / w;
      t.ir[(size_t)k * t.mp_ir + x] = (float)(wk * std::cos(a) * s);
      t.ir[(size_t)(half + k) * t.mp_ir + x] = edge ? 0.0f : (float)(-wk * std::sin(a) * s);
    }
  }
  return t;
}

template <bool IN_F16, bool OUT_F16, bool ADD>
ien_status line_pass(hipStream_t s, int lines, const LinePass &p) {
  const dim3 grid((unsigned)lines, (unsigned)((p.C + 31) / 32));
  hipLaunchKernelGGL((k_line_mfma<IN_F16, OUT_F16, ADD>), grid, dim3(THREADS), 0, s, p);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
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
  if (e == hipSuccess && 2 * height <= MFMA_MAX_K && width + 1 <= MFMA_MAX_K &&
      2 * (width / 2 + 1) <= MFMA_MAX_K) {
    const Tables t = pass_tables((int)height, (int)width);
    f->mp_fr = t.mp_fr;
    f->mp_fc = t.mp_fc;
    f->mp_ir = t.mp_ir;
    auto put = [&](float **d, const std::vector<float> &v) {
      hipError_t r = hipMalloc((void **)d, v.size() * 4);
      return r == hipSuccess ? hipMemcpy(*d, v.data(), v.size() * 4, hipMemcpyHostToDevice) : r;
    };
    e = put(&f->d_fr, t.fr);
    if (e == hipSuccess) e = put(&f->d_fc, t.fc);
    if (e == hipSuccess) e = put(&f->d_ic, t.ic);
    if (e == hipSuccess) e = put(&f->d_ir, t.ir);
  }
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
  (void)hipFree(f->d_fr);
  (void)hipFree(f->d_fc);
  (void)hipFree(f->d_ic);
  (void)hipFree(f->d_ir);
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
  if (f->d_fr) {
    LinePass rows{d_x, d_work, ch, w, w + (w & 1), w, 2 * half, half, f->mp_fr,
                  (long)w * (long)stride, (long)stride, 0, (long)half * 2 * ch, 2L * ch, ch, f->d_fr};
    ien_status st = line_pass<true, false, false>(s, h, rows);
    if (st != IEN_OK) return st;
    LinePass cols{d_work, d_spectrum, ch, 2 * h, 2 * h, h, 2 * h, h, f->mp_fc,
                  2L * ch, (long)half * 2 * ch, ch, 2L * ch, (long)half * 2 * ch, ch, f->d_fc};
    return line_pass<false, true, false>(s, half, cols);
  }
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
  if (f->d_ic) {
    LinePass cols{d_spectrum, d_work, ch, 2 * h, 2 * h, h, 2 * h, h, f->mp_fc,
                  2L * ch, (long)half * 2 * ch, ch, 2L * ch, (long)half * 2 * ch, ch, f->d_ic};
    ien_status st = line_pass<true, false, false>(s, half, cols);
    if (st != IEN_OK) return st;
    LinePass rows{d_work, d_out, ch, 2 * half, 2 * half, half, w, w, f->mp_ir,
                  (long)half * 2 * ch, 2L * ch, ch, (long)w * (long)stride, (long)stride, 0, f->d_ir};
    return line_pass<false, true, true>(s, h, rows);
  }
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
