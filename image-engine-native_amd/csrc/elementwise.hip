// elementwise.hip -- the memory-bound passes around the products:
// half conversions (half.rs), LayerNorm / GELU / sigmoid (math.rs), the
// Real-ESRGAN pixel shuffle with the repeated input (realesrgan-native
// network.rs:115-141, shaders/shuffle.comp) and the depthwise convolution.
//
// All of them are HBM-bound: each thread moves 16-byte vectors where the
// layout allows, rows are reduced within one wave64 (no LDS round trip),
// and grids are sized to the work, not to the CU count.

#include "ien_internal.h"

namespace ien {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f_e(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ uint16_t f2h_e(float f) {
  _Float16 v = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

static unsigned grid_for(size_t items, unsigned per_block) {
  size_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > (1u << 30)) g = 1u << 30;
  return (unsigned)g;
}

// ---- half.rs:50-79 floats_to_halves / halves_to_f32 ----------------------
__global__ void k_f2h(const float *__restrict__ src, uint16_t *__restrict__ dst, size_t n) {
  const bool aligned = (((uintptr_t)src & 15) | ((uintptr_t)dst & 7)) == 0;
  size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  for (; i < n; i += (size_t)gridDim.x * blockDim.x * 4) {
    if (aligned && i + 4 <= n) {
      float4v v = *(const float4v *)(src + i);
      uint16_t h[4] = {f2h_e(v[0]), f2h_e(v[1]), f2h_e(v[2]), f2h_e(v[3])};
      uint2 o;
      __builtin_memcpy(&o, h, 8);
      *(uint2 *)(dst + i) = o;
    } else {
      for (size_t j = i; j < n && j < i + 4; j++) dst[j] = f2h_e(src[j]);
    }
  }
}

__global__ void k_h2f(const uint16_t *__restrict__ src, float *__restrict__ dst, size_t n) {
  const bool aligned = (((uintptr_t)src & 7) | ((uintptr_t)dst & 15)) == 0;
  size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  for (; i < n; i += (size_t)gridDim.x * blockDim.x * 4) {
    if (aligned && i + 4 <= n) {
      uint2 o = *(const uint2 *)(src + i);
      uint16_t h[4];
      __builtin_memcpy(h, &o, 8);
      float4v v = {h2f_e(h[0]), h2f_e(h[1]), h2f_e(h[2]), h2f_e(h[3])};
      *(float4v *)(dst + i) = v;
    } else {
      for (size_t j = i; j < n && j < i + 4; j++) dst[j] = h2f_e(src[j]);
    }
  }
}

// ---- realesrgan network.rs:115-141: pixel shuffle x4 plus the input ------
// One thread per output pixel: out(4y+i, 4x+j, c) = last(y, x, 16c+4i+j)
// + image(y, x, c).  Consecutive threads write consecutive output pixels.
__global__ void k_shuffle_add(const uint16_t *__restrict__ last, long last_stride,
                              const float *__restrict__ image, int width, int height,
                              float *__restrict__ out) {
  const long ow = 4L * width, total = ow * 4L * height;
  for (long o = (long)blockIdx.x * blockDim.x + threadIdx.x; o < total;
       o += (long)gridDim.x * blockDim.x) {
    long oy = o / ow, ox = o - oy * ow;
    long y = oy >> 2, x = ox >> 2;
    int i = (int)(oy & 3), j = (int)(ox & 3);
    long p = y * width + x;
    const uint16_t *l = last + p * last_stride + 4 * i + j;
    const float *im = image + p * 3;
    out[o * 3 + 0] = h2f_e(l[0]) + im[0];
    out[o * 3 + 1] = h2f_e(l[16]) + im[1];
    out[o * 3 + 2] = h2f_e(l[32]) + im[2];
  }
}

// ---- math.rs:95-116 LayerNorm: one wave per row, two passes over ---------
// registers, f32 statistics, epsilon 1e-5.
__global__ __launch_bounds__(256) void k_layer_norm(uint16_t *__restrict__ x, long rows, int c,
                                                    long stride, const float *__restrict__ gamma,
                                                    const float *__restrict__ beta) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  uint16_t *r = x + row * stride;
  constexpr int MAXV = 48;  // up to 64 * 48 = 3072 channels per row
  float v[MAXV];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXV; k++) {
    int idx = lane + 64 * k;
    v[k] = idx < c ? h2f_e(r[idx]) : 0.0f;
    sum += v[k];
  }
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float mean = sum / (float)c;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXV; k++) {
    int idx = lane + 64 * k;
    float d = idx < c ? v[k] - mean : 0.0f;
    sq += d * d;
  }
  for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
  const float inv = 1.0f / sqrtf(sq / (float)c + 1e-5f);
#pragma unroll
  for (int k = 0; k < MAXV; k++) {
    int idx = lane + 64 * k;
    if (idx < c) r[idx] = f2h_e((v[k] - mean) * inv * gamma[idx] + beta[idx]);
  }
}

// ---- math.rs:136-152 GELU and the logistic function in place -------------
__device__ __forceinline__ float gelu_e(float x) {
  // math.rs:41-75 (Eigen's generic_fast_erf_float coefficients).
  float z = fminf(fmaxf(x * 0.70710678118654752f, -4.0f), 4.0f);
  float z2 = z * z;
  float p = -2.7261423e-10f;
  p = p * z2 + 2.7706814e-08f;
  p = p * z2 + -2.101024e-06f;
  p = p * z2 + -5.6925064e-05f;
  p = p * z2 + -7.3499063e-04f;
  p = p * z2 + -2.9546e-03f;
  p = p * z2 + -1.6096033e-02f;
  float q = -1.4566072e-05f;
  q = q * z2 + -2.1337406e-04f;
  q = q * z2 + -1.682827e-03f;
  q = q * z2 + -7.373329e-03f;
  q = q * z2 + -1.426474e-02f;
  return 0.5f * x * (1.0f + z * p / q);
}

__global__ void k_unary(uint16_t *__restrict__ x, size_t n, int op) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    float v = h2f_e(x[i]);
    if (op == 0) {
      v = gelu_e(v);
    } else {
      float e = __expf(-fabsf(v));
      float s = e / (e + 1.0f);
      v = v > 0.0f ? 1.0f - s : s;
    }
    x[i] = f2h_e(v);
  }
}

// ---- depthwise size x size convolution (no reference implementation) ----
// NCHW: one block per 32-row band of one channel plane; the band's input
// halo is staged in LDS as floats, and each thread computes 16 outputs of
// one row from a register window, so each input value is read from HBM
// once (plus the halo) and from LDS (size + 15) / 16 times per output row.
template <int KSZ>
__global__ __launch_bounds__(256) void k_depthwise_nchw(const uint16_t *__restrict__ x, int H,
                                                        int W, int C,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ bias,
                                                        uint16_t *__restrict__ y) {
  constexpr int BR = 32, P = KSZ / 2;
  constexpr int MAXW = 256;  // widest supported row
  __shared__ float tile[(BR + KSZ - 1) * (MAXW + KSZ - 1)];
  const int bands = (H + BR - 1) / BR;
  const int c = blockIdx.x / bands, band = blockIdx.x % bands;
  const int y0 = band * BR;
  const int TW = W + KSZ - 1;
  const uint16_t *plane = x + (long)c * H * W;
  for (int e = threadIdx.x; e < (BR + KSZ - 1) * TW; e += 256) {
    int ty = e / TW, tx = e - ty * TW;
    int iy = y0 + ty - P, ix = tx - P;
    tile[e] = (iy >= 0 && iy < H && ix >= 0 && ix < W) ? h2f_e(plane[(long)iy * W + ix]) : 0.0f;
  }
  float wk[KSZ * KSZ];
#pragma unroll
  for (int t = 0; t < KSZ * KSZ; t++) wk[t] = w[t * C + c];
  const float b = bias ? bias[c] : 0.0f;
  __syncthreads();
  const int groups = (W + 15) / 16;
  for (int item = threadIdx.x; item < BR * groups; item += 256) {
    int r = item / groups, g = item - r * groups;
    int oy = y0 + r;
    if (oy >= H) continue;
    int x0 = g * 16;
    float acc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) acc[q] = b;
#pragma unroll
    for (int ky = 0; ky < KSZ; ky++) {
      float win[16 + KSZ - 1];
      const float *row = tile + (r + ky) * TW + x0;
#pragma unroll
      for (int q = 0; q < 16 + KSZ - 1; q++) win[q] = (x0 + q < TW) ? row[q] : 0.0f;
#pragma unroll
      for (int kx = 0; kx < KSZ; kx++)
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] += win[q + kx] * wk[ky * KSZ + kx];
    }
    uint16_t *out = y + (long)c * H * W + (long)oy * W + x0;
    if (x0 + 16 <= W && (((uintptr_t)out) & 15) == 0) {
      uint16_t h[16];
#pragma unroll
      for (int q = 0; q < 16; q++) h[q] = f2h_e(acc[q]);
      u32x4 v0, v1;
      __builtin_memcpy(&v0, h, 16);
      __builtin_memcpy(&v1, h + 8, 16);
      *(u32x4 *)out = v0;
      *(u32x4 *)(out + 8) = v1;
    } else {
      for (int q = 0; q < 16 && x0 + q < W; q++) out[q] = f2h_e(acc[q]);
    }
  }
}

// NHWC: one thread per (pixel, channel), channels fastest (coalesced).
__global__ void k_depthwise_nhwc(const uint16_t *__restrict__ x, int H, int W, int C,
                                 const float *__restrict__ w, int ksz,
                                 const float *__restrict__ bias, uint16_t *__restrict__ y) {
  const long total = (long)H * W * C;
  const int P = ksz / 2;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    int c = (int)(i % C);
    long p = i / C;
    int oy = (int)(p / W), ox = (int)(p % W);
    float acc = bias ? bias[c] : 0.0f;
    for (int t = 0; t < ksz * ksz; t++) {
      int iy = oy + t / ksz - P, ix = ox + t % ksz - P;
      if (iy >= 0 && iy < H && ix >= 0 && ix < W)
        acc += h2f_e(x[((long)iy * W + ix) * C + c]) * w[t * C + c];
    }
    y[i] = f2h_e(acc);
  }
}

}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_floats_to_halves(ien_ctx *ctx, const float *d_src, uint16_t *d_dst, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_src && d_dst)), IEN_ERR_INPUT, "null argument");
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_f2h, dim3(grid_for(n, 1024)), dim3(256), 0, ctx->stream, d_src, d_dst, n);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_halves_to_floats(ien_ctx *ctx, const uint16_t *d_src, float *d_dst, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_src && d_dst)), IEN_ERR_INPUT, "null argument");
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_h2f, dim3(grid_for(n, 1024)), dim3(256), 0, ctx->stream, d_src, d_dst, n);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_pixel_shuffle_add(ien_ctx *ctx, const uint16_t *d_last, size_t last_stride,
                                 const float *d_image, size_t width, size_t height,
                                 float *d_out) {
  IEN_CHECK(ctx && d_last && d_image && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(width > 0 && height > 0, IEN_ERR_INPUT, "empty %zu x %zu image", width, height);
  IEN_CHECK(last_stride >= 48, IEN_ERR_INPUT, "last layer stride %zu under 48", last_stride);
  size_t total = width * height * 16;
  hipLaunchKernelGGL(k_shuffle_add, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, d_last,
                     (long)last_stride, d_image, (int)width, (int)height, d_out);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_layer_norm(ien_ctx *ctx, uint16_t *d_x, size_t rows, size_t c, size_t stride,
                          const float *d_gamma, const float *d_beta) {
  IEN_CHECK(ctx && d_x && d_gamma && d_beta, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(c > 0 && c <= 3072 && stride >= c, IEN_ERR_INPUT, "rows of %zu values", c);
  if (rows == 0) return IEN_OK;
  hipLaunchKernelGGL(k_layer_norm, dim3(grid_for(rows, 4)), dim3(256), 0, ctx->stream, d_x,
                     (long)rows, (int)c, (long)stride, d_gamma, d_beta);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_gelu(ien_ctx *ctx, uint16_t *d_x, size_t n) {
  IEN_CHECK(ctx && (n == 0 || d_x), IEN_ERR_INPUT, "null argument");
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_unary, dim3(grid_for(n, 1024)), dim3(256), 0, ctx->stream, d_x, n, 0);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_sigmoid(ien_ctx *ctx, uint16_t *d_x, size_t n) {
  IEN_CHECK(ctx && (n == 0 || d_x), IEN_ERR_INPUT, "null argument");
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_unary, dim3(grid_for(n, 1024)), dim3(256), 0, ctx->stream, d_x, n, 1);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_depthwise(ien_ctx *ctx, const uint16_t *d_x, size_t height, size_t width,
                         size_t channels, ien_layout layout, const float *d_w, size_t size,
                         const float *d_bias, uint16_t *d_y) {
  IEN_CHECK(ctx && d_x && d_w && d_y, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(height > 0 && width > 0 && channels > 0, IEN_ERR_INPUT, "empty input");
  IEN_CHECK(size % 2 == 1 && size <= 7, IEN_ERR_INPUT, "depthwise size %zu", size);
  if (layout == IEN_LAYOUT_NCHW && size == 7 && width <= 256) {
    unsigned blocks = (unsigned)(channels * ((height + 31) / 32));
    hipLaunchKernelGGL(k_depthwise_nchw<7>, dim3(blocks), dim3(256), 0, ctx->stream, d_x,
                       (int)height, (int)width, (int)channels, d_w, d_bias, d_y);
  } else if (layout == IEN_LAYOUT_NCHW && size == 3 && width <= 256) {
    unsigned blocks = (unsigned)(channels * ((height + 31) / 32));
    hipLaunchKernelGGL(k_depthwise_nchw<3>, dim3(blocks), dim3(256), 0, ctx->stream, d_x,
                       (int)height, (int)width, (int)channels, d_w, d_bias, d_y);
  } else {
    IEN_CHECK(layout == IEN_LAYOUT_NHWC, IEN_ERR_INPUT,
              "NCHW depthwise of size %zu or rows over 256 pixels", size);
    size_t total = height * width * channels;
    hipLaunchKernelGGL(k_depthwise_nhwc, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream,
                       d_x, (int)height, (int)width, (int)channels, d_w, (int)size, d_bias, d_y);
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // extern "C"
