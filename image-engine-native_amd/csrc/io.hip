// io.hip -- 8-bit image I/O of the models' Model::run entry points, on the
// device: to_float / to_byte (realesrgan-native lib.rs:292-300, the same in
// scunet-native lib.rs), LaMa's mask binarisation and the compositing that
// keeps the known pixels (lama-native lib.rs:138-155), and BiRefNet's
// ImageNet normalisation (birefnet-native lib.rs:111-116).
//
// Every pass is HBM-bound and trivially parallel: a thread takes quads of 4
// consecutive values (4 bytes, one 16-byte float access), 4 quads a step,
// 256 quads apart, so that each wave instruction reads or writes one
// contiguous run and each thread has 4 loads in flight; a scalar path
// covers the ragged end and unaligned pointers.

#include <cmath>

#include "ien_internal.h"

namespace ien {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

unsigned grid_for16(size_t n) {
  size_t g = (n + 16 * 256 - 1) / (16 * 256);
  if (g < 1) g = 1;
  if (g > (1u << 20)) g = 1u << 20;
  return (unsigned)g;
}

bool aligned16(const void *a, const void *b) {
  return ((((uintptr_t)a) | ((uintptr_t)b)) & 15) == 0;
}

// lib.rs:292-295 to_float: f32::from(v) / 255.0 (correctly rounded).
__device__ __forceinline__ float to_float(uint8_t v) { return (float)v / 255.0f; }

// lib.rs:297-300 to_byte: (v.clamp(0, 1) * 255).round() as u8 -- rounding
// half away from zero; a NaN saturates to 0 as Rust's `as u8` does.
__device__ __forceinline__ uint8_t to_byte(float v) {
  if (!(v == v)) return 0;
  const float c = fminf(fmaxf(v, 0.0f), 1.0f);
  return (uint8_t)roundf(c * 255.0f);
}

typedef uint8_t byte4 __attribute__((ext_vector_type(4)));

// The quads of n values: load(q) for the 4 quads of a step first, then
// put(q, loaded) (q < n / 4); then the last n % 4 values one by one
// (tail(j), block 0).
template <typename V, typename Load, typename Put, typename Tail>
__device__ __forceinline__ void quads(size_t n, Load load, Put put, Tail tail) {
  const size_t nq = n / 4;
  for (size_t b = (size_t)blockIdx.x * 1024; b < nq; b += (size_t)gridDim.x * 1024) {
    V v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const size_t q = b + threadIdx.x + 256 * k;
      if (q < nq) v[k] = load(q);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const size_t q = b + threadIdx.x + 256 * k;
      if (q < nq) put(q, v[k]);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n % 4) tail(4 * nq + threadIdx.x);
}

// Every value one by one (pointers not aligned for the quads).
template <typename F>
__device__ __forceinline__ void singles(size_t n, F f) {
  for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < n;
       j += (size_t)gridDim.x * blockDim.x)
    f(j);
}

__global__ void k_bytes_to_floats(const uint8_t *__restrict__ src, float *__restrict__ dst,
                                  size_t n, int vec) {
  auto one = [&](size_t j) { dst[j] = to_float(src[j]); };
  if (!vec) return singles(n, one);
  quads<byte4>(
      n, [&](size_t q) { return *(const byte4 *)(src + 4 * q); },
      [&](size_t q, byte4 b) {
        *(float4v *)(dst + 4 * q) = float4v{to_float(b[0]), to_float(b[1]), to_float(b[2]), to_float(b[3])};
      },
      one);
}

__global__ void k_floats_to_bytes(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                  size_t n, int vec) {
  auto one = [&](size_t j) { dst[j] = to_byte(src[j]); };
  if (!vec) return singles(n, one);
  quads<float4v>(
      n, [&](size_t q) { return *(const float4v *)(src + 4 * q); },
      [&](size_t q, float4v f) {
        *(byte4 *)(dst + 4 * q) = byte4{to_byte(f[0]), to_byte(f[1]), to_byte(f[2]), to_byte(f[3])};
      },
      one);
}

// lama-native lib.rs:142: f32::from(u8::from(m != 0)).
__global__ void k_mask_bytes(const uint8_t *__restrict__ src, float *__restrict__ dst, size_t n,
                             int vec) {
  auto bit = [](uint8_t m) { return m ? 1.0f : 0.0f; };
  auto one = [&](size_t j) { dst[j] = bit(src[j]); };
  if (!vec) return singles(n, one);
  quads<byte4>(
      n, [&](size_t q) { return *(const byte4 *)(src + 4 * q); },
      [&](size_t q, byte4 b) { *(float4v *)(dst + 4 * q) = float4v{bit(b[0]), bit(b[1]), bit(b[2]), bit(b[3])}; },
      one);
}

// birefnet-native lib.rs:113-116: (f32::from(v) / 255.0 - MEAN[c]) / STD[c]
// for colour c = value index mod 3 of interleaved RGB, in f32.
struct Stats {
  float mean[3], std[3];
};

__device__ __forceinline__ float normalized(uint8_t v, int c, const Stats &s) {
  return (to_float(v) - s.mean[c]) / s.std[c];
}

__global__ void k_normalize_bytes(const uint8_t *__restrict__ src, float *__restrict__ dst,
                                  size_t n, Stats s, int vec) {
  auto one = [&](size_t j) { dst[j] = normalized(src[j], (int)(j % 3), s); };
  if (!vec) return singles(n, one);
  quads<byte4>(
      n, [&](size_t q) { return *(const byte4 *)(src + 4 * q); },
      [&](size_t q, byte4 b) {
        int c = (int)((4 * q) % 3);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[e] = normalized(b[e], c, s);
          c = c == 2 ? 0 : c + 1;
        }
        *(float4v *)(dst + 4 * q) = float4v{v[0], v[1], v[2], v[3]};
      },
      one);
}

// lama-native lib.rs:147-155: the known pixels keep their bytes, the holes
// (mask byte not 0) take the prediction as bytes.  Values of interleaved
// RGB: value i belongs to pixel i / 3.
struct Composite {
  byte4 rgb;
  float4v pred;
};

__global__ void k_composite_bytes(const uint8_t *__restrict__ rgb, const uint8_t *__restrict__ mask,
                                  const float *__restrict__ pred, uint8_t *__restrict__ out,
                                  size_t n, int vec) {
  auto one = [&](size_t j) { out[j] = mask[j / 3] ? to_byte(pred[j]) : rgb[j]; };
  if (!vec) return singles(n, one);
  quads<Composite>(
      n,
      [&](size_t q) { return Composite{*(const byte4 *)(rgb + 4 * q), *(const float4v *)(pred + 4 * q)}; },
      [&](size_t q, Composite c) {
        byte4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = mask[(4 * q + e) / 3] ? to_byte(c.pred[e]) : c.rgb[e];
        *(byte4 *)(out + 4 * q) = o;
      },
      one);
}

}  // namespace

// Host launchers shared with the model drivers.
ien_status bytes_to_floats(ien_ctx *ctx, const uint8_t *src, float *dst, size_t n) {
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_bytes_to_floats, dim3(grid_for16(n)), dim3(256), 0, ctx->stream, src, dst,
                     n, (int)aligned16(src, dst));
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status floats_to_bytes(ien_ctx *ctx, const float *src, uint8_t *dst, size_t n) {
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_floats_to_bytes, dim3(grid_for16(n)), dim3(256), 0, ctx->stream, src, dst,
                     n, (int)aligned16(src, dst));
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status mask_bytes(ien_ctx *ctx, const uint8_t *src, float *dst, size_t n) {
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_mask_bytes, dim3(grid_for16(n)), dim3(256), 0, ctx->stream, src, dst, n,
                     (int)aligned16(src, dst));
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status normalize_bytes(ien_ctx *ctx, const uint8_t *src, size_t pixels, const float mean[3],
                           const float deviation[3], float *dst) {
  const size_t n = pixels * 3;
  if (n == 0) return IEN_OK;
  Stats s;
  for (int c = 0; c < 3; c++) {
    s.mean[c] = mean[c];
    s.std[c] = deviation[c];
  }
  hipLaunchKernelGGL(k_normalize_bytes, dim3(grid_for16(n)), dim3(256), 0, ctx->stream, src, dst,
                     n, s, (int)aligned16(src, dst));
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status composite_bytes(ien_ctx *ctx, const uint8_t *rgb, const uint8_t *mask,
                           const float *pred, size_t pixels, uint8_t *out) {
  const size_t n = pixels * 3;
  if (n == 0) return IEN_OK;
  const bool vec = aligned16(rgb, out) && aligned16(pred, pred);
  hipLaunchKernelGGL(k_composite_bytes, dim3(grid_for16(n)), dim3(256), 0, ctx->stream, rgb, mask,
                     pred, out, n, (int)vec);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_bytes_to_floats(ien_ctx *ctx, const uint8_t *d_src, float *d_dst, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_src && d_dst)), IEN_ERR_INPUT, "null argument");
  return bytes_to_floats(ctx, d_src, d_dst, n);
}

ien_status ien_floats_to_bytes(ien_ctx *ctx, const float *d_src, uint8_t *d_dst, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_src && d_dst)), IEN_ERR_INPUT, "null argument");
  return floats_to_bytes(ctx, d_src, d_dst, n);
}

ien_status ien_mask_bytes(ien_ctx *ctx, const uint8_t *d_mask, float *d_dst, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_mask && d_dst)), IEN_ERR_INPUT, "null argument");
  return mask_bytes(ctx, d_mask, d_dst, n);
}

ien_status ien_normalize_bytes(ien_ctx *ctx, const uint8_t *d_rgb, size_t pixels,
                               const float mean[3], const float deviation[3], float *d_dst) {
  IEN_CHECK(ctx && mean && deviation && (pixels == 0 || (d_rgb && d_dst)), IEN_ERR_INPUT,
            "null argument");
  return normalize_bytes(ctx, d_rgb, pixels, mean, deviation, d_dst);
}

ien_status ien_composite_bytes(ien_ctx *ctx, const uint8_t *d_rgb, const uint8_t *d_mask,
                               const float *d_pred, size_t pixels, uint8_t *d_out) {
  IEN_CHECK(ctx && (pixels == 0 || (d_rgb && d_mask && d_pred && d_out)), IEN_ERR_INPUT,
            "null argument");
  return composite_bytes(ctx, d_rgb, d_mask, d_pred, pixels, d_out);
}

}  // extern "C"
