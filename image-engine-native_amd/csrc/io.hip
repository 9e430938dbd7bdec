// io.hip -- 8-bit image I/O of the models' Model::run entry points, on the
// device: to_float / to_byte (realesrgan-native lib.rs:292-300, the same in
// scunet-native lib.rs), LaMa's mask binarisation and the compositing that
// keeps the known pixels (lama-native lib.rs:138-155), and BiRefNet's
// ImageNet normalisation (birefnet-native lib.rs:111-116).
//
// Every pass is HBM-bound and trivially parallel: a thread owns 16
// consecutive bytes (one 16-byte load or store) and the floats they map to
// (four 16-byte accesses), with a scalar path for a ragged end or
// unaligned pointers.

#include <cmath>

#include "ien_internal.h"

namespace ien {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint8_t byte16 __attribute__((ext_vector_type(16)));

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

__global__ void k_bytes_to_floats(const uint8_t *__restrict__ src, float *__restrict__ dst,
                                  size_t n, int vec) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < n;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (vec && i + 16 <= n) {
      const byte16 b = *(const byte16 *)(src + i);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float4v f = {to_float(b[4 * q]), to_float(b[4 * q + 1]), to_float(b[4 * q + 2]),
                     to_float(b[4 * q + 3])};
        *(float4v *)(dst + i + 4 * q) = f;
      }
    } else {
      for (size_t j = i; j < n && j < i + 16; j++) dst[j] = to_float(src[j]);
    }
  }
}

__global__ void k_floats_to_bytes(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                  size_t n, int vec) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < n;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (vec && i + 16 <= n) {
      float4v f[4];
#pragma unroll
      for (int q = 0; q < 4; q++) f[q] = *(const float4v *)(src + i + 4 * q);
      byte16 b;
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) b[4 * q + e] = to_byte(f[q][e]);
      *(byte16 *)(dst + i) = b;
    } else {
      for (size_t j = i; j < n && j < i + 16; j++) dst[j] = to_byte(src[j]);
    }
  }
}

// lama-native lib.rs:142: f32::from(u8::from(m != 0)).
__global__ void k_mask_bytes(const uint8_t *__restrict__ src, float *__restrict__ dst, size_t n,
                             int vec) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < n;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (vec && i + 16 <= n) {
      const byte16 b = *(const byte16 *)(src + i);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float4v f = {b[4 * q] ? 1.0f : 0.0f, b[4 * q + 1] ? 1.0f : 0.0f,
                     b[4 * q + 2] ? 1.0f : 0.0f, b[4 * q + 3] ? 1.0f : 0.0f};
        *(float4v *)(dst + i + 4 * q) = f;
      }
    } else {
      for (size_t j = i; j < n && j < i + 16; j++) dst[j] = src[j] ? 1.0f : 0.0f;
    }
  }
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
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < n;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (vec && i + 16 <= n) {
      const byte16 b = *(const byte16 *)(src + i);
      int c = (int)(i % 3);
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        v[e] = normalized(b[e], c, s);
        c = c == 2 ? 0 : c + 1;
      }
#pragma unroll
      for (int q = 0; q < 4; q++)
        *(float4v *)(dst + i + 4 * q) = float4v{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
      for (size_t j = i; j < n && j < i + 16; j++) dst[j] = normalized(src[j], (int)(j % 3), s);
    }
  }
}

// lama-native lib.rs:147-155: the known pixels keep their bytes, the holes
// (mask byte not 0) take the prediction as bytes.  Values of interleaved
// RGB: value i belongs to pixel i / 3.
__global__ void k_composite_bytes(const uint8_t *__restrict__ rgb, const uint8_t *__restrict__ mask,
                                  const float *__restrict__ pred, uint8_t *__restrict__ out,
                                  size_t n, int vec) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < n;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (vec && i + 16 <= n) {
      const byte16 b = *(const byte16 *)(rgb + i);
      float4v f[4];
#pragma unroll
      for (int q = 0; q < 4; q++) f[q] = *(const float4v *)(pred + i + 4 * q);
      byte16 o;
#pragma unroll
      for (int e = 0; e < 16; e++)
        o[e] = mask[(i + e) / 3] ? to_byte(f[e / 4][e % 4]) : b[e];
      *(byte16 *)(out + i) = o;
    } else {
      for (size_t j = i; j < n && j < i + 16; j++) out[j] = mask[j / 3] ? to_byte(pred[j]) : rgb[j];
    }
  }
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
