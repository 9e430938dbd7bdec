// resample.hip -- the memory-bound resampling passes: align-corners
// bilinear resize (crates/birefnet-native/src/decoder.rs:436-522), the
// model-input padding (scunet-native network.rs:356-379, lama-native
// network.rs:336-370) and the crop back to the image.

#include "conv_common.h"

namespace ien {
namespace {

// decoder.rs:467-488 axis: taps and weights of one output coordinate.
struct Tap {
  int i0, i1;
  float d1, d2;  // distance to i0 (the weight of i1), to i1 (the weight of i0)
};

__device__ __forceinline__ Tap axis_tap(int out, int len_in, int len_out) {
  float pos = len_out == 1 ? 0.0f : (float)out * (float)(len_in - 1) / (float)(len_out - 1);
  pos = fminf(fmaxf(pos, 0.0f), (float)(len_in - 1));
  Tap t;
  t.i0 = (int)pos;
  t.i1 = min(t.i0 + 1, len_in - 1);
  if (t.i0 == t.i1) {
    t.d1 = 0.5f;
    t.d2 = 0.5f;
  } else {
    t.d1 = fabsf(pos - (float)t.i0);
    t.d2 = fabsf(pos - (float)t.i1);
  }
  return t;
}

struct ResizeArgs {
  const uint16_t *src;
  int sh, sw;
  long sstride;
  int c;
  void *dst;
  int dh, dw;
  long dstride;
  int out_f32, add;
};

__device__ __forceinline__ void put(const ResizeArgs &a, long at, float v) {
  if (a.out_f32) {
    float *d = (float *)a.dst + at;
    *d = a.add ? *d + v : v;
  } else {
    uint16_t *d = (uint16_t *)a.dst + at;
    *d = f2h(a.add ? h2f(*d) + v : v);
  }
}

// One thread per output pixel and 8-channel chunk: four 16-byte loads, the
// blend in f32, one 16-byte store of halves or two of floats (with the old
// values loaded the same way when adding).  32-bit indexing (the host
// checks the item count), the output type and the add fixed per instance.
template <bool F32, bool ADD>
__global__ __launch_bounds__(256) void k_resize8(ResizeArgs a, int per, int items) {
  const int item = blockIdx.x * 256 + threadIdx.x;
  if (item >= items) return;
  const int pix = item / per, k = item - pix * per;
  const int y = pix / a.dw, x = pix - y * a.dw;
  const Tap ty = axis_tap(y, a.sh, a.dh), tx = axis_tap(x, a.sw, a.dw);
  const float w11 = tx.d2 * ty.d2, w21 = tx.d1 * ty.d2, w12 = tx.d2 * ty.d1, w22 = tx.d1 * ty.d1;
  const int ss = (int)a.sstride;
  const uint16_t *s0 = a.src + (ty.i0 * a.sw) * ss + 8 * k, *s1 = a.src + (ty.i1 * a.sw) * ss + 8 * k;
  const u32x4 r11 = *(const u32x4 *)(s0 + tx.i0 * ss), r21 = *(const u32x4 *)(s0 + tx.i1 * ss);
  const u32x4 r12 = *(const u32x4 *)(s1 + tx.i0 * ss), r22 = *(const u32x4 *)(s1 + tx.i1 * ss);
  const long out = (long)pix * a.dstride + 8 * k;
  float old[8] = {};
  if constexpr (ADD) {
    if constexpr (F32) {
      const float4v o0 = *(const float4v *)((const float *)a.dst + out);
      const float4v o1 = *(const float4v *)((const float *)a.dst + out + 4);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        old[e] = o0[e];
        old[4 + e] = o1[e];
      }
    } else {
      const u32x4 o = *(const u32x4 *)((const uint16_t *)a.dst + out);
      uint16_t h[8];
      __builtin_memcpy(h, &o, 16);
#pragma unroll
      for (int e = 0; e < 8; e++) old[e] = h2f(h[e]);
    }
  }
  uint16_t h11[8], h21[8], h12[8], h22[8];
  __builtin_memcpy(h11, &r11, 16);
  __builtin_memcpy(h21, &r21, 16);
  __builtin_memcpy(h12, &r12, 16);
  __builtin_memcpy(h22, &r22, 16);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float b = w11 * h2f(h11[e]) + w21 * h2f(h21[e]) + w12 * h2f(h12[e]) + w22 * h2f(h22[e]);
    v[e] = ADD ? old[e] + b : b;
  }
  if constexpr (F32) {
    *(float4v *)((float *)a.dst + out) = float4v{v[0], v[1], v[2], v[3]};
    *(float4v *)((float *)a.dst + out + 4) = float4v{v[4], v[5], v[6], v[7]};
  } else {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = f2h(v[e]);
    u32x4 w;
    __builtin_memcpy(&w, o, 16);
    *(u32x4 *)((uint16_t *)a.dst + out) = w;
  }
}

// One thread per output pixel and 8-channel chunk (VEC) or channel.
template <bool VEC>
__global__ __launch_bounds__(256) void k_resize(ResizeArgs a) {
  const int per = VEC ? a.c / 8 : a.c;
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  if (item >= (long)a.dh * a.dw * per) return;
  const long pix = item / per;
  const int k = (int)(item - pix * per);
  const int y = (int)(pix / a.dw), x = (int)(pix - (long)y * a.dw);
  const Tap ty = axis_tap(y, a.sh, a.dh), tx = axis_tap(x, a.sw, a.dw);
  const float w11 = tx.d2 * ty.d2, w21 = tx.d1 * ty.d2, w12 = tx.d2 * ty.d1, w22 = tx.d1 * ty.d1;
  const long p11 = ((long)ty.i0 * a.sw + tx.i0) * a.sstride, p21 = ((long)ty.i0 * a.sw + tx.i1) * a.sstride;
  const long p12 = ((long)ty.i1 * a.sw + tx.i0) * a.sstride, p22 = ((long)ty.i1 * a.sw + tx.i1) * a.sstride;
  const long out = pix * a.dstride;
  if constexpr (VEC) {
    float v11[8], v21[8], v12[8], v22[8];
    auto ld = [&](long p, float *v) {
      const u32x4 raw = *(const u32x4 *)(a.src + p + 8 * k);
      uint16_t h[8];
      __builtin_memcpy(h, &raw, 16);
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = h2f(h[e]);
    };
    ld(p11, v11);
    ld(p21, v21);
    ld(p12, v12);
    ld(p22, v22);
#pragma unroll
    for (int e = 0; e < 8; e++)
      put(a, out + 8 * k + e, w11 * v11[e] + w21 * v21[e] + w12 * v12[e] + w22 * v22[e]);
  } else {
    const float v = w11 * h2f(a.src[p11 + k]) + w21 * h2f(a.src[p21 + k]) +
                    w12 * h2f(a.src[p12 + k]) + w22 * h2f(a.src[p22 + k]);
    put(a, out + k, v);
  }
}

// One thread per padded pixel.
__global__ __launch_bounds__(256) void k_pad_image(int mode, const float *__restrict__ image,
                                                   const float *__restrict__ mask, int width,
                                                   int height, int pw, int ph,
                                                   uint16_t *__restrict__ out, long stride) {
  const long pix = (long)blockIdx.x * 256 + threadIdx.x;
  if (pix >= (long)ph * pw) return;
  const int y = (int)(pix / pw), x = (int)(pix - (long)y * pw);
  uint16_t *o = out + pix * stride;
  if (mode == IEN_PAD_REPLICATE) {
    const long p = (long)min(y, height - 1) * width + min(x, width - 1);
#pragma unroll
    for (int ch = 0; ch < 3; ch++) o[ch] = f2h(image[p * 3 + ch]);
  } else {
    const int sy = y < height ? y : 2 * height - 1 - y;
    const int sx = x < width ? x : 2 * width - 1 - x;
    const long p = (long)sy * width + sx;
    const float m = mask[p];
#pragma unroll
    for (int ch = 0; ch < 3; ch++) o[ch] = f2h(image[p * 3 + ch] * (1.0f - m));
    o[3] = f2h(m);
  }
}

__global__ __launch_bounds__(256) void k_crop(const uint16_t *__restrict__ map, int map_width,
                                              long stride, int width, int height, int channels,
                                              float *__restrict__ out) {
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  if (item >= (long)height * width * channels) return;
  const long pix = item / channels;
  const int ch = (int)(item - pix * channels);
  const int y = (int)(pix / width), x = (int)(pix - (long)y * width);
  out[item] = h2f(map[((long)y * map_width + x) * stride + ch]);
}

// 2 x 2 gather: one thread per output row and 8-channel chunk of one of
// the four pixels.
__global__ __launch_bounds__(256) void k_gather_2x2(const uint16_t *__restrict__ map, int h2,
                                                    int w2, int width, int c, long stride,
                                                    int col_major, uint16_t *__restrict__ rows) {
  const int chunks = c >> 3;
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  if (item >= (long)h2 * w2 * 4 * chunks) return;
  const long r = item / (4 * chunks);
  const int rest = (int)(item - r * 4 * chunks), q = rest / chunks, k = rest - q * chunks;
  const int yy = 2 * (int)(r / w2), xx = 2 * (int)(r - (r / w2) * w2);
  const int dy = col_major ? (q & 1) : (q >> 1), dx = col_major ? (q >> 1) : (q & 1);
  *(u32x4 *)(rows + (r * 4 + q) * c + 8 * k) =
      *(const u32x4 *)(map + ((long)(yy + dy) * width + xx + dx) * stride + 8 * k);
}

// 2 x 2 scatter: one thread per input pixel, sub-pixel and 8-channel chunk.
__global__ __launch_bounds__(256) void k_scatter_2x2(const uint16_t *__restrict__ rows,
                                                     long row_stride, int h, int w, int c,
                                                     uint16_t *__restrict__ map, long stride) {
  const int chunks = c >> 3;
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  if (item >= (long)h * w * 4 * chunks) return;
  const long r = item / (4 * chunks);
  const int rest = (int)(item - r * 4 * chunks), q = rest / chunks, k = rest - q * chunks;
  const int y = (int)(r / w), x = (int)(r - (r / w) * w);
  const long pixel = (long)(2 * y + (q >> 1)) * (2 * w) + 2 * x + (q & 1);
  *(u32x4 *)(map + pixel * stride + 8 * k) = *(const u32x4 *)(rows + r * row_stride + q * c + 8 * k);
}

// x += y, 8 halves per thread (a scalar tail).
__global__ __launch_bounds__(256) void k_add(uint16_t *__restrict__ x,
                                             const uint16_t *__restrict__ y, long n) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    u32x4 a = *(const u32x4 *)(x + i), b = *(const u32x4 *)(y + i);
    uint16_t ha[8], hb[8];
    __builtin_memcpy(ha, &a, 16);
    __builtin_memcpy(hb, &b, 16);
#pragma unroll
    for (int e = 0; e < 8; e++) ha[e] = f2h(h2f(ha[e]) + h2f(hb[e]));
    __builtin_memcpy(&a, ha, 16);
    *(u32x4 *)(x + i) = a;
  } else {
    for (long j = i; j < n; j++) x[j] = f2h(h2f(x[j]) + h2f(y[j]));
  }
}

unsigned grid256(long items) { return (unsigned)((items + 255) / 256); }

bool a16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_resize(ien_ctx *ctx, const uint16_t *d_src, size_t sh, size_t sw, size_t src_stride,
                      size_t c, void *d_dst, size_t dh, size_t dw, size_t dst_stride,
                      ien_out_type out_type, int add) {
  IEN_CHECK(ctx && d_src && d_dst, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(sh >= 1 && sw >= 1 && dh >= 1 && dw >= 1 && c >= 1, IEN_ERR_INPUT,
            "resize %zu x %zu -> %zu x %zu of %zu channels", sh, sw, dh, dw, c);
  IEN_CHECK(src_stride >= c && dst_stride >= c, IEN_ERR_INPUT, "strides below the channels");
  IEN_CHECK(out_type == IEN_OUT_F16 || out_type == IEN_OUT_F32, IEN_ERR_INPUT, "output type");
  IEN_CHECK(sh < (1u << 30) && sw < (1u << 30) && dh < (1u << 30) && dw < (1u << 30),
            IEN_ERR_INPUT, "sides");
  ResizeArgs a{d_src, (int)sh, (int)sw, (long)src_stride, (int)c, d_dst, (int)dh, (int)dw,
               (long)dst_stride, out_type == IEN_OUT_F32, add != 0};
  const bool vec = c % 8 == 0 && src_stride % 8 == 0 && ((uintptr_t)d_src & 15) == 0;
  const long items = (long)dh * dw * (vec ? c / 8 : c);
  if (items == 0) return IEN_OK;
  // Whole 16-byte stores: the output aligned and its pixels whole chunks
  // apart; every index in 32 bits.
  const size_t osize = out_type == IEN_OUT_F32 ? 4 : 2;
  const bool store16 = vec && ((uintptr_t)d_dst & 15) == 0 && (dst_stride * osize) % 16 == 0 &&
                       sh * sw * src_stride < (1u << 31) && items < (1L << 31);
  if (store16) {
    const int per = (int)(c / 8), n = (int)items;
    const dim3 grid(grid256(items)), block(256);
    auto kernel = out_type == IEN_OUT_F32 ? (add ? k_resize8<true, true> : k_resize8<true, false>)
                                          : (add ? k_resize8<false, true> : k_resize8<false, false>);
    hipLaunchKernelGGL(kernel, grid, block, 0, ctx->stream, a, per, n);
  } else if (vec)
    hipLaunchKernelGGL(k_resize<true>, dim3(grid256(items)), dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(k_resize<false>, dim3(grid256(items)), dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_pad_image(ien_ctx *ctx, ien_pad_mode mode, const float *d_image,
                         const float *d_mask, size_t width, size_t height, size_t multiple,
                         uint16_t *d_out, size_t stride) {
  IEN_CHECK(ctx && d_image && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(mode == IEN_PAD_REPLICATE || (mode == IEN_PAD_SYMMETRIC_MASKED && d_mask),
            IEN_ERR_INPUT, "pad mode %d (the symmetric mode needs the mask)", (int)mode);
  IEN_CHECK(width >= 1 && height >= 1 && multiple >= 1 && width < (1u << 30) &&
                height < (1u << 30),
            IEN_ERR_INPUT, "image %zu x %zu, multiple %zu", width, height, multiple);
  const size_t ph = (height + multiple - 1) / multiple * multiple;
  const size_t pw = (width + multiple - 1) / multiple * multiple;
  const size_t channels = mode == IEN_PAD_REPLICATE ? 3 : 4;
  IEN_CHECK(stride >= channels, IEN_ERR_INPUT, "stride %zu below %zu channels", stride, channels);
  // Mirroring reflects at most a whole side.
  IEN_CHECK(mode == IEN_PAD_REPLICATE || (ph - height <= height && pw - width <= width),
            IEN_ERR_INPUT, "image %zu x %zu too small to mirror to %zu x %zu", width, height, pw,
            ph);
  hipLaunchKernelGGL(k_pad_image, dim3(grid256((long)(ph * pw))), dim3(256), 0, ctx->stream,
                     (int)mode, d_image, d_mask, (int)width, (int)height, (int)pw, (int)ph, d_out,
                     (long)stride);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_crop(ien_ctx *ctx, const uint16_t *d_map, size_t map_width, size_t stride,
                    size_t width, size_t height, size_t channels, float *d_out) {
  IEN_CHECK(ctx && d_map && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(width >= 1 && height >= 1 && channels >= 1 && width <= map_width &&
                stride >= channels && width < (1u << 30) && height < (1u << 30),
            IEN_ERR_INPUT, "crop %zu x %zu x %zu of a map %zu wide", width, height, channels,
            map_width);
  hipLaunchKernelGGL(k_crop, dim3(grid256((long)(height * width * channels))), dim3(256), 0,
                     ctx->stream, d_map, (int)map_width, (long)stride, (int)width, (int)height,
                     (int)channels, d_out);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_gather_2x2(ien_ctx *ctx, const uint16_t *d_map, size_t height, size_t width,
                          size_t c, size_t stride, ien_order order, uint16_t *d_rows) {
  IEN_CHECK(ctx && d_map && d_rows, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(height >= 2 && width >= 2 && height % 2 == 0 && width % 2 == 0 && height < (1u << 30) &&
                width < (1u << 30),
            IEN_ERR_INPUT, "2 x 2 gather of a %zu x %zu map", width, height);
  IEN_CHECK(c >= 8 && c % 8 == 0 && stride >= c && stride % 8 == 0 && a16(d_map) && a16(d_rows),
            IEN_ERR_INPUT, "%zu channels, stride %zu (multiples of 8, 16-byte aligned)", c, stride);
  IEN_CHECK(order == IEN_ORDER_ROW_MAJOR || order == IEN_ORDER_COLUMN_MAJOR, IEN_ERR_INPUT,
            "order %d", (int)order);
  const long items = (long)(height / 2) * (width / 2) * 4 * (c / 8);
  hipLaunchKernelGGL(k_gather_2x2, dim3(grid256(items)), dim3(256), 0, ctx->stream, d_map,
                     (int)(height / 2), (int)(width / 2), (int)width, (int)c, (long)stride,
                     order == IEN_ORDER_COLUMN_MAJOR ? 1 : 0, d_rows);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_scatter_2x2(ien_ctx *ctx, const uint16_t *d_rows, size_t row_stride,
                           size_t height, size_t width, size_t c, uint16_t *d_map,
                           size_t stride) {
  IEN_CHECK(ctx && d_rows && d_map, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(height >= 1 && width >= 1 && height < (1u << 29) && width < (1u << 29), IEN_ERR_INPUT,
            "2 x 2 scatter of a %zu x %zu grid", width, height);
  IEN_CHECK(c >= 8 && c % 8 == 0 && row_stride >= 4 * c && row_stride % 8 == 0 && stride >= c &&
                stride % 8 == 0 && a16(d_map) && a16(d_rows),
            IEN_ERR_INPUT, "%zu channels, strides %zu / %zu", c, row_stride, stride);
  const long items = (long)height * width * 4 * (c / 8);
  hipLaunchKernelGGL(k_scatter_2x2, dim3(grid256(items)), dim3(256), 0, ctx->stream, d_rows,
                     (long)row_stride, (int)height, (int)width, (int)c, d_map, (long)stride);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_add(ien_ctx *ctx, uint16_t *d_x, const uint16_t *d_y, size_t n) {
  IEN_CHECK(ctx && (n == 0 || (d_x && d_y)), IEN_ERR_INPUT, "null argument");
  IEN_CHECK(a16(d_x) && a16(d_y), IEN_ERR_INPUT, "alignment (16 bytes)");
  if (n == 0) return IEN_OK;
  hipLaunchKernelGGL(k_add, dim3(grid256((long)((n + 7) / 8))), dim3(256), 0, ctx->stream, d_x,
                     d_y, (long)n);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // extern "C"
