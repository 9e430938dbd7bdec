// elementwise.hip -- the memory-bound passes around the products:
// half conversions (half.rs), LayerNorm / GELU / sigmoid (math.rs), the
// Real-ESRGAN pixel shuffle with the repeated input (realesrgan-native
// network.rs:115-141, shaders/shuffle.comp) and the depthwise convolution.
//
// All of them are HBM-bound: each thread moves 16-byte vectors where the
// layout allows, rows are reduced within one wave64 (no LDS round trip),
// and grids are sized to the work, not to the CU count.

#include "ien_internal.h"
#include "lanes.h"

namespace ien {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

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

// The same sums a workgroup per run of up to 64 input pixels of one row:
// their 48-half records come in as 16-byte loads (staged in LDS), each
// thread (pixel, sub-row i) builds its 12 output floats into the LDS copy
// of the 4 output rows (4 x 3 KiB), and those go out as 16-byte stores,
// consecutive threads on consecutive chunks of a row.  Grid: x over runs
// of 64 pixels, y over input rows.  Needs 16-byte aligned pixel records
// and output.
constexpr int SHUF_PX = 64;
__global__ __launch_bounds__(256) void k_shuffle_add16(const uint16_t *__restrict__ last,
                                                       long last_stride,
                                                       const float *__restrict__ image, int width,
                                                       float *__restrict__ out) {
  __shared__ uint4 rec[SHUF_PX * 6];          // 48 halves a pixel
  __shared__ float4v rows[4 * SHUF_PX * 3];   // 4 rows of 4 SHUF_PX pixels x RGB
  const int t = threadIdx.x, y = blockIdx.y, x0 = blockIdx.x * SHUF_PX;
  const int n = min(SHUF_PX, width - x0);  // pixels in this run
  const long p0 = (long)y * width + x0;
  for (int q = t; q < n * 6; q += 256)
    rec[q] = *(const uint4 *)(last + (p0 + q / 6) * last_stride + 8 * (q % 6));
  __syncthreads();
  {
    const int px = t >> 2, i = t & 3;
    if (px < n) {
      const uint16_t *h = (const uint16_t *)(rec + px * 6);
      const float im[3] = {image[3 * (p0 + px)], image[3 * (p0 + px) + 1],
                           image[3 * (p0 + px) + 2]};
      float v[12];
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int c = 0; c < 3; c++) v[3 * j + c] = h2f_e(h[16 * c + 4 * i + j]) + im[c];
#pragma unroll
      for (int k = 0; k < 3; k++)
        rows[(i * SHUF_PX + px) * 3 + k] = float4v{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
    }
  }
  __syncthreads();
  for (int q = t; q < 4 * n * 3; q += 256) {
    const int i = q / (3 * n), c = q - i * 3 * n;
    *(float4v *)(out + 12L * width * (4L * y + i) + 12L * x0 + 4 * c) = rows[i * SHUF_PX * 3 + c];
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
  sum = group_sum<64>(sum);
  const float mean = sum / (float)c;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXV; k++) {
    int idx = lane + 64 * k;
    float d = idx < c ? v[k] - mean : 0.0f;
    sq += d * d;
  }
  sq = group_sum<64>(sq);
  const float inv = 1.0f / sqrtf(sq / (float)c + 1e-5f);
#pragma unroll
  for (int k = 0; k < MAXV; k++) {
    int idx = lane + 64 * k;
    if (idx < c) r[idx] = f2h_e((v[k] - mean) * inv * gamma[idx] + beta[idx]);
  }
}

// The same with L lanes per row (a power of two, at most 64) and Q chunks
// of 8 channels per lane, 16-byte loads and stores: rows of 8-aligned
// channels at 8-aligned strides.  A lane's gamma and beta are requested
// with its row, so their latency overlaps the row's.  The reductions stay
// inside the row's aligned lane group.
// Rows are read from `src` (sstride apart) and written to x (stride
// apart); the two may be the same rows (in place).  With g2w > 0 row r is
// instead the 2 x 2 pixel group (2 (r / g2w) + dy, 2 (r % g2w) + dx) of a
// map 2 g2w wide (pixels sstride apart, c / 4 channels each), in
// column-major order: channel block q = dy + 2 dx (ien_gather_2x2's
// column-major rows, gathered as they are read).
template <int L, int Q>
__global__ __launch_bounds__(256) void k_layer_norm_vec(const uint16_t *src, long sstride,
                                                        uint16_t *x, long rows, int c, long stride,
                                                        const float *__restrict__ gamma,
                                                        const float *__restrict__ beta, int g2w) {
  const int sub = threadIdx.x & (L - 1);
  const long row = ((long)blockIdx.x * 256 + threadIdx.x) / L;
  if (row >= rows) return;  // whole lane groups leave together
  const uint16_t *rs = src + row * sstride;
  uint16_t *r = x + row * stride;
  // Chunk k of the row (8 channels).
  auto chunk_at = [&](int k) -> const uint16_t * {
    if (g2w == 0) return rs + 8 * k;
    const int qc = (c >> 5), q = k / qc, kk = k - q * qc;  // c / 4 channels a block
    const long ry = row / g2w, rx = row - ry * g2w;
    const long pixel = (2 * ry + (q & 1)) * (2L * g2w) + 2 * rx + (q >> 1);
    return src + pixel * sstride + 8 * kk;
  };
  const int chunks = c >> 3;
  float v[8 * Q];
  float4 g[2 * Q], b[2 * Q];
  u32x4 raw[Q];
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int k = min(sub + L * q, chunks - 1);  // (lanes past the row repeat its last chunk)
    raw[q] = *(const u32x4 *)chunk_at(k);
    g[2 * q] = *(const float4 *)(gamma + 8 * k);
    g[2 * q + 1] = *(const float4 *)(gamma + 8 * k + 4);
    b[2 * q] = *(const float4 *)(beta + 8 * k);
    b[2 * q + 1] = *(const float4 *)(beta + 8 * k + 4);
  }
  float sum = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int k = sub + L * q;
    if (k < chunks) {
      uint16_t h[8];
      __builtin_memcpy(h, &raw[q], 16);
#pragma unroll
      for (int e = 0; e < 8; e++) v[8 * q + e] = h2f_e(h[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) v[8 * q + e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) sum += v[8 * q + e];
  }
  sum = group_sum<L>(sum);
  const float mean = sum / (float)c;
  float sq = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; q++)
    if (sub + L * q < chunks) {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = v[8 * q + e] - mean;
        sq += d * d;
      }
    }
  sq = group_sum<L>(sq);
  const float inv = 1.0f / sqrtf(sq / (float)c + 1e-5f);
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int k = sub + L * q;
    if (k < chunks) {
      const float4 g0 = g[2 * q], g1 = g[2 * q + 1], b0 = b[2 * q], b1 = b[2 * q + 1];
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; e++) h[e] = f2h_e((v[8 * q + e] - mean) * inv * gg[e] + bb[e]);
      u32x4 raw;
      __builtin_memcpy(&raw, h, 16);
      *(u32x4 *)(r + 8 * k) = raw;
    }
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
// NCHW: one block per 32-row band of one channel plane (rows up to 256).
//  - The band plus its halo rows go to LDS as f32 with KSZ / 2 zero columns
//    each side: every thread first issues all of its 16-byte loads
//    (addresses clamped into the plane, padding decided at the store), then
//    converts and stores them.
//  - Each thread computes a 4 x 4 block of outputs: for each of the
//    4 + KSZ - 1 input rows it reads 4 + KSZ - 1 floats once and does the
//    4 x KSZ multiply-adds of that row per output row; the weights are
//    uniform per block (scalar registers).
template <int KSZ, bool VEC>
__global__ __launch_bounds__(256) void k_depthwise_nchw(const uint16_t *__restrict__ x, int H,
                                                        int W, int C,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ bias,
                                                        uint16_t *__restrict__ y) {
  constexpr int BR = 32, P = KSZ / 2, MAXW = 256;
  constexpr int TH = BR + KSZ - 1;             // tile rows
  constexpr int TW = MAXW + KSZ - 1 + 1;       // tile pitch (floats), odd: banks spread
  __shared__ float tile[TH * TW];
  const int bands = (H + BR - 1) / BR;
  const int c = blockIdx.x / bands, band = blockIdx.x - c * bands;
  const int y0 = band * BR;
  const uint16_t *plane = x + (long)c * H * W;

  // Stage: rows y0 - P .. y0 + BR + P - 1 of the plane, 8 pixels per item
  // (VEC: rows of whole 16-byte groups) or one.
  if constexpr (VEC) {
    const int chunks = W / 8;
    const int items = TH * chunks;
    constexpr int PER = (TH * (MAXW / 8) + 255) / 256;
    u32x4 raw[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int e = min(threadIdx.x + 256 * k, items - 1);
      const int ty = e / chunks, ch = e - ty * chunks;
      const int iy = min(max(y0 + ty - P, 0), H - 1);
      raw[k] = *(const u32x4 *)(plane + (long)iy * W + 8 * ch);
    }
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int e = threadIdx.x + 256 * k;
      if (e >= items) break;
      const int ty = e / chunks, ch = e - ty * chunks;
      const int iy = y0 + ty - P;
      const bool row_ok = iy >= 0 && iy < H;
      uint16_t h[8];
      __builtin_memcpy(h, &raw[k], 16);
      float *dst = tile + ty * TW + P + 8 * ch;
#pragma unroll
      for (int q = 0; q < 8; q++) dst[q] = row_ok ? h2f_e(h[q]) : 0.0f;
    }
  } else {
    for (int e = threadIdx.x; e < TH * W; e += 256) {
      const int ty = e / W, xx = e - ty * W;
      const int iy = y0 + ty - P;
      tile[ty * TW + P + xx] = iy >= 0 && iy < H ? h2f_e(plane[(long)iy * W + xx]) : 0.0f;
    }
  }
  // Zero columns left and right of the plane's row (P each).
  for (int e = threadIdx.x; e < TH * 2 * P; e += 256) {
    const int ty = e / (2 * P), q = e - ty * 2 * P;
    tile[ty * TW + (q < P ? q : W + q)] = 0.0f;
  }
  float wk[KSZ * KSZ];
#pragma unroll
  for (int t = 0; t < KSZ * KSZ; t++) wk[t] = w[t * C + c];
  const float b = bias ? bias[c] : 0.0f;
  __syncthreads();

  // Compute: 4 x 4 output blocks, (BR / 4) x (W / 4) of them.
  const int gx = (W + 3) / 4;
  for (int item = threadIdx.x; item < (BR / 4) * gx; item += 256) {
    const int r0 = 4 * (item / gx), x0 = 4 * (item - (item / gx) * gx);
    if (y0 + r0 >= H) continue;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = b;
#pragma unroll
    for (int ry = 0; ry < 4 + KSZ - 1; ry++) {
      float win[4 + KSZ - 1];
      const float *row = tile + (r0 + ry) * TW + x0;
#pragma unroll
      for (int q = 0; q < 4 + KSZ - 1; q++) win[q] = row[q];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int ky = ry - i;
        if (ky < 0 || ky >= KSZ) continue;
#pragma unroll
        for (int kx = 0; kx < KSZ; kx++)
#pragma unroll
          for (int j = 0; j < 4; j++) acc[i][j] += win[j + kx] * wk[ky * KSZ + kx];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int oy = y0 + r0 + i;
      if (oy >= H) break;
      uint16_t *out = y + (long)c * H * W + (long)oy * W + x0;
      if (VEC && x0 + 4 <= W) {
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = f2h_e(acc[i][j]);
        uint2 v;
        __builtin_memcpy(&v, h, 8);
        *(uint2 *)out = v;
      } else {
        for (int j = 0; j < 4 && x0 + j < W; j++) out[j] = f2h_e(acc[i][j]);
      }
    }
  }
}

// NCHW depthwise on MFMA, for rows of a multiple of 32 pixels (<= 256):
// per channel and kernel row ky, the 1-D convolution of an input row is a
// banded (Toeplitz) product, so a 32 x 32 output tile (32 rows y, 32
// columns x from x0) is
//   out[y][x] = sum_ky sum_{j < 48} in[y + ky - P][x0 - 8 + j] T_ky[j][x],
//   T_ky[j][x] = w[ky][j - 8 - x + P] (zero outside the kernel),
// 3 v_mfma_f32_32x32x16_f16 per ky: A = the input rows (16-byte reads of the
// f16 band staged in LDS, 8 zero columns left and 16 right), B = T_ky in
// registers (the weights rounded to f16; products are exact and sums f32).
// The B fragments depend on the lane's column only: each block puts its
// channel's 49 weights in LDS (loaded in the same batch as the input band:
// one memory latency per block), spreads them into a zero-padded band per
// ky, and every lane reads its 8 values of T_ky[16 s + 8 h + i][x] from
// there.  The 8 values start at any half, so the band is kept in 8 copies
// shifted by one half each: the lane reads copy (start mod 8) at a 16-byte
// aligned address (unaligned LDS reads stall).  A block covers 32 rows, one
// tile per wave.  C lane l holds column
// x = l % 32 (coalesced 2-byte stores), register r row 8 (r / 4) + 4 (l / 32)
// + r % 4.  Wave w takes columns 32 w .. 32 w + 31.
template <int KSZ>
__global__ __launch_bounds__(512) void k_depthwise_mfma(const uint16_t *__restrict__ x, int H,
                                                        int W, int C,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ bias,
                                                        uint16_t *__restrict__ y) {
  constexpr int P = KSZ / 2, BR = 32, TH = BR + KSZ - 1, MAXW = 256;
  constexpr int WB = 96, WOFF = 40;  // weight band: T value at kx sits at kx + WOFF
  constexpr int BATCH = 8;           // loads in flight per thread (covers TH rows of MAXW)
  __shared__ __attribute__((aligned(16))) uint16_t tile[TH * (MAXW + 24)];
  __shared__ __attribute__((aligned(16))) uint16_t wband[8 * KSZ * WB];
  __shared__ float wl[KSZ * KSZ];
  const int pitch = W + 24;  // halves; input column x sits at x + 8
  const int bands = (H + BR - 1) / BR;
  const int c = blockIdx.x / bands, band = blockIdx.x - c * bands, y0 = band * BR;
  const uint16_t *plane = x + (long)c * H * W;
  const int nt = blockDim.x;

  // Stage rows y0 - P .. y0 + BR + P - 1, 16-byte chunks (chunk k of an LDS
  // row is input columns 8 k - 8 .. 8 k - 1), and the weights: all loads of
  // a thread first, from clamped addresses, zeros decided at the store.
  const int chunks = pitch / 8, items = TH * chunks;
  const float wmine = w[min((int)threadIdx.x, KSZ * KSZ - 1) * C + c];
  for (int base = threadIdx.x; base < items; base += BATCH * nt) {
    u32x4 raw[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; b++) {
      const int e = min(base + b * nt, items - 1);
      const int ty = e / chunks, k = e - ty * chunks;
      const int iy = min(max(y0 + ty - P, 0), H - 1);
      const int ix = min(max(8 * k - 8, 0), W - 8);
      raw[b] = *(const u32x4 *)(plane + (long)iy * W + ix);
    }
#pragma unroll
    for (int b = 0; b < BATCH; b++) {
      const int e = base + b * nt;
      if (e >= items) break;
      const int ty = e / chunks, k = e - ty * chunks;
      const int iy = y0 + ty - P;
      const bool ok = iy >= 0 && iy < H && k >= 1 && 8 * k <= W;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      *(u32x4 *)(tile + ty * pitch + 8 * k) = ok ? raw[b] : zero;
    }
  }
  if (threadIdx.x < KSZ * KSZ) wl[threadIdx.x] = wmine;
  const float b = bias ? bias[c] : 0.0f;
  __syncthreads();
  // The weight band (kx outside the kernel: zero), every entry of every
  // copy written, 8 per thread and item: copy k holds at t the band value of
  // t + k.
  for (int e = threadIdx.x; e < KSZ * WB; e += nt) {  // e = (k, ky, 8-entry group)
    const int k = e / (KSZ * WB / 8), rest = e - k * (KSZ * WB / 8);
    const int ky = rest / (WB / 8), q = rest - ky * (WB / 8);
    const int kx0 = 8 * q + k - WOFF;
    uint16_t h[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int kx = kx0 + j;
      h[j] = f2h_e(kx >= 0 && kx < KSZ ? wl[ky * KSZ + min(max(kx, 0), KSZ - 1)] : 0.0f);
    }
    u32x4 v;
    __builtin_memcpy(&v, h, 16);
    *(u32x4 *)(wband + (k * KSZ + ky) * WB + 8 * q) = v;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
  const int x0 = 32 * (threadIdx.x >> 6);
  // B fragments: element i of step s is T_ky at kx = 16 s + 8 h + i - 8 - x + P.
  half8 tb[KSZ][3];
#pragma unroll
  for (int ky = 0; ky < KSZ; ky++)
#pragma unroll
    for (int s = 0; s < 3; s++) {
      const int t0 = WOFF + 16 * s + 8 * hf - 8 - l32 + P;  // 1 + P .. 79 + P
      const int k = t0 & 7;
      tb[ky][s] = *(const half8 *)(wband + (k * KSZ + ky) * WB + (t0 - k));
    }

  uint16_t *out = y + (long)c * H * W + x0 + l32;
  const bool full = y0 + BR <= H;
#pragma unroll
  for (int t = 0; t < BR / 32; t++) {
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = b;
#pragma unroll
    for (int ky = 0; ky < KSZ; ky++)
#pragma unroll
      for (int s = 0; s < 3; s++) {
        const half8 a =
            *(const half8 *)(tile + (32 * t + l32 + ky) * pitch + x0 + 16 * s + 8 * hf);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, tb[ky][s], acc, 0, 0, 0);
      }
    if (full) {
#pragma unroll
      for (int r = 0; r < 16; r++)
        out[(long)(y0 + 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3)) * W] = f2h_e(acc[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int oy = y0 + 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (oy < H) out[(long)oy * W] = f2h_e(acc[r]);
      }
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
  IEN_CHECK(width < (1u << 28) && height < (1u << 28), IEN_ERR_INPUT, "image of %zu x %zu",
            width, height);
  if (last_stride % 8 == 0 && (((uintptr_t)d_last | (uintptr_t)d_out) & 15) == 0 &&
      height <= 65535) {  // input rows on the grid's y
    const dim3 grid((unsigned)((width + SHUF_PX - 1) / SHUF_PX), (unsigned)height);
    hipLaunchKernelGGL(k_shuffle_add16, grid, dim3(256), 0, ctx->stream, d_last, (long)last_stride,
                       d_image, (int)width, d_out);
  } else {
    size_t total = width * height * 16;
    hipLaunchKernelGGL(k_shuffle_add, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, d_last,
                       (long)last_stride, d_image, (int)width, (int)height, d_out);
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_layer_norm(ien_ctx *ctx, uint16_t *d_x, size_t rows, size_t c, size_t stride,
                          const float *d_gamma, const float *d_beta) {
  IEN_CHECK(ctx && d_x && d_gamma && d_beta, IEN_ERR_INPUT, "null argument");
  return layer_norm_to(ctx, d_x, stride, d_x, stride, rows, c, d_gamma, d_beta, 0);
}

}  // extern "C"

namespace ien {

ien_status layer_norm_to(ien_ctx *ctx, const uint16_t *d_src, size_t sstride, uint16_t *d_x,
                         size_t stride, size_t rows, size_t c, const float *d_gamma,
                         const float *d_beta, int gather_w2) {
  IEN_CHECK(c > 0 && c <= 3072 && stride >= c && sstride >= (gather_w2 ? c / 4 : c),
            IEN_ERR_INPUT, "rows of %zu values", c);
  if (rows == 0) return IEN_OK;
  const bool vec = c % 8 == 0 && stride % 8 == 0 && sstride % 8 == 0 &&
                   (((uintptr_t)d_x | (uintptr_t)d_src) & 15) == 0 &&
                   ((uintptr_t)d_gamma & 15) == 0 && ((uintptr_t)d_beta & 15) == 0;
  IEN_CHECK(vec || (d_src == d_x && gather_w2 == 0), IEN_ERR_INPUT,
            "LayerNorm into other rows: 8-aligned channels and strides, 16-byte aligned rows");
  IEN_CHECK(gather_w2 >= 0 && (gather_w2 == 0 || (c % 32 == 0 && rows % gather_w2 == 0)),
            IEN_ERR_INPUT, "2 x 2 groups of %zu channels over %zu rows", c, rows);
  if (vec) {
    // Lanes: the largest power of two dividing the chunks (no idle lanes)
    // when that leaves at most 3 chunks a lane, else the chunks rounded up
    // to a power of two (at most 64 lanes, up to 6 chunks each).
    const int chunks = (int)(c / 8);
    int lanes = std::min(chunks & -chunks, 64), q = (chunks + lanes - 1) / lanes;
    if (q > 3) {
      lanes = 1;
      while (lanes < chunks && lanes < 64) lanes *= 2;
      q = (chunks + lanes - 1) / lanes;  // at most 6 (c <= 3072)
    }
    const size_t threads = rows * (size_t)lanes;
    const dim3 grid((unsigned)((threads + 255) / 256));
    using K = void (*)(const uint16_t *, long, uint16_t *, long, int, long, const float *,
                       const float *, int);
    static const K table[7][3] = {
        {k_layer_norm_vec<1, 1>, k_layer_norm_vec<1, 2>, k_layer_norm_vec<1, 3>},
        {k_layer_norm_vec<2, 1>, k_layer_norm_vec<2, 2>, k_layer_norm_vec<2, 3>},
        {k_layer_norm_vec<4, 1>, k_layer_norm_vec<4, 2>, k_layer_norm_vec<4, 3>},
        {k_layer_norm_vec<8, 1>, k_layer_norm_vec<8, 2>, k_layer_norm_vec<8, 3>},
        {k_layer_norm_vec<16, 1>, k_layer_norm_vec<16, 2>, k_layer_norm_vec<16, 3>},
        {k_layer_norm_vec<32, 1>, k_layer_norm_vec<32, 2>, k_layer_norm_vec<32, 3>},
        {k_layer_norm_vec<64, 1>, k_layer_norm_vec<64, 2>, k_layer_norm_vec<64, 3>}};
    int level = 0;
    while ((1 << level) < lanes) level++;
    const K k = q <= 3 ? table[level][q - 1] : k_layer_norm_vec<64, 6>;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, ctx->stream, d_src, (long)sstride, d_x, (long)rows,
                       (int)c, (long)stride, d_gamma, d_beta, gather_w2);
    IEN_HIP(hipGetLastError());
    return IEN_OK;
  }
  hipLaunchKernelGGL(k_layer_norm, dim3(grid_for(rows, 4)), dim3(256), 0, ctx->stream, d_x,
                     (long)rows, (int)c, (long)stride, d_gamma, d_beta);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien

extern "C" {

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
  // The band kernel: 16-byte loads and 8-byte stores for rows of a multiple
  // of 8 pixels in 16-byte aligned planes, element by element otherwise.
  const bool bands = layout == IEN_LAYOUT_NCHW && width <= 256 && (size == 7 || size == 3);
  const bool vec = width % 8 == 0 && ((uintptr_t)d_x & 15) == 0 && ((uintptr_t)d_y & 7) == 0;
  if (bands && vec && width % 32 == 0) {
    // Toeplitz products on MFMA: one wave per 32 columns of a 32-row band.
    unsigned blocks = (unsigned)(channels * ((height + 31) / 32));
    hipLaunchKernelGGL(size == 7 ? k_depthwise_mfma<7> : k_depthwise_mfma<3>, dim3(blocks),
                       dim3((unsigned)(2 * width)), 0, ctx->stream, d_x, (int)height, (int)width,
                       (int)channels, d_w, d_bias, d_y);
  } else if (bands) {
    void (*k)(const uint16_t *, int, int, int, const float *, const float *, uint16_t *) =
        size == 7 ? (vec ? k_depthwise_nchw<7, true> : k_depthwise_nchw<7, false>)
                  : (vec ? k_depthwise_nchw<3, true> : k_depthwise_nchw<3, false>);
    unsigned blocks = (unsigned)(channels * ((height + 31) / 32));
    hipLaunchKernelGGL(k, dim3(blocks), dim3(256), 0, ctx->stream, d_x, (int)height, (int)width,
                       (int)channels, d_w, d_bias, d_y);
  } else {
    IEN_CHECK(layout == IEN_LAYOUT_NHWC, IEN_ERR_INPUT,
              "NCHW depthwise of size %zu, rows over 256 pixels or not a multiple of 8", size);
    size_t total = height * width * channels;
    hipLaunchKernelGGL(k_depthwise_nhwc, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream,
                       d_x, (int)height, (int)width, (int)channels, d_w, (int)size, d_bias, d_y);
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // extern "C"
