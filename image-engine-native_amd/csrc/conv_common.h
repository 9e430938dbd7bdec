// conv_common.h -- definitions shared by the convolution kernels
// (conv.hip: general implicit GEMM; conv_res.hip: resident weights).
#pragma once

#include <algorithm>
#include <cstring>

#include "ien_internal.h"

#pragma clang diagnostic ignored "-Winline-asm"  // m0 is written by the LDS loads

namespace ien {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct ConvArgs {
  const uint16_t *x;
  int H, W, C;
  int xs;  // NHWC: halves between pixels; NCHW: halves between planes
  int rows_mode;
  int M;  // rows_mode: number of input rows (= output pixels)
  int pad_reflect;
  int noff;
  int offy[4], offx[4];
  int OH, OW;
  int p_begin, p_end;  // output pixel range [row0, row0 + rows)
  int ty_begin, tiles_x, tiles_y, tiles_n;
  const uint16_t *wp;
  const uint16_t *zeros;  // 4 KiB of zeros: the source of padding pixels
  int KB;  // k fragments (16) of the packed weights
  int NB;  // n fragments (32), a multiple of 4
  int N;
  const float *bias;
  const float *slope;
  void *y;
  int ys;
  int out_nchw, out_f32, act, accumulate;
  // Split-K: blockIdx.y takes channel chunks [kchunks y, kchunks (y + 1)),
  // and with ksplit > 1 the launch writes raw f32 sums (no bias) to
  // y + y_index * (p_end - p_begin) * ys, NHWC; a finishing pass adds them.
  // With `part` set instead, each split writes its sums to part and counts
  // itself in on tile_count[blockIdx.x]; the tile's last split adds them
  // in split order and runs the epilogue itself (no finishing pass).
  int ksplit, kchunks;
  float *part;
  int *tile_count;
  // NHWC f16 outputs in 16-byte groups: a map (rows ys apart) added to the
  // rounded result and rounded again, or null.
  const uint16_t *add2;
  // The same outputs, whole maps, not split over K: 0, or 1 + 2 py + px to
  // write output pixel (y, x) to pixel (2 y + py, 2 x + px) of a map
  // 2 OH x 2 OW (pixels ys apart), one phase of a transposed convolution.
  int phase;
  // Tile order: 0 = output channels fastest (each XCD's band of blocks
  // covers a few pixel tiles at every channel tile), 1 = pixels fastest
  // (a band covers few channel tiles at every pixel tile: for weights
  // larger than the inputs, so each XCD's L2 fetches its share of them once).
  int n_major;
};

__device__ __forceinline__ int reflect_idx(int i, int n) {
  int last = n - 1;
  int a = i < 0 ? -i : i;
  int b = 2 * last - i;
  return a < b ? a : b;
}

// math.rs:41-75: exact GELU through erf(x) = x P(x^2) / Q(x^2) on [-4, 4]
// with Eigen's generic_fast_erf_float coefficients.
__device__ __forceinline__ float gelu_f(float x) {
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
  // q lies in [-2.40, -0.0142] on the clamped range: the hardware
  // reciprocal (1 ulp) in place of a correctly rounded division changes the
  // quotient by at most 2 ulp of f32, far below the f16 the results are
  // stored in.
  return 0.5f * x * (1.0f + z * p * __builtin_amdgcn_rcpf(q));
}

__device__ __forceinline__ float sigmoid_f(float x) {
  // math.rs:33-39: from exp(-|x|) so neither tail cancels.
  float e = __expf(-fabsf(x));
  float s = e / (e + 1.0f);
  return x > 0.0f ? 1.0f - s : s;
}

// `slope` is the PReLU slope of this value's channel.
__device__ __forceinline__ float activate(float v, int act, float slope) {
  switch (act) {
    case IEN_ACT_RELU: return v > 0.0f ? v : 0.0f;
    case IEN_ACT_PRELU: return v < 0.0f ? v * slope : v;
    case IEN_ACT_GELU: return gelu_f(v);
    case IEN_ACT_SIGMOID: return sigmoid_f(v);
    default: return v;
  }
}

// The activation as a compile-time choice (one epilogue per kernel).
template <int ACT>
__device__ __forceinline__ float act_c(float v, float slope) {
  if constexpr (ACT == IEN_ACT_RELU) return v > 0.0f ? v : 0.0f;
  else if constexpr (ACT == IEN_ACT_PRELU) {
    // v < 0 ? v slope : v as a bit select on v's sign (no compare, so no
    // mask register per value); only -0 with a negative slope differs (+0).
    // One v_bfi_b32 does the select ((m & a) | (~m & b)), which the
    // compiler otherwise spells as three instructions.
    const int m = __builtin_bit_cast(int, v) >> 31;
    int r;
    asm("v_bfi_b32 %0, %1, %2, %3"
        : "=v"(r)
        : "v"(m), "v"(__builtin_bit_cast(int, v * slope)), "v"(__builtin_bit_cast(int, v)));
    return __builtin_bit_cast(float, r);
  }
  else if constexpr (ACT == IEN_ACT_GELU) return gelu_f(v);
  else if constexpr (ACT == IEN_ACT_SIGMOID) return sigmoid_f(v);
  else return v;
}

__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) {
  _Float16 v = (_Float16)f;  // round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// XCD-aware order: block b runs on XCD b % 8; give each XCD a contiguous
// band of the logical tile order when the grid divides evenly.
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  if ((nblocks & 7) != 0) return b;
  return (b & 7) * (nblocks >> 3) + (b >> 3);
}

typedef int int4v __attribute__((ext_vector_type(4)));

// A raw buffer resource over `bytes` (< 2^31) bytes at `p`: offsets past
// the end read 0 and drop stores.
__device__ __forceinline__ int4v buffer_rsrc(const void *p, long bytes) {
  const unsigned long long a = (unsigned long long)p;
  int4v r;
  r.x = (int)(unsigned)a;
  r.y = (int)((a >> 32) & 0xffff);
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}

// The same, read from lane 0: for callers whose pointer and size the
// compiler cannot prove uniform, so that the inline assembly below gets the
// resource in SGPRs.
__device__ __forceinline__ int4v uniform_rsrc(const void *p, long bytes) {
  int4v r = buffer_rsrc(p, bytes);
  r.x = __builtin_amdgcn_readfirstlane(r.x);
  r.y = __builtin_amdgcn_readfirstlane(r.y);
  r.z = __builtin_amdgcn_readfirstlane(r.z);
  return r;
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Buffer loads straight into LDS, issued from inline assembly: lane l's
// bytes from buffer offset `off` land at LDS `wave_base` + (16 or 4) l.
// `wave_base` must be uniform.  Counted by vmcnt but invisible to the
// compiler (its own waits after such loads flush whole counters), so the
// kernel waits for them itself (wait_vm).  Loads complete in order.
__device__ __forceinline__ void dma_lds(int4v rsrc, unsigned wave_base, int off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(wave_base), "v"(off), "s"(rsrc) : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(int4v rsrc, unsigned wave_base, int off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :: "s"(wave_base), "v"(off), "s"(rsrc) : "memory", "m0");
}

// This wave's LDS accesses done (lgkmcnt(0)), then the workgroup barrier,
// without the release fence of __syncthreads, which also waits for every
// outstanding global load (vmcnt(0)) and so for the loads a pipelined
// kernel keeps in flight across the barrier.  Only for LDS handoffs:
// global stores made before it are not ordered for the other waves.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) alone.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// Global -> LDS staging, BATCH independent loads in flight per thread
// before any of them is written: with one wave per SIMD nothing else hides
// a load's latency, so a load-wait-store loop would pay it every time.
// `load(e)` must load unconditionally from a valid address (padding is
// decided in `store(e, v)`), so that no branch separates the loads.
template <int BATCH, typename Load, typename Store>
__device__ __forceinline__ void staged_copy(int total, int tid, Load load, Store store) {
  for (int base = tid; base < total; base += 256 * BATCH) {
    u32x4 v[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; b++) v[b] = load(min(base + b * 256, total - 1));
#pragma unroll
    for (int b = 0; b < BATCH; b++) {
      const int e = base + b * 256;
      if (e < total) store(e, v[b]);
    }
  }
}

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at lds + 16 l, so a wave
// fills one contiguous KiB; no register holds the data and nothing waits
// until s_waitcnt vmcnt.  `lds` must be the same for the whole wave.
__device__ __forceinline__ void dma16(const void *src, void *lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

// conv.hip: the pass after a split-K product -- the ksplit f32 partial sums
// of `rows` x a.N outputs (rows `pitch` floats apart, split z after z rows
// x pitch, in the context's workspace) added in order, then bias, old
// output when accumulating and activation into a.y.
ien_status splitk_finish(ien_ctx *ctx, int ksplit, long rows, int pitch, const ConvArgs &a);

// rows.hip: products over rows (1 x 1, NHWC f16 in and out) with K a
// multiple of 32, N of 8, 16-byte aligned rows and enough tiles to fill
// the chip.
bool rows_supported(const ConvArgs &a, long rows);
ien_status launch_rows(ien_ctx *ctx, const ConvArgs &a);

// conv_res.hip: the resident-weight kernel for NHWC inputs of 16, 32 or 64
// channels with k x k (k = 1, 3) zero-padded taps and K = k k C <= 640.
bool resident_supported(int ks, int stride, int c, int nchw, int reflect, int noff, int rows_mode,
                        long in_bytes);
ien_status launch_resident(ien_ctx *ctx, ConvArgs a, int ks);

// conv_small.hip: NHWC convolutions of 4 input channels (dense taps x
// channels K) and of 64 input channels into N outputs with N x ks <= 32
// ((output, kx) pairs as the MFMA rows); stride 1, zero or reflect padding,
// whole output images.
bool narrow_supported(const ConvArgs &a, int ks, int stride, int nchw, int noff, int rows_mode);
ien_status launch_narrow(ien_ctx *ctx, ConvArgs a, int ks);
bool few_supported(const ConvArgs &a, int ks, int stride, int nchw, int noff, int rows_mode);
ien_status launch_few(ien_ctx *ctx, ConvArgs a, int ks);

// conv_nchw.hip: 1x1 products of whole NCHW f16 planes into NCHW f16
// planes (pixels a multiple of 8, 16-byte aligned planes), not accumulating.
bool nchw1_supported(const ConvArgs &a, int ks, int stride, long rows);
ien_status launch_nchw1(ien_ctx *ctx, const ConvArgs &a);
// The same file: zero-padded 3x3 convolutions of 64 NCHW f16 channels into
// 64, and of 128 into 128 (whole maps, widths a multiple of 8), not
// accumulating.
bool nchw3_supported(const ConvArgs &a, int ks, int stride, long rows);
ien_status launch_nchw3(ien_ctx *ctx, const ConvArgs &a);
bool nchw3q_supported(const ConvArgs &a, int ks, int stride, long rows);
ien_status launch_nchw3q(ien_ctx *ctx, const ConvArgs &a);

}  // namespace ien
