// conv.hip -- convolution and dense products as implicit GEMM on gfx950
// f16 MFMA (v_mfma_f32_32x32x16_f16) with f32 accumulation.
//
// Replaces the reference's matrix product (crates/native-engine/src/gemm.rs
// multiply, every conv and linear layer of the CPU path) and its Vulkan
// shaders (realesrgan-native shaders/conv_*.comp, scunet-native
// shaders/conv3.comp and gemm*.comp, lama-native shaders/conv*.comp,
// birefnet-native shaders/gemm*.comp).
//
// Shape of the GEMM: M = output pixels (row-major), N = output channels,
// K = taps x input channels, taps outer and channels inner (gemm.rs:
// "the reduction runs over taps in order, channels within each").
//
// One workgroup = 4 wave64s computes a TR x TC tile of output pixels for
// BN = 32 * NBW * NSPLIT output channels.  Per chunk of CK input channels it
// stages the tile's input halo ((TR-1) S + KS) x ((TC-1) S + KS) pixels in
// LDS, NHWC with a padded pixel stride (CK + 8 halves) so the A-fragment
// reads (16 bytes per lane, 32 consecutive pixels) hit distinct banks, then
// walks taps x 16-channel steps: A fragments from LDS (one ds_read_b128 per
// lane), B fragments straight from the packed weights in global memory
// (L2-resident, one 16-byte load per lane, prefetched a step ahead), one
// MFMA per (M-block, N-block).  The epilogue stages f32 results per wave in
// LDS and writes 16-byte vectors: bias, the old output when accumulating,
// then the activation, as gemm.rs:583-666 orders them.
//
// Block ids are remapped so that each XCD (blocks are dealt round-robin to
// the 8 XCDs) gets a contiguous band of tiles: neighbouring tiles share halo
// rows, which then stay in that XCD's L2.

#include <cstring>

#include "ien_internal.h"

namespace ien {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct ConvArgs {
  const uint16_t *x;
  int H, W, C;
  long xs;
  int rows_mode;
  long M;  // rows_mode: number of input rows (= output pixels)
  int pad_reflect;
  int noff;
  int offy[4], offx[4];
  int OH, OW;
  long p_begin, p_end;  // output pixel range [row0, row0 + rows)
  int ty_begin, tiles_x, tiles_y, tiles_n;
  const uint16_t *wp;
  int KB;  // k fragments (16) of the packed weights
  int NB;  // n fragments (32), a multiple of 4
  int N;
  const float *bias;
  const float *slope;
  void *y;
  long ys;
  int out_nchw, out_f32, act, accumulate;
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
  return 0.5f * x * (1.0f + z * p / q);
}

__device__ __forceinline__ float sigmoid_f(float x) {
  // math.rs:33-39: from exp(-|x|) so neither tail cancels.
  float e = __expf(-fabsf(x));
  float s = e / (e + 1.0f);
  return x > 0.0f ? 1.0f - s : s;
}

__device__ __forceinline__ float activate(float v, int act, const float *slope, int n) {
  switch (act) {
    case IEN_ACT_RELU: return v > 0.0f ? v : 0.0f;
    case IEN_ACT_PRELU: return v < 0.0f ? v * slope[n] : v;
    case IEN_ACT_GELU: return gelu_f(v);
    case IEN_ACT_SIGMOID: return sigmoid_f(v);
    default: return v;
  }
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

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW>
struct ConvCfg {
  static constexpr int NSPLIT = 4 / MSPLIT;
  static constexpr int BN = 32 * NBW * NSPLIT;
  static constexpr int MB = TR * TC / 32;       // M-blocks per tile
  static constexpr int MBW = MB / MSPLIT;       // M-blocks per wave
  static constexpr int EXT = KS == 0 ? 2 : KS;  // offset taps read one pixel on
  static constexpr int HR = (TR - 1) * S + EXT;
  static constexpr int HC = (TC - 1) * S + EXT;
  static constexpr int CKP = VEC ? CK + 8 : CK;  // LDS halves per halo pixel
  static constexpr int HALO_HALVES = HR * HC * CKP;
  static constexpr int STAGE_FLOATS = 4 * MBW * 32 * 36;  // 4 waves x (MBW*32 px) x (32+4)
  static constexpr int LDS_BYTES =
      HALO_HALVES * 2 > STAGE_FLOATS * 4 ? HALO_HALVES * 2 : STAGE_FLOATS * 4;
  static_assert(MB % MSPLIT == 0, "M-blocks must split evenly over waves");
  static_assert(TC % 32 == 0, "tile columns are whole M-blocks");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW>
__global__ __launch_bounds__(256) void conv_mfma(ConvArgs a) {
  using Cfg = ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW>;
  constexpr int HR = Cfg::HR, HC = Cfg::HC, CKP = Cfg::CKP, MBW = Cfg::MBW;
  constexpr int P = KS == 0 ? 0 : KS / 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[Cfg::LDS_BYTES];
  uint16_t *halo = (uint16_t *)lds_raw;

  const int nblocks = gridDim.x;
  const int bid = xcd_remap(blockIdx.x, nblocks);
  const int tn = bid % a.tiles_n;
  const int t = bid / a.tiles_n;
  const int tx = t % a.tiles_x;
  const int ty = t / a.tiles_x + a.ty_begin;
  const int oy0 = ty * TR, ox0 = tx * TC;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int mg = wave % MSPLIT, ng = wave / MSPLIT;
  const int nblk0 = tn * (Cfg::BN / 32) + ng * NBW;  // first 32-channel block of this wave
  const int T = KS == 0 ? a.noff : KS * KS;

  floatx16 acc[MBW][NBW];
#pragma unroll
  for (int i = 0; i < MBW; i++)
#pragma unroll
    for (int j = 0; j < NBW; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  // Halo origin in input pixels.
  const int iy0 = oy0 * S - P, ix0 = ox0 * S - P;

  // Offset of input pixel (iy, ix), or -1 for a zero (padding, outside).
  auto resolve = [&](int iy, int ix) -> long {
    if (a.rows_mode) {
      long r = (long)iy * a.W + ix;
      if (iy < 0 || ix < 0 || ix >= a.W || r >= a.M) return -1;
      return r * a.xs;
    }
    if (iy < 0 || iy >= a.H || ix < 0 || ix >= a.W) {
      if (!a.pad_reflect || KS == 0) return -1;
      // Clamped as well: halo pixels that feed no stored output may lie
      // further out than one reflection reaches, and must stay in bounds.
      iy = min(max(reflect_idx(iy, a.H), 0), a.H - 1);
      ix = min(max(reflect_idx(ix, a.W), 0), a.W - 1);
    }
    long p = (long)iy * a.W + ix;
    return IN_NCHW ? p : p * a.xs;
  };

  for (int c0 = 0; c0 < a.C; c0 += CK) {
    const int cc = min(CK, a.C - c0);
    __syncthreads();
    // ---- global -> LDS: the halo of this channel chunk ----
    if (VEC && !IN_NCHW) {
      const int vpp = cc >> 3;  // 16-byte vectors per pixel
      const int total = HR * HC * vpp;
      for (int e = tid; e < total; e += 256) {
        int hp = e / vpp, v = e - hp * vpp;
        int hy = hp / HC, hx = hp - hy * HC;
        long off = resolve(iy0 + hy, ix0 + hx);
        u32x4 val = {0u, 0u, 0u, 0u};
        if (off >= 0) val = *(const u32x4 *)(a.x + off + c0 + 8 * v);
        *(u32x4 *)(halo + hp * CKP + 8 * v) = val;
      }
    } else if (!IN_NCHW) {
      const int total = HR * HC * cc;
      for (int e = tid; e < total; e += 256) {
        int hp = e / cc, c = e - hp * cc;
        int hy = hp / HC, hx = hp - hy * HC;
        long off = resolve(iy0 + hy, ix0 + hx);
        halo[hp * CKP + c] = off >= 0 ? a.x[off + c0 + c] : (uint16_t)0;
      }
    } else {
      // NCHW: pixels fastest, so neighbouring lanes read neighbouring halves.
      const int total = HR * HC * cc;
      for (int e = tid; e < total; e += 256) {
        int c = e / (HR * HC), hp = e - c * (HR * HC);
        int hy = hp / HC, hx = hp - hy * HC;
        long off = resolve(iy0 + hy, ix0 + hx);
        halo[hp * CKP + c] = off >= 0 ? a.x[(long)(c0 + c) * a.xs + off] : (uint16_t)0;
      }
    }
    __syncthreads();

    // ---- MFMA over taps x 16-channel steps of this chunk ----
    if (VEC) {
      const int kcs = cc >> 4;
      const int steps = T * kcs;
      const uint16_t *wbase = a.wp + (long)lane * 8;
      auto kb_of = [&](int s) {
        int tap = s / kcs, kc = s - tap * kcs;
        return (tap * a.C + c0) / 16 + kc;
      };
      half8 bcur[NBW], bnext[NBW];
#pragma unroll
      for (int j = 0; j < NBW; j++)
        bcur[j] = *(const half8 *)(wbase + ((long)(nblk0 + j) * a.KB + kb_of(0)) * 512);
      for (int s = 0; s < steps; s++) {
        if (s + 1 < steps) {
          int kbn = kb_of(s + 1);
#pragma unroll
          for (int j = 0; j < NBW; j++)
            bnext[j] = *(const half8 *)(wbase + ((long)(nblk0 + j) * a.KB + kbn) * 512);
        }
        const int tap = s / kcs, kc = s - tap * kcs;
        int dy, dx;
        if constexpr (KS == 0) {
          dy = a.offy[tap];
          dx = a.offx[tap];
        } else {
          dy = tap / KS;
          dx = tap - dy * KS;
        }
        half8 av[MBW];
#pragma unroll
        for (int i = 0; i < MBW; i++) {
          const int mb = mg * MBW + i;
          const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (lane & 31);
          const int hp = (r * S + dy) * HC + cx * S + dx;
          av[i] = *(const half8 *)(halo + hp * CKP + kc * 16 + 8 * (lane >> 5));
        }
#pragma unroll
        for (int i = 0; i < MBW; i++)
#pragma unroll
          for (int j = 0; j < NBW; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bcur[j], acc[i][j], 0, 0, 0);
        if (s + 1 < steps) {
#pragma unroll
          for (int j = 0; j < NBW; j++) bcur[j] = bnext[j];
        }
      }
    } else {
      // Small channel counts (one chunk holds them all): K flattened over
      // (tap, channel) as the reference orders it, 16 at a time.
      const int K = T * cc;
      const int kbs = (K + 15) / 16;
      for (int kb = 0; kb < kbs; kb++) {
        half8 bv[NBW];
#pragma unroll
        for (int j = 0; j < NBW; j++)
          bv[j] = *(const half8 *)(a.wp + ((long)(nblk0 + j) * a.KB + kb) * 512 + lane * 8);
        half8 av[MBW];
#pragma unroll
        for (int i = 0; i < MBW; i++) {
          const int mb = mg * MBW + i;
          const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (lane & 31);
#pragma unroll
          for (int q = 0; q < 8; q++) {
            int k = kb * 16 + 8 * (lane >> 5) + q;
            uint16_t hv = 0;
            if (k < K) {
              int tap = k / cc, c = k - tap * cc;
              int dy, dx;
              if constexpr (KS == 0) {
                dy = a.offy[tap];
                dx = a.offx[tap];
              } else {
                dy = tap / KS;
                dx = tap - dy * KS;
              }
              hv = halo[((r * S + dy) * HC + cx * S + dx) * CKP + c];
            }
            _Float16 f;
            __builtin_memcpy(&f, &hv, 2);
            av[i][q] = f;
          }
        }
#pragma unroll
        for (int i = 0; i < MBW; i++)
#pragma unroll
          for (int j = 0; j < NBW; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: stage per wave in LDS, then 8 outputs per lane ----
  __syncthreads();
  float *stage = (float *)lds_raw + wave * (MBW * 32 * 36);
#pragma unroll
  for (int j = 0; j < NBW; j++) {
    const int nbase = (nblk0 + j) * 32;
    if (nbase >= a.N) break;  // wave-uniform
    // C fragment: lane holds column n = lane % 32 and rows
    // 8 (r / 4) + 4 (lane / 32) + r % 4 of each 32x32 block.
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int m = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        stage[(i * 32 + m) * 36 + (lane & 31)] = acc[i][j][r];
      }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const int g = lane & 3;  // 8-channel group
    const int n = nbase + 8 * g;
    for (int q = lane >> 2; q < MBW * 32; q += 16) {
      const int mb = mg * MBW + q / 32;
      const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (q & 31);
      const int oy = oy0 + r, ox = ox0 + cx;
      long p = (long)oy * a.OW + ox;
      bool valid = oy < a.OH && ox < a.OW && p >= a.p_begin && p < a.p_end;
      if (!valid || n >= a.N) continue;
      const long rel = p - a.p_begin;
      float v[8];
      const float4v s0 = *(const float4v *)(stage + q * 36 + 8 * g);
      const float4v s1 = *(const float4v *)(stage + q * 36 + 8 * g + 4);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[e] = s0[e];
        v[4 + e] = s1[e];
      }
      const int nv = min(8, a.N - n);
      if (!a.out_nchw) {
        const long base = rel * a.ys + n;
        if (a.out_f32) {
          float *yo = (float *)a.y + base;
#pragma unroll
          for (int e = 0; e < 8; e++)
            if (e < nv) {
              float o = v[e] + a.bias[n + e];
              if (a.accumulate) o += yo[e];
              yo[e] = activate(o, a.act, a.slope, n + e);
            }
        } else {
          uint16_t *yo = (uint16_t *)a.y + base;
          const bool vec = nv == 8 && (((uintptr_t)yo & 15) == 0);
          uint16_t old[8];
          if (a.accumulate) {
            if (vec) {
              u32x4 ov = *(const u32x4 *)yo;
              __builtin_memcpy(old, &ov, 16);
            } else {
              for (int e = 0; e < nv; e++) old[e] = yo[e];
            }
          }
          uint16_t outv[8];
#pragma unroll
          for (int e = 0; e < 8; e++) {
            float o = v[e] + a.bias[min(n + e, a.N - 1)];
            if (a.accumulate && e < nv) o += h2f(old[e]);
            outv[e] = f2h(activate(o, a.act, a.slope, min(n + e, a.N - 1)));
          }
          if (vec) {
            u32x4 ov;
            __builtin_memcpy(&ov, outv, 16);
            *(u32x4 *)yo = ov;
          } else {
            for (int e = 0; e < nv; e++) yo[e] = outv[e];
          }
        }
      } else {
        // NCHW: channel planes `ys` apart.
        for (int e = 0; e < nv; e++) {
          const long at = (long)(n + e) * a.ys + rel;
          float o = v[e] + a.bias[n + e];
          if (a.out_f32) {
            float *yo = (float *)a.y + at;
            if (a.accumulate) o += *yo;
            *yo = activate(o, a.act, a.slope, n + e);
          } else {
            uint16_t *yo = (uint16_t *)a.y + at;
            if (a.accumulate) o += h2f(*yo);
            *yo = f2h(activate(o, a.act, a.slope, n + e));
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW>
static ien_status run_cfg(ien_ctx *ctx, ConvArgs a) {
  using Cfg = ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW>;
  // Tile grid over the requested pixel range.
  const long first_row = a.p_begin / a.OW, last_row = (a.p_end - 1) / a.OW;
  a.ty_begin = (int)(first_row / TR);
  const int ty_end = (int)(last_row / TR) + 1;
  a.tiles_y = ty_end - a.ty_begin;
  a.tiles_x = (a.OW + TC - 1) / TC;
  a.tiles_n = (a.N + Cfg::BN - 1) / Cfg::BN;
  long blocks = (long)a.tiles_y * a.tiles_x * a.tiles_n;
  IEN_CHECK(blocks > 0 && blocks < (1L << 31), IEN_ERR_INPUT, "grid of %ld tiles", blocks);
  // The packed weights must cover every fragment the tiles touch.
  IEN_CHECK(a.tiles_n * (Cfg::BN / 32) <= a.NB, IEN_ERR_INPUT, "weights narrower than the tile");
  hipLaunchKernelGGL((conv_mfma<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW>), dim3((unsigned)blocks),
                     dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status launch_conv(ien_ctx *ctx, const ConvCall &c) {
  const ien_matrix *w = c.w;
  IEN_CHECK(w && w->d_packed, IEN_ERR_INPUT, "no weights");
  const int T = c.noff ? c.noff : c.ks * c.ks;
  IEN_CHECK((size_t)T * c.C == w->k, IEN_ERR_INPUT,
            "input does not match the weights: %d taps x %d channels, k = %zu", T, c.C, w->k);
  IEN_CHECK(c.rows > 0, IEN_ERR_INPUT, "no rows");
  ConvArgs a;
  std::memset(&a, 0, sizeof a);
  a.x = c.x;
  a.H = c.H;
  a.W = c.W;
  a.C = c.C;
  a.xs = c.xs;
  a.rows_mode = c.rows_mode;
  a.pad_reflect = c.pad_reflect;
  a.noff = c.noff;
  for (int i = 0; i < 4; i++) {
    a.offy[i] = c.offy[i];
    a.offx[i] = c.offx[i];
  }
  a.OH = c.OH;
  a.OW = c.OW;
  a.p_begin = c.row0;
  a.p_end = c.row0 + c.rows;
  a.wp = w->d_packed;
  a.KB = w->kb;
  a.NB = w->nb;
  a.N = (int)w->n;
  a.bias = w->d_bias;
  a.slope = c.slope;
  a.y = c.y;
  a.ys = c.ys;
  a.out_nchw = c.out_nchw;
  a.out_f32 = c.out_f32;
  a.act = c.act;
  a.accumulate = c.accumulate;
  IEN_CHECK(c.act != IEN_ACT_PRELU || c.slope, IEN_ERR_INPUT, "PReLU without slopes");

  const bool nchw = c.in_nchw != 0;
  // 16-channel MFMA steps; NHWC halo loads of 16 bytes need aligned pixels.
  const bool vec = c.C % 16 == 0 &&
                   (nchw || (c.xs % 8 == 0 && ((uintptr_t)c.x & 15) == 0));
  if (c.rows_mode) {
    // Input::Rows: a virtual image TC wide, rows in order.
    IEN_CHECK(!nchw && c.ks == 1 && c.noff == 0, IEN_ERR_INPUT, "rows are NHWC, one tap");
    constexpr int TC = 32;
    a.W = TC;
    a.OW = TC;
    a.M = c.row0 + c.rows;
    a.H = a.OH = (int)((a.M + TC - 1) / TC);
    if (vec) return run_cfg<1, 1, 4, 32, 4, 2, 64, true, false>(ctx, a);
    IEN_CHECK(c.C <= 64, IEN_ERR_INPUT, "rows of %d values (not a multiple of 16, over 64)", c.C);
    return run_cfg<1, 1, 4, 32, 4, 2, 64, false, false>(ctx, a);
  }
  IEN_CHECK(vec || c.C <= 16, IEN_ERR_INPUT,
            "%d channels: a multiple of 16, or at most 16", c.C);
  if (c.noff) {
    IEN_CHECK(!nchw, IEN_ERR_INPUT, "offset taps read NHWC");
    for (int i = 0; i < c.noff; i++)
      IEN_CHECK(c.offy[i] >= 0 && c.offy[i] <= 1 && c.offx[i] >= 0 && c.offx[i] <= 1,
                IEN_ERR_INPUT, "offsets past one pixel");
    if (vec) return run_cfg<0, 1, 4, 32, 4, 2, 64, true, false>(ctx, a);
    return run_cfg<0, 1, 4, 32, 4, 2, 16, false, false>(ctx, a);
  }
#define IEN_CONV_LAYOUTS(KS, S, TR, TC, MS, NBW, CK, V)                            \
  return nchw ? run_cfg<KS, S, TR, TC, MS, NBW, CK, V, true>(ctx, a)               \
              : run_cfg<KS, S, TR, TC, MS, NBW, CK, V, false>(ctx, a)
  if (c.ks == 3 && c.stride == 1) {
    if (!vec) IEN_CONV_LAYOUTS(3, 1, 4, 32, 4, 2, 16, false);
    if (c.OW % 96 == 0 && c.C <= 64) IEN_CONV_LAYOUTS(3, 1, 4, 96, 4, 2, 64, true);
    IEN_CONV_LAYOUTS(3, 1, 4, 32, 4, 2, 64, true);
  }
  if (c.ks == 3 && c.stride == 2) {
    if (!vec) return run_cfg<3, 2, 4, 32, 4, 2, 16, false, false>(ctx, a);
    return run_cfg<3, 2, 4, 32, 4, 2, 32, true, false>(ctx, a);
  }
  if (c.ks == 1 && c.stride == 1) {
    IEN_CHECK(vec, IEN_ERR_INPUT, "1x1 products over %d channels", c.C);
    IEN_CONV_LAYOUTS(1, 1, 4, 32, 4, 2, 64, true);
  }
  if (c.ks == 7 && c.stride == 1) {
    IEN_CHECK(!nchw, IEN_ERR_INPUT, "7x7 convolutions read NHWC");
    if (!vec) return run_cfg<7, 1, 4, 32, 4, 2, 16, false, false>(ctx, a);
    return run_cfg<7, 1, 4, 32, 4, 2, 32, true, false>(ctx, a);
  }
#undef IEN_CONV_LAYOUTS
  return fail(IEN_ERR_INPUT, "no kernel for %dx%d stride %d convolutions", c.ks, c.ks, c.stride);
}

// Fill a ConvCall from the op-level descriptors.
static ien_status describe(const ien_input *in, size_t row0, size_t rows, const ien_matrix *w,
                           ConvCall *c) {
  IEN_CHECK(in && w, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(in->data, IEN_ERR_INPUT, "null input data");
  c->x = (const uint16_t *)in->data;
  c->w = w;
  c->row0 = (long)row0;
  c->rows = (long)rows;
  if (in->kind == IEN_INPUT_ROWS) {
    IEN_CHECK(in->stride >= w->k, IEN_ERR_INPUT, "row stride %zu under k = %zu", in->stride, w->k);
    c->rows_mode = 1;
    c->C = (int)w->k;
    c->xs = (long)in->stride;
    c->ks = 1;
    c->stride = 1;
    return IEN_OK;
  }
  IEN_CHECK(in->kind == IEN_INPUT_IMAGE, IEN_ERR_INPUT, "input kind %d", (int)in->kind);
  IEN_CHECK(in->height > 0 && in->width > 0 && in->height < (1u << 20) && in->width < (1u << 20),
            IEN_ERR_INPUT, "%zu x %zu image", in->width, in->height);
  c->H = (int)in->height;
  c->W = (int)in->width;
  c->C = (int)in->channels;
  c->xs = (long)in->stride;
  c->in_nchw = in->layout == IEN_LAYOUT_NCHW;
  if (c->in_nchw)
    IEN_CHECK(in->stride >= in->height * in->width, IEN_ERR_INPUT, "plane stride under h x w");
  else
    IEN_CHECK(in->stride >= in->channels, IEN_ERR_INPUT, "pixel stride under channels");
  c->pad_reflect = in->pad == IEN_PAD_REFLECT;
  if (in->taps == IEN_TAPS_CONV) {
    IEN_CHECK(in->size % 2 == 1 && in->step > 0, IEN_ERR_INPUT, "size %zu step %zu", in->size,
              in->step);
    IEN_CHECK(!c->pad_reflect || (in->size / 2 < in->height && in->size / 2 < in->width),
              IEN_ERR_INPUT, "reflect padding past a %zu x %zu image", in->width, in->height);
    c->ks = (int)in->size;
    c->stride = (int)in->step;
    c->OH = (int)((in->height - 1) / in->step + 1);
    c->OW = (int)((in->width - 1) / in->step + 1);
  } else {
    IEN_CHECK(in->count >= 1 && in->count <= 4, IEN_ERR_INPUT, "%zu offsets", in->count);
    c->noff = (int)in->count;
    for (size_t i = 0; i < in->count; i++) {
      c->offy[i] = (int)in->offsets[i][0];
      c->offx[i] = (int)in->offsets[i][1];
    }
    c->ks = 0;
    c->stride = 1;
    c->OH = (int)in->height;
    c->OW = (int)in->width;
  }
  IEN_CHECK(row0 + rows <= (size_t)c->OH * c->OW, IEN_ERR_INPUT, "rows %zu..%zu past %d pixels",
            row0, row0 + rows, c->OH * c->OW);
  return IEN_OK;
}

}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_multiply_ex(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                           const ien_matrix *w, const ien_output *out, ien_act act,
                           const float *d_slope, int accumulate) {
  IEN_CHECK(ctx && out && out->data, IEN_ERR_INPUT, "null argument");
  if (rows == 0) return IEN_OK;
  ConvCall c;
  ien_status s = describe(input, row0, rows, w, &c);
  if (s != IEN_OK) return s;
  c.y = out->data;
  c.ys = (long)out->stride;
  c.out_nchw = out->layout == IEN_LAYOUT_NCHW;
  c.out_f32 = out->type == IEN_OUT_F32;
  if (c.out_nchw)
    IEN_CHECK(out->stride >= rows, IEN_ERR_INPUT, "plane stride under the rows");
  else
    IEN_CHECK(out->stride >= w->n, IEN_ERR_INPUT, "output stride %zu under n = %zu", out->stride,
              w->n);
  c.act = act;
  c.slope = d_slope;
  c.accumulate = accumulate;
  return launch_conv(ctx, c);
}

ien_status ien_multiply(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                        const ien_matrix *w, void *d_out, size_t stride, ien_act act,
                        int accumulate) {
  IEN_CHECK(act == IEN_ACT_NONE || act == IEN_ACT_RELU || act == IEN_ACT_GELU, IEN_ERR_INPUT,
            "multiply takes Act::{None, Relu, Gelu}");
  ien_output out = {d_out, stride, IEN_LAYOUT_NHWC, IEN_OUT_F16};
  return ien_multiply_ex(ctx, input, row0, rows, w, &out, act, nullptr, accumulate);
}

ien_status ien_conv3(ien_ctx *ctx, const ien_input *input, const ien_matrix *w, void *d_out,
                     size_t stride, int accumulate, ien_act finish, const float *d_slope) {
  IEN_CHECK(input && input->kind == IEN_INPUT_IMAGE && input->taps == IEN_TAPS_CONV &&
                input->size == 3 && input->step == 1,
            IEN_ERR_INPUT, "conv3 needs a 3x3 stride-1 convolution");
  IEN_CHECK(finish == IEN_ACT_NONE || finish == IEN_ACT_RELU || finish == IEN_ACT_PRELU,
            IEN_ERR_INPUT, "finish %d", (int)finish);
  ien_output out = {d_out, stride, IEN_LAYOUT_NHWC, IEN_OUT_F16};
  return ien_multiply_ex(ctx, input, 0, input->height * input->width, w, &out, finish, d_slope,
                         accumulate);
}

}  // extern "C"
