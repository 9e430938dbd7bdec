// conv_res.hip -- resident-weight persistent convolution on gfx950 MFMA.
//
// For NHWC inputs of 16, 32 or 64 channels with 1x1 or 3x3 zero-padded
// taps (K = k k C <= 576): Real-ESRGAN's body layers (crates/realesrgan-
// native/src/network.rs:96-109, gemm.rs multiply semantics) and the 1x1
// products of that width.
//
// One workgroup per CU, 8 waves (2 per SIMD: the second wave hides the
// other's MFMA and LDS latency and doubles the LDS read rate), persistent
// over 2 x 64-pixel output tiles, all 64 output channels of a tile.
//  - Prologue: the 64 channels' weight fragments go global -> LDS by
//    direct-to-LDS loads (one contiguous KiB per wave instruction, read once
//    per CU from L2), then each wave copies its 32-channel slice into VGPRs
//    (A operand of v_mfma_f32_32x32x16_f16: the packing is the A layout, so
//    the product is C^T = W^T X^T) and the LDS is reused for activations.
//  - Per tile: wait for the tile's halo (double-buffered, loaded by
//    direct-to-LDS loads issued one tile ahead, 16-byte chunks XOR-swizzled
//    per pixel so the B-operand reads are conflict-free); write the previous
//    tile's results from the LDS staging buffer to HBM as full 128-byte
//    lines; run the tile's MFMAs (each wave: one 32-pixel x 32-channel block,
//    two accumulator chains); stage bias + activation results as f16.
// Bias then activation, or bias, old output, activation when accumulating:
// the order of gemm.rs:583-666.

#include "conv_common.h"

namespace ien {

template <int KS, int C>
struct Res8 {
  static constexpr int TR = 2, TC = 64;  // output tile: 2 rows of 64 pixels
  static constexpr int STEPS = KS * KS * C / 16;
  static constexpr int HR = TR + KS - 1, HC = TC + KS - 1;
  static constexpr int PB = C * 2, NCH = PB / 16, RPB = 256 / PB;
  static constexpr int HALO = (HR * HC * PB + 1023) / 1024 * 1024;
  static constexpr int SPX = 64 + 8;                  // staged halves per pixel (padded)
  static constexpr int STAGE = TR * TC * SPX * 2;     // bytes
  static constexpr int WBYTES = 2 * STEPS * 1024;     // B fragments of 64 channels
  static constexpr int MAIN = 2 * HALO + STAGE;
  static constexpr int PARAM = MAIN > WBYTES ? MAIN : WBYTES;  // bias, slopes after this
  static constexpr int LDS = PARAM + 2 * 64 * 4;
  static_assert(C == 16 || C == 32 || C == 64, "power-of-two chunk swizzle");
  static_assert(STEPS <= 36, "weights must fit in registers");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int KS, int C, int ACT>
__global__ __launch_bounds__(512) void conv_res8(ConvArgs a) {
  using R = Res8<KS, C>;
  constexpr int STEPS = R::STEPS, HC = R::HC, PB = R::PB, P = KS / 2;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[R::LDS];
  unsigned char *stage = lds + 2 * R::HALO;
  float *bias_l = (float *)(lds + R::PARAM), *slope_l = bias_l + 64;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int mg = wave & 3, ng = wave >> 2;  // 32-pixel block, 32-channel half
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int tn = lb % a.tiles_n;            // this block's 64-channel tile
  const int per_n = gridDim.x / a.tiles_n;  // blocks sharing it
  const int tiles_m = a.tiles_x * a.tiles_y;

  // ---- prologue: weights through LDS into VGPRs; bias and slopes to LDS ----
  for (int f = wave; f < 2 * STEPS; f += 8) {
    const int jn = f / STEPS, s = f - jn * STEPS;
    dma16(a.wp + ((tn * 2 + jn) * a.KB + s) * 512 + lane * 8, lds + f * 1024);
  }
  if (tid < 64) {
    const int n = tn * 64 + tid;  // < NB * 32: the bias is padded
    bias_l[tid] = a.bias[n];
    slope_l[tid] = ACT == IEN_ACT_PRELU ? a.slope[min(n, a.N - 1)] : 0.0f;
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  half8 wr[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; s++)
    wr[s] = *(const half8 *)(lds + (ng * STEPS + s) * 1024 + lane * 16);
  __syncthreads();  // every wave holds its weights: the LDS is free

  // Halo pixel of tap (0, 0) for the lane's pixel; tile pixel of the lane.
  const int tpix = (mg >> 1) * 64 + (mg & 1) * 32 + (lane & 31);
  const int apix = (mg >> 1) * HC + (mg & 1) * 32 + (lane & 31);

  auto origin = [&](int mt, int &oy0, int &ox0) {
    oy0 = (mt / a.tiles_x + a.ty_begin) * R::TR;
    ox0 = (mt % a.tiles_x) * R::TC;
  };

  auto load_halo = [&](int mt, unsigned char *buf) {
    int oy0, ox0;
    origin(mt, oy0, ox0);
    for (int g = wave; g < R::HALO / 1024; g += 8) {
      const int byte = g * 1024 + lane * 16;
      const int hp = byte / PB, slot = (byte % PB) / 16;
      const uint16_t *src = a.zeros;
      if (hp < R::HR * HC) {
        const int hy = hp / HC, hx = hp - hy * HC;
        const int iy = oy0 + hy - P, ix = ox0 + hx - P;
        if (iy >= 0 && iy < a.H && ix >= 0 && ix < a.W)
          src = a.x + (iy * a.W + ix) * a.xs + 8 * (slot ^ ((hp / R::RPB) & (R::NCH - 1)));
      }
      dma16(src, buf + g * 1024);
    }
  };

  // The staged tile to HBM: 16 bytes (8 channels of one pixel) per item,
  // 8 items per pixel, so a wave writes 8 whole pixels (full lines).
  auto store_tile = [&](int mt) {
    int oy0, ox0;
    origin(mt, oy0, ox0);
    for (int v = tid; v < R::TR * R::TC * 8; v += 512) {
      const int tp = v >> 3, chunk = v & 7;
      const int oy = oy0 + tp / R::TC, ox = ox0 + tp % R::TC;
      const int p = oy * a.OW + ox;
      const int n0 = tn * 64 + chunk * 8;
      if (oy >= a.OH || ox >= a.OW || p < a.p_begin || p >= a.p_end || n0 >= a.N) continue;
      const int rel = p - a.p_begin;
      u32x4 hv = *(const u32x4 *)(stage + (tp * R::SPX + chunk * 8) * 2);
      uint16_t *yo = (uint16_t *)a.y + (long)rel * a.ys + n0;
      if (!a.accumulate && !a.out_f32 && !a.out_nchw && n0 + 8 <= a.N &&
          (((uintptr_t)yo) & 15) == 0) {
        *(u32x4 *)yo = hv;
        continue;
      }
      uint16_t h[8];
      __builtin_memcpy(h, &hv, 16);
      for (int e = 0; e < 8 && n0 + e < a.N; e++) {
        const long at = a.out_nchw ? (long)(n0 + e) * a.ys + rel : (long)rel * a.ys + n0 + e;
        float o = h2f(h[e]);
        const float sl = slope_l[chunk * 8 + e];
        if (a.out_f32) {
          float *yf = (float *)a.y + at;
          if (a.accumulate) o = act_c<ACT>(o + *yf, sl);
          *yf = o;
        } else {
          uint16_t *yh = (uint16_t *)a.y + at;
          if (a.accumulate) o = act_c<ACT>(o + h2f(*yh), sl);
          *yh = f2h(o);
        }
      }
    }
  };

  auto mma = [&](const unsigned char *buf, floatx16 &acc_a, floatx16 &acc_b) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      acc_a[r] = 0.0f;
      acc_b[r] = 0.0f;
    }
    auto frag = [&](int s) {
      const int tap = s / (C / 16), kc = s % (C / 16);
      const int p = apix + (tap / KS) * HC + tap % KS;
      const int c = 2 * kc + (lane >> 5);
      return *(const half8 *)(buf + p * PB + 16 * (c ^ ((p / R::RPB) & (R::NCH - 1))));
    };
    half8 xv[2];
    xv[0] = frag(0);
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      if (s + 1 < STEPS) xv[(s + 1) & 1] = frag(s + 1);
      __builtin_amdgcn_sched_barrier(0);
      if (s & 1)
        acc_b = __builtin_amdgcn_mfma_f32_32x32x16_f16(wr[s], xv[s & 1], acc_b, 0, 0, 0);
      else
        acc_a = __builtin_amdgcn_mfma_f32_32x32x16_f16(wr[s], xv[s & 1], acc_a, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // C^T fragment: the lane holds pixel lane % 32 of its block and channels
  // 32 ng + 8 g + 4 (lane / 32) + e of the tile.
  auto stage_tile = [&](const floatx16 &acc_a, const floatx16 &acc_b) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int ch = ng * 32 + 8 * g + 4 * (lane >> 5);
      const float4v b4 = *(const float4v *)(bias_l + ch);
      const float4v s4 = *(const float4v *)(slope_l + ch);
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float v = acc_a[4 * g + e] + acc_b[4 * g + e] + b4[e];
        if (!a.accumulate) v = act_c<ACT>(v, s4[e]);
        h[e] = f2h(v);
      }
      uint2 o;
      __builtin_memcpy(&o, h, 8);
      *(uint2 *)(stage + (tpix * R::SPX + ch) * 2) = o;
    }
  };

  int mt = lb / a.tiles_n;
  if (mt < tiles_m) load_halo(mt, lds);
  int prev = -1;
  bool odd = false;
  while (mt < tiles_m) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this tile's halo has landed
    __syncthreads();  // ... for every wave; the staging holds the previous tile
    const int next = mt + per_n;
    if (next < tiles_m) load_halo(next, odd ? lds : lds + R::HALO);
    if (prev >= 0) store_tile(prev);
    floatx16 acc_a, acc_b;
    mma(odd ? lds + R::HALO : lds, acc_a, acc_b);
    __syncthreads();  // every wave has read the staging
    stage_tile(acc_a, acc_b);
    prev = mt;
    mt = next;
    odd = !odd;
  }
  __syncthreads();
  if (prev >= 0) store_tile(prev);
}

bool resident_supported(int ks, int stride, int c, int nchw, int reflect, int noff, int rows_mode) {
  return (ks == 1 || ks == 3) && stride == 1 && (c == 16 || c == 32 || c == 64) && !nchw &&
         !reflect && noff == 0 && !rows_mode && ks * ks * c / 16 <= 36;
}

template <int KS, int C>
static ien_status run_res8(ien_ctx *ctx, ConvArgs a) {
  using R = Res8<KS, C>;
  void (*kernel)(ConvArgs) = nullptr;
  switch (a.act) {
    case IEN_ACT_RELU: kernel = conv_res8<KS, C, IEN_ACT_RELU>; break;
    case IEN_ACT_PRELU: kernel = conv_res8<KS, C, IEN_ACT_PRELU>; break;
    case IEN_ACT_GELU: kernel = conv_res8<KS, C, IEN_ACT_GELU>; break;
    case IEN_ACT_SIGMOID: kernel = conv_res8<KS, C, IEN_ACT_SIGMOID>; break;
    default: kernel = conv_res8<KS, C, IEN_ACT_NONE>; break;
  }
  const int first_row = a.p_begin / a.OW, last_row = (a.p_end - 1) / a.OW;
  a.ty_begin = first_row / R::TR;
  a.tiles_y = last_row / R::TR + 1 - a.ty_begin;
  a.tiles_x = (a.OW + R::TC - 1) / R::TC;
  a.tiles_n = (a.N + 63) / 64;
  IEN_CHECK(a.tiles_n * 2 <= a.NB, IEN_ERR_INPUT, "weights narrower than the tile");
  const long tiles_m = (long)a.tiles_y * a.tiles_x;
  // One workgroup per CU; every channel tile gets as many, a multiple of 8
  // (the XCDs) where there are that many.
  long per_n = std::min<long>(tiles_m, std::max<long>(1, ctx->cus / a.tiles_n));
  if (per_n >= 8) per_n = per_n / 8 * 8;
  const long blocks = per_n * a.tiles_n;
  IEN_CHECK(blocks > 0 && blocks < (1L << 31), IEN_ERR_INPUT, "grid of %ld", blocks);
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(512), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status launch_resident(ien_ctx *ctx, ConvArgs a, int ks) {
  if (ks == 3) {
    switch (a.C) {
      case 16: return run_res8<3, 16>(ctx, a);
      case 32: return run_res8<3, 32>(ctx, a);
      default: return run_res8<3, 64>(ctx, a);
    }
  }
  switch (a.C) {
    case 16: return run_res8<1, 16>(ctx, a);
    case 32: return run_res8<1, 32>(ctx, a);
    default: return run_res8<1, 64>(ctx, a);
  }
}

}  // namespace ien
