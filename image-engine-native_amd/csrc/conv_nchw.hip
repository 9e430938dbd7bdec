// conv_nchw.hip -- 1x1 products of NCHW f16 maps into NCHW f16 maps on
// gfx950 (gemm.rs:514-667 multiply on an Image input of one tap, channel
// planes in and out): Y[n][p] = act(sum_c W[c][n] X[c][p] + b[n]).
//
// NCHW puts the pixels of one channel next to each other, while an MFMA
// operand needs eight consecutive reduction (channel) values in a lane.  The
// general kernel turns each 16-byte group of a channel row into eight
// two-byte LDS writes; this one transposes in registers instead: a thread
// loads 8 pixels of 4 channels (four 16-byte loads, 8 lanes per 128-byte
// line), permutes them into 8 pixels x 4 channels (16 v_perm_b32) and
// writes each pixel's 4 channels as one 8-byte LDS store into a
// pixel-major tile [pixel][channel], whose rows are the B operand of
// v_mfma_f32_32x32x16_f16 as plain 16-byte reads.
//
// Workgroup: 4 waves, 128 output channels x 64 pixels; wave w computes
// output channels 32 w .. 32 w + 31 over both 32-pixel blocks.  K runs in
// chunks of 128 channels, double-buffered: chunk i + 1's loads (pixels
// into registers, weight fragments straight into LDS) are issued before
// chunk i's products.  Results are staged in LDS and stored as whole
// 128-byte output rows.

#include "conv_common.h"

namespace ien {
namespace {

constexpr int TN = 128, TP = 64, KC = 128;
constexpr int XPITCH = KC + 8;                     // halves per staged pixel
constexpr int X_BYTES = TP * XPITCH * 2;           // 17408
constexpr int W_BYTES = (TN / 32) * (KC / 16) * 1024;  // 32768
constexpr int STAGE = X_BYTES + W_BYTES;
constexpr int YPITCH = TP + 8;                     // halves per staged output row
static_assert(X_BYTES % 1024 == 0, "weight fragments on whole KiB");
static_assert(TN * YPITCH * 2 <= STAGE, "output staging within a stage");

struct NchwArgs {
  const uint16_t *x;
  int xs, C, P;  // plane stride (halves), channels, pixels (a multiple of 8)
  const uint16_t *wp;
  int KB;
  const uint16_t *zeros;
  const float *bias, *slope;
  int N;
  uint16_t *y;
  int ys;
};

template <int ACT>
__global__ __launch_bounds__(256) void k_nchw1(NchwArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * STAGE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int p0 = blockIdx.x * TP, nt = blockIdx.y;
  const int chunks = (a.C + KC - 1) / KC;
  // This thread's part of a chunk's pixels: channels 4 cg .. 4 cg + 3 of
  // the chunk, pixels 8 pg .. 8 pg + 7 of the tile.
  const int cg = tid >> 3, pg = tid & 7;
  const int px = min(p0 + 8 * pg, a.P - 8);  // a valid group (masked at the store)
  auto load_x = [&](int ch, u32x4 *v) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // Channels past C read the zero page (no select after the load, which
      // would make the compiler wait for it at once).
      const int c = ch * KC + 4 * cg + i;
      v[i] = *(const u32x4 *)(c < a.C ? a.x + (long)c * a.xs + px : a.zeros);
    }
  };
  // Pixel j's four channels: the low (even j) or high (odd j) halves of
  // dword j / 2 of each channel's group.
  auto store_x = [&](int s, const u32x4 *v) {
    uint16_t *xt = (uint16_t *)(lds + s * STAGE) + 4 * cg;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
      uint2 o;
      o.x = __builtin_amdgcn_perm(v[1][j >> 1], v[0][j >> 1], sel);
      o.y = __builtin_amdgcn_perm(v[3][j >> 1], v[2][j >> 1], sel);
      *(uint2 *)(xt + (8 * pg + j) * XPITCH) = o;
    }
  };
  // The chunk's weight fragments [n block j][k step], 8 a wave.
  auto dma_w = [&](int ch, int s) {
#pragma unroll
    for (int f = wave; f < 32; f += 4) {
      const int j = f >> 3, kb = ch * (KC / 16) + (f & 7);
      const uint16_t *src = kb < a.KB ? a.wp + ((long)(4 * nt + j) * a.KB + kb) * 512 + lane * 8
                                      : a.zeros + lane * 8;
      dma16(src, lds + s * STAGE + X_BYTES + f * 1024);
    }
  };

  // The epilogue's bias and slopes for this lane's 16 output channels,
  // requested first (rows 8 q + 4 hi .. + 3 of the wave's 32).
  float4v bias[4], slope[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int n = TN * nt + 32 * wave + 8 * q + 4 * hi;  // < the bias's padded length
    bias[q] = *(const float4v *)(a.bias + n);
    slope[q] = a.slope ? float4v{a.slope[min(n, a.N - 1)], a.slope[min(n + 1, a.N - 1)],
                                 a.slope[min(n + 2, a.N - 1)], a.slope[min(n + 3, a.N - 1)]}
                       : float4v{0.0f, 0.0f, 0.0f, 0.0f};
  }
  floatx16 acc[2] = {};
  u32x4 cur[4], nxt[4];
  load_x(0, cur);
  dma_w(0, 0);
  for (int ch = 0; ch < chunks; ch++) {
    const int s = ch & 1;
    if (ch + 1 < chunks) {
      load_x(ch + 1, nxt);
      dma_w(ch + 1, s ^ 1);
      wait_vm<12>();  // chunk ch's 4 loads and 8 fragments have landed
    } else {
      wait_vm<0>();
    }
    store_x(s, cur);
    lds_barrier();
    const unsigned char *wa = lds + s * STAGE + X_BYTES + wave * 8 * 1024 + lane * 16;
    const uint16_t *xb = (const uint16_t *)(lds + s * STAGE) + col * XPITCH + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < KC / 16; ks++) {
      const half8 w = *(const half8 *)(wa + ks * 1024);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w, *(const half8 *)(xb + 16 * ks), acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          w, *(const half8 *)(xb + 32 * XPITCH + 16 * ks), acc[1], 0, 0, 0);
    }
    lds_barrier();  // stage s is free for chunk ch + 2
#pragma unroll
    for (int i = 0; i < 4; i++) cur[i] = nxt[i];
  }
  // Epilogue: D[n][p] + bias, activation, f16, staged as [n][p]; then 8
  // lanes store one 128-byte output row.
  uint16_t *ys = (uint16_t *)lds;
#pragma unroll
  for (int pb = 0; pb < 2; pb++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int n = 32 * wave + 8 * (r >> 2) + 4 * hi + (r & 3);
      const float v = acc[pb][r] + bias[r >> 2][r & 3];
      ys[n * YPITCH + 32 * pb + col] = f2h(act_c<ACT>(v, slope[r >> 2][r & 3]));
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TN * TP / 8 / 256; i++) {
    const int q = tid + 256 * i, n = q >> 3, part = q & 7;
    const int ng = TN * nt + n, p = p0 + 8 * part;
    if (ng < a.N && p < a.P)
      *(u32x4 *)(a.y + (long)ng * a.ys + p) = *(const u32x4 *)(ys + n * YPITCH + 8 * part);
  }
}

}  // namespace

bool nchw1_supported(const ConvArgs &a, int ks, int stride, long rows) {
  const long P = (long)a.H * a.W;
  return ks == 1 && stride == 1 && !a.rows_mode && !a.pad_reflect && a.noff == 0 && a.out_nchw &&
         !a.out_f32 && !a.accumulate && a.p_begin == 0 && rows == P && P % 8 == 0 && a.C % 16 == 0 &&
         a.xs % 8 == 0 && a.ys % 8 == 0 && (((uintptr_t)a.x | (uintptr_t)a.y) & 15) == 0 &&
         (long)a.C * a.xs < (1L << 31) && (long)a.N * a.ys < (1L << 31);
}

ien_status launch_nchw1(ien_ctx *ctx, const ConvArgs &a) {
  NchwArgs n{a.x, a.xs, a.C, a.H * a.W, a.wp, a.KB, a.zeros, a.bias, a.slope, a.N, (uint16_t *)a.y,
             a.ys};
  const dim3 grid((unsigned)((n.P + TP - 1) / TP), (unsigned)((a.N + TN - 1) / TN));
  switch (a.act) {
    case IEN_ACT_RELU: hipLaunchKernelGGL(k_nchw1<IEN_ACT_RELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_GELU: hipLaunchKernelGGL(k_nchw1<IEN_ACT_GELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_PRELU: hipLaunchKernelGGL(k_nchw1<IEN_ACT_PRELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_SIGMOID:
      hipLaunchKernelGGL(k_nchw1<IEN_ACT_SIGMOID>, grid, dim3(256), 0, ctx->stream, n);
      break;
    default: hipLaunchKernelGGL(k_nchw1<IEN_ACT_NONE>, grid, dim3(256), 0, ctx->stream, n); break;
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien
