// conv_nchw.hip -- 1x1 products and 3x3 64 -> 64 convolutions of NCHW f16
// maps into NCHW f16 maps on gfx950 (gemm.rs:514-667 multiply on an Image
// input, channel planes in and out): Y[n][p] = act(sum_c W[c][n] X[c][p] +
// b[n]) for one tap; the 3x3 kernel is further down.
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


// ---- 3x3 convolutions of 64 channels into 64 (NCHW in and out) ----
//
// One workgroup of 4 waves per tile of 4 output rows x 96 pixels, the
// layer's whole K: its 72 KiB of weight fragments (both 32-channel output
// blocks, 36 k steps each) land straight in LDS, and the tile's 6 x 98
// pixel halo is transposed in registers (4 channels x 8 pixels -> 8 pixels
// x 4 channels, as k_nchw1 does) into a pixel-major LDS tile of 144-byte
// pixels, whose 32 consecutive pixels are an A fragment read without bank
// conflicts.  Wave w computes tile row w: 3 pixel blocks x 2 channel
// blocks, so each k step reads 5 fragments for 6 MFMAs.
//
// K runs in two channel halves (taps, then 16-channel steps within each,
// the general kernel's order for 32-channel chunks): both halves' loads
// are issued at once, and the second half's pixels are transposed after
// the first half's products, which hide its loads.  Results are staged in
// LDS (where the halo was) and leave as 16-byte stores along pixel rows.
constexpr int N3_TR = 4, N3_TC = 96, N3_HR = 6, N3_HC = 98, N3_GROUPS = 14;
constexpr int N3_PX = 72;  // halves per halo pixel: 64 channels + 8 of padding
// Halves per halo row: 16 past the pixels, so that rows 2 k and 2 k + 1
// sit 16 banks apart (their halves of one transpose write share a cycle).
constexpr int N3_RP = N3_HC * N3_PX + 16;
constexpr int N3_HALO = N3_HR * N3_RP * 2;             // 84864
constexpr int N3_WFRAGS = 2 * 36;                      // 2 channel blocks x 36 k steps
constexpr int N3_LDS = N3_HALO + N3_WFRAGS * 1024;     // 158592
constexpr int N3_UNITS = N3_HR * N3_GROUPS * 8;        // per half: (row, 8-pixel group, channel quad)
constexpr int N3_ITEMS = (N3_UNITS + 255) / 256;
constexpr int N3_YP = N3_TC + 8;                       // halves per staged output row
static_assert(N3_HALO % 1024 == 0 || N3_HALO % 16 == 0, "fragments 16-byte aligned");
static_assert(N3_LDS <= 160 * 1024, "LDS budget");
static_assert(N3_GROUPS * 8 >= N3_HC + 7, "groups cover the halo columns");
static_assert(N3_TR * 64 * N3_YP * 2 <= N3_HALO, "output staging within the halo");
static_assert(N3_HR % 2 == 0, "row pairs");

struct Nchw3Args {
  const uint16_t *x;
  int xs, H, W;  // plane stride (halves), map size (W a multiple of 8)
  const uint16_t *wp;
  int KB;
  const uint16_t *zeros;
  const float *bias, *slope;
  uint16_t *y;
  int ys;
  int tiles_x, tiles;
};

template <int ACT>
__global__ __launch_bounds__(256) void k_nchw3(Nchw3Args a) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[N3_LDS];
  uint16_t *halo = (uint16_t *)lds;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int t = xcd_remap(blockIdx.x, a.tiles);
  const int y0 = (t / a.tiles_x) * N3_TR, x0 = (t % a.tiles_x) * N3_TC;

  float bias[2], slope[2];
#pragma unroll
  for (int nb = 0; nb < 2; nb++) {
    bias[nb] = a.bias[32 * nb + col];
    slope[nb] = ACT == IEN_ACT_PRELU ? a.slope[32 * nb + col] : 0.0f;
  }

  // Half h's weight fragments: blocks nb, taps, its two 16-channel steps
  // (fragment nb KB + 4 tap + 2 h + g of the packed matrix), 9 a wave,
  // straight into LDS at the same fragment index.
  const int4v wrs = uniform_rsrc(a.wp, 72L * 1024);
  const unsigned wlds = lds_addr(lds + N3_HALO);
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // in SGPRs: the LDS base is one
  auto dma_w = [&](int h) {
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const int e = 4 * i + wv, nb = e / 18, tg = e % 18;
      const int f = nb * 36 + (tg >> 1) * 4 + 2 * h + (tg & 1);
      dma_lds(wrs, wlds + f * 1024, f * 1024 + lane * 16);
    }
  };
  // Half h's halo units: rows 2 p + rr (input row y0 - 1 + that), group g
  // (input pixels x0 - 8 + 8 g ..+ 7), channels 32 h + 4 q ..+ 3.  Lanes
  // 0-7 of each 16 take the quads of one row, 8-15 the next row's, so a
  // transpose write of 16 lanes fills 32 distinct banks.  Groups outside
  // the map read the zero page.
  u32x4 v[2][N3_ITEMS][4];
  auto unit = [&](int u, int &r, int &g, int &q) {
    q = u & 7;
    const int rr = (u >> 3) & 1, gp = u >> 4, p = gp / N3_GROUPS;
    g = gp - p * N3_GROUPS;
    r = 2 * p + rr;
  };
  auto load_x = [&](int h) {
#pragma unroll
    for (int j = 0; j < N3_ITEMS; j++) {
      int r, g, q;
      const int u = tid + 256 * j;
      unit(u, r, g, q);
      const int iy = y0 - 1 + r, gx = x0 - 8 + 8 * g;
      const bool ok = u < N3_UNITS && iy >= 0 && iy < a.H && gx >= 0 && gx < a.W;
#pragma unroll
      for (int i = 0; i < 4; i++)
        v[h][j][i] = *(const u32x4 *)(ok ? a.x + (long)(32 * h + 4 * q + i) * a.xs +
                                               (long)iy * a.W + gx
                                         : a.zeros);
    }
  };
  auto store_x = [&](int h) {
#pragma unroll
    for (int j = 0; j < N3_ITEMS; j++) {
      int r, g, q;
      const int u = tid + 256 * j;
      unit(u, r, g, q);
      // Pixel e of the group is halo column 8 g + e - 7.
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int hc = 8 * g + e - 7;
        const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
        uint2 o;
        o.x = __builtin_amdgcn_perm(v[h][j][1][e >> 1], v[h][j][0][e >> 1], sel);
        o.y = __builtin_amdgcn_perm(v[h][j][3][e >> 1], v[h][j][2][e >> 1], sel);
        if (u < N3_UNITS && hc >= 0 && hc < N3_HC)
          *(uint2 *)(halo + r * N3_RP + hc * N3_PX + 32 * h + 4 * q) = o;
      }
    }
  };

  // Row `wave` of the tile: pixel blocks b (32 b ..+ 31), channel blocks nb.
  floatx16 acc[3][2] = {};
  const uint16_t *ab = halo + wave * N3_RP + col * N3_PX + 8 * hi;
  const uint16_t *wb = (const uint16_t *)(lds + N3_HALO) + lane * 8;
  auto products = [&](int h) {
    // Step s: tap s / 2, channels 32 h + 16 (s % 2) ..+ 15.
    auto frag = [&](int s, half8 *av, half8 *bv) {
      const int tap = s >> 1, g = 2 * h + (s & 1), dy = tap / 3, dx = tap % 3;
#pragma unroll
      for (int b = 0; b < 3; b++)
        av[b] = *(const half8 *)(ab + dy * N3_RP + (32 * b + dx) * N3_PX + 16 * g);
#pragma unroll
      for (int nb = 0; nb < 2; nb++) bv[nb] = *(const half8 *)(wb + (nb * 36 + tap * 4 + g) * 512);
    };
    half8 av[2][3], bv[2][2];
    frag(0, av[0], bv[0]);
#pragma unroll
    for (int s = 0; s < 18; s++) {
      if (s + 1 < 18) frag(s + 1, av[(s + 1) & 1], bv[(s + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < 3; b++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
          acc[b][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s & 1][b], bv[s & 1][nb],
                                                              acc[b][nb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  dma_w(0);
  load_x(0);
  dma_w(1);
  load_x(1);
  wait_vm<9 + 4 * N3_ITEMS>();  // half 0's fragments and pixels have landed
  store_x(0);
  lds_barrier();
  products(0);
  wait_vm<0>();
  store_x(1);
  lds_barrier();
  products(1);
  lds_barrier();  // every wave is done with the halo: it becomes the output staging

  // D[pixel][channel]: accumulator r holds pixel 8 (r / 4) + 4 hi + r % 4
  // of the block, channel col; staged [row][channel][pixel].
  uint16_t *ys = halo + wave * 64 * N3_YP;
#pragma unroll
  for (int b = 0; b < 3; b++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        uint2 o;
        const float v0 = act_c<ACT>(acc[b][nb][4 * r4 + 0] + bias[nb], slope[nb]);
        const float v1 = act_c<ACT>(acc[b][nb][4 * r4 + 1] + bias[nb], slope[nb]);
        const float v2 = act_c<ACT>(acc[b][nb][4 * r4 + 2] + bias[nb], slope[nb]);
        const float v3 = act_c<ACT>(acc[b][nb][4 * r4 + 3] + bias[nb], slope[nb]);
        o.x = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
        o.y = (uint32_t)f2h(v2) | ((uint32_t)f2h(v3) << 16);
        *(uint2 *)(ys + (32 * nb + col) * N3_YP + 32 * b + 8 * r4 + 4 * hi) = o;
      }
  lds_barrier();
  // 12 16-byte pieces per (row, channel): 3072 a tile, 12 a thread.
#pragma unroll
  for (int i = 0; i < N3_TR * 64 * 12 / 256; i++) {
    const int e = tid + 256 * i, k = e % 12, rn = e / 12, row = rn >> 6, n = rn & 63;
    const int oy = y0 + row, ox = x0 + 8 * k;
    if (oy < a.H && ox < a.W)
      *(u32x4 *)(a.y + (long)n * a.ys + (long)oy * a.W + ox) =
          *(const u32x4 *)(halo + rn * N3_YP + 8 * k);
  }
}

// ---- 3x3 convolutions of 128 channels into 128 (NCHW in and out) ----
//
// One workgroup of 4 waves per tile of 2 output rows x 96 pixels and one
// half (64) of the output channels; the two halves of a pixel tile are
// neighbours in the XCD-aware order, so the second finds the halo in the
// first's L2.  K runs in four 32-channel quarters (taps, then 16-channel
// steps within each: the general kernel's order at 32-channel chunks)
// through two LDS buffers: a quarter's 36 KiB of weight fragments land by
// buffer loads straight into LDS, and its 4 x 98 pixel halo is loaded into
// registers and transposed (4 channels x 8 pixels -> 8 pixels x 4
// channels, as k_nchw1 does) into a pixel-major tile of 80-byte pixels.
// While quarter i is multiplied, quarter i + 1 sits in the other buffer
// and quarter i + 2's halo is in flight in registers.  Wave w computes
// row w / 2 of the tile against channel block w % 2 of the half: 3 pixel
// blocks, 4 fragments read for 3 MFMAs a k step.
constexpr int Q_TR = 2, Q_TC = 96, Q_HR = 4, Q_HC = 98, Q_GROUPS = 14;
constexpr int Q_PX = 40;           // halves per halo pixel: 32 channels + 8
constexpr int Q_RP = Q_HC * Q_PX;  // halves per halo row: rows 40 banks apart
constexpr int Q_HALO = (Q_HR * Q_RP * 2 + 1023) / 1024 * 1024;  // 31744
constexpr int Q_WFRAGS = 2 * 18;                                // 2 channel blocks x 9 taps x 2 steps
constexpr int Q_BUF = Q_HALO + Q_WFRAGS * 1024;                 // 68608
constexpr int Q_LDS = 2 * Q_BUF;                                // 137216
constexpr int Q_UNITS = Q_HR * Q_GROUPS * 8;  // per quarter: (row, 8-pixel group, channel quad)
constexpr int Q_ITEMS = (Q_UNITS + 255) / 256;
constexpr int Q_YP = Q_TC + 8;  // halves per staged output row
static_assert(Q_LDS <= 160 * 1024, "LDS budget");
static_assert(Q_GROUPS * 8 >= Q_HC + 7, "groups cover the halo columns");
static_assert(Q_TR * 64 * Q_YP * 2 <= Q_HALO, "output staging within a halo buffer");
static_assert(Q_HR % 2 == 0, "row pairs");

struct Nchw3qArgs {
  const uint16_t *x;
  int xs, H, W;          // plane stride (halves), map size (W a multiple of 8)
  const uint16_t *wp;    // packed 1152 x 128 fragments, 72 k steps a channel block
  const uint16_t *zeros;
  const float *bias, *slope;
  uint16_t *y;
  int ys;
  int tiles_x, tiles;    // pixel tiles across; tiles = 2 x pixel tiles
};

template <int ACT>
__global__ __launch_bounds__(256) void k_nchw3q(Nchw3qArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[Q_LDS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int t = xcd_remap(blockIdx.x, a.tiles), nh = t & 1, pt = t >> 1;
  const int y0 = (pt / a.tiles_x) * Q_TR, x0 = (pt % a.tiles_x) * Q_TC;
  const int row = wave >> 1, nb = wave & 1;
  const int och = 64 * nh + 32 * nb + col;
  const float bias = a.bias[och];
  const float slope = ACT == IEN_ACT_PRELU ? a.slope[och] : 0.0f;

  // Quarter q's weight fragments of this half: LDS slot e = b 18 + 2 tap + g
  // holds packed fragment (2 nh + b) 72 + 8 tap + 2 q + g; 9 a wave.
  const int4v wrs = uniform_rsrc(a.wp + (size_t)nh * 2 * 72 * 512, 2L * 72 * 1024);
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // in SGPRs: the LDS base is one
  auto dma_w = [&](int q, int buf) {
    const unsigned base = lds_addr(lds + buf * Q_BUF + Q_HALO);
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const int e = 4 * i + wv, b = e / 18, tg = e % 18;
      const int f = b * 72 + (tg >> 1) * 8 + 2 * q + (tg & 1);
      dma_lds(wrs, base + e * 1024, f * 1024 + lane * 16);
    }
  };
  // Halo units of a quarter: rows 2 p + rr (input row y0 - 1 + that), group
  // g (input pixels x0 - 8 + 8 g ..+ 7), channels 32 q + 4 c4 ..+ 3.  Lanes
  // 0-7 of each 16 take the quads of one row, 8-15 the next row's.  Groups
  // outside the map read the zero page.
  auto unit = [&](int u, int &r, int &g, int &c4) {
    c4 = u & 7;
    const int rr = (u >> 3) & 1, gp = u >> 4, p = gp / Q_GROUPS;
    g = gp - p * Q_GROUPS;
    r = 2 * p + rr;
  };
  auto load_x = [&](int q, u32x4 (&v)[Q_ITEMS][4]) {
#pragma unroll
    for (int j = 0; j < Q_ITEMS; j++) {
      int r, g, c4;
      const int u = tid + 256 * j;
      unit(u, r, g, c4);
      const int iy = y0 - 1 + r, gx = x0 - 8 + 8 * g;
      const bool ok = u < Q_UNITS && iy >= 0 && iy < a.H && gx >= 0 && gx < a.W;
#pragma unroll
      for (int i = 0; i < 4; i++)
        v[j][i] = *(const u32x4 *)(ok ? a.x + (long)(32 * q + 4 * c4 + i) * a.xs +
                                            (long)iy * a.W + gx
                                      : a.zeros);
    }
  };
  auto store_x = [&](const u32x4 (&v)[Q_ITEMS][4], int buf) {
    uint16_t *halo = (uint16_t *)(lds + buf * Q_BUF);
#pragma unroll
    for (int j = 0; j < Q_ITEMS; j++) {
      int r, g, c4;
      const int u = tid + 256 * j;
      unit(u, r, g, c4);
      // Pixel e of the group is halo column 8 g + e - 7.
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int hc = 8 * g + e - 7;
        const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
        uint2 o;
        o.x = __builtin_amdgcn_perm(v[j][1][e >> 1], v[j][0][e >> 1], sel);
        o.y = __builtin_amdgcn_perm(v[j][3][e >> 1], v[j][2][e >> 1], sel);
        if (u < Q_UNITS && hc >= 0 && hc < Q_HC)
          *(uint2 *)(halo + r * Q_RP + hc * Q_PX + 4 * c4) = o;
      }
    }
  };

  // Pixel blocks b (32 b ..+ 31) of tile row `row`, channel block nb.
  floatx16 acc[3] = {};
  auto products = [&](int buf) {
    const uint16_t *ab = (const uint16_t *)(lds + buf * Q_BUF) + row * Q_RP + col * Q_PX + 8 * hi;
    const uint16_t *wb = (const uint16_t *)(lds + buf * Q_BUF + Q_HALO) + nb * 18 * 512 + lane * 8;
    // Step s: tap s / 2, channels 16 (s % 2) ..+ 15 of the quarter.
    auto frag = [&](int s, half8 *av, half8 &bv) {
      const int tap = s >> 1, g = s & 1, dy = tap / 3, dx = tap % 3;
#pragma unroll
      for (int b = 0; b < 3; b++)
        av[b] = *(const half8 *)(ab + dy * Q_RP + (32 * b + dx) * Q_PX + 16 * g);
      bv = *(const half8 *)(wb + (2 * tap + g) * 512);
    };
    half8 av[2][3], bv[2];
    frag(0, av[0], bv[0]);
#pragma unroll
    for (int s = 0; s < 18; s++) {
      if (s + 1 < 18) frag(s + 1, av[(s + 1) & 1], bv[(s + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < 3; b++)
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s & 1][b], bv[s & 1], acc[b], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  u32x4 va[Q_ITEMS][4], vb[Q_ITEMS][4];
  dma_w(0, 0);
  load_x(0, va);
  dma_w(1, 1);
  load_x(1, vb);
  wait_vm<9 + 4 * Q_ITEMS>();  // quarter 0's fragments and pixels have landed
  store_x(va, 0);
  lds_barrier();
  load_x(2, va);
  products(0);
  wait_vm<4 * Q_ITEMS>();  // quarter 1's (quarter 2's pixels still in flight)
  store_x(vb, 1);
  lds_barrier();  // every wave is done with buffer 0
  dma_w(2, 0);
  load_x(3, vb);
  products(1);
  wait_vm<4 * Q_ITEMS>();  // quarter 2's (quarter 3's pixels still in flight)
  store_x(va, 0);
  lds_barrier();  // every wave is done with buffer 1
  dma_w(3, 1);
  products(0);
  wait_vm<0>();
  store_x(vb, 1);
  lds_barrier();  // every wave is done with buffer 0: its halo becomes the output staging
  products(1);

  // D[pixel][channel]: accumulator r holds pixel 8 (r / 4) + 4 hi + r % 4
  // of the block, channel col; staged [row][channel of the half][pixel].
  uint16_t *ys = (uint16_t *)lds + (row * 64 + 32 * nb + col) * Q_YP;
#pragma unroll
  for (int b = 0; b < 3; b++)
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      uint2 o;
      const float v0 = act_c<ACT>(acc[b][4 * r4 + 0] + bias, slope);
      const float v1 = act_c<ACT>(acc[b][4 * r4 + 1] + bias, slope);
      const float v2 = act_c<ACT>(acc[b][4 * r4 + 2] + bias, slope);
      const float v3 = act_c<ACT>(acc[b][4 * r4 + 3] + bias, slope);
      o.x = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
      o.y = (uint32_t)f2h(v2) | ((uint32_t)f2h(v3) << 16);
      *(uint2 *)(ys + 32 * b + 8 * r4 + 4 * hi) = o;
    }
  lds_barrier();
  // 12 16-byte pieces per (row, channel): 1536 a tile, 6 a thread.
#pragma unroll
  for (int i = 0; i < Q_TR * 64 * 12 / 256; i++) {
    const int e = tid + 256 * i, k = e % 12, rn = e / 12, rr = rn >> 6, n = rn & 63;
    const int oy = y0 + rr, ox = x0 + 8 * k;
    if (oy < a.H && ox < a.W)
      *(u32x4 *)(a.y + (long)(64 * nh + n) * a.ys + (long)oy * a.W + ox) =
          *(const u32x4 *)((const uint16_t *)lds + rn * Q_YP + 8 * k);
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

bool nchw3_supported(const ConvArgs &a, int ks, int stride, long rows) {
  const long P = (long)a.H * a.W;
  return ks == 3 && stride == 1 && a.C == 64 && a.N == 64 && a.KB == 36 && !a.rows_mode &&
         !a.pad_reflect && a.noff == 0 && a.out_nchw && !a.out_f32 && !a.accumulate &&
         a.p_begin == 0 && rows == P && a.OH == a.H && a.OW == a.W && a.W % 8 == 0 &&
         a.xs % 8 == 0 && a.ys % 8 == 0 && (((uintptr_t)a.x | (uintptr_t)a.y) & 15) == 0 &&
         a.xs >= P && a.ys >= P && 64L * a.xs < (1L << 31) && 64L * a.ys < (1L << 31);
}

ien_status launch_nchw3(ien_ctx *ctx, const ConvArgs &a) {
  Nchw3Args n{a.x, a.xs, a.H, a.W, a.wp, a.KB, a.zeros, a.bias, a.slope, (uint16_t *)a.y, a.ys,
              (a.W + N3_TC - 1) / N3_TC, 0};
  n.tiles = n.tiles_x * ((a.H + N3_TR - 1) / N3_TR);
  const dim3 grid((unsigned)n.tiles);
  switch (a.act) {
    case IEN_ACT_RELU: hipLaunchKernelGGL(k_nchw3<IEN_ACT_RELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_GELU: hipLaunchKernelGGL(k_nchw3<IEN_ACT_GELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_PRELU: hipLaunchKernelGGL(k_nchw3<IEN_ACT_PRELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_SIGMOID:
      hipLaunchKernelGGL(k_nchw3<IEN_ACT_SIGMOID>, grid, dim3(256), 0, ctx->stream, n);
      break;
    default: hipLaunchKernelGGL(k_nchw3<IEN_ACT_NONE>, grid, dim3(256), 0, ctx->stream, n); break;
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

bool nchw3q_supported(const ConvArgs &a, int ks, int stride, long rows) {
  const long P = (long)a.H * a.W;
  return ks == 3 && stride == 1 && a.C == 128 && a.N == 128 && a.KB == 72 && !a.rows_mode &&
         !a.pad_reflect && a.noff == 0 && a.out_nchw && !a.out_f32 && !a.accumulate &&
         a.p_begin == 0 && rows == P && a.OH == a.H && a.OW == a.W && a.W % 8 == 0 &&
         a.xs % 8 == 0 && a.ys % 8 == 0 && (((uintptr_t)a.x | (uintptr_t)a.y) & 15) == 0 &&
         a.xs >= P && a.ys >= P && 128L * a.xs < (1L << 31) && 128L * a.ys < (1L << 31);
}

ien_status launch_nchw3q(ien_ctx *ctx, const ConvArgs &a) {
  Nchw3qArgs n{a.x, a.xs, a.H, a.W, a.wp, a.zeros, a.bias, a.slope, (uint16_t *)a.y, a.ys,
               (a.W + Q_TC - 1) / Q_TC, 0};
  n.tiles = 2 * n.tiles_x * ((a.H + Q_TR - 1) / Q_TR);
  const dim3 grid((unsigned)n.tiles);
  switch (a.act) {
    case IEN_ACT_RELU: hipLaunchKernelGGL(k_nchw3q<IEN_ACT_RELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_GELU: hipLaunchKernelGGL(k_nchw3q<IEN_ACT_GELU>, grid, dim3(256), 0, ctx->stream, n); break;
    case IEN_ACT_PRELU:
      hipLaunchKernelGGL(k_nchw3q<IEN_ACT_PRELU>, grid, dim3(256), 0, ctx->stream, n);
      break;
    case IEN_ACT_SIGMOID:
      hipLaunchKernelGGL(k_nchw3q<IEN_ACT_SIGMOID>, grid, dim3(256), 0, ctx->stream, n);
      break;
    default: hipLaunchKernelGGL(k_nchw3q<IEN_ACT_NONE>, grid, dim3(256), 0, ctx->stream, n); break;
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien
