// spectral.hip -- the spectral branch of LaMa's fast Fourier convolution in
// three launches (crates/lama-native/src/network.rs:205-245, Ffc::run):
//
//   spectral  = ReLU(x_global spectral_in + b)              1x1, 384 -> 192
//   spectrum  = rfftn(spectral), "ortho"                     fourier.rs:291-344
//   filtered  = ReLU(spectrum fourier + b)                   1x1 over spectrum pixels, 384 -> 384
//   spectral += irfftn(filtered), "ortho"                    fourier.rs:347-403
//   out       = ReLU(out + spectral spectral_out)            1x1, 192 -> 384, accumulated
//
// for maps of at most 64 x 64 (LaMa's eighth scale up to 512 x 512 images).
// The unfused path (fourier.hip and four products) takes seven dependent
// launches, each a load -> compute -> store chain of a few microseconds on a
// map of 1.5 MB; here:
//
//   front  (one workgroup per map row and 64-channel group): the spectral_in
//          product for the row's pixels, bias, ReLU, f16 (the spectral map,
//          also stored for the residual), then the row transform of those
//          channels: R[y][m][c], m < w the real parts of columns 0 .. w / 2
//          and the imaginary parts of columns 1 .. w - half (the others are
//          zero for a real row), f32.
//   columns (one workgroup per spectrum column and group of 32 channels):
//          the column's R for every row and channel, the complex transform
//          down the column (x 1 / sqrt(h w)) for all 192 channels into f16
//          (the spectrum), the fourier product for the group's real and
//          imaginary output channels with bias and ReLU into f16 (filtered),
//          and their inverse column transform: U[y][k][re | im], f32.
//   back   (one workgroup per map row and 128-channel output group): the
//          row's U, its inverse real transform (irfftn's C2R rule: the
//          imaginary parts of column 0 and, for an even width, column w / 2
//          are not read; x 1 / sqrt(h w)), added to the spectral map in f32
//          and rounded to f16, then the spectral_out product accumulated onto
//          the cross output with ReLU.
//
// Every product runs on v_mfma_f32_32x32x16_f16.  The transforms are real
// matrix products with tables built in double on the host; to keep their
// sums at f32 accuracy, an f32 operand v enters as the two halves
// hi = f16(v), lo = f16(v - hi) and each table entry likewise, and a product
// sums hi.hi + lo.hi + hi.lo (|error| about 2^-22 of the terms): the split is
// one more stretch of the reduction (K) dimension.  f32 intermediates are
// scaled by powers of two before the split (R by 2^-6, U by 2^-8, undone in
// the tables) so that no half overflows.  The rounding points are those of
// the unfused path: the spectral map, the spectrum and the filtered spectrum
// in f16, the transforms' sums in f32.
//
// The MFMA reduction dimension has to run along a lane's registers, so
// every intermediate is laid out with the next reduction's index
// contiguous: the spectral row transposed in LDS ([channel][x]), R and U
// transposed into LDS as they are loaded (eight rows of four channels per
// thread, written as 16-byte rows of eight points), the spectrum row-major
// over channels ([ky][c']) for the fourier product, its output transposed
// ([n][ky]) for the inverse columns.

#include <cmath>
#include <vector>

#include "conv_common.h"

namespace ien {
namespace {

constexpr int GLOBAL_C = 384;  // the FFC's global channels (the product's input)
constexpr int SPEC = 192;      // spectral channels
constexpr int SPEC2 = 384;     // spectrum values per pixel: re x 192 | im x 192
constexpr int MAX_SIDE = 64;
constexpr float RSCALE = 1.0f / 64, USCALE = 1.0f / 256;
constexpr int COLUMN_GROUPS = 6;  // 32 channels a columns workgroup
constexpr int BACK_GROUPS = 3;    // 128 output channels a back workgroup

__device__ __forceinline__ half8 ld8(const uint16_t *p) { return *(const half8 *)p; }
__device__ __forceinline__ floatx16 mfma16(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void st4h(uint16_t *p, float a, float b, float c, float d) {
  uint2 v;
  v.x = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
  v.y = (uint32_t)f2h(c) | ((uint32_t)f2h(d) << 16);
  *(uint2 *)p = v;
}
// Eight f32 values (pre-scaled) as the hi and lo halves.
__device__ __forceinline__ void split8(const float *v, half8 &hi, half8 &lo) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const _Float16 a = (_Float16)v[j];
    hi[j] = a;
    lo[j] = (_Float16)(v[j] - (float)a);
  }
}

// ---- front: spectral_in product and the row transform ---------------------

struct FrontArgs {
  const uint16_t *x;
  int xs;  // halves between pixels of x
  int h, w, xp, mb;  // xp: w rounded up to 16; mb: 32-row blocks of R (w)
  const uint16_t *w_in;
  int kb_in;
  const float *b_in;
  const uint16_t *tf;  // A fragments [mb][2 xp / 16]: hi, then lo table
  uint16_t *s;         // spectral map, channel-major per row: [h][192][w]
  float *r;            // [h][w][192]
};

constexpr int SP = MAX_SIDE + 8;  // halves per transposed spectral row
// LDS of the front workgroup (bytes): the row's pixels [x][48 chunks of 16
// bytes], chunk c of pixel x at slot c ^ (x % 16), so that the 16 lanes of
// a fragment read that take one chunk of 16 pixels fall on distinct banks;
// the group's weight fragments [n block][k step]; the table's fragments
// [m block][step]; the spectral row transposed [channel][x].
constexpr int F_PIX = 0, F_W = 48 * 1024, F_T = 96 * 1024, F_ST = 112 * 1024;
constexpr int FRONT_LDS = F_ST + 64 * SP * 2;

__global__ __launch_bounds__(256) void k_spectral_front(FrontArgs p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[FRONT_LDS];
  uint16_t *st = (uint16_t *)(lds + F_ST);
  const int y = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  constexpr int KS = GLOBAL_C / 16;
  const int ks_t = p.xp / 8;  // 2 xp / 16 <= 8 table steps
  // Every global byte the workgroup reads is requested once, straight into
  // LDS (one KiB a wave instruction, consecutive 16-byte chunks of a pixel
  // row, weight fragment or table fragment).
  {
    const uint16_t *row = p.x + (long)y * p.w * p.xs;
    for (int f = wave; f < 48; f += 4) {
      const int q = 64 * f + lane, x = q / 48, c = (q - 48 * x) ^ (x & 15);
      dma16(row + (long)min(x, p.w - 1) * p.xs + 8 * c, lds + F_PIX + f * 1024);
    }
    const uint16_t *wg = p.w_in + (long)(2 * g) * p.kb_in * 512 + lane * 8;
    for (int f = wave; f < 2 * KS; f += 4) {
      const int nblk = f / KS, ks = f - nblk * KS;
      dma16(wg + ((long)nblk * p.kb_in + ks) * 512, lds + F_W + f * 1024);
    }
    for (int f = wave; f < p.mb * ks_t; f += 4) {
      const int mblk = f / ks_t, i = f - mblk * ks_t;
      dma16(p.tf + (long)f * 512 + lane * 8, lds + F_T + (mblk * 8 + i) * 1024);
    }
  }
  const int nblk = wave & 1, xblk = wave >> 1;  // the product's block
  float4v bias[4];
#pragma unroll
  for (int q = 0; q < 4; q++) bias[q] = *(const float4v *)(p.b_in + 64 * g + nblk * 32 + 8 * q + 4 * hi);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the direct-to-LDS loads have landed
  __syncthreads();
  {
    // D[n][x] = sum_k W[k][n] x[x][k]: the weights as the A operand, pixels
    // as the B operand (eight consecutive channels of a pixel per lane).
    if (xblk * 32 < p.w) {
      const int x = xblk * 32 + col, sx = x & 15;
      const unsigned char *wa = lds + F_W + nblk * KS * 1024 + lane * 16;
      const unsigned char *xa = lds + F_PIX + x * 768;
      floatx16 acc = {};
#pragma unroll
      for (int i = 0; i < KS; i++)
        acc = mfma16(*(const half8 *)(wa + i * 1024), *(const half8 *)(xa + (((2 * i + hi) ^ sx) << 4)), acc);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int n0 = nblk * 32 + 8 * q + 4 * hi;  // channel within the group
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = fmaxf(acc[4 * q + j] + bias[q][j], 0.0f);
        if (x < p.w) {
          uint16_t *sr = p.s + ((long)y * SPEC + 64 * g + n0) * p.w + x;
#pragma unroll
          for (int j = 0; j < 4; j++) sr[(long)j * p.w] = f2h(v[j]);
        }
        if (x < p.xp) {
#pragma unroll
          for (int j = 0; j < 4; j++) st[(n0 + j) * SP + x] = x < p.w ? f2h(v[j]) : (uint16_t)0;
        }
      }
    }
  }
  __syncthreads();
  {
    // D[m][c] = sum_x F[m][x] S[x][c], the table (hi, then lo) as the A
    // operand, the spectral row (twice) as the B operand.
    const int cblk = wave & 1, mblk = wave >> 1;
    if (mblk < p.mb) {
      const int c = cblk * 32 + col;
      const unsigned char *ta = lds + F_T + mblk * 8 * 1024 + lane * 16;
      floatx16 acc = {};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (i < ks_t) {
          const int x0 = (16 * i + 8 * hi) % p.xp;
          acc = mfma16(*(const half8 *)(ta + i * 1024), ld8(st + c * SP + x0), acc);
        }
      }
      float *out = p.r + (long)y * p.w * SPEC + 64 * g + c;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = mblk * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (m < p.w) out[(long)m * SPEC] = acc[r];
      }
    }
  }
}

// ---- columns: column transform, fourier product, inverse columns ----------

struct ColumnArgs {
  const float *r;
  int h, w, half, yp, nba;  // yp: h rounded up to 16; nba: 32-blocks of 2h
  const uint16_t *ta;       // B fragments [nba][4 yp / 16]: (hi | lo, part, y)
  const uint16_t *tc;       // B fragments [nba][4 yp / 16]: (hi | lo, part, ky)
  const uint16_t *wf;
  int kb_f;
  const float *b_f;
  float *u;  // [h][half][384]
};

constexpr int RP = MAX_SIDE + 8;                        // halves per transposed R row
constexpr int R_PLANE = SPEC2 * RP;                     // one of the hi / lo planes
constexpr int ZP = SPEC2 + 8;                           // halves per spectrum row
constexpr int COL_LDS = 2 * R_PLANE + MAX_SIDE * ZP;    // halves: 160768 bytes
constexpr int US_OFF = 8192, US_P = 36;                 // U staging (halves offset, floats a row)

__global__ __launch_bounds__(512) void k_spectral_columns(ColumnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[COL_LDS];
  uint16_t *rhi = lds, *rlo = lds + R_PLANE, *z = lds + 2 * R_PLANE;
  // After the column transform, over rhi: the filtered spectrum [2 x 32][RP]
  // and the inverse columns' outputs [2h][US_P] f32 on their way out.
  uint16_t *pt = lds;
  float *ustage = (float *)(lds + US_OFF);
  // Block b runs on XCD b % 8: the groups of column k all take XCD k % 8,
  // so the column's R comes from memory once and from that XCD's L2 after.
  // Slots past the last column exit at once.
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int k = xcd + 8 * (slot / COLUMN_GROUPS), g = slot % COLUMN_GROUPS, tid = threadIdx.x;
  if (k >= p.half) return;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int h = p.h, yp = p.yp, ysteps = yp / 16, ks2 = 2 * ysteps;
  constexpr int CG = SPEC / COLUMN_GROUPS, KF = SPEC2 / 16, YS = MAX_SIDE / 16;
  // Roles: every wave takes a quarter of the column transform's outputs
  // (column block nb = w % 4, channel blocks w / 4 + 2 j); waves 0 .. 3
  // then the fourier product (row block w / 2, real or imaginary outputs
  // w % 2), waves 4 .. 7 the inverse columns (column block w - 4).  The
  // column transform's table fragments (hi and lo for each part and y step)
  // and the product's bias are requested first, then R.
  const int nb = wave & 3;
  half8 thi[2][YS], tlo[2][YS];
  {
    const uint16_t *tb = p.ta + (long)min(nb, p.nba - 1) * 2 * ks2 * 512 + lane * 8;
#pragma unroll
    for (int part = 0; part < 2; part++)
#pragma unroll
      for (int ys = 0; ys < YS; ys++) {
        const int s = part * ysteps + min(ys, ysteps - 1);
        thi[part][ys] = ld8(tb + s * 512);
        tlo[part][ys] = ld8(tb + (ks2 + s) * 512);
      }
  }
  const int pb = wave >> 1, ppart = wave & 1;  // fourier product block
  const int nbm = (ppart * SPEC + CG * g) / 32;
  const float bias = p.b_f[nbm * 32 + col];
  // R of this column for every row: the real parts at row k of R, the
  // imaginary ones at row half + k - 1 (none for k = 0 or k > w - half),
  // scaled and split into [part 192 + c][y].  At most two items a thread,
  // both loaded before either is stored.
  {
    const int mim = (k >= 1 && k <= p.w - p.half) ? p.half + k - 1 : -1;
    const int yg = yp / 8, per_part = (SPEC / 4) * yg, items = 2 * per_part;
    float4v v[2][8];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int it = min(tid + 512 * b, items - 1);
      const int part = it / per_part, rem = it - part * per_part;
      const int c4 = rem / yg, y0 = (rem % yg) * 8;
      const int m = part ? mim : k;
      const int at0 = (y0 * p.w + m) * SPEC + 4 * c4, step = p.w * SPEC;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const bool ok = m >= 0 && y0 + j < h;
        v[b][j] = *(const float4v *)(p.r + (ok ? at0 + j * step : 0));
        if (!ok) v[b][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int it = tid + 512 * b;
      if (it < items) {
        const int part = it / per_part, rem = it - part * per_part;
        const int c4 = rem / yg, y0 = (rem % yg) * 8;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
          float f[8];
#pragma unroll
          for (int j = 0; j < 8; j++) f[j] = v[b][j][cc] * RSCALE;
          half8 vh, vl;
          split8(f, vh, vl);
          const int row = part * SPEC + 4 * c4 + cc;
          *(half8 *)(rhi + row * RP + y0) = vh;
          *(half8 *)(rlo + row * RP + y0) = vl;
        }
      }
    }
  }
  __syncthreads();
  // Column transform: D[c][(part', ky)] = sum over (part, y) of
  // (Rhi Thi + Rlo Thi + Rhi Tlo)[part][c][y] x [(part, y)][(part', ky)].
  floatx16 acc[3] = {};
  if (nb < p.nba) {
    const int cb0 = wave >> 2;
#pragma unroll
    for (int ys = 0; ys < YS; ys++) {
      if (ys < ysteps) {
#pragma unroll
        for (int part = 0; part < 2; part++) {
          const int off = (part * SPEC + 32 * cb0 + col) * RP + ys * 16 + 8 * hi;
#pragma unroll
          for (int j = 0; j < 3; j++) {
            const half8 ah = ld8(rhi + off + 64 * j * RP), al = ld8(rlo + off + 64 * j * RP);
            acc[j] = mfma16(ah, thi[part][ys], acc[j]);
            acc[j] = mfma16(al, thi[part][ys], acc[j]);
            acc[j] = mfma16(ah, tlo[part][ys], acc[j]);
          }
        }
      }
    }
  }
  // The next phase's operands, requested before this phase's results are
  // stored: the fourier weights (waves 0 .. 3), the inverse table (4 .. 7).
  const int mbs = (h + 31) / 32;
  const int nbc = wave - 4;  // inverse columns block
  half8 wf[KF];
  if (wave < 4) {
    const uint16_t *wb = p.wf + (long)nbm * p.kb_f * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < KF; i++) wf[i] = ld8(wb + i * 512);
  } else {
    // Slot (t, part, ys) holds the fragment of step t ks2 + part ysteps + ys.
    const uint16_t *tb = p.tc + (long)min(max(nbc, 0), p.nba - 1) * 2 * ks2 * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < 4 * YS; i++) {
      const int t = i / (2 * YS), part = (i / YS) & 1, ys = min(i % YS, ysteps - 1);
      wf[i] = ld8(tb + (t * ks2 + part * ysteps + ys) * 512);
    }
  }
  if (nb < p.nba) {
    const int cb0 = wave >> 2;
    const int n = nb * 32 + col;
    if (n < 2 * h) {
      const int pp = n >= h, ky = n - pp * h;
      uint16_t *zr = z + ky * ZP + pp * SPEC;
#pragma unroll
      for (int j = 0; j < 3; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int c0 = 32 * (cb0 + 2 * j) + 8 * q + 4 * hi;
          st4h(zr + c0, acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]);
        }
    }
  }
  __syncthreads();
  // Fourier product over the spectrum pixels of this column for the
  // group's output channels (CG real parts, CG imaginary parts):
  // D[ky][n] = sum_c' Z[ky][c'] W[c'][n], bias, ReLU, f16, into [n][ky].
  if (wave < 4 && pb < mbs) {
    const uint16_t *za = z + (pb * 32 + col) * ZP + 8 * hi;
    floatx16 d = {};
#pragma unroll
    for (int i = 0; i < KF; i++) d = mfma16(ld8(za + 16 * i), wf[i], d);
    uint16_t *dst = pt + (ppart * CG + col) * RP;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int ky0 = pb * 32 + 8 * q + 4 * hi;
      if (ky0 < yp) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = ky0 + j < h ? fmaxf(d[4 * q + j] + bias, 0.0f) : 0.0f;
        st4h(dst + ky0, v[0], v[1], v[2], v[3]);
      }
    }
  }
  __syncthreads();
  // Inverse columns: D[c][(part', y)] = sum over (term, part, ky) of
  // P[part][c][ky] Ti_term[(part, ky)][(part', y)]; terms hi, lo; staged as
  // [(part', y)][c] for whole-line stores.
  if (wave >= 4 && nbc < p.nba) {
    floatx16 d = {};
#pragma unroll
    for (int i = 0; i < 4 * YS; i++) {
      const int part = (i / YS) & 1, ys = i % YS;
      if (ys < ysteps) d = mfma16(ld8(pt + (part * CG + col) * RP + ys * 16 + 8 * hi), wf[i], d);
    }
    const int n = nbc * 32 + col;
#pragma unroll
    for (int q = 0; q < 4; q++)
      *(float4v *)(ustage + n * US_P + 8 * q + 4 * hi) =
          float4v{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
  }
  __syncthreads();
  // U[y][k][part' 192 + 32 g + c]: 8 lanes write one 128-byte line.
  for (int q = tid; q < 2 * h * 8; q += 512) {
    const int n = q >> 3, c4 = q & 7;
    const int pp = n >= h, yy = n - pp * h;
    *(float4v *)(p.u + ((yy * p.half + k) * SPEC2 + pp * SPEC + CG * g + 4 * c4)) =
        *(const float4v *)(ustage + n * US_P + 4 * c4);
  }
}

// ---- back: inverse rows, residual, spectral_out product -------------------

struct BackArgs {
  const float *u;
  int h, w, half, mp, nbx;  // mp: w rounded up to 16; nbx: 32-blocks of w
  const uint16_t *tr;       // B fragments [nbx][2 mp / 16]: (hi | lo, m)
  const uint16_t *s;        // spectral map [h][192][w]
  const uint16_t *wo;
  int kb_o;
  uint16_t *out;
  int ys;
  // Where the result goes (rows ys apart, out's layout) and a map added to
  // it after the ReLU and rounding, rounded again (or null).
  uint16_t *dst;
  const uint16_t *add;
};

constexpr int UP = MAX_SIDE + 8;
constexpr int U_PLANE = SPEC * UP;
constexpr int S2P = SPEC + 8;
constexpr int OBP = 136;  // halves a pixel of the staged output (128 + a pad chunk)
// LDS of the back workgroup (bytes): U's hi and lo planes [c][m] (later the
// staged output [x][OBP]), the updated spectral row [x][c], the group's
// spectral_out fragments [n block][k step], the spectral row [c][x].
constexpr int B_S2 = 2 * U_PLANE * 2, B_W = B_S2 + MAX_SIDE * S2P * 2;
constexpr int B_ST = B_W + 4 * 12 * 1024, BACK_LDS = B_ST + SPEC * MAX_SIDE * 2;
static_assert(B_W % 1024 == 0 && B_ST % 1024 == 0, "DMA targets on whole KiB");
static_assert(MAX_SIDE * OBP * 2 <= B_S2, "staged output over U");

__global__ __launch_bounds__(256) void k_spectral_back(BackArgs p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[BACK_LDS];
  uint16_t *uhi = (uint16_t *)lds, *ulo = uhi + U_PLANE, *s2 = (uint16_t *)(lds + B_S2);
  uint16_t *ob = (uint16_t *)lds;  // after the inverse rows
  const uint16_t *srow = (const uint16_t *)(lds + B_ST);
  const int y = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int msteps = p.mp / 16, w = p.w;
  constexpr int MS = MAX_SIDE / 16, NG = SPEC2 / BACK_GROUPS, KO = SPEC / 16;
  static_assert(NG / 32 * KO == 48, "spectral_out fragments of a group");
  // Roles: in the inverse rows, wave w takes column block nb = w % nbx and
  // channel blocks w / nbx + (4 / nbx) j (at most three); in the
  // spectral_out product, blocks w and w + 4 of (output block, column
  // block).  Requested first: the weights and the spectral row straight
  // into LDS, the table into registers, then U.
  const int nb = wave % p.nbx, cstep = 4 / p.nbx, cb0 = wave / p.nbx;
  const int nblocks = (NG / 32) * p.nbx;
  {
    const uint16_t *wg = p.wo + (long)((NG * g) / 32) * p.kb_o * 512 + lane * 8;
    for (int f = wave; f < NG / 32 * KO; f += 4) {
      const int nbl = f / KO, i = f - nbl * KO;
      dma16(wg + ((long)nbl * p.kb_o + i) * 512, lds + B_W + f * 1024);
    }
    const uint16_t *sg = p.s + (long)y * SPEC * w;
    const int chunks = SPEC * w / 8;
    for (int f = wave; f * 64 < chunks; f += 4) dma16(sg + 8 * min(64 * f + lane, chunks - 1), lds + B_ST + f * 1024);
  }
  half8 thi[MS], tlo[MS];
  {
    const uint16_t *tb = p.tr + (long)nb * 2 * msteps * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < MS; i++) {
      thi[i] = ld8(tb + min(i, msteps - 1) * 512);
      tlo[i] = ld8(tb + (msteps + min(i, msteps - 1)) * 512);
    }
  }
  // U of this row in the order of R's rows (m < half: real parts of column
  // m; half <= m < w: imaginary parts of column m - half + 1), scaled and
  // split into [c][m].  At most two items a thread, both loaded first.
  {
    const int mg = p.mp / 8, items = (SPEC / 4) * mg;
    float4v v[2][8];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int it = min(tid + 256 * b, items - 1);
      const int c4 = it / mg, m0 = (it % mg) * 8;
      const int row0 = y * p.half * SPEC2 + 4 * c4;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int m = m0 + j;
        const bool ok = m < w, im = m >= p.half;
        const int at = im ? (m - p.half + 1) * SPEC2 + SPEC : m * SPEC2;
        v[b][j] = *(const float4v *)(p.u + row0 + (ok ? at : 0));
        if (!ok) v[b][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int it = tid + 256 * b;
      if (it < items) {
        const int c4 = it / mg, m0 = (it % mg) * 8;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
          float f[8];
#pragma unroll
          for (int j = 0; j < 8; j++) f[j] = v[b][j][cc] * USCALE;
          half8 vh, vl;
          split8(f, vh, vl);
          *(half8 *)(uhi + (4 * c4 + cc) * UP + m0) = vh;
          *(half8 *)(ulo + (4 * c4 + cc) * UP + m0) = vl;
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the direct-to-LDS loads have landed
  __syncthreads();
  // Inverse rows: D[c][x] = sum over m of (Uhi Thi + Ulo Thi + Uhi Tlo)[c][m]
  // x [m][x].  Then + the spectral map, f16, into [x][c].
  {
    const int x = nb * 32 + col, xc = min(x, w - 1);
#pragma unroll
    for (int j = 0; j < 3; j++) {
      const int cb = cb0 + cstep * j;
      if (cb < SPEC / 32) {
        floatx16 acc = {};
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
          if (ms < msteps) {
            const int off = (cb * 32 + col) * UP + ms * 16 + 8 * hi;
            const half8 ah = ld8(uhi + off), al = ld8(ulo + off);
            acc = mfma16(ah, thi[ms], acc);
            acc = mfma16(al, thi[ms], acc);
            acc = mfma16(ah, tlo[ms], acc);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int c0 = cb * 32 + 8 * q + 4 * hi;
          const uint16_t *sc = srow + c0 * w + xc;
          st4h(s2 + x * S2P + c0, acc[4 * q] + h2f(sc[0]), acc[4 * q + 1] + h2f(sc[w]),
               acc[4 * q + 2] + h2f(sc[2 * w]), acc[4 * q + 3] + h2f(sc[3 * w]));
        }
      }
    }
  }
  __syncthreads();
  // The cross output of this row's group channels, into [x][OBP] over U
  // (16 data chunks and a pad chunk a pixel), behind the product below.
  {
    const uint16_t *og = p.out + (long)y * w * p.ys + NG * g;
    for (int f = wave; f * 64 < 17 * w; f += 4) {
      const int q = 64 * f + lane, x = min(q / 17, w - 1), c = q % 17;
      dma16(og + (long)x * p.ys + 8 * (c & 15), lds + f * 1024);
    }
  }
  // The residual this row's results are added to (when there is one): at
  // most 4 of its 16-byte items a thread (16 w items, w <= 64), requested
  // now so that their latency passes behind the product below.
  constexpr int AITEMS = 16 * MAX_SIDE / 256;
  const long orow = (long)y * w * p.ys + NG * g;
  u32x4 addv[AITEMS];
  if (p.add) {
#pragma unroll
    for (int i = 0; i < AITEMS; i++) {
      const int q = tid + 256 * i, x = min(q >> 4, w - 1), c = q & 15;
      addv[i] = *(const u32x4 *)(p.add + orow + (long)x * p.ys + 8 * c);
    }
  }
  // spectral_out: D[n][x] = sum_c W[c][n] S2[x][c], the weights as the A
  // operand; out = ReLU(out + D), staged in LDS.
  floatx16 dacc[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int b = wave + 4 * j;
    dacc[j] = floatx16{};
    if (b < nblocks) {
      const int nbl = b / p.nbx, xb = b % p.nbx;
      const uint16_t *sb = s2 + (xb * 32 + col) * S2P + 8 * hi;
      const unsigned char *wa = lds + B_W + nbl * KO * 1024 + lane * 16;
#pragma unroll
      for (int i = 0; i < KO; i++) dacc[j] = mfma16(*(const half8 *)(wa + i * 1024), ld8(sb + 16 * i), dacc[j]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the staged cross output has landed
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int b = wave + 4 * j;
    if (b < nblocks) {
      const int nbl = b / p.nbx, x = (b % p.nbx) * 32 + col;
      uint16_t *o = ob + x * OBP + nbl * 32;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint16_t *e = o + 8 * q + 4 * hi;
        const uint2 ov = *(const uint2 *)e;
        st4h(e, fmaxf(h2f((uint16_t)ov.x) + dacc[j][4 * q], 0.0f),
             fmaxf(h2f((uint16_t)(ov.x >> 16)) + dacc[j][4 * q + 1], 0.0f),
             fmaxf(h2f((uint16_t)ov.y) + dacc[j][4 * q + 2], 0.0f),
             fmaxf(h2f((uint16_t)(ov.y >> 16)) + dacc[j][4 * q + 3], 0.0f));
      }
    }
  }
  __syncthreads();
  // 16 lanes write one pixel's 256 bytes.
  {
    uint16_t *og = p.dst + orow;
    if (p.add) {
#pragma unroll
      for (int i = 0; i < AITEMS; i++) {
        const int q = tid + 256 * i, x = q >> 4, c = q & 15;
        if (q < 16 * w) {
          uint16_t o[8], h[8];
          *(u32x4 *)o = *(const u32x4 *)(ob + x * OBP + 8 * c);
          *(u32x4 *)h = addv[i];
#pragma unroll
          for (int e = 0; e < 8; e++) o[e] = f2h(h2f(o[e]) + h2f(h[e]));
          *(u32x4 *)(og + (long)x * p.ys + 8 * c) = *(const u32x4 *)o;
        }
      }
    } else {
      for (int q = tid; q < 16 * w; q += 256) {
        const int x = q >> 4, c = q & 15;
        *(u32x4 *)(og + (long)x * p.ys + 8 * c) = *(const u32x4 *)(ob + x * OBP + 8 * c);
      }
    }
  }
}

// ---- host: the tables ------------------------------------------------------

float half_bits_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1f;
  const uint32_t m = h & 0x3ffu;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 0x400u), e - 25);
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

// term 0: f16(v); term 1: f16(v - f16(v)).
uint16_t split_half(double v, int term) {
  const float f = (float)v;
  const uint16_t hi = f32_to_half(f);
  return term == 0 ? hi : f32_to_half(f - half_bits_to_float(hi));
}

// Fragments of an MFMA operand: fragment (blk, ks) holds value(32 blk + l %
// 32, 16 ks + 8 (l / 32) + i) at lane l, element i (the layout of both the A
// operand, rows x k, and the B operand, columns x k).
template <typename F>
std::vector<uint16_t> operand(int blocks, int ksteps, F value) {
  std::vector<uint16_t> out((size_t)blocks * ksteps * 512);
  for (int blk = 0; blk < blocks; blk++)
    for (int ks = 0; ks < ksteps; ks++)
      for (int l = 0; l < 64; l++)
        for (int i = 0; i < 8; i++)
          out[((size_t)blk * ksteps + ks) * 512 + l * 8 + i] =
              value(32 * blk + l % 32, 16 * ks + 8 * (l / 32) + i);
  return out;
}

int up16(int n) { return (n + 15) / 16 * 16; }

}  // namespace
}  // namespace ien

using namespace ien;

struct ien_spectral {
  ien_ctx *ctx = nullptr;
  int h = 0, w = 0, half = 0, xp = 0, yp = 0, mb = 0, nba = 0, nbx = 0;
  uint16_t *d_tf = nullptr, *d_ta = nullptr, *d_tc = nullptr, *d_tr = nullptr;
};

namespace ien {

bool spectral_shapes(const ien_matrix *in, const ien_matrix *f, const ien_matrix *out) {
  return in && f && out && in->k == GLOBAL_C && in->n == SPEC && in->d_bias && f->k == SPEC2 &&
         f->n == SPEC2 && f->d_bias && out->k == SPEC && out->n == SPEC2;
}

ien_status spectral_rows(const ien_spectral *sp, const uint16_t *x, long xs,
                         const ien_matrix *m_in, uint16_t *spectral, float *r) {
  ien_ctx *ctx = sp->ctx;
  FrontArgs a{x, (int)xs, sp->h, sp->w, sp->xp, sp->mb, m_in->d_packed, m_in->kb, m_in->d_bias,
              sp->d_tf, spectral, r};
  hipLaunchKernelGGL(k_spectral_front, dim3((unsigned)sp->h, SPEC / 64), dim3(256), 0, ctx->stream,
                     a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status spectral_columns(const ien_spectral *sp, const ien_matrix *m_f, const float *r,
                            float *u) {
  ien_ctx *ctx = sp->ctx;
  ColumnArgs c{r, sp->h, sp->w, sp->half, sp->yp, sp->nba, sp->d_ta, sp->d_tc, m_f->d_packed,
               m_f->kb, m_f->d_bias, u};
  const unsigned column_blocks = 8u * COLUMN_GROUPS * (unsigned)((sp->half + 7) / 8);
  hipLaunchKernelGGL(k_spectral_columns, dim3(column_blocks), dim3(512), 0, ctx->stream, c);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status spectral_front(const ien_spectral *sp, const uint16_t *x, long xs,
                          const ien_matrix *m_in, const ien_matrix *m_f, uint16_t *spectral,
                          float *r, float *u) {
  const ien_status st = spectral_rows(sp, x, xs, m_in, spectral, r);
  return st == IEN_OK ? spectral_columns(sp, m_f, r, u) : st;
}

ien_status spectral_back(const ien_spectral *sp, const ien_matrix *m_out, const uint16_t *spectral,
                         const float *u, uint16_t *out, long ys, uint16_t *dst,
                         const uint16_t *add) {
  ien_ctx *ctx = sp->ctx;
  IEN_CHECK((((uintptr_t)dst | (uintptr_t)add) & 15) == 0, IEN_ERR_INPUT,
            "spectral output and added map 16-byte aligned");
  BackArgs b{u, sp->h, sp->w, sp->half, sp->xp, sp->nbx, sp->d_tr, spectral, m_out->d_packed,
             m_out->kb, out, (int)ys, dst ? dst : out, add};
  hipLaunchKernelGGL(k_spectral_back, dim3((unsigned)sp->h, BACK_GROUPS), dim3(256), 0,
                     ctx->stream, b);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

size_t spectral_r_floats(const ien_spectral *sp) { return (size_t)sp->h * sp->w * SPEC; }
size_t spectral_u_floats(const ien_spectral *sp) { return (size_t)sp->h * sp->half * SPEC2; }

}  // namespace ien

extern "C" {

ien_status ien_spectral_new(ien_ctx *ctx, size_t height, size_t width, ien_spectral **out) {
  IEN_CHECK(ctx && out, IEN_ERR_INPUT, "null argument");
  *out = nullptr;
  IEN_CHECK(height >= 1 && width >= 1 && height <= MAX_SIDE && width <= MAX_SIDE, IEN_ERR_INPUT,
            "spectral unit of %zu x %zu (sides 1 .. %d)", width, height, MAX_SIDE);
  IEN_HIP(hipSetDevice(ctx->device));
  const int h = (int)height, w = (int)width, half = w / 2 + 1;
  ien_spectral *sp = new ien_spectral;
  sp->ctx = ctx;
  sp->h = h;
  sp->w = w;
  sp->half = half;
  sp->xp = up16(w);
  sp->yp = up16(h);
  sp->mb = (w + 31) / 32;
  sp->nba = (2 * h + 31) / 32;
  sp->nbx = (w + 31) / 32;
  const double tau = 6.283185307179586476925, s = 1.0 / std::sqrt((double)h * w);
  const int xp = sp->xp, yp = sp->yp;
  // Row transform (A operand, rows m of R): cos for the real parts of
  // columns m < half, -sin for the imaginary parts of columns m - half + 1.
  const std::vector<uint16_t> tf = operand(sp->mb, 2 * xp / 16, [&](int m, int kk) -> uint16_t {
    const int term = kk / xp, x = kk % xp;
    if (m >= w || x >= w) return 0;
    const int col = m < half ? m : m - half + 1;
    const double a = tau * (double)((long)col * x % w) / w;
    return split_half(m < half ? std::cos(a) : -std::sin(a), term);
  });
  // Column transform (B operand, columns (part', ky)), x 1 / sqrt(h w) x 64:
  // (a + i b) e^{-i theta}.  K: (term, part, y), terms hi, lo.
  const std::vector<uint16_t> ta = operand(sp->nba, 4 * yp / 16, [&](int n, int kk) -> uint16_t {
    const int term = kk / (2 * yp), part = (kk % (2 * yp)) / yp, y = kk % yp;
    if (n >= 2 * h || y >= h) return 0;
    const int pp = n / h, ky = n % h;
    const double a = tau * (double)((long)ky * y % h) / h, c = std::cos(a), sn = std::sin(a);
    const double v = pp == 0 ? (part == 0 ? c : sn) : (part == 0 ? -sn : c);
    return split_half(v * s * 64.0, term);
  });
  // Inverse columns (B operand, columns (part', y)): (a + i b) e^{+i theta}.
  // K: (term, part, ky), terms hi, lo.
  const std::vector<uint16_t> tc = operand(sp->nba, 4 * yp / 16, [&](int n, int kk) -> uint16_t {
    const int term = kk / (2 * yp), part = (kk % (2 * yp)) / yp, ky = kk % yp;
    if (n >= 2 * h || ky >= h) return 0;
    const int pp = n / h, y = n % h;
    const double a = tau * (double)((long)ky * y % h) / h, c = std::cos(a), sn = std::sin(a);
    const double v = pp == 0 ? (part == 0 ? c : -sn) : (part == 0 ? sn : c);
    return split_half(v, term);
  });
  // Inverse rows (B operand, columns x), x 1 / sqrt(h w) x 256: the real
  // parts of column k times w_k cos, the imaginary parts times -w_k sin,
  // w_k = 1 for column 0 and (even w) w / 2, else 2.  K: (term, m), terms
  // hi, lo.
  const std::vector<uint16_t> tr = operand(sp->nbx, 2 * xp / 16, [&](int x, int kk) -> uint16_t {
    const int term = kk / xp, m = kk % xp;
    if (x >= w || m >= w) return 0;
    const int col = m < half ? m : m - half + 1;
    const double wk = (col == 0 || 2 * col == w) ? 1.0 : 2.0;
    const double a = tau * (double)((long)col * x % w) / w;
    const double v = m < half ? wk * std::cos(a) : -wk * std::sin(a);
    return split_half(v * s * 256.0, term);
  });
  auto put = [](uint16_t **d, const std::vector<uint16_t> &v) {
    hipError_t e = hipMalloc((void **)d, v.size() * 2);
    return e == hipSuccess ? hipMemcpy(*d, v.data(), v.size() * 2, hipMemcpyHostToDevice) : e;
  };
  hipError_t e = put(&sp->d_tf, tf);
  if (e == hipSuccess) e = put(&sp->d_ta, ta);
  if (e == hipSuccess) e = put(&sp->d_tc, tc);
  if (e == hipSuccess) e = put(&sp->d_tr, tr);
  if (e != hipSuccess) {
    ien_spectral_free(sp);
    return fail(IEN_ERR_GPU, "spectral tables: %s", hipGetErrorString(e));
  }
  *out = sp;
  return IEN_OK;
}

void ien_spectral_free(ien_spectral *sp) {
  if (!sp) return;
  (void)hipFree(sp->d_tf);
  (void)hipFree(sp->d_ta);
  (void)hipFree(sp->d_tc);
  (void)hipFree(sp->d_tr);
  delete sp;
}

size_t ien_spectral_work(const ien_spectral *sp) {
  return sp ? spectral_r_floats(sp) + spectral_u_floats(sp) : 0;
}

ien_status ien_spectral_run(const ien_spectral *sp, const uint16_t *d_x, size_t stride,
                            const ien_matrix *spectral_in, const ien_matrix *fourier,
                            const ien_matrix *spectral_out, uint16_t *d_spectral, float *d_work,
                            uint16_t *d_out, size_t out_stride) {
  IEN_CHECK(sp && d_x && d_spectral && d_work && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(spectral_shapes(spectral_in, fourier, spectral_out), IEN_ERR_INPUT,
            "spectral matrices must be %d x %d with bias, %d x %d with bias and %d x %d", GLOBAL_C,
            SPEC, SPEC2, SPEC2, SPEC, SPEC2);
  IEN_CHECK(stride >= GLOBAL_C && stride % 8 == 0 && ((uintptr_t)d_x & 15) == 0, IEN_ERR_INPUT,
            "input pixel stride %zu (a multiple of 8 >= %d, 16-byte aligned)", stride, GLOBAL_C);
  IEN_CHECK(out_stride >= SPEC2 && out_stride % 8 == 0 && ((uintptr_t)d_out & 15) == 0 &&
                ((uintptr_t)d_spectral & 15) == 0 && ((uintptr_t)d_work & 15) == 0,
            IEN_ERR_INPUT, "output pixel stride %zu (a multiple of 8 >= %d), alignment", out_stride,
            SPEC2);
  float *r = d_work, *u = d_work + spectral_r_floats(sp);
  ien_status st = spectral_front(sp, d_x, (long)stride, spectral_in, fourier, d_spectral, r, u);
  if (st == IEN_OK)
    st = spectral_back(sp, spectral_out, d_spectral, u, d_out, (long)out_stride, nullptr, nullptr);
  return st;
}

}  // extern "C"
