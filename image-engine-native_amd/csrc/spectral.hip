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
  uint16_t *s;         // spectral map [h][w][192]
  float *r;            // [h][w][192]
};

constexpr int SP = MAX_SIDE + 8;  // halves per transposed spectral row

__global__ __launch_bounds__(256) void k_spectral_front(FrontArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t st[64 * SP];
  const int y = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  {
    // D[n][x] = sum_k W[k][n] x[x][k]: the weights as the A operand, pixels
    // as the B operand (eight consecutive channels of a pixel per lane).
    const int nblk = wave & 1, xblk = wave >> 1;
    if (xblk * 32 < p.w) {
      const int x = min(xblk * 32 + col, p.w - 1);
      const uint16_t *xa = p.x + ((long)y * p.w + x) * p.xs + 8 * hi;
      const uint16_t *wa = p.w_in + (long)(2 * g + nblk) * p.kb_in * 512 + lane * 8;
      floatx16 acc = {};
      constexpr int KS = GLOBAL_C / 16;
      half8 a[KS], b[KS];
#pragma unroll
      for (int i = 0; i < KS; i++) {
        a[i] = ld8(wa + i * 512);
        b[i] = ld8(xa + i * 16);
      }
#pragma unroll
      for (int i = 0; i < KS; i++) acc = mfma16(a[i], b[i], acc);
      const int xo = xblk * 32 + col;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int n0 = nblk * 32 + 8 * q + 4 * hi;  // channel within the group
        const float *bias = p.b_in + 64 * g + n0;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = fmaxf(acc[4 * q + j] + bias[j], 0.0f);
        if (xo < p.w) st4h(p.s + ((long)y * p.w + xo) * SPEC + 64 * g + n0, v[0], v[1], v[2], v[3]);
        if (xo < p.xp) {
#pragma unroll
          for (int j = 0; j < 4; j++) st[(n0 + j) * SP + xo] = xo < p.w ? f2h(v[j]) : (uint16_t)0;
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
      const int c = cblk * 32 + col, ks_n = p.xp / 8;  // 2 xp / 16 <= 8
      const uint16_t *ta = p.tf + (long)mblk * ks_n * 512 + lane * 8;
      half8 a[8];
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = ld8(ta + min(i, ks_n - 1) * 512);
      floatx16 acc = {};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (i < ks_n) {
          const int x0 = (16 * i + 8 * hi) % p.xp;
          acc = mfma16(a[i], ld8(st + c * SP + x0), acc);
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
  const uint16_t *ta;       // B fragments [nba][6 yp / 16]
  const uint16_t *tc;       // B fragments [nba][4 yp / 16]
  const uint16_t *wf;
  int kb_f;
  const float *b_f;
  float *u;  // [h][half][384]
};

constexpr int RP = MAX_SIDE + 8;                        // halves per transposed R row
constexpr int R_PLANE = SPEC2 * RP;                     // one of the hi / lo planes
constexpr int ZP = SPEC2 + 8;                           // halves per spectrum row
constexpr int COL_LDS = 2 * R_PLANE + MAX_SIDE * ZP;    // halves: 160768 bytes

__global__ __launch_bounds__(512) void k_spectral_columns(ColumnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[COL_LDS];
  uint16_t *rhi = lds, *rlo = lds + R_PLANE, *z = lds + 2 * R_PLANE;
  uint16_t *pt = lds;  // after the column transform: filtered, [2 x 32][RP], over rhi
  const int k = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int h = p.h, yp = p.yp, ysteps = yp / 16;
  constexpr int CG = SPEC / COLUMN_GROUPS;
  // R of this column for every row: the real parts at row k of R, the
  // imaginary ones at row half + k - 1 (none for k = 0 or k > w - half),
  // scaled and split into [part 192 + c][y].
  {
    const int mim = (k >= 1 && k <= p.w - p.half) ? p.half + k - 1 : -1;
    const int yg = yp / 8, items = 2 * (SPEC / 4) * yg;
    for (int it = tid; it < items; it += 512) {
      const int part = it / ((SPEC / 4) * yg), rem = it % ((SPEC / 4) * yg);
      const int c4 = rem / yg, y0 = (rem % yg) * 8;
      const int m = part ? mim : k;
      float4v v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const bool ok = m >= 0 && y0 + j < h;
        v[j] = *(const float4v *)(p.r + ((long)(ok ? y0 + j : 0) * p.w + (ok ? m : 0)) * SPEC + 4 * c4);
        if (!ok) v[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int cc = 0; cc < 4; cc++) {
        float f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = v[j][cc] * RSCALE;
        half8 vh, vl;
        split8(f, vh, vl);
        const int row = part * SPEC + 4 * c4 + cc;
        *(half8 *)(rhi + row * RP + y0) = vh;
        *(half8 *)(rlo + row * RP + y0) = vl;
      }
    }
  }
  __syncthreads();
  // Column transform: D[c][(part', ky)] = sum over (term, part, y) of
  // R_term[part][c][y] T_term[(part, y)][(part', ky)]; terms hi.hi, lo.hi,
  // hi.lo.  Wave w: output columns nb = w % 4, channel blocks w / 4 + 2 j.
  {
    const int nb = wave & 3, ksa = 6 * ysteps;
    if (nb < p.nba) {
      const int cb0 = wave >> 2;
      const uint16_t *tb = p.ta + (long)nb * ksa * 512 + lane * 8;
      floatx16 acc[3] = {};
      half8 bn = ld8(tb);
      for (int ks = 0; ks < ksa; ks++) {
        const half8 b = bn;
        if (ks + 1 < ksa) bn = ld8(tb + (ks + 1) * 512);
        const int t = ks / (2 * ysteps), part = (ks / ysteps) & 1;
        const int y0 = (ks % ysteps) * 16 + 8 * hi;
        const uint16_t *plane = (t == 1 ? rlo : rhi) + (part * SPEC + 32 * cb0 + col) * RP + y0;
#pragma unroll
        for (int j = 0; j < 3; j++) acc[j] = mfma16(ld8(plane + 64 * j * RP), b, acc[j]);
      }
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
  }
  __syncthreads();
  // Fourier product over the spectrum pixels of this column for the
  // group's output channels (CG real parts, CG imaginary parts):
  // D[ky][n] = sum_c' Z[ky][c'] W[c'][n], bias, ReLU, f16, into [n][ky].
  {
    const int mbs = (h + 31) / 32;
    for (int b = wave; b < 2 * mbs; b += 8) {
      const int mb = b >> 1, part = b & 1;
      const int nbm = (part * SPEC + CG * g) / 32;
      const uint16_t *wb = p.wf + (long)nbm * p.kb_f * 512 + lane * 8;
      const uint16_t *za = z + (mb * 32 + col) * ZP + 8 * hi;
      floatx16 acc = {};
      constexpr int KS = SPEC2 / 16;
#pragma unroll
      for (int s0 = 0; s0 < KS; s0 += 8) {
        half8 bw[8];
#pragma unroll
        for (int i = 0; i < 8; i++) bw[i] = ld8(wb + (s0 + i) * 512);
#pragma unroll
        for (int i = 0; i < 8; i++) acc = mfma16(ld8(za + 16 * (s0 + i)), bw[i], acc);
      }
      const float bias = p.b_f[nbm * 32 + col];
      uint16_t *dst = pt + (part * CG + col) * RP;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int ky0 = mb * 32 + 8 * q + 4 * hi;
        if (ky0 < yp) {
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; j++) v[j] = ky0 + j < h ? fmaxf(acc[4 * q + j] + bias, 0.0f) : 0.0f;
          st4h(dst + ky0, v[0], v[1], v[2], v[3]);
        }
      }
    }
  }
  __syncthreads();
  // Inverse columns: D[c][(part', y)] = sum over (term, part, ky) of
  // P[part][c][ky] Ti_term[(part, ky)][(part', y)]; terms hi, lo.
  {
    const int ksc = 4 * ysteps;
    for (int nb = wave; nb < p.nba; nb += 8) {
      const uint16_t *tb = p.tc + (long)nb * ksc * 512 + lane * 8;
      floatx16 acc = {};
      half8 bn = ld8(tb);
      for (int ks = 0; ks < ksc; ks++) {
        const half8 b = bn;
        if (ks + 1 < ksc) bn = ld8(tb + (ks + 1) * 512);
        const int part = (ks / ysteps) & 1, ky0 = (ks % ysteps) * 16 + 8 * hi;
        acc = mfma16(ld8(pt + (part * CG + col) * RP + ky0), b, acc);
      }
      const int n = nb * 32 + col;
      if (n < 2 * h) {
        const int pp = n >= h, yy = n - pp * h;
        float *dst = p.u + ((long)yy * p.half + k) * SPEC2 + pp * SPEC + CG * g;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int c0 = 8 * q + 4 * hi;
          *(float4v *)(dst + c0) =
              float4v{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        }
      }
    }
  }
}

// ---- back: inverse rows, residual, spectral_out product -------------------

struct BackArgs {
  const float *u;
  int h, w, half, mp, nbx;  // mp: w rounded up to 16; nbx: 32-blocks of w
  const uint16_t *tr;       // B fragments [nbx][3 mp / 16]
  const uint16_t *s;        // spectral map [h][w][192]
  const uint16_t *wo;
  int kb_o;
  uint16_t *out;
  int ys;
};

constexpr int UP = MAX_SIDE + 8;
constexpr int U_PLANE = SPEC * UP;
constexpr int S2P = SPEC + 8;
constexpr int BACK_LDS = 2 * U_PLANE + MAX_SIDE * S2P;  // halves: 80896 bytes

__global__ __launch_bounds__(256) void k_spectral_back(BackArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[BACK_LDS];
  uint16_t *uhi = lds, *ulo = lds + U_PLANE, *s2 = lds + 2 * U_PLANE;
  const int y = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, col = lane & 31, hi = lane >> 5;
  const int msteps = p.mp / 16;
  // U of this row in the order of R's rows (m < half: real parts of column
  // m; half <= m < w: imaginary parts of column m - half + 1), scaled and
  // split into [c][m].
  {
    const int mg = p.mp / 8, items = (SPEC / 4) * mg;
    for (int it = tid; it < items; it += 256) {
      const int c4 = it / mg, m0 = (it % mg) * 8;
      float4v v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int m = m0 + j;
        const bool ok = m < p.w, im = m >= p.half;
        const int kk = ok ? (im ? m - p.half + 1 : m) : 0;
        v[j] = *(const float4v *)(p.u + ((long)y * p.half + kk) * SPEC2 + (ok && im ? SPEC : 0) + 4 * c4);
        if (!ok) v[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int cc = 0; cc < 4; cc++) {
        float f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = v[j][cc] * USCALE;
        half8 vh, vl;
        split8(f, vh, vl);
        *(half8 *)(uhi + (4 * c4 + cc) * UP + m0) = vh;
        *(half8 *)(ulo + (4 * c4 + cc) * UP + m0) = vl;
      }
    }
  }
  __syncthreads();
  // Inverse rows: D[c][x] = sum over (term, m) of U_term[c][m] Tr_term[m][x];
  // terms hi.hi, lo.hi, hi.lo.  Then + the spectral map, f16, into [x][c].
  {
    const int ksr = 3 * msteps;
    const int nb = wave % p.nbx, cstep = 4 / p.nbx;
    const uint16_t *tb = p.tr + (long)nb * ksr * 512 + lane * 8;
    const int x = nb * 32 + col, xc = min(x, p.w - 1);
    const uint16_t *sp = p.s + ((long)y * p.w + xc) * SPEC;
    for (int cb = wave / p.nbx; cb < SPEC / 32; cb += cstep) {
      floatx16 acc = {};
      half8 bn = ld8(tb);
      for (int ks = 0; ks < ksr; ks++) {
        const half8 b = bn;
        if (ks + 1 < ksr) bn = ld8(tb + (ks + 1) * 512);
        const int t = ks / msteps, m0 = (ks % msteps) * 16 + 8 * hi;
        acc = mfma16(ld8((t == 1 ? ulo : uhi) + (cb * 32 + col) * UP + m0), b, acc);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int c0 = cb * 32 + 8 * q + 4 * hi;
        const uint2 old = *(const uint2 *)(sp + c0);
        st4h(s2 + x * S2P + c0, acc[4 * q] + h2f((uint16_t)old.x),
             acc[4 * q + 1] + h2f((uint16_t)(old.x >> 16)), acc[4 * q + 2] + h2f((uint16_t)old.y),
             acc[4 * q + 3] + h2f((uint16_t)(old.y >> 16)));
      }
    }
  }
  __syncthreads();
  // spectral_out: D[n][x] = sum_c W[c][n] S2[x][c], the weights as the A
  // operand; out = ReLU(out + D).
  {
    constexpr int NG = SPEC2 / BACK_GROUPS, KS = SPEC / 16;
    for (int b = wave; b < (NG / 32) * p.nbx; b += 4) {
      const int nbl = b / p.nbx, xb = b % p.nbx;
      const int nbm = (NG * g) / 32 + nbl;
      const uint16_t *wa = p.wo + (long)nbm * p.kb_o * 512 + lane * 8;
      const uint16_t *sb = s2 + (xb * 32 + col) * S2P + 8 * hi;
      half8 a[KS];
#pragma unroll
      for (int i = 0; i < KS; i++) a[i] = ld8(wa + i * 512);
      floatx16 acc = {};
#pragma unroll
      for (int i = 0; i < KS; i++) acc = mfma16(a[i], ld8(sb + 16 * i), acc);
      const int x = xb * 32 + col;
      if (x < p.w) {
        uint16_t *o = p.out + ((long)y * p.w + x) * p.ys + nbm * 32;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int n0 = 8 * q + 4 * hi;
          const uint2 old = *(const uint2 *)(o + n0);
          st4h(o + n0, fmaxf(h2f((uint16_t)old.x) + acc[4 * q], 0.0f),
               fmaxf(h2f((uint16_t)(old.x >> 16)) + acc[4 * q + 1], 0.0f),
               fmaxf(h2f((uint16_t)old.y) + acc[4 * q + 2], 0.0f),
               fmaxf(h2f((uint16_t)(old.y >> 16)) + acc[4 * q + 3], 0.0f));
        }
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

ien_status spectral_front(const ien_spectral *sp, const uint16_t *x, long xs,
                          const ien_matrix *m_in, const ien_matrix *m_f, uint16_t *spectral,
                          float *r, float *u) {
  ien_ctx *ctx = sp->ctx;
  FrontArgs a{x, (int)xs, sp->h, sp->w, sp->xp, sp->mb, m_in->d_packed, m_in->kb, m_in->d_bias,
              sp->d_tf, spectral, r};
  hipLaunchKernelGGL(k_spectral_front, dim3((unsigned)sp->h, SPEC / 64), dim3(256), 0, ctx->stream,
                     a);
  IEN_HIP(hipGetLastError());
  ColumnArgs c{r, sp->h, sp->w, sp->half, sp->yp, sp->nba, sp->d_ta, sp->d_tc, m_f->d_packed,
               m_f->kb, m_f->d_bias, u};
  hipLaunchKernelGGL(k_spectral_columns, dim3((unsigned)sp->half, COLUMN_GROUPS), dim3(512), 0,
                     ctx->stream, c);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status spectral_back(const ien_spectral *sp, const ien_matrix *m_out, const uint16_t *spectral,
                         const float *u, uint16_t *out, long ys) {
  ien_ctx *ctx = sp->ctx;
  BackArgs b{u, sp->h, sp->w, sp->half, sp->xp, sp->nbx, sp->d_tr, spectral, m_out->d_packed,
             m_out->kb, out, (int)ys};
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
  // (a + i b) e^{-i theta}.  K: (term, part, y), terms hi, hi, lo.
  const std::vector<uint16_t> ta = operand(sp->nba, 6 * yp / 16, [&](int n, int kk) -> uint16_t {
    const int term = kk / (2 * yp), part = (kk % (2 * yp)) / yp, y = kk % yp;
    if (n >= 2 * h || y >= h) return 0;
    const int pp = n / h, ky = n % h;
    const double a = tau * (double)((long)ky * y % h) / h, c = std::cos(a), sn = std::sin(a);
    const double v = pp == 0 ? (part == 0 ? c : sn) : (part == 0 ? -sn : c);
    return split_half(v * s * 64.0, term == 2 ? 1 : 0);
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
  // hi, hi, lo.
  const std::vector<uint16_t> tr = operand(sp->nbx, 3 * xp / 16, [&](int x, int kk) -> uint16_t {
    const int term = kk / xp, m = kk % xp;
    if (x >= w || m >= w) return 0;
    const int col = m < half ? m : m - half + 1;
    const double wk = (col == 0 || 2 * col == w) ? 1.0 : 2.0;
    const double a = tau * (double)((long)col * x % w) / w;
    const double v = m < half ? wk * std::cos(a) : -wk * std::sin(a);
    return split_half(v * s * 256.0, term == 2 ? 1 : 0);
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
  IEN_CHECK(out_stride >= SPEC2 && out_stride % 4 == 0 && ((uintptr_t)d_out & 7) == 0 &&
                ((uintptr_t)d_spectral & 15) == 0 && ((uintptr_t)d_work & 15) == 0,
            IEN_ERR_INPUT, "output pixel stride %zu (a multiple of 4 >= %d), alignment", out_stride,
            SPEC2);
  float *r = d_work, *u = d_work + spectral_r_floats(sp);
  ien_status st = spectral_front(sp, d_x, (long)stride, spectral_in, fourier, d_spectral, r, u);
  if (st == IEN_OK) st = spectral_back(sp, spectral_out, d_spectral, u, d_out, (long)out_stride);
  return st;
}

}  // extern "C"
