// rows.hip -- products over rows of pixels (1 x 1 convolutions and
// Input::Rows, gemm.rs:272-283) on gfx950: out[r] = act(x[r] W + bias
// (+ old out[r] when accumulating)), x f16 rows `xs` halves apart, W packed
// as MFMA B fragments (ien_matrix), f16 rows out.
//
// A workgroup of 4 waves computes a 128-row x BN-column tile (BN = 128:
// each wave 64 x 64, 2 x 2 blocks of v_mfma_f32_32x32x16_f16; BN = 64: each
// wave 32 x 64).  K runs in chunks of KC channels through a 3-stage LDS
// ring: every wave issues its share of the chunk's direct-to-LDS buffer
// loads (16 bytes a lane, 1 KiB a wave instruction) two chunks ahead, so
// one barrier per chunk suffices and the loads of two chunks are always in
// flight.  The loads are inline assembly the compiler does not see (its
// own waits after such loads would flush the whole counter); loads
// complete in order, so waiting until LPC are outstanding means all but
// the next chunk's have landed.  The buffer range check returns zeros for
// rows past the end.
//  - x rows are staged [row][16-byte slot] with the slots XOR-swizzled by
//    row, so the 32 rows of an A-fragment read fall on distinct banks; the
//    swizzle is applied to the source address, since a wave's loads fill a
//    contiguous KiB.
//  - W fragments are copied as packed (1 KiB per fragment, lane order).
//  - Epilogue: acc + bias staged as f32 in LDS, 64 rows at a time, then
//    per 16-byte item (8 channels of a row) the old output (loaded first,
//    all at once) and the activation, one loop per activation: the order of
//    gemm.rs:583-666.
// Chunks of 32 channels keep the ring at 48 KiB (BN = 128), so several
// workgroups share a CU and hide each other's latency.
// Tiles are dealt XCD-aware with N fastest, so a tile row's x stays in its
// XCD's L2 for every column tile.
// Planes: the rows may come from two maps (channels k1 .. K from x2, rows
// xs2 apart) and go to two (columns n1 .. N to y2, rows ys2 apart), so that
// the two halves of a map that two streams work on share no cache line.

#include "conv_common.h"
#include "window_geo.h"

namespace ien {
namespace {

struct RowsArgs {
  const uint16_t *x;  // row 0 of the range
  int xs;             // halves between rows
  int M, K;           // rows, reduction depth (a multiple of KC)
  const uint16_t *wp;
  int KB, NB, N;      // packed 16-deep and 32-wide blocks, columns
  const float *bias, *slope;
  uint16_t *y;        // output row 0
  int ys;
  const uint16_t *x2;  // channels k1 .. K (k1 = K: x only), rows xs2 apart
  int xs2, k1;
  uint16_t *y2;        // columns n1 .. N (n1 = N: y only), rows ys2 apart
  int ys2, n1;
  // 2 x 2 regroupings (0: none).  g2w: row r is the 2 x 2 group of pixels
  // (2 (r / g2w) + dy, 2 (r % g2w) + dx) of a map 2 g2w wide (pixels xs
  // apart), channel block q = 2 dy + dx of K / 4 channels each.  s2w: the
  // rows are the pixels of a map s2w wide; column block q of N / 4 goes to
  // pixel (2 (r / s2w) + q / 2, 2 (r % s2w) + q % 2) of a map 2 s2w wide
  // (pixels ys apart).
  int g2w, s2w;
  uint16_t *ydup;  // gathered rows: a second copy of the output (rows ys apart), or null
  const uint16_t *add2;  // MODE 3: a map added to the rounded result (rows ys apart)
  WinGeo wg;             // MODE 4: row r is token r % n of window r / n of y's map
  int act, accumulate;
  int tiles_n, tiles;
  // Split-K (gridDim.y splits of kchunks chunks): raw f32 sums of split z
  // at part + (z M + row) pitch, no bias, for the finishing pass.
  float *part;
  int pitch, kchunks;
};

template <int BM_, int BN, int KC>
struct RowsCfg {
  static constexpr int BM = BM_;
  static constexpr int SLOTS = KC / 8;                   // 16-byte slots per staged row
  static constexpr int A_BYTES = BM * KC * 2;
  static constexpr int B_BYTES = BN * KC * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int STAGES = 3;
  static constexpr int A_LOADS = A_BYTES / 1024 / 4;     // per wave and chunk
  static constexpr int B_LOADS = B_BYTES / 1024 / 4;
  static constexpr int LPC = A_LOADS + B_LOADS;
  static constexpr int SP = BN + 4;                      // staged f32 row pitch
  static constexpr int LDS = STAGES * STAGE > 64 * SP * 4 ? STAGES * STAGE : 64 * SP * 4;
  static constexpr int WM = BN == 128 ? BM / 64 : 1;      // 32-row blocks per wave
  static constexpr int HALVES = BM / 64;                 // 64-row staging passes
  static constexpr int ITEMS = BM * BN / 8 / 256;        // 16-byte output items per thread
  static_assert(A_LOADS * 4 * 1024 == A_BYTES && B_LOADS * 4 * 1024 == B_BYTES, "load split");
};

// Slot of 16-byte chunk g of staged row r.
template <int SLOTS>
__device__ __forceinline__ int swz(int r, int g) {
  return g ^ ((SLOTS == 8 ? r : r >> 1) & (SLOTS - 1));
}

// MODE 0: plain rows; 1: 2 x 2 gathered rows (g2w); 2: rows scattered over
// 2 x 2 output pixels (s2w); 3: plain rows whose f16 result gets add2 added
// and is rounded again (a separate map addition after the product); 4: rows
// are window tokens whose rounded result is added onto their map pixel
// (ien_window_scatter_add after the product), tokens past the edge dropped.
template <int BM, int BN, int KC, int MODE>
__global__ __launch_bounds__(256) void k_rows(RowsArgs a) {
  using R = RowsCfg<BM, BN, KC>;
  static_assert(BM == 128 || BN == 128, "64-row tiles are 128 columns wide");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[R::LDS];
  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = t / a.tiles_n, tn = t - tm * a.tiles_n;
  const int m0 = tm * R::BM;
  const unsigned l0 = lds_addr(lds);
  const int4v xr = buffer_rsrc(a.x, (long)a.M * (MODE == 1 ? 4 : 1) * a.xs * 2);
  const int4v xr2 = buffer_rsrc(a.x2, (long)a.M * a.xs2 * 2);
  const int4v wr = buffer_rsrc(a.wp, (long)a.NB * a.KB * 1024);
  const int c_begin = blockIdx.y * a.kchunks;
  const int chunks = min(a.K / KC - c_begin, a.kchunks);  // this split's chunks
  // Gathered rows: the pixel of each A load's row at channel block 0.
  int gpix[R::A_LOADS];
  if constexpr (MODE == 1) {
#pragma unroll
    for (int i = 0; i < R::A_LOADS; i++) {
      const int m = m0 + (wave + 4 * i) * (1024 / (KC * 2)) + lane / R::SLOTS;
      const int yy = m / a.g2w;
      gpix[i] = 4 * yy * a.g2w + 2 * (m - yy * a.g2w);
    }
  }

  // Chunk c into stage s: A rows m0 .. m0 + BM - 1, channels c KC .. + KC - 1;
  // B fragments of column blocks tn BN / 32 .. and k blocks c KC / 16 ...
  auto issue = [&](int lc, int s) {
    const int c = c_begin + lc;
    const unsigned base = l0 + s * R::STAGE;
    const bool second = c * KC >= a.k1;  // (uniform: k1 is a multiple of KC)
    const int4v sr = second ? xr2 : xr;
    const int rs = second ? a.xs2 : a.xs, c0 = second ? c * KC - a.k1 : c * KC;
#pragma unroll
    for (int i = 0; i < R::A_LOADS; i++) {
      const int d = wave + 4 * i;                 // KiB of the A stage
      const int row = d * (1024 / (KC * 2)) + lane / R::SLOTS;
      const int slot = lane % R::SLOTS;
      const int g = swz<R::SLOTS>(row, slot);      // the chunk this slot holds
      int off = ((m0 + row) * rs + c0 + 8 * g) * 2;
      if constexpr (MODE == 1) {
        const int cin = a.K >> 2, q = c0 / cin;
        off = ((gpix[i] + (q >> 1) * 2 * a.g2w + (q & 1)) * rs + c0 - q * cin + 8 * g) * 2;
      }
      dma_lds(sr, __builtin_amdgcn_readfirstlane(base + d * 1024), off);
    }
#pragma unroll
    for (int i = 0; i < R::B_LOADS; i++) {
      const int f = wave + 4 * i;                 // fragment (j, q) of the chunk
      const int j = f / (KC / 16), q = f % (KC / 16);
      const int nb = tn * (BN / 32) + j, kb = c * (KC / 16) + q;
      dma_lds(wr, __builtin_amdgcn_readfirstlane(base + R::A_BYTES + f * 1024),
               (nb * a.KB + kb) * 1024 + lane * 16);
    }
  };

  const int wm = BN == 128 ? (wave & 1) : wave;   // block of WM 32-row blocks
  const int wn = BN == 128 ? (wave >> 1) : 0;     // 64-column block
  // The epilogue's bias for this lane's two columns, requested now so that
  // its latency hides behind the products (padded to whole 32-column blocks).
  float bias_r[2];
#pragma unroll
  for (int j = 0; j < 2; j++) bias_r[j] = a.bias[tn * BN + (wn * 2 + j) * 32 + l32];
  floatx16 acc[R::WM][2];
#pragma unroll
  for (int i = 0; i < R::WM; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = floatx16{};

  issue(0, 0);
  if (chunks > 1) issue(1, 1);
  for (int c = 0; c < chunks; c++) {  // c: this split's chunk index
    if (c + 1 < chunks)
      wait_vm<R::LPC>();  // all but chunk c + 1's loads
    else
      wait_vm<0>();
    __syncthreads();  // chunk c visible; every wave is done with chunk c - 1
    if (c + 2 < chunks) issue(c + 2, (c + 2) % 3);
    const unsigned char *sa = lds + (c % 3) * R::STAGE;
    const unsigned char *sb = sa + R::A_BYTES;
#pragma unroll
    for (int q = 0; q < KC / 16; q++) {
      half8 af[R::WM], bf[2];
#pragma unroll
      for (int i = 0; i < R::WM; i++) {
        const int row = (wm * R::WM + i) * 32 + l32;
        af[i] = *(const half8 *)(sa + row * KC * 2 + swz<R::SLOTS>(row, 2 * q + hf) * 16);
      }
#pragma unroll
      for (int j = 0; j < 2; j++)
        bf[j] = *(const half8 *)(sb + ((wn * 2 + j) * (KC / 16) + q) * 1024 + lane * 16);
#pragma unroll
      for (int i = 0; i < R::WM; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }
  __syncthreads();  // every wave is done with the stages

  if (a.part) {  // split-K: raw sums, 32 bytes per item
    float *st = (float *)lds;
    const int owner = BM == 64 ? 0 : BN == 128 ? wm : wm >> 1;
#pragma unroll
    for (int half = 0; half < R::HALVES; half++) {
      if (half) __syncthreads();
      if (owner == half) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
          for (int i = 0; i < R::WM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++)
              st[((wm * R::WM + i) * 32 - 64 * half + 8 * (r >> 2) + 4 * hf + (r & 3)) * R::SP +
                 (wn * 2 + j) * 32 + l32] = acc[i][j][r];
      }
      __syncthreads();
#pragma unroll
      for (int e = half * R::ITEMS / R::HALVES; e < (half + 1) * R::ITEMS / R::HALVES; e++) {
        const int v = tid + 256 * e, row = v / (BN / 8), c8 = 8 * (v % (BN / 8));
        if (m0 + row >= a.M) continue;
        const float *sr = st + (row - 64 * half) * R::SP + c8;
        float *q = a.part + ((long)blockIdx.y * a.M + m0 + row) * a.pitch + tn * BN + c8;
        *(float4v *)q = *(const float4v *)sr;
        *(float4v *)(q + 4) = *(const float4v *)(sr + 4);
      }
    }
    return;
  }

  // 16-byte items: row v / (BN / 8), channels 8 (v % (BN / 8)) ..., items
  // of staging pass h in rows 64 h .. 64 h + 63.  The old outputs are loaded
  // first, so their latency overlaps the staging.
  // Output item (row, col .. col + 7) in y or, past column n1, in y2
  // (n1 is a multiple of 8).
  auto out_at = [&](int row, int col) {
    if constexpr (MODE == 2) {
      const int cout = a.N >> 2, q = col / cout, y = row / a.s2w;
      const long pixel = (long)(2 * y + (q >> 1)) * (2 * a.s2w) + 2 * (row - y * a.s2w) + (q & 1);
      return a.y + pixel * a.ys + (col - q * cout);
    }
    return col < a.n1 ? a.y + (long)row * a.ys + col : a.y2 + (long)row * a.ys2 + (col - a.n1);
  };
  // MODE 4: the map pixel of an output row, or null past the map's edge.
  auto win_dst = [&](int row, int col) -> uint16_t * {
    const int w = row / a.wg.n, src = win_source(a.wg, w, row - w * a.wg.n);
    return src < 0 ? nullptr : a.y + (long)src * a.ys + col;
  };
  u32x4 old[R::ITEMS], old2[MODE >= 3 ? R::ITEMS : 1];
  if constexpr (MODE == 4) {
#pragma unroll
    for (int e = 0; e < R::ITEMS; e++) {
      const int v = tid + 256 * e, row = v / (BN / 8), col = tn * BN + 8 * (v % (BN / 8));
      const uint16_t *q = m0 + row < a.M && col < a.N ? win_dst(m0 + row, col) : nullptr;
      old2[e] = *(const u32x4 *)(q ? q : a.y);
    }
  }
  if constexpr (MODE == 3) {
#pragma unroll
    for (int e = 0; e < R::ITEMS; e++) {
      const int v = tid + 256 * e, row = v / (BN / 8), col = tn * BN + 8 * (v % (BN / 8));
      const bool ok = m0 + row < a.M && col < a.N;
      old2[e] = *(const u32x4 *)(a.add2 + (ok ? (long)(m0 + row) * a.ys + col : 0));
    }
  }
  if (a.accumulate) {
#pragma unroll
    for (int e = 0; e < R::ITEMS; e++) {
      const int v = tid + 256 * e, row = v / (BN / 8), col = tn * BN + 8 * (v % (BN / 8));
      const bool ok = m0 + row < a.M && col < a.N;
      old[e] = *(const u32x4 *)(ok ? out_at(m0 + row, col) : a.y);
    }
  }
  float *st = (float *)lds;
  auto store = [&](auto actf, int half) {
#pragma unroll
    for (int e = half * R::ITEMS / R::HALVES; e < (half + 1) * R::ITEMS / R::HALVES; e++) {
      const int v = tid + 256 * e, row = v / (BN / 8), c8 = 8 * (v % (BN / 8));
      const int col = tn * BN + c8;
      if (m0 + row >= a.M || col >= a.N) continue;
      uint16_t *dst = nullptr;
      if constexpr (MODE == 4) {
        dst = win_dst(m0 + row, col);
        if (!dst) continue;
      } else {
        dst = out_at(m0 + row, col);
      }
      const float *sr = st + (row - 64 * half) * R::SP + c8;
      const float4v s0 = *(const float4v *)sr, s1 = *(const float4v *)(sr + 4);
      float v8[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      if (a.accumulate) {
        uint16_t h[8];
        __builtin_memcpy(h, &old[e], 16);
#pragma unroll
        for (int k = 0; k < 8; k++) v8[k] += h2f(h[k]);
      }
      uint16_t o[8];
#pragma unroll
      for (int k = 0; k < 8; k++) o[k] = f2h(actf(v8[k], col + k));
      if constexpr (MODE >= 3) {
        uint16_t h2[8];
        __builtin_memcpy(h2, &old2[e], 16);
#pragma unroll
        for (int k = 0; k < 8; k++) o[k] = f2h(h2f(o[k]) + h2f(h2[k]));
      }
      __builtin_memcpy(dst, o, 16);
      if constexpr (MODE == 1)
        if (a.ydup) __builtin_memcpy(a.ydup + (long)(m0 + row) * a.ys + col, o, 16);
    }
  };
  // acc + bias as f32 rows in LDS, 64 rows at a time.
  const int owner = BM == 64 ? 0 : BN == 128 ? wm : wm >> 1;  // the 64 rows this wave computed
#pragma unroll
  for (int half = 0; half < R::HALVES; half++) {
    if (half) __syncthreads();  // the first half is read
    if (owner == half) {
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int col = (wn * 2 + j) * 32 + l32;
        const float b = bias_r[j];
#pragma unroll
        for (int i = 0; i < R::WM; i++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            st[((wm * R::WM + i) * 32 - 64 * half + 8 * (r >> 2) + 4 * hf + (r & 3)) * R::SP + col] =
                acc[i][j][r] + b;
      }
    }
    __syncthreads();
    switch (a.act) {
      case IEN_ACT_RELU: store([&](float v, int) { return act_c<IEN_ACT_RELU>(v, 0.0f); }, half); break;
      case IEN_ACT_GELU: store([&](float v, int) { return act_c<IEN_ACT_GELU>(v, 0.0f); }, half); break;
      case IEN_ACT_SIGMOID:
        store([&](float v, int) { return act_c<IEN_ACT_SIGMOID>(v, 0.0f); }, half);
        break;
      case IEN_ACT_PRELU:
        store([&](float v, int col) { return act_c<IEN_ACT_PRELU>(v, a.slope[col]); }, half);
        break;
      default: store([&](float v, int) { return v; }, half); break;
    }
  }
}

// Split-K when the tiles leave three quarters of the CUs idle, or any CU
// idle with K at least 1536 deep: about two workgroups per CU, each split at
// least 256 deep.  (Splitting products that already fill most CUs, such as
// SCUNet's 1024-deep fc2 over 192 tiles, cost more in partial sums and the
// finishing pass than it gained.)
template <int BM, int BN, int KC, int MODE = 0>
ien_status launch(ien_ctx *ctx, RowsArgs a, const ConvArgs &c) {
  a.tiles_n = (a.N + BN - 1) / BN;
  a.tiles = (a.M + BM - 1) / BM * a.tiles_n;
  const int chunks = a.K / KC;
  a.pitch = a.tiles_n * BN;
  int ksplit = 1;
  // (The finishing pass writes one map, row by row; gathered rows are
  // split like any others.)
  const bool planes = a.k1 < a.K || a.n1 < a.N || MODE >= 2;
  if (!planes && chunks >= 16 && (4 * a.tiles <= ctx->cus || (a.K >= 1536 && a.tiles < ctx->cus))) {
    ksplit = std::min(chunks / 8, (2 * ctx->cus + a.tiles - 1) / a.tiles);
    while (ksplit > 1 && (size_t)ksplit * a.M * a.pitch > ctx->splitk_floats) ksplit--;
  }
  a.kchunks = (chunks + ksplit - 1) / ksplit;
  ksplit = (chunks + a.kchunks - 1) / a.kchunks;
  a.part = ksplit > 1 ? ctx->splitk : nullptr;
  hipLaunchKernelGGL((k_rows<BM, BN, KC, MODE>), dim3((unsigned)a.tiles, (unsigned)ksplit), dim3(256), 0,
                     ctx->stream, a);
  IEN_HIP(hipGetLastError());
  if (ksplit == 1) return IEN_OK;
  const ien_status st = splitk_finish(ctx, ksplit, a.M, a.pitch, c);
  if (st != IEN_OK || !a.ydup) return st;
  // The finishing pass writes one map: the second copy follows it.
  IEN_HIP(hipMemcpy2DAsync(a.ydup, (size_t)a.ys * 2, a.y, (size_t)a.ys * 2, (size_t)a.N * 2,
                           (size_t)a.M, hipMemcpyDeviceToDevice, ctx->stream));
  return IEN_OK;
}

}  // namespace

// Tiles of 128 rows when they number at least 128, else 64-row tiles when
// those number at least 96, or at least 8 with K 512 deep (split-K); below
// that the general kernel serves.
static long tiles_of(long rows, int bm, int n) { return (rows + bm - 1) / bm * ((n + 127) / 128); }

bool rows_supported(const ConvArgs &a, long rows) {
  const bool aligned = (((uintptr_t)a.x) & 15) == 0 && (((uintptr_t)a.y) & 15) == 0;
  const long t64 = tiles_of(rows, 64, a.N);
  const bool enough = tiles_of(rows, 128, a.N) >= 128 || t64 >= 96 || (t64 >= 8 && a.C >= 512);
  return aligned && !a.out_f32 && !a.out_nchw && a.C % 32 == 0 && a.N % 8 == 0 && a.xs % 8 == 0 &&
         a.ys % 8 == 0 && (long)a.xs * (rows + 128) * 2 <= 0x7fff0000L &&
         (long)a.NB * a.KB * 1024 <= 0x7fff0000L && enough;
}

// Rows p_begin .. p_end of x (row stride xs) times the packed weights into
// rows 0 .. of y; a.C is the reduction depth.
ien_status launch_rows(ien_ctx *ctx, const ConvArgs &c) {
  RowsArgs a{};
  a.x = c.x + (long)c.p_begin * c.xs;
  a.xs = c.xs;
  a.M = c.p_end - c.p_begin;
  a.K = c.C;
  a.wp = c.wp;
  a.KB = c.KB;
  a.NB = c.NB;
  a.N = c.N;
  a.bias = c.bias;
  a.slope = c.slope;
  a.y = (uint16_t *)c.y;
  a.ys = c.ys;
  a.x2 = a.x;
  a.xs2 = a.xs;
  a.k1 = a.K;
  a.y2 = a.y;
  a.ys2 = a.ys;
  a.n1 = a.N;
  a.act = c.act;
  a.accumulate = c.accumulate;
  // Columns over 64: 64-row tiles (four workgroups a CU, twice the tiles of
  // 128-row ones; measured faster on every model shape); up to 64 columns:
  // 128 x 64 tiles.
  if (c.N > 64 || tiles_of(a.M, 128, a.N) < 128) return launch<64, 128, 32>(ctx, a, c);
  return launch<128, 64, 32>(ctx, a, c);
}

ien_status launch_rows_planes(ien_ctx *ctx, const RowsPlanes &p) {
  const ien_matrix *w = p.w;
  IEN_CHECK(w && w->d_packed && p.rows > 0, IEN_ERR_INPUT, "rows planes: no weights or rows");
  const int K = (int)w->k, N = (int)w->n;
  IEN_CHECK(K % 32 == 0 && p.k1 % 32 == 0 && p.k1 > 0 && p.k1 <= K && N % 8 == 0 &&
                p.n1 % 8 == 0 && p.n1 > 0 && p.n1 <= N,
            IEN_ERR_INPUT, "rows planes: k %d split at %d, n %d split at %d", K, p.k1, N, p.n1);
  const bool gather = p.gather_w2 > 0, scatter = p.scatter_w > 0;
  IEN_CHECK(p.gather_w2 >= 0 && p.scatter_w >= 0 &&
                (!gather || (p.k1 == K && K % 128 == 0 && p.rows % p.gather_w2 == 0)) &&
                (!scatter || (p.n1 == N && N % 32 == 0 && p.rows % p.scatter_w == 0 && !p.accumulate)) &&
                (!p.ydup || (gather && p.n1 == N && ((uintptr_t)p.ydup & 15) == 0 && !p.accumulate)) &&
                (!p.add || (!gather && !scatter && p.n1 == N && ((uintptr_t)p.add & 15) == 0)) &&
                (!p.windows ||
                 (!gather && !scatter && !p.add && !p.accumulate && p.n1 == N &&
                  p.rows == p.windows->windows * p.windows->n && p.windows->windows < (1L << 31) &&
                  (long)p.windows->height * p.windows->width * p.ys * 2 <= 0x7fff0000L)),
            IEN_ERR_INPUT, "rows planes: 2 x 2 regrouping of k %d / n %d over %ld rows", K, N, p.rows);
  // A gathered row reads K / 4 channels of each pixel; a scattered one
  // writes N / 4.
  const int kx = gather ? K / 4 : p.k1, ny = scatter ? N / 4 : p.n1;
  const long xrows = gather ? 4 * p.rows : p.rows, yrows = scatter ? 4 * p.rows : p.rows;
  const uintptr_t ptrs = (uintptr_t)p.x | (uintptr_t)p.x2 | (uintptr_t)p.y | (uintptr_t)p.y2;
  IEN_CHECK((ptrs & 15) == 0 && p.xs % 8 == 0 && p.xs2 % 8 == 0 && p.ys % 8 == 0 &&
                p.ys2 % 8 == 0 && p.xs >= kx && p.xs2 >= K - p.k1 && p.ys >= ny &&
                p.ys2 >= N - p.n1,
            IEN_ERR_INPUT, "rows planes: alignment or strides");
  IEN_CHECK((long)p.xs * (xrows + 512) * 2 <= 0x7fff0000L &&
                (long)p.xs2 * (p.rows + 128) * 2 <= 0x7fff0000L &&
                (long)p.ys * (yrows + 512) * 2 <= 0x7fff0000L &&
                (long)p.ys2 * (p.rows + 128) * 2 <= 0x7fff0000L,
            IEN_ERR_INPUT, "rows planes over 2 GiB");
  RowsArgs a{};
  a.x = p.x;
  a.xs = p.xs;
  a.x2 = p.x2;
  a.xs2 = p.xs2;
  a.k1 = p.k1;
  a.M = (int)p.rows;
  a.K = K;
  a.wp = w->d_packed;
  a.KB = w->kb;
  a.NB = w->nb;
  a.N = N;
  a.bias = w->d_bias;
  a.y = p.y;
  a.ys = p.ys;
  a.y2 = p.y2;
  a.ys2 = p.ys2;
  a.n1 = p.n1;
  a.g2w = p.gather_w2;
  a.s2w = p.scatter_w;
  a.ydup = p.ydup;
  a.add2 = p.add;
  a.act = IEN_ACT_NONE;
  a.accumulate = p.accumulate;
  // The output as the split-K finishing pass reads it (one map: no planes
  // split-K).
  ConvArgs c{};
  c.N = N;
  c.bias = w->d_bias;
  c.y = p.y;
  c.ys = p.ys;
  c.act = IEN_ACT_NONE;
  c.accumulate = p.accumulate;
  if (gather) return launch<64, 128, 32, 1>(ctx, a, c);
  if (p.add) return launch<64, 128, 32, 3>(ctx, a, c);
  if (p.windows) {
    a.wg = *p.windows;
    return launch<64, 128, 32, 4>(ctx, a, c);
  }
  if (scatter) return launch<64, 128, 32, 2>(ctx, a, c);
  if (N > 64 || tiles_of(a.M, 128, a.N) < 128) return launch<64, 128, 32>(ctx, a, c);
  return launch<128, 64, 32>(ctx, a, c);
}

}  // namespace ien
