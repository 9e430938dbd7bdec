// join_split.hip -- one SCUNet block boundary in one pass over the pixels
// (crates/scunet-native/src/network.rs:156-215, which runs the block's
// join and the next block's split on one chunk of pixels so that they do
// not stream the whole map in and out between them):
//
//   x' = x + join([y_conv | y_swin]) + join bias      (f16, stored to x)
//   [y_conv' | y_swin'] = split(x') + split bias       (f16, into the planes)
//
// for maps of C = 64 or 128 channels, the split map kept as two planes of
// C / 2 channels.  The results are the separate row products' bit for bit:
// each sum runs over the k steps in order from zero, then the bias, then
// (join) the old x, rounded once to f16; the split reads the rounded x'.
//
// A persistent workgroup of 4 waves keeps both products' weight fragments
// in LDS (loaded once) and walks 64-pixel tiles: the next tile's split-map
// rows and x rows land straight in LDS (global_load_lds) while this tile is
// multiplied.  Products are D[channel][pixel] = W^T X^T on
// v_mfma_f32_32x32x16_f16 (the packed weight fragments as the A operand,
// the staged rows as B), so a lane holds 4 consecutive channels of one
// pixel: the join's epilogue reads the old x as one 8-byte LDS read and
// writes x' as one 8-byte LDS write, into a tile that is both the split's
// B operand and the source of x's 16-byte stores.  Staged rows are
// 16-byte slots XOR-swizzled by row (slot = chunk ^ (row & 7)), so the 8
// rows of a 16-byte fragment read sit on distinct banks.  A tile's stores
// are issued at the start of the next tile, after its loads are waited
// for, so that the wait never includes the stores just made.

#include "conv_common.h"

namespace ien {
namespace {

template <int C>
struct JsCfg {
  static constexpr int BM = 64;                    // pixels a tile
  static constexpr int SLOTS = C / 8;              // 16-byte slots a staged row
  static constexpr int ROWB = C * 2;               // bytes a staged row
  static constexpr int TILE = BM * ROWB;           // one staged tile
  static constexpr int NB = C / 32;                // 32-channel blocks
  static constexpr int KS = C / 16;                // k steps
  static constexpr int WFR = NB * KS;              // fragments of one product
  static constexpr int OFF_WS = WFR * 1024;        // the split's fragments (the join's at 0)
  static constexpr int OFF_BUF = 2 * WFR * 1024;   // two buffers: [split-map rows][x rows]
  static constexpr int OFF_X = OFF_BUF + 4 * TILE; // x' tile
  static constexpr int OFF_Y = OFF_X + TILE;       // split output staging
  static constexpr int LDS = OFF_Y + TILE;
  static constexpr int NBW = NB / 2;               // channel blocks a wave (2 pixel blocks)
  static constexpr int LPT = 2 * TILE / 1024 / 4;  // loads a wave per tile
  static constexpr int ITEMS = BM * SLOTS / 256;   // 16-byte store pieces a thread per tile
  static_assert(C == 64 || C == 128, "64 or 128 channels");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(WFR % 4 == 0 && (2 * TILE) % 4096 == 0, "whole KiB a wave");
};

struct JsArgs {
  const uint16_t *yc, *ysw;  // split-map planes, rows C / 2 apart (read, then overwritten)
  uint16_t *x;               // the map, rows C apart (updated in place)
  int M;                     // pixels
  const uint16_t *wj, *ws;   // packed fragments, KB = C / 16
  const float *bj, *bs;      // biases (padded to whole 32-channel blocks)
  const uint16_t *zeros;
  int tiles;
};

template <int C>
__device__ __forceinline__ int slot_of(int row, int chunk) {
  return chunk ^ (row & 7);
}

template <int C>
__global__ __launch_bounds__(256) void k_join_split(JsArgs a) {
  using J = JsCfg<C>;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[J::LDS];
  const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pb = wave & 1;  // pixel block of the tile
  constexpr int HALF = C / 2;

  // Both products' fragments, once: fragment f = nb KB + kb of a packed
  // matrix, nb < NB, are its first WFR KiB.
#pragma unroll
  for (int i = 0; i < J::WFR / 4; i++) {
    const int f = 4 * i + wave;
    dma16(a.wj + (long)f * 512 + lane * 8, lds + f * 1024);
    dma16(a.ws + (long)f * 512 + lane * 8, lds + J::OFF_WS + f * 1024);
  }
  // This lane's biases: channels 32 nb + 8 g + 4 hi ..+ 3 of its blocks.
  float4v bj[J::NBW][4], bs[J::NBW][4];
#pragma unroll
  for (int j = 0; j < J::NBW; j++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int n = 32 * ((wave >> 1) + 2 * j) + 8 * g + 4 * hi;
      bj[j][g] = *(const float4v *)(a.bj + n);
      bs[j][g] = *(const float4v *)(a.bs + n);
    }

  // Tile t's rows into buffer b: the split map's chunks (the first half
  // from yc, the second from ysw) and x's, slots swizzled by row; rows
  // past the end read the zero page.
  auto issue = [&](int t, int b) {
    unsigned char *base = lds + J::OFF_BUF + b * 2 * J::TILE;
#pragma unroll
    for (int i = 0; i < J::LPT; i++) {
      const int d = 4 * i + wave;                     // KiB of the buffer
      const int piece = (d % (J::TILE / 1024)) * 64 + lane;
      const int row = piece / J::SLOTS, slot = piece % J::SLOTS;
      const int chunk = slot_of<C>(row, slot);        // the swizzle is its own inverse
      const long m = (long)t * J::BM + row;
      const uint16_t *src;
      if (d < J::TILE / 1024)
        src = chunk < J::SLOTS / 2 ? a.yc + m * HALF + 8 * chunk : a.ysw + m * HALF + 8 * chunk - HALF;
      else
        src = a.x + m * C + 8 * chunk;
      dma16(m < a.M ? src : a.zeros, base + d * 1024);
    }
  };
  // Stores of tile t from the x' tile and the staging: 16-byte pieces,
  // consecutive threads on consecutive slots of a row.
  auto store = [&](int t) {
    const unsigned char *xs = lds + J::OFF_X, *ys = lds + J::OFF_Y;
#pragma unroll
    for (int i = 0; i < J::ITEMS; i++) {
      const int e = tid + 256 * i, row = e / J::SLOTS, chunk = e % J::SLOTS;
      const long m = (long)t * J::BM + row;
      if (m >= a.M) continue;
      const int off = row * J::ROWB + 16 * slot_of<C>(row, chunk);
      *(u32x4 *)(a.x + m * C + 8 * chunk) = *(const u32x4 *)(xs + off);
      uint16_t *dst = chunk < J::SLOTS / 2 ? (uint16_t *)a.yc + m * HALF + 8 * chunk
                                           : (uint16_t *)a.ysw + m * HALF + 8 * chunk - HALF;
      *(u32x4 *)dst = *(const u32x4 *)(ys + off);
    }
  };
  // The products of one tile: B = the staged rows at `rows`, A = the
  // fragments at `w`; acc[j] is channel block (wave / 2) + 2 j.
  const int prow = 32 * pb + l32;  // this lane's pixel row of the tile
  auto products = [&](const unsigned char *rows, const unsigned char *w, floatx16 *acc) {
#pragma unroll
    for (int j = 0; j < J::NBW; j++) acc[j] = floatx16{};
#pragma unroll
    for (int ks = 0; ks < J::KS; ks++) {
      const half8 bv = *(const half8 *)(rows + prow * J::ROWB + 16 * slot_of<C>(prow, 2 * ks + hi));
#pragma unroll
      for (int j = 0; j < J::NBW; j++) {
        const int nb = (wave >> 1) + 2 * j;
        const half8 av = *(const half8 *)(w + (nb * J::KS + ks) * 1024 + lane * 16);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[j], 0, 0, 0);
      }
    }
  };
  // Byte offset in a staged tile of channels 32 nb + 8 g + 4 hi ..+ 3 of
  // this lane's pixel.
  auto quad_at = [&](int nb, int g) {
    return prow * J::ROWB + 16 * slot_of<C>(prow, 4 * nb + g) + 8 * hi;
  };

  int t = blockIdx.x;
  if (t < a.tiles) issue(t, 0);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 0; t < a.tiles; i++, t += gridDim.x) {
    const int b = i & 1;
    lds_barrier();  // every wave is done with the last tile's LDS
    const int next = t + gridDim.x;
    if (next < a.tiles) {
      issue(next, b ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<J::LPT>();  // all but the next tile's loads (and the fragments at first)
    } else {
      wait_vm<0>();
    }
    lds_barrier();  // this tile's rows (and the fragments) are visible
    if (i > 0) store(t - gridDim.x);
    const unsigned char *buf = lds + J::OFF_BUF + b * 2 * J::TILE;
    floatx16 acc[J::NBW];
    products(buf, lds, acc);
    lds_barrier();  // the last tile's x' and staging are stored
    // x' = f16((acc + join bias) + old x), into the x' tile.
#pragma unroll
    for (int j = 0; j < J::NBW; j++) {
      const int nb = (wave >> 1) + 2 * j;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int off = quad_at(nb, g);
        const uint2 old = *(const uint2 *)(buf + J::TILE + off);
        const uint16_t o0 = (uint16_t)old.x, o1 = (uint16_t)(old.x >> 16);
        const uint16_t o2 = (uint16_t)old.y, o3 = (uint16_t)(old.y >> 16);
        uint2 v;
        v.x = (uint32_t)f2h(acc[j][4 * g + 0] + bj[j][g][0] + h2f(o0)) |
              ((uint32_t)f2h(acc[j][4 * g + 1] + bj[j][g][1] + h2f(o1)) << 16);
        v.y = (uint32_t)f2h(acc[j][4 * g + 2] + bj[j][g][2] + h2f(o2)) |
              ((uint32_t)f2h(acc[j][4 * g + 3] + bj[j][g][3] + h2f(o3)) << 16);
        *(uint2 *)(lds + J::OFF_X + off) = v;
      }
    }
    lds_barrier();  // x' complete
    products(lds + J::OFF_X, lds + J::OFF_WS, acc);
    // The split's f16 results into the staging.
#pragma unroll
    for (int j = 0; j < J::NBW; j++) {
      const int nb = (wave >> 1) + 2 * j;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        uint2 v;
        v.x = (uint32_t)f2h(acc[j][4 * g + 0] + bs[j][g][0]) |
              ((uint32_t)f2h(acc[j][4 * g + 1] + bs[j][g][1]) << 16);
        v.y = (uint32_t)f2h(acc[j][4 * g + 2] + bs[j][g][2]) |
              ((uint32_t)f2h(acc[j][4 * g + 3] + bs[j][g][3]) << 16);
        *(uint2 *)(lds + J::OFF_Y + quad_at(nb, g)) = v;
      }
    }
  }
  // The last tile's stores.
  if (blockIdx.x < a.tiles) {
    lds_barrier();
    const int last = blockIdx.x + (int)((a.tiles - 1 - blockIdx.x) / gridDim.x) * gridDim.x;
    store(last);
  }
}

}  // namespace

bool join_split_supported(const JoinSplit &p) {
  const int c = p.c;
  if (c != 64 && c != 128) return false;
  if (!p.join || !p.split || !p.join->d_packed || !p.split->d_packed) return false;
  const ien_matrix *m[2] = {p.join, p.split};
  for (const ien_matrix *w : m)
    if ((int)w->k != c || (int)w->n != c || w->kb != c / 16 || w->nb < c / 32) return false;
  const uintptr_t ptrs = (uintptr_t)p.yc | (uintptr_t)p.ysw | (uintptr_t)p.x;
  return (ptrs & 15) == 0 && p.rows > 0 && p.rows < (1L << 30);
}

ien_status launch_join_split(ien_ctx *ctx, const JoinSplit &p) {
  IEN_CHECK(join_split_supported(p), IEN_ERR_INPUT, "join + split over %d channels", p.c);
  JsArgs a{p.yc, p.ysw, p.x, (int)p.rows, p.join->d_packed, p.split->d_packed,
           p.join->d_bias, p.split->d_bias, ctx->zeros, 0};
  a.tiles = (int)((p.rows + 63) / 64);
  // Workgroups a CU: two of 64 KiB at 64 channels, one of 160 KiB at 128.
  const int per_cu = p.c == 64 ? 2 : 1;
  const unsigned grid = (unsigned)std::min<long>(a.tiles, (long)per_cu * ctx->cus);
  if (p.c == 64)
    hipLaunchKernelGGL(k_join_split<64>, dim3(grid), dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(k_join_split<128>, dim3(grid), dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien
