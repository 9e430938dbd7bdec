// conv_res.hip -- resident-weight persistent convolution on gfx950 MFMA.
//
// For NHWC inputs of 16, 32 or 64 channels with 1x1 or 3x3 zero-padded
// taps (K = k k C <= 576): Real-ESRGAN's body layers (crates/realesrgan-
// native/src/network.rs:96-109, gemm.rs multiply semantics) and the 1x1
// products of that width.
//
// One workgroup per CU, 8 waves (2 per SIMD), persistent over 2 x 64-pixel
// output tiles, all 64 output channels of a tile; wave w computes 32 pixels
// (block w % 4) by 32 channels (half w / 4) with v_mfma_f32_32x32x16_f16.
// The packed weights are the A operand, so the product is C^T = W^T X^T,
// and each wave keeps its 32 channels' weights in VGPRs for all its tiles.
//  - Every global read is a buffer load straight into LDS, issued from
//    inline assembly: the compiler neither sees nor waits for them (its
//    waits after such loads flush whole counters), so the kernel counts
//    them itself.  Loads complete in order, so waiting until at most n
//    vector-memory operations are outstanding means all loads but the last
//    n issued have landed, stores in between or not.  The range check of
//    the buffer loads supplies the zero padding.
//  - Halo pixels are stored with a 16-byte pad chunk, so the 32 pixels of a
//    B fragment fall on distinct LDS banks and every fragment of a tap is a
//    fixed offset from the lane's base (ds_read_b128 with an immediate).
//  - Three halo buffers: tile t+2's halo is loaded while tile t computes,
//    which covers the memory latency of a whole tile.
//  - Per tile t, one barrier, then one unrolled, branch-free MFMA sequence
//    (one accumulator chain seeded with the bias) into which are
//    interleaved: tile t+2's halo loads; tile t-1's epilogue (activation,
//    f16, into a staging buffer) from the accumulators kept since; tile
//    t-2's stores from the other staging buffer (16-byte buffer stores of
//    whole 128-byte pixel rows; the range check drops items outside the
//    output).
// Bias then activation, or bias, old output, activation when accumulating:
// the order of gemm.rs:583-666.

#include "conv_common.h"

namespace ien {

// H32: outputs of at most 32 channels, not accumulating -- every wave on
// the one 32-channel half, over tiles of 4 rows of 64 pixels.
template <int KS, int C, bool H32 = false>
struct Res8 {
  static constexpr int TR = H32 ? 4 : 2, TC = 64;  // output tile: TR rows of 64 pixels
  static constexpr int CH = H32 ? 32 : 64;         // output channels of a tile
  static constexpr int IPX = CH / 8;               // 16-byte items of a staged pixel
  static constexpr int STEPS = KS * KS * C / 16;
  static constexpr int HR = TR + KS - 1, HC = TC + KS - 1, HPIX = HR * HC;
  // Halo pixel stride: the channels plus one 16-byte pad chunk.
  static constexpr int PB = C * 2 + 16;
  // Whole 8 KiB, so that each of the 8 waves issues the same number of
  // 1 KiB loads per halo.
  static constexpr int HALO = (HPIX * PB + 8191) / 8192 * 8192;
  static constexpr int HIT = HALO / 8192;     // halo loads per wave
  static constexpr int SPX = CH + 8;          // staged halves per pixel (padded)
  static constexpr int STAGE = TR * TC * SPX * 2;
  static constexpr int WBYTES = CH / 32 * STEPS * 1024;  // B fragments of the tile's channels
  // LDS: 3 halo buffers | 2 staging buffers | bias (1 KiB) | slopes (1 KiB).
  // In the prologue the weights sit over halo 2 and the staging buffers.
  static constexpr int STG = 3 * HALO;
  static constexpr int PARAM = STG + 2 * STAGE;
  static constexpr int WOFF = 2 * HALO;
  // When they fit: two buffers for the old outputs of an accumulating tile
  // (its 16-byte store items, in item order).
  static constexpr int OLDB = TR * TC * IPX * 16;
  static constexpr int OLD = PARAM + 2048;
  static constexpr bool OLD_LDS = OLD + 2 * OLDB <= 160 * 1024;
  static constexpr int LDS = OLD_LDS ? OLD + 2 * OLDB : PARAM + 2048;
  static constexpr int SITEMS = TR * TC * IPX / 512;  // 16-byte stores per thread and tile
  static constexpr int DEPTH = 3;                   // fragment prefetch
  static_assert(C == 16 || C == 32 || C == 64, "channels");
  static_assert(STEPS <= 36, "weights must fit in registers");
  static_assert(WOFF + WBYTES <= PARAM, "prologue weights overlap the parameters");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(SITEMS * 512 == TR * TC * IPX, "store split");
  static_assert(2 * HIT < 64, "vmcnt range");
};

// ACT: the activation of a plain launch (0 .. 4), or 8 + the activation an
// accumulating launch applies after adding the old output (its staged sums
// are not activated).  Both compile-time: a run-time switch per element in
// the epilogue breaks the straight-line MFMA sequence it is interleaved
// into.
template <int KS, int C, int ACT, bool H32 = false>
__global__ __launch_bounds__(512) void conv_res8(ConvArgs a) {
  using R = Res8<KS, C, H32>;
  constexpr int EACT = ACT >= 8 ? IEN_ACT_NONE : ACT;  // on the staged sums
  constexpr int AACT = ACT >= 8 ? ACT - 8 : IEN_ACT_NONE;  // after the old output
  constexpr int IPX = R::IPX, CH = R::CH, NJ = CH / 32;
  constexpr int STEPS = R::STEPS, HC = R::HC, PB = R::PB, P = KS / 2, DEPTH = R::DEPTH;
  constexpr int HIT = R::HIT;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[R::LDS];
  const float *bias_l = (const float *)(lds + R::PARAM), *slope_l = bias_l + 256;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // 32-pixel block, 32-channel half
  const int mg = H32 ? wave : wave & 3, ng = H32 ? 0 : wave >> 2;
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int tn = lb % a.tiles_n;            // this block's CH-channel tile
  const int per_n = gridDim.x / a.tiles_n;  // blocks sharing it
  const int tiles_m = a.tiles_x * a.tiles_y;
  const unsigned lds0 = lds_addr(lds);

  auto origin = [&](int mt, int &oy0, int &ox0) {
    oy0 = (mt / a.tiles_x + a.ty_begin) * R::TR;
    ox0 = (mt % a.tiles_x) * R::TC;
  };

  // Part i of a tile's halo: wave w fills KiB w + 8 i of the buffer; lane l
  // its 16 bytes at 16 l, which belong to halo pixel hp, chunk ch (offsets
  // past the input read the zeros of the pad chunk and padding pixels).
  constexpr int OOB = 0x7ffffff0;
  const int4v xr = buffer_rsrc(a.x, (int)((long)a.H * a.W * a.xs * 2));
  auto load_halo = [&](int i, int oy0, int ox0, int buf) {
    const int g = wave + 8 * i;
    const int byte = g * 1024 + lane * 16;
    const int hp = byte / PB, ch = (byte - hp * PB) >> 4;
    const int hy = hp / HC, hx = hp - hy * HC;
    const int iy = oy0 + hy - P, ix = ox0 + hx - P;
    const bool ok = hp < R::HPIX && ch < C / 8 && (unsigned)iy < (unsigned)a.H &&
                    (unsigned)ix < (unsigned)a.W;
    const int off = ok ? ((iy * a.W + ix) * a.xs + 8 * ch) * 2 : OOB;
    dma_lds(xr, __builtin_amdgcn_readfirstlane(lds0 + buf * R::HALO + g * 1024), off);
  };
  auto load_tile = [&](int mtl, int buf) {
    int oy0, ox0;
    origin(mtl, oy0, ox0);
#pragma unroll
    for (int i = 0; i < HIT; i++) load_halo(i, oy0, ox0, buf);
  };

  // ---- prologue: bias, slopes, weights, then the halos of the first two
  // tiles (the second is the first again when there is none) ----
  if (wave == 0) {  // lanes 0-15: the 64 biases of the tile (padded to NB * 32)
    dma_lds(buffer_rsrc(a.bias, a.NB * 32 * 4), __builtin_amdgcn_readfirstlane(lds0 + R::PARAM),
            lane < 16 ? (tn * CH + 4 * lane) * 4 : OOB);
  } else if (wave == 1) {  // lanes 0-15: the slopes (zeros unless PReLU)
    dma_lds(buffer_rsrc(a.slope, a.act == IEN_ACT_PRELU ? a.N * 4 : 0),
            __builtin_amdgcn_readfirstlane(lds0 + R::PARAM + 1024),
            lane < 16 ? (tn * CH + 4 * lane) * 4 : OOB);
  }
  {
    const int4v wrs = buffer_rsrc(a.wp, a.NB * a.KB * 1024);
    for (int f = wave; f < NJ * STEPS; f += 8) {
      const int jn = f / STEPS, s = f - jn * STEPS;
      dma_lds(wrs, __builtin_amdgcn_readfirstlane(lds0 + R::WOFF + f * 1024),
              ((tn * NJ + jn) * a.KB + s) * 1024 + lane * 16);
    }
  }
  int mt = lb / a.tiles_n;
  const bool any = mt < tiles_m;
  if (any) {
    load_tile(mt, 0);
    load_tile(mt + per_n < tiles_m ? mt + per_n : mt, 1);
  }
  wait_vm<2 * HIT>();  // bias, slopes, weights (the halos may be in flight)
  __syncthreads();
  half8 wr[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; s++)
    wr[s] = *(const half8 *)(lds + R::WOFF + (ng * STEPS + s) * 1024 + lane * 16);
  if (any)
    wait_vm<HIT>();  // the first tile's halo
  else
    wait_vm<0>();  // no tile: nothing may still be writing LDS at the end
  __syncthreads();  // ... of every wave; the weights are in registers

  const int tpix = (mg >> 1) * 64 + (mg & 1) * 32 + (lane & 31);
  const int abase = ((mg >> 1) * HC + (mg & 1) * 32 + (lane & 31)) * PB + 16 * (lane >> 5);

  // Plain f16 NHWC outputs of whole 16-byte chunks below 2 GiB go out as
  // buffer stores; anything else element by element (store_slow).
  const long out_bytes = (long)(a.p_end - a.p_begin) * a.ys * 2;
  const bool plain = !a.out_f32 && !a.out_nchw && a.N % 8 == 0 && a.ys % 8 == 0 &&
                     (((uintptr_t)a.y) & 15) == 0 && out_bytes <= 0x7fff0000L;
  // Accumulating into such outputs: the old items of tile t-1 are loaded
  // straight into LDS in iteration t (before its halo loads, so the wait at
  // the end of the iteration covers them) and added in iteration t+1.
  const bool accum = plain && a.accumulate && R::OLD_LDS;
  const bool fast = plain && (!a.accumulate || accum);
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(a.y, 0, fast ? (int)out_bytes : 0, 0x00020000);
  const int4v yl = buffer_rsrc(a.y, accum ? (int)out_bytes : 0);

  // Byte offset of output item j of this thread (16 bytes: 8 channels of
  // one pixel; 8 consecutive threads write one pixel's 128 bytes), or OOB.
  auto item_off = [&](int j, int mts, bool valid) -> int {
    int oy0, ox0;
    origin(mts, oy0, ox0);
    const int v = tid + 512 * j, tp = v / IPX, chunk = v % IPX;
    const int oy = oy0 + tp / R::TC, ox = ox0 + tp % R::TC;
    const int p = oy * a.OW + ox;
    const int n0 = tn * CH + chunk * 8;
    const bool ok = valid && oy < a.OH && ox < a.OW && p >= a.p_begin && p < a.p_end && n0 < a.N;
    return ok ? ((p - a.p_begin) * a.ys + n0) * 2 : OOB;
  };
  auto item_src = [&](int j, const unsigned char *stage) {
    const int v = tid + 512 * j;
    return *(const u32x4 *)(stage + ((v / IPX) * R::SPX + (v % IPX) * 8) * 2);
  };
  auto old_buf = [&](int k) { return lds + R::OLD + k * R::OLDB; };
  // Old items of tile mts into old buffer k (8 KiB per round of items).
  auto load_old = [&](int mts, int k) {
#pragma unroll
    for (int j = 0; j < R::SITEMS; j++)
      dma_lds(yl, __builtin_amdgcn_readfirstlane(lds0 + R::OLD + k * R::OLDB + (512 * j + 64 * wave) * 16),
              item_off(j, mts, true));
  };
  // Staged sum + old item, activated, for an accumulating store.
  auto add_old = [&](int j, u32x4 sv, const unsigned char *ob) {
    const int v = tid + 512 * j, chunk = v % IPX;
    const u32x4 ov = *(const u32x4 *)(ob + 16 * v);
    uint16_t h[8], o[8];
    __builtin_memcpy(h, &sv, 16);
    __builtin_memcpy(o, &ov, 16);
#pragma unroll
    for (int e = 0; e < 8; e++)
      h[e] = f2h(act_c<AACT>(h2f(h[e]) + h2f(o[e]), slope_l[chunk * 8 + e]));
    __builtin_memcpy(&sv, h, 16);
    return sv;
  };

  // Accumulating, NCHW or ragged outputs: the staged sums (bias included,
  // no activation when accumulating) by whole 16-byte chunks where the
  // output is f16 NHWC with 8-aligned rows, else element by element.
  const bool vec8 = !a.out_f32 && !a.out_nchw && a.ys % 8 == 0 && (((uintptr_t)a.y) & 15) == 0;
  auto store_slow = [&](int mts, const unsigned char *stage) {
    int oy0, ox0;
    origin(mts, oy0, ox0);
    for (int v = tid; v < R::TR * R::TC * IPX; v += 512) {
      const int tp = v / IPX, chunk = v % IPX;
      const int oy = oy0 + tp / R::TC, ox = ox0 + tp % R::TC;
      const int p = oy * a.OW + ox;
      const int n0 = tn * CH + chunk * 8;
      if (oy >= a.OH || ox >= a.OW || p < a.p_begin || p >= a.p_end || n0 >= a.N) continue;
      const int rel = p - a.p_begin;
      u32x4 hv = *(const u32x4 *)(stage + (tp * R::SPX + chunk * 8) * 2);
      uint16_t h[8];
      __builtin_memcpy(h, &hv, 16);
      if (vec8 && n0 + 8 <= a.N) {
        u32x4 *yv = (u32x4 *)((uint16_t *)a.y + (long)rel * a.ys + n0);
        if (a.accumulate) {
          const u32x4 ov = *yv;
          uint16_t oh[8];
          __builtin_memcpy(oh, &ov, 16);
#pragma unroll
          for (int e = 0; e < 8; e++)
            h[e] = f2h(act_c<AACT>(h2f(h[e]) + h2f(oh[e]), slope_l[chunk * 8 + e]));
          __builtin_memcpy(&hv, h, 16);
        }
        *yv = hv;
        continue;
      }
      for (int e = 0; e < 8 && n0 + e < a.N; e++) {
        const long at = a.out_nchw ? (long)(n0 + e) * a.ys + rel : (long)rel * a.ys + n0 + e;
        float o = h2f(h[e]);
        uint16_t *yh = (uint16_t *)a.y + at;
        if (a.accumulate) o = act_c<AACT>(o + h2f(*yh), slope_l[chunk * 8 + e]);
        *yh = f2h(o);
      }
    }
  };

  // One of the 4 epilogue groups of a finished tile.  C^T fragment: the
  // lane holds pixel lane % 32 of its block; register 4 g + e is channel
  // 32 ng + 8 g + 4 (lane / 32) + e.  (When accumulating, EACT is none: the
  // sum is staged and activated after the old output.)
  auto epilogue = [&](const floatx16 &acc, int g, unsigned char *stage) {
    const int ch = ng * 32 + 8 * g + 4 * (lane >> 5);
    const float4v s4 = *(const float4v *)(slope_l + ch);
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) h[e] = f2h(act_c<EACT>(acc[4 * g + e], s4[e]));
    uint2 o;
    __builtin_memcpy(&o, h, 8);
    *(uint2 *)(stage + (tpix * R::SPX + ch) * 2) = o;
  };

  auto bias_acc = [&]() {
    floatx16 acc;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const float4v b4 = *(const float4v *)(bias_l + ng * 32 + 8 * g + 4 * (lane >> 5));
#pragma unroll
      for (int e = 0; e < 4; e++) acc[4 * g + e] = b4[e];
    }
    return acc;
  };

  // The MFMA sequence of tile t on halo buffer `cur`, with tile t+2's halo
  // loads into buffer `nxt` and (unless FIRST: no earlier tile) tile t-1's
  // epilogue and tile t-2's stores spread over the steps.
  auto mma = [&](auto first, int cur, int nxt, int nmt, bool dma, const floatx16 &acc1,
                 unsigned char *stage1, const int *soff, const unsigned char *stage2,
                 int old_mt, int old_wr, const unsigned char *old_rd) {
    constexpr bool FIRST = decltype(first)::value;
    int noy0, nox0;
    origin(nmt, noy0, nox0);
    const unsigned char *bp = lds + cur * R::HALO + abase;
    auto frag = [&](int s) {
      const int tap = s / (C / 16), kc = s % (C / 16);
      return *(const half8 *)(bp + ((tap / KS) * HC + tap % KS) * PB + 32 * kc);
    };
    u32x4 sv[R::SITEMS];
    // Event e at step e * STEPS / NEV, in this order: staged reads of tile
    // t-2, the first halo load, the stores of tile t-2, the other halo
    // loads, the epilogue groups of tile t-1.
    constexpr int NS = R::SITEMS, NEV = FIRST ? HIT : 2 * NS + HIT + 4;
    auto event = [&](int e) {
      if constexpr (FIRST) {
        if (dma) load_halo(e, noy0, nox0, nxt);
      } else {
        if (e < NS) {
          if (e == 0 && accum) load_old(old_mt, old_wr);  // before this tile's halo loads
          sv[e] = item_src(e, stage2);
          if (accum) sv[e] = add_old(e, sv[e], old_rd);
        } else if (e == NS) {
          if (dma) load_halo(0, noy0, nox0, nxt);
        } else if (e < 2 * NS + 1) {
          const int j = e - NS - 1;
          __builtin_amdgcn_raw_buffer_store_b128(sv[j], yr, soff[j], 0, 0);
        } else if (e < 2 * NS + HIT) {
          if (dma) load_halo(e - 2 * NS, noy0, nox0, nxt);
        } else {
          epilogue(acc1, e - 2 * NS - HIT, stage1);
        }
      }
    };
    floatx16 acc = bias_acc();
    half8 xv[DEPTH + 1];
#pragma unroll
    for (int s = 0; s < DEPTH && s < STEPS; s++) xv[s] = frag(s);
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      if (s + DEPTH < STEPS) xv[(s + DEPTH) % (DEPTH + 1)] = frag(s + DEPTH);
#pragma unroll
      for (int e = 0; e < NEV; e++)
        if (e * STEPS / NEV == s) event(e);
      __builtin_amdgcn_sched_barrier(0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wr[s], xv[s % (DEPTH + 1)], acc, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
  };

  // Iteration t: halo buffer t % 3 holds tile t (t+1's is in flight, t+2's
  // is loaded here into buffer (t + 2) % 3, which held tile t-1); staging
  // buffer t % 2 receives tile t-1 and buffer (t + 1) % 2 holds tile t-2.
  auto stage_buf = [&](int k) { return lds + R::STG + k * R::STAGE; };
  floatx16 acc1 = {};
  int mt1 = -1, mt2 = -1;  // the tiles one and two iterations back
  int t = 0, h = 0;        // h = t % 3
  while (mt < tiles_m) {
    const int far = mt + 2 * per_n;
    const bool dma = far < tiles_m;  // a uniform branch: no load without a tile
    const int h2 = h == 0 ? 2 : h - 1;  // (t + 2) % 3
    floatx16 acc;
    if (t == 0) {
      acc = mma(std::true_type{}, h, h2, far, dma, acc1, nullptr, nullptr, nullptr, 0, 0, nullptr);
    } else {
      const int par = t & 1;
      unsigned char *st1 = stage_buf(par);
      const unsigned char *st2 = stage_buf(par ^ 1);
      if (mt2 >= 0 && !fast) store_slow(mt2, st2);
      int soff[R::SITEMS];
#pragma unroll
      for (int j = 0; j < R::SITEMS; j++)
        soff[j] = item_off(j, mt2 < 0 ? mt : mt2, mt2 >= 0 && fast);
      acc = mma(std::false_type{}, h, h2, far, dma, acc1, st1, soff, st2, mt1, t & 1,
                old_buf((t - 1) & 1));
    }
    acc1 = acc;
    mt2 = mt1;
    mt1 = mt;
    mt += per_n;
    t++;
    h = h == 2 ? 0 : h + 1;
    // Tile t+1's halo (loaded before this iteration's HIT loads, which may
    // be in flight; without them the stores in between could be counted
    // in their place, so then wait for everything).
    if (dma)
      wait_vm<HIT>();
    else
      wait_vm<0>();
    __syncthreads();  // ... of every wave; staging written, buffers read
  }
  // Drain: tile t-2's stores and tile t-1's epilogue, then tile t-1's stores.
  const int par = t & 1;
  if (mt2 >= 0) {
    if (fast) {
#pragma unroll
      for (int j = 0; j < R::SITEMS; j++) {
        u32x4 sv = item_src(j, stage_buf(par ^ 1));
        if (accum) sv = add_old(j, sv, old_buf((t - 1) & 1));
        __builtin_amdgcn_raw_buffer_store_b128(sv, yr, item_off(j, mt2, true), 0, 0);
      }
    } else {
      store_slow(mt2, stage_buf(par ^ 1));
    }
  }
  if (mt1 >= 0) {
    if (accum) load_old(mt1, t & 1);
#pragma unroll
    for (int g = 0; g < 4; g++) epilogue(acc1, g, stage_buf(par));
  }
  if (accum) wait_vm<0>();  // tile t-1's old items
  __syncthreads();
  if (mt1 >= 0) {
    if (fast) {
#pragma unroll
      for (int j = 0; j < R::SITEMS; j++) {
        u32x4 sv = item_src(j, stage_buf(par));
        if (accum) sv = add_old(j, sv, old_buf(t & 1));
        __builtin_amdgcn_raw_buffer_store_b128(sv, yr, item_off(j, mt1, true), 0, 0);
      }
    } else {
      store_slow(mt1, stage_buf(par));
    }
  }
}

bool resident_supported(int ks, int stride, int c, int nchw, int reflect, int noff, int rows_mode,
                        long in_bytes) {
  // Buffer-load offsets are 32-bit: inputs below 2 GiB.
  return (ks == 1 || ks == 3) && stride == 1 && (c == 16 || c == 32 || c == 64) && !nchw &&
         !reflect && noff == 0 && !rows_mode && ks * ks * c / 16 <= 36 && in_bytes <= 0x7fff0000L;
}

template <int KS, int C, bool H32 = false>
static ien_status run_res8(ien_ctx *ctx, ConvArgs a) {
  using R = Res8<KS, C, H32>;
  void (*kernel)(ConvArgs) = nullptr;
  // Accumulating: the sums are staged and activated after the old output
  // (ACT 8 + the activation); the tall-tile H32 form never accumulates.
  switch (a.act + (a.accumulate && !H32 ? 8 : 0)) {
    case IEN_ACT_RELU: kernel = conv_res8<KS, C, IEN_ACT_RELU, H32>; break;
    case IEN_ACT_PRELU: kernel = conv_res8<KS, C, IEN_ACT_PRELU, H32>; break;
    case IEN_ACT_GELU: kernel = conv_res8<KS, C, IEN_ACT_GELU, H32>; break;
    case IEN_ACT_SIGMOID: kernel = conv_res8<KS, C, IEN_ACT_SIGMOID, H32>; break;
    case 8 + IEN_ACT_NONE: kernel = conv_res8<KS, C, 8 + IEN_ACT_NONE, H32>; break;
    case 8 + IEN_ACT_RELU: kernel = conv_res8<KS, C, 8 + IEN_ACT_RELU, H32>; break;
    case 8 + IEN_ACT_PRELU: kernel = conv_res8<KS, C, 8 + IEN_ACT_PRELU, H32>; break;
    case 8 + IEN_ACT_GELU: kernel = conv_res8<KS, C, 8 + IEN_ACT_GELU, H32>; break;
    case 8 + IEN_ACT_SIGMOID: kernel = conv_res8<KS, C, 8 + IEN_ACT_SIGMOID, H32>; break;
    default: kernel = conv_res8<KS, C, IEN_ACT_NONE, H32>; break;
  }
  const int first_row = a.p_begin / a.OW, last_row = (a.p_end - 1) / a.OW;
  a.ty_begin = first_row / R::TR;
  a.tiles_y = last_row / R::TR + 1 - a.ty_begin;
  a.tiles_x = (a.OW + R::TC - 1) / R::TC;
  a.tiles_n = (a.N + R::CH - 1) / R::CH;
  IEN_CHECK(a.tiles_n * (R::CH / 32) <= a.NB, IEN_ERR_INPUT, "weights narrower than the tile");
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
      case 32:
        // At most 32 outputs, not accumulating: every wave on them, tiles
        // of 4 rows (the old-output buffers of accumulating tiles would not
        // fit beside the larger halos).
        if (a.N <= 32 && !a.accumulate) return run_res8<3, 32, true>(ctx, a);
        return run_res8<3, 32>(ctx, a);
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
