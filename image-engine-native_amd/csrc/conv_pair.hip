// conv_pair.hip -- consecutive 3x3 64 -> 64 convolutions, each with bias
// and PReLU, two per tile pass: pairs of Real-ESRGAN's body layers
// (crates/realesrgan-native/src/network.rs:96-109; gemm.rs multiply order).
//
// A launch of one such layer at 256 x 384 spends about as long on fixed
// costs (the gap after the previous kernel, the weights landing, the last
// stores draining) as on its products; a pair pays them once, and a chain
// of pairs (the whole body in one launch) once for all of them.
//
// One workgroup of 8 waves (two per SIMD) computes a 16 x 24 tile of a
// pair's second layer:
//  - The input halo, 20 x 28 pixels of 64 channels, is loaded straight into
//    LDS (zeros outside the image, from the buffer range check), each pixel
//    followed by a 16-byte pad chunk and each row by 224 bytes, so that
//    the B fragments of packed pixel blocks read LDS without bank conflicts.
//  - Phase 1: the first layer on the 18 x 26 pixels the second one reads,
//    packed row after row into 15 blocks of 32 (each lane addresses its own
//    pixel, so a block may span rows and only the halo itself is computed
//    twice).  Pixels outside the image are stored as zeros: the second
//    layer's zero padding.  The results go to LDS as f16, rounded as the
//    map between two separate launches would hold them.
//  - Phase 2: the second layer on the 16 x 24 output pixels (12 blocks).
// Wave w takes the 32 output channels of half w / 4 and the blocks w % 4,
// w % 4 + 4, ...; it holds that half of one layer's packed weights in
// registers (36 fragments, the A operand of v_mfma_f32_32x32x16_f16, so the
// product is C^T = W^T X^T), each layer's loaded once per workgroup into
// LDS and from there into registers.  Every accumulator is seeded with the
// bias and sums the 36 steps (9 taps x 16 channels, taps first) in the
// order of the one-layer resident kernel, so a pair gives the same bits as
// two launches of it.
//
// A chain runs P pairs in one launch with one workgroup per tile, all
// resident at once (at most one per CU).  A tile keeps its pair output in
// LDS as the centre of the next pair's halo and exchanges only the 2-pixel
// ring with its 8 neighbours: after pair k it stores the outer 2 rows and
// columns of its output to border map k % 2 and, once those stores are
// complete, publishes epoch k + 1; pair k + 1 waits until each neighbour's
// epoch reaches k + 1 and loads its ring from that map.  The neighbours may
// run on other XCDs, whose L2 caches are not kept coherent with this one:
// the border stores, the ring loads and the epoch words all use device
// scope (the sc1 cache policy: written through to, and read from, the
// device's point of coherence), so no cache-wide write-back or invalidate
// is needed.  A neighbour only publishes after it has
// read its own ring from the other map, so a border map is never rewritten
// while a reader still needs it.  Every wait is bounded by a wall-clock
// limit; a tile that runs out sets an abort word that every other waiting
// tile sees, so all workgroups end (the run reports the failure).  The last
// pair stores the whole tile.  Each workgroup counts itself out as its last
// act; the last one out returns the epochs, the abort word and the count to
// zero, so the next chain on the stream starts from clear flags without a
// launch of its own for them.

#include "conv_common.h"

namespace ien {
namespace {

constexpr int C = 64;                      // channels in, between and out
constexpr int OTR = 16, OTC = 24;          // output tile
constexpr int MR = OTR + 2, MC = OTC + 2;  // first layer's pixels: 18 x 26
constexpr int IR = OTR + 4, IC = OTC + 4;  // input halo: 20 x 28
constexpr int PB = 2 * C + 16;             // bytes of a staged pixel
// Staged rows end with padding, which with 144-byte pixels (16
// consecutive pixels on disjoint banks) makes a block's step from the last
// pixel of one of its rows to the first of the next land on the banks of a
// one-pixel step, so no B-fragment read conflicts even where a block spans
// rows: the first layer's results are read in rows of 24 (of 26), the halo
// in rows of 26 (of 28) by a single pair and, interior first, in rows of
// 22 by a chain.
constexpr int MROW = MC * PB + 224;  // bytes a staged row of the first layer's results
constexpr int MPIX = MR * MC, OPIX = OTR * OTC;
constexpr int WBYTES = 2 * (9 * C / 16) * 1024;  // both halves of a layer
constexpr int STEPS = 9 * C / 16;
constexpr int MBLK = (MPIX + 31) / 32, OBLK = OPIX / 32;
constexpr int WAVES = 8, THREADS = 64 * WAVES;
constexpr int WLOADS = WBYTES / (1024 * WAVES);  // 1 KiB weight loads per wave
constexpr int INNER = (MR - 4) * (MC - 4);       // first-layer pixels that read no halo ring
constexpr int MAXPAIRS = 16;
#ifndef IEN_PAIR_PREFETCH
#define IEN_PAIR_PREFETCH 1
#endif
constexpr int PREFETCH = IEN_PAIR_PREFETCH;  // steps a B fragment is loaded ahead of its products
static_assert((MROW - 23 * PB) % 256 == PB, "first layer's rows");
static_assert(MBLK <= 16 && OBLK == 12 && INNER >= 8 * 32, "block split over the waves");
static_assert(WLOADS * 1024 * WAVES == WBYTES, "weight loads");

// LDS layout: the halo, then the first layer's results (its weights before
// them), then the biases and slopes of both layers.
template <bool CHAIN>
struct Geo {
  static constexpr int HROW = IC * PB + (CHAIN ? 160 : 224);  // bytes a staged halo row
  static constexpr int HALO = IR * HROW;
  static constexpr int MID = HALO;
  static constexpr int PARAM = MID + std::max(MR * MROW, WBYTES);
  static constexpr int LDS = PARAM + 4 * C * 4;
  static constexpr int HLOADS = (HALO + 1024 * WAVES - 1) / (1024 * WAVES);  // 1 KiB loads a wave
  static constexpr int RSPAN = (2 * HROW + 1023) / 1024;  // 1 KiB loads of two ring rows
  static_assert(LDS <= 160 * 1024 && HALO % 16 == 0, "LDS budget");
  static_assert((HROW - ((CHAIN ? MC - 4 : MC) - 1) * PB) % 256 == PB, "halo rows");
  static_assert(HLOADS + WLOADS < 64, "load split");
  static_assert((WAVES - 1 + WAVES * (HLOADS - 2)) * 1024 + 1024 <= HALO, "halo loads before the last");
  static_assert(WBYTES <= HALO, "second layer's weights in the halo");
};

// The first layer's pixel i (of MPIX) in a pass order: row-major, or for a
// chain the INNER pixels that read only the halo's centre first (rows 2 ..
// 15, columns 2 .. 23, row-major), then rows 0, 1, then columns 0, 1, 24,
// 25 of rows 2 .. 15, then rows 16, 17.
template <bool CHAIN>
__device__ __forceinline__ int first_pixel(int i) {
  if (!CHAIN) return i;
  if (i < INNER) return (2 + i / (MC - 4)) * MC + 2 + i % (MC - 4);
  i -= INNER;
  if (i < 2 * MC) return i;
  i -= 2 * MC;
  if (i < 4 * (MR - 4)) {
    const int c = i & 3;
    return (2 + (i >> 2)) * MC + (c < 2 ? c : c + MC - 4);
  }
  return (MR - 2) * MC + i - 4 * (MR - 4);
}

struct PairArgs {
  const uint16_t *x;  // H x W x 64 f16 input (pixels 64 halves apart)
  uint16_t *y;        // the same shape: the last pair's output
  int H, W, tiles_x, tiles_y;
  int KB;     // fragments along k of each layer (36)
  int pairs;  // 1, or the chain's length
  // Layer 2 k and 2 k + 1 of pair k: packed weights (fragment (kb, nb) at
  // (nb KB + kb) 512 halves), biases and PReLU slopes (64 each).
  const uint16_t *w[2 * MAXPAIRS];
  const float *b[2 * MAXPAIRS], *s[2 * MAXPAIRS];
  // Chain only: the border maps (pair k stores to border[k % 2]); the
  // flags: the abort word, the failure word (raised to this launch's
  // sequence number `seq` when a wait gives up, never lowered, so the host
  // tells which launches failed without clearing it), the count of
  // workgroups done, then the tile epochs (tiles_x tiles_y words); all but
  // the failure word are zero at launch and again at the end; and the
  // wall-clock ticks (100 MHz) a wait for neighbours may take (negative: no
  // wait succeeds, every tile with a neighbour gives up at its first wait --
  // the failure path on demand).
  uint16_t *border[2];
  int *flags;
  int seq;
  long spin_limit;
  // Chain only, optional (wl null: none): a final 3x3 64 -> 48 layer
  // (weights packed with n padded, bias; no activation) whose 48 channels
  // are pixel-shuffled x4 and added to the f32 RGB image (H x W x 3) into
  // out ((4 H) x (4 W) x 3 f32) instead of the last pair storing its map.
  const uint16_t *wl;
  const float *bl;
  const float *image;
  float *out;
  // Chain only, optional (w0 null: none): the first layer, 3x3 over the
  // image's RGB and a zero fourth channel (weights packed with k = 36 in
  // 3 fragments, bias, PReLU slopes), computed by the first pair on its
  // halo from the f32 image instead of reading x.
  const uint16_t *w0;
  const float *b0, *s0;
};

constexpr int OOB = 0x7ffffff0;
constexpr int SC1 = 16;  // cache policy bits of a device-scope buffer access

// dma_lds at device scope (sc1): the load bypasses copies in this XCD's
// caches that another XCD's device-scope stores may have made stale.
__device__ __forceinline__ void dma_lds_device(int4v rsrc, unsigned wave_base, int off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen sc1 lds"
               :: "s"(wave_base), "v"(off), "s"(rsrc) : "memory", "m0");
}

template <bool CHAIN>
__global__ __launch_bounds__(THREADS) void conv_pair(PairArgs a) {
  using G = Geo<CHAIN>;
  constexpr int HROW = G::HROW, HALO = G::HALO, MID = G::MID, PARAM = G::PARAM;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[G::LDS];
  __shared__ int go;  // chain: 1 when every neighbour is ready
  __shared__ float img[CHAIN ? OTR * OTC * 3 : 1];  // chain: the final layer's image tile
  float *par = (float *)(lds + PARAM);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = wave >> 2, grp = wave & 3;  // channel half, block group
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int ty = tile / a.tiles_x, tx = tile % a.tiles_x;
  const int y0 = ty * OTR, x0 = tx * OTC;
  const unsigned lds0 = lds_addr(lds);
  const long map_bytes = (long)a.H * a.W * C * 2;

  // Lane l's 16 bytes of fragment (step s, channel half hf): rows 16 s +
  // 8 (l / 32) .. + 7 of output channel 32 hf + l % 32.
  half8 w[STEPS];
  // A layer's fragments of both halves, (hf 36 + s) KiB from `at`, once per
  // workgroup.
  auto stage_weights = [&](const uint16_t *wp, int at) {
    const int4v wr = buffer_rsrc(wp, WBYTES);
#pragma unroll
    for (int i = 0; i < WLOADS; i++) {
      const int f = wave + WAVES * i;
      dma_lds(wr, __builtin_amdgcn_readfirstlane(lds0 + at + f * 1024), f * 1024 + lane * 16);
    }
  };
  auto params = [&](int k) {
    if (tid < C) {
      par[tid] = a.b[2 * k][tid];
      par[C + tid] = a.s[2 * k][tid];
      par[2 * C + tid] = a.b[2 * k + 1][tid];
      par[3 * C + tid] = a.s[2 * k + 1][tid];
    }
  };
  // Global offset of chunk ch (8 channels) of halo pixel (hy, hx), or OOB
  // for the pad chunk and pixels outside the image.
  auto halo_src = [&](int hy, int hx, int ch) {
    const int gy = y0 - 2 + hy, gx = x0 - 2 + hx;
    const bool ok = hx < IC && ch < 8 && (unsigned)gy < (unsigned)a.H && (unsigned)gx < (unsigned)a.W;
    return ok ? ((gy * a.W + gx) * C + 8 * ch) * 2 : OOB;
  };

  // The accumulators of a block, seeded with the bias: register 4 g + e is
  // channel 32 hf + 8 g + 4 (lane / 32) + e of pixel lane % 32.
  auto seed = [&](const float *bias) {
    floatx16 acc;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const float4v b4 = *(const float4v *)(bias + 32 * hf + 8 * g + 4 * (lane >> 5));
#pragma unroll
      for (int e = 0; e < 4; e++) acc[4 * g + e] = b4[e];
    }
    return acc;
  };
  // acc[j] += W^T X^T over the 36 steps for NB blocks whose lane bases are
  // base[j] in a staged map of rows ROW bytes apart.  With STREAM the
  // weights come into w from their staging at `wat` in step with the B
  // fragments (the first products after a layer's weights are staged), so
  // that their loads overlap the products instead of preceding them.
  auto products = [&](auto nblocks, auto row, const int *base, floatx16 *acc, auto stream,
                      int wat) {
    constexpr int NB = decltype(nblocks)::value, ROW = decltype(row)::value;
    constexpr bool STREAM = decltype(stream)::value;
    constexpr int DEPTH = PREFETCH;  // steps the B fragments are loaded ahead
    auto frag = [&](int j, int s) {
      const int tap = s / 4, kc = s % 4;
      return *(const half8 *)(lds + base[j] + (tap / 3) * ROW + (tap % 3) * PB + 32 * kc);
    };
    half8 xv[NB][DEPTH + 1];
#pragma unroll
    for (int s = 0; s < DEPTH; s++) {
      if (STREAM) w[s] = *(const half8 *)(lds + wat + (hf * STEPS + s) * 1024 + lane * 16);
#pragma unroll
      for (int j = 0; j < NB; j++) xv[j][s] = frag(j, s);
    }
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      if (s + DEPTH < STEPS) {
        if (STREAM)
          w[s + DEPTH] = *(const half8 *)(lds + wat + (hf * STEPS + s + DEPTH) * 1024 + lane * 16);
#pragma unroll
        for (int j = 0; j < NB; j++) xv[j][(s + DEPTH) % (DEPTH + 1)] = frag(j, s + DEPTH);
      }
#pragma unroll
      for (int j = 0; j < NB; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s], xv[j][s % (DEPTH + 1)], acc[j], 0, 0, 0);
      // Keeps each step's loads ahead of the products they feed: left to
      // itself the scheduler sinks them to just before their use, and every
      // product then waits out an LDS round trip.
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using streamed = std::true_type;
  using held = std::false_type;
  // The PReLU slopes of the lane's 16 channels, the same for every block.
  auto slopes = [&](const float *slope, float4v *s4) {
#pragma unroll
    for (int g = 0; g < 4; g++) s4[g] = *(const float4v *)(slope + 32 * hf + 8 * g + 4 * (lane >> 5));
  };
  // Activation and f16 of a block's accumulators, all bits cleared where
  // keep is 0: out[g] holds channels 32 hf + 8 g + 4 (lane / 32) .. + 3 of
  // pixel lane % 32.
  auto finish = [&](const floatx16 &acc, const float4v *s4, unsigned keep, uint2 *out) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; e++) h[e] = f2h(act_c<IEN_ACT_PRELU>(acc[4 * g + e], s4[g][e]));
      __builtin_memcpy(&out[g], h, 8);
      out[g].x &= keep;
      out[g].y &= keep;
    }
  };
  // Pass `pass` of phase 1: the first layer on blocks grp + 4 (2 pass + j),
  // j < 2, of its pixels in first_pixel order; blocks past the last are
  // computed on its final pixel and dropped.  Results to LDS as f16
  // (zeros outside the image: the second layer's padding).  Pass 0 streams
  // the layer's weights from their staging in MID.  after() runs once the
  // products are issued, before the results are stored: pass 0's waits for
  // every wave to hold its weights (MID then takes the results), pass 1's
  // for every wave to be done with the halo and stages the next weights
  // there, behind this pass's epilogue.
  auto first_pass = [&](auto pass_c, auto after) {
    constexpr int pass = decltype(pass_c)::value;
    int base[2], pix[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = 32 * (grp + 4 * (2 * pass + j)) + (lane & 31);
      const int pc = first_pixel<CHAIN>(i < MPIX ? i : MPIX - 1);
      pix[j] = i < MPIX ? pc : -1;
      base[j] = (pc / MC) * HROW + (pc % MC) * PB + 16 * (lane >> 5);
    }
    floatx16 acc[2] = {seed(par), seed(par)};
    products(std::integral_constant<int, 2>{}, std::integral_constant<int, HROW>{}, base, acc,
             std::integral_constant<bool, pass == 0>{}, MID);
    __builtin_amdgcn_sched_barrier(0);
    after();
    float4v s4[4];
    slopes(par + C, s4);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int p = pix[j];
      if (p < 0) continue;
      const int gy = y0 - 1 + p / MC, gx = x0 - 1 + p % MC;
      const bool inside = (unsigned)gy < (unsigned)a.H && (unsigned)gx < (unsigned)a.W;
      uint2 o[4];
      finish(acc[j], s4, inside ? ~0u : 0u, o);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int ch = 32 * hf + 8 * g + 4 * (lane >> 5);
        *(uint2 *)(lds + MID + (p / MC) * MROW + (p % MC) * PB + ch * 2) = o[g];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // The products of the 3 output blocks of a wave (grp, grp + 4, grp + 8:
  // 32 output pixels q each), seeded with `bias`, on a staged map whose
  // output pixel q's tap (0, 0) is at base_of(q) (rows ROW bytes apart):
  // two blocks, then one, each passed to emit(j, acc) as soon as its
  // products are issued, so that no more than two blocks' accumulators and
  // fragments are live beside the weights.  The first two stream the
  // layer's weights from their staging at `wat`, which emit may overwrite
  // once every wave has them (the barrier after those products).
  auto three_blocks = [&](auto row, const float *bias, int wat, auto base_of, auto emit) {
    {
      int base[2];
#pragma unroll
      for (int j = 0; j < 2; j++) base[j] = base_of(32 * (grp + 4 * j) + (lane & 31));
      floatx16 acc[2] = {seed(bias), seed(bias)};
      products(std::integral_constant<int, 2>{}, row, base, acc, streamed{}, wat);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // every wave holds its weights: emit may overwrite their staging
      emit(0, acc[0]);
      emit(1, acc[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    int base[1] = {base_of(32 * (grp + 8) + (lane & 31))};
    floatx16 acc[1] = {seed(bias)};
    products(std::integral_constant<int, 1>{}, row, base, acc, held{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    emit(2, acc[0]);
  };

  // Chain, first pair with a first layer: the first layer's outputs on the
  // whole 20 x 28 halo, from the image patch around it (22 x 30 pixels of
  // f16 RGB and a zero fourth channel) and the layer's 6 fragments, both
  // staged in MID; as the separate 4-channel kernel computes them (one
  // v_mfma_f32_32x32x16_f16 step covers 4 taps of 4 channels, lane half h
  // reading taps 4 s + 2 h and 4 s + 2 h + 1; taps 9 .. 11 read tap 0
  // against zero weights), PReLU, zeros outside the image.
  constexpr int PR = IR + 2, PC = IC + 2;  // the patch: 22 x 30
  auto first_layer = [&]() {
    for (int i = tid; i < PR * PC; i += THREADS) {
      const int gy = y0 - 3 + i / PC, gx = x0 - 3 + i % PC;
      uint16_t h[4] = {0, 0, 0, 0};
      if ((unsigned)gy < (unsigned)a.H && (unsigned)gx < (unsigned)a.W) {
        const float *im = a.image + ((long)gy * a.W + gx) * 3;
        h[0] = f2h(im[0]);
        h[1] = f2h(im[1]);
        h[2] = f2h(im[2]);
      }
      uint2 v;
      __builtin_memcpy(&v, h, 8);
      *(uint2 *)(lds + MID + i * 8) = v;
    }
    constexpr int W0AT = MID + PR * PC * 8;  // the fragments after the patch
    static_assert((MID + PR * PC * 8) % 16 == 0 && PR * PC * 8 + 6 * 1024 <= WBYTES, "patch");
    if (wave < 6) {
      const int4v w0r = buffer_rsrc(a.w0, 6 * 1024);
      dma_lds(w0r, __builtin_amdgcn_readfirstlane(lds0 + W0AT + wave * 1024), wave * 1024 + lane * 16);
    }
    if (tid < C) {
      par[tid] = a.b0[tid];
      par[C + tid] = a.s0[tid];
    }
    wait_vm<0>();
    __syncthreads();
    half8 w0[3];
#pragma unroll
    for (int s = 0; s < 3; s++) w0[s] = *(const half8 *)(lds + W0AT + (hf * 3 + s) * 1024 + lane * 16);
    float4v s4[4];
    slopes(par + C, s4);
    auto tap = [](int t) { return t < 9 ? ((t / 3) * PC + t % 3) * 8 : 0; };
    for (int blk = grp; blk * 32 < IR * IC; blk += 4) {
      const int p = 32 * blk + (lane & 31), pc = p < IR * IC ? p : IR * IC - 1;
      const int hy = pc / IC, hx = pc % IC;
      const unsigned char *pb = lds + MID + (hy * PC + hx) * 8;
      floatx16 acc = seed(par);
#pragma unroll
      for (int s = 0; s < 3; s++) {
        const int t0 = 4 * s + 2 * (lane >> 5);
        typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
        const u32x2v q0 = *(const u32x2v *)(pb + tap(t0)), q1 = *(const u32x2v *)(pb + tap(t0 + 1));
        const u32x4 raw = {q0[0], q0[1], q1[0], q1[1]};
        half8 xb;
        __builtin_memcpy(&xb, &raw, 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0[s], xb, acc, 0, 0, 0);
      }
      if (p >= IR * IC) continue;
      const int gy = y0 - 2 + hy, gx = x0 - 2 + hx;
      const bool inside = (unsigned)gy < (unsigned)a.H && (unsigned)gx < (unsigned)a.W;
      uint2 o[4];
      finish(acc, s4, inside ? ~0u : 0u, o);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int ch = 32 * hf + 8 * g + 4 * (lane >> 5);
        *(uint2 *)(lds + hy * HROW + hx * PB + ch * 2) = o[g];
      }
    }
    __syncthreads();  // the halo is complete; MID and the parameters are free
  };

  int *abort_word = CHAIN ? a.flags : nullptr;
  int *epochs = CHAIN ? a.flags + 3 : nullptr;
  // Chain: the workgroup's last act on every way out.  Only wave 0 writes
  // the flags (the epoch stores, the abort and failure words); every wave
  // reads the epochs and the abort word, always before the barrier that
  // ends a ring wait, so once wave 0 counts the workgroup out no access of
  // it to the flags remains.  The count's release orders wave 0's flag
  // stores before it, and the workgroup that brings it to the grid size
  // (every other one has left) clears the flags.
  auto leave = [&]() {
    if (wave != 0) return;
    int done = 0;
    if (lane == 0)
      done = __hip_atomic_fetch_add(a.flags + 2, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    done = __builtin_amdgcn_readfirstlane(done);
    if (done != (int)gridDim.x - 1) return;
    for (int i = lane; i < (int)gridDim.x; i += 64)
      __hip_atomic_store(epochs + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0) {
      __hip_atomic_store(abort_word, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.flags + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  const int pairs = CHAIN ? a.pairs : 1;
  // Chain: lane n < 9 (n != 4) of a wave watches neighbour (ty + n / 3 - 1,
  // tx + n % 3 - 1): its epoch word, or null where there is none.
  auto neighbour = [&]() -> const int * {
    if (lane < 9 && lane != 4) {
      const int ny = ty + lane / 3 - 1, nx = tx + lane % 3 - 1;
      if (ny >= 0 && ny < a.tiles_y && nx >= 0 && nx < a.tiles_x) return epochs + ny * a.tiles_x + nx;
    }
    return nullptr;
  };
  // Chain: this wave's share of the loads of the halo's 2-pixel ring from
  // the neighbours' border map (k - 1) % 2, at device scope.  A load fills
  // one contiguous KiB of LDS, 16 bytes a lane: staged chunk q of a run of
  // pixels is chunk q % 9 of pixel q / 9 (chunk 8, the pad, and pixels
  // outside the image read zeros).
  auto ring_loads = [&](int k) {
    // The lane index through an opaque move: the offsets below are then
    // computed where they are used rather than kept live (or spilled) from
    // the kernel's start, so that no spill reload, whose wait would also
    // wait for every load in flight, lands between these loads.
    int lane;
    asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(tid & 63));
    const int4v rr = buffer_rsrc(a.border[(k - 1) & 1], map_bytes);
    auto src = [&](int gy, int gx, int c) {
      const bool ok = c < 8 && (unsigned)gx < (unsigned)a.W && (unsigned)gy < (unsigned)a.H;
      return ok ? ((gy * a.W + gx) * C + 8 * c) * 2 : OOB;
    };
    // Halo rows 0, 1, 18, 19 whole: 28 pixels, 252 chunks, 4 loads a row
    // (the last 4 lanes of the fourth write zeros into the row's padding).
    for (int i = wave; i < 16; i += WAVES) {
      const int r = i >> 2, part = i & 3, hy = r < 2 ? r : r + IR - 4;
      const int q = 64 * part + lane, p = (int)((unsigned)q / 9u);
      dma_lds_device(rr, __builtin_amdgcn_readfirstlane(lds0 + hy * HROW + part * 1024),
                     q < 9 * IC ? src(y0 - 2 + hy, x0 - 2 + p, q - 9 * p) : OOB);
    }
    // Pixels 0, 1 and 26, 27 of rows 2 .. 17: 18 chunks (lanes 0 .. 17) a load.
    for (int i = wave; i < 2 * (IR - 4); i += WAVES) {
      const int hy = 2 + (i >> 1), hx0 = (i & 1) ? IC - 2 : 0;
      const int p = lane >= 9 ? 1 : 0;
      if (lane < 18)
        dma_lds_device(rr, __builtin_amdgcn_readfirstlane(lds0 + hy * HROW + hx0 * PB),
                       src(y0 - 2 + hy, x0 - 2 + hx0 + p, lane - 9 * p));
    }
  };
  // Chain: the ring of pair k.  Each wave waits for its neighbours' epoch k
  // (lane n for neighbour n) and issues its share of the loads, then waits
  // for them; the barrier follows.  False when a wait gave up: wave 0 then
  // raises the abort word (which every waiting tile watches) and the
  // failure word.
  auto ring = [&](int k) {
    bool fail = false;
    if (const int *f = neighbour()) {
      const unsigned long long t0 = wall_clock64();
      while (a.spin_limit < 0 ||
             __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < k) {
        if (__hip_atomic_load(abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
            (long)(wall_clock64() - t0) > a.spin_limit) {
          fail = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    if (__builtin_amdgcn_ballot_w64(fail) != 0) {
      if (lane == 0) go = 0;
    } else {
      ring_loads(k);
    }
    wait_vm<0>();
    __syncthreads();
    if (go != 0) return true;
    if (tid == 0) {
      __hip_atomic_store(abort_word, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_max(abort_word + 1, a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return false;
  };
  if (CHAIN && tid == 0) go = 1;  // (seen after the first pair's opening barrier)
  // A chain's final layer adds the tile's image rows (24 pixels x RGB,
  // 288 bytes each): into their own LDS array now, so that the loads are
  // long done when the tail needs them (the first pair's waits cover them);
  // rows past the image read zeros.
  if constexpr (CHAIN) {
    if (a.wl) {
      const int4v ir = buffer_rsrc(a.image, (long)a.H * a.W * 12);
      const unsigned i0 = lds_addr(img);
      for (int i = wave; i < 2 * OTR; i += WAVES) {
        const int r = i >> 1, part = i & 1, e = 64 * part + lane;
        if (e < OTC * 3)
          dma_lds4(ir, __builtin_amdgcn_readfirstlane(i0 + (r * OTC * 3 + 64 * part) * 4),
                   y0 + r < a.H ? (((y0 + r) * a.W + x0) * 3 + e) * 4 : OOB);
      }
    }
  }
  for (int k = 0; k < pairs; k++) {
    // ---- the first layer's weights (where its results will go) and, for
    // a single pair or a chain's first, the whole halo from the input; a
    // chain's later pairs find the weights staged and the halo's centre
    // left in LDS by the pair before ----
    if (CHAIN && k == 0 && a.w0) {
      first_layer();
      stage_weights(a.w[0], MID);
    } else if (!CHAIN || k == 0) {
      stage_weights(a.w[2 * k], MID);
      // KiB g of the halo: lane l's 16 bytes belong to halo row hy, pixel
      // hx, chunk ch (chunk 8 and the row padding read zeros, as do
      // offsets past the input); lanes past the halo's end load nothing.
      const int4v xr = buffer_rsrc(a.x, map_bytes);
#pragma unroll
      for (int i = 0; i < G::HLOADS; i++) {
        const int g = wave + WAVES * i, byte = g * 1024 + lane * 16;
        const int hy = byte / HROW, within = byte - hy * HROW;
        const int hx = within / PB, ch = (within - hx * PB) >> 4;
        if (i < G::HLOADS - 1 || byte < HALO)  // only the last KiB runs past the halo
          dma_lds(xr, __builtin_amdgcn_readfirstlane(lds0 + g * 1024), halo_src(hy, hx, ch));
      }
    }
    params(k);
    wait_vm<0>();  // (a chain's later pairs: also the previous border stores)
    __syncthreads();
    if (CHAIN && k > 0 && tid == 0)  // publish epoch k: this tile's pair k - 1 border is out
      __hip_atomic_store(epochs + tile, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- phase 1: the first layer on the 18 x 26 pixels in two passes;
    // a chain's first pass reads only the halo's centre, and the ring
    // comes in between the passes ----
    first_pass(std::integral_constant<int, 0>{}, [] {
      __syncthreads();  // every wave holds its weights: MID may take the results
    });
    if (CHAIN && k > 0 && !ring(k)) {  // (no load of this workgroup is in flight here)
      leave();
      return;
    }
    // ---- and the second layer's weights, staged where the halo was ----
    first_pass(std::integral_constant<int, 1>{}, [&] {
      __syncthreads();  // every wave is done with the halo
      stage_weights(a.w[2 * k + 1], 0);
    });
    wait_vm<0>();
    __syncthreads();  // the first layer's results complete, the weights staged

    // ---- phase 2: the second layer on the 16 x 24 outputs, blocks grp,
    // grp + 4, grp + 8 ----
    auto mid_base = [&](int q) { return MID + (q / OTC) * MROW + (q % OTC) * PB + 16 * (lane >> 5); };
    float4v s4[4];
    slopes(par + 3 * C, s4);

    if constexpr (!CHAIN) {
      // Each wave's 96 pixels of its 32 channels go out through LDS (its
      // own 6 KiB where the halo was), so that a lane stores 16 bytes and
      // 4 lanes a pixel's 64 contiguous bytes.  Staged pixel wp = 32 j +
      // l % 32 holds its 4 chunks of 8 channels at chunk c ^ (wp / 4 % 4),
      // which keeps both the writes (16 pixels, one chunk) and the reads
      // (4 pixels, 4 chunks) free of bank conflicts.
      unsigned char *stage = lds + wave * (OBLK / 4) * 32 * 64;
      three_blocks(std::integral_constant<int, MROW>{}, par + 2 * C, 0, mid_base,
                   [&](int j, const floatx16 &acc) {
        uint2 o[4];
        finish(acc, s4, ~0u, o);
        const int wp = 32 * j + (lane & 31);
#pragma unroll
        for (int pr = 0; pr < 2; pr++) {
          // Lanes < 32 hold channels 16 pr + 0..3 (o[2 pr]) and 16 pr +
          // 8..11 (o[2 pr + 1]), lanes >= 32 the runs 4 above; swapping the
          // upper half's o[2 pr] with the lower half's o[2 pr + 1] gives
          // lane l < 32 channels 16 pr + 0..7 and lane l + 32 channels
          // 16 pr + 8..15.
          const auto sx = __builtin_amdgcn_permlane32_swap(o[2 * pr].x, o[2 * pr + 1].x, false, false);
          const auto sy = __builtin_amdgcn_permlane32_swap(o[2 * pr].y, o[2 * pr + 1].y, false, false);
          const uint4 v = {sx[0], sy[0], sx[1], sy[1]};
          const int c = 2 * pr + (lane >> 5);
          *(uint4 *)(stage + wp * 64 + 16 * (c ^ ((wp >> 2) & 3))) = v;
        }
      });
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const __amdgpu_buffer_rsrc_t yr =
          __builtin_amdgcn_make_buffer_rsrc(a.y, 0, (int)map_bytes, 0x00020000);
#pragma unroll
      for (int i = 0; i < 6; i++) {
        const int v = lane + 64 * i, wp = v >> 2, c = v & 3;
        const uint4 d = *(const uint4 *)(stage + wp * 64 + 16 * (c ^ ((wp >> 2) & 3)));
        const int q = 32 * (grp + 4 * (wp >> 5)) + (wp & 31);
        const int gy = y0 + q / OTC, gx = x0 + q % OTC;
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 dv = {d.x, d.y, d.z, d.w};
        __builtin_amdgcn_raw_buffer_store_b128(
            dv, yr, gy < a.H && gx < a.W ? (gy * a.W + gx) * C * 2 + 64 * hf + 16 * c : OOB, 0, 0);
      }
    } else {
      // The results become the centre of the next pair's halo (zeros
      // outside the image: its padding).
      const bool last = k == pairs - 1 && !a.wl;  // (a final layer follows the last pair)
      const __amdgpu_buffer_rsrc_t br =
          __builtin_amdgcn_make_buffer_rsrc(a.border[k & 1], 0, (int)map_bytes, 0x00020000);
      three_blocks(std::integral_constant<int, MROW>{}, par + 2 * C, 0, mid_base,
                   [&](int j, const floatx16 &acc) {
        const int q = 32 * (grp + 4 * j) + (lane & 31), r = q / OTC, col = q % OTC;
        const bool inside = y0 + r < a.H && x0 + col < a.W;
        uint2 o[4];
        finish(acc, s4, inside ? ~0u : 0u, o);
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int ch = 32 * hf + 8 * g + 4 * (lane >> 5);
          *(uint2 *)(lds + (2 + r) * HROW + (2 + col) * PB + ch * 2) = o[g];
        }
      });
      __syncthreads();  // the centre is complete; the first layer's results are read
      if (last) {
        // The whole tile out, 16 bytes a lane (8 lanes a pixel).
        const __amdgpu_buffer_rsrc_t yr =
            __builtin_amdgcn_make_buffer_rsrc(a.y, 0, (int)map_bytes, 0x00020000);
        for (int v = tid; v < OPIX * 8; v += THREADS) {
          const int c = v & 7, b = v >> 3, r = b / OTC, col = b % OTC;
          const uint4 d = *(const uint4 *)(lds + (2 + r) * HROW + (2 + col) * PB + 16 * c);
          const int gy = y0 + r, gx = x0 + col;
          typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
          const u32x4 dv = {d.x, d.y, d.z, d.w};
          __builtin_amdgcn_raw_buffer_store_b128(
              dv, yr, gy < a.H && gx < a.W ? (gy * a.W + gx) * C * 2 + 16 * c : OOB, 0, 0);
        }
      } else {
        // The pixels of the outer 2 rows (0, 1, 14, 15) and columns (0, 1,
        // 22, 23), which the neighbours read, to border map k % 2 at device
        // scope, with the next pair's first weights staged behind them
        // (their completion, and so the epoch, is awaited at the next
        // pair's start).  (Stored straight from the registers during phase
        // 2 instead, they cost more than this pass.)
        // All of a thread's chunks are read from LDS before any is stored.
        constexpr int CHUNKS = (4 * OTC + 4 * (OTR - 4)) * 8;
        constexpr int PER = (CHUNKS + THREADS - 1) / THREADS;
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        u32x4 dv[PER];
        int at[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
          const int v = tid + THREADS * i, vc = v < CHUNKS ? v : CHUNKS - 1;
          const int c = vc & 7, b = vc >> 3;
          int r, col;
          if (b < 4 * OTC) {
            r = b / OTC;
            r = r < 2 ? r : r + OTR - 4;
            col = b % OTC;
          } else {
            r = 2 + ((b - 4 * OTC) >> 2);
            col = (b - 4 * OTC) & 3;
            col = col < 2 ? col : col + OTC - 4;
          }
          const uint4 d = *(const uint4 *)(lds + (2 + r) * HROW + (2 + col) * PB + 16 * c);
          dv[i] = u32x4{d.x, d.y, d.z, d.w};
          const int gy = y0 + r, gx = x0 + col;
          at[i] = v < CHUNKS && gy < a.H && gx < a.W ? (gy * a.W + gx) * C * 2 + 16 * c : OOB;
        }
#pragma unroll
        for (int i = 0; i < PER; i++) __builtin_amdgcn_raw_buffer_store_b128(dv[i], br, at[i], 0, SC1);
        stage_weights(k + 1 < pairs ? a.w[2 * k + 2] : a.wl, MID);
      }
    }
  }

  if constexpr (CHAIN) {
    if (!a.wl) {
      leave();
      return;
    }
    // ---- the final layer on the 16 x 24 tile, read from the halo (its
    // 1-pixel ring inside the 2-pixel one), no activation; then the pixel
    // shuffle x4 plus the image, as f32 RGB ----
    const int k = pairs;
    if (tid < C) par[tid] = a.bl[tid];  // zero past channel 48
    wait_vm<0>();  // the last border stores (the image rows landed long ago)
    __syncthreads();
    if (tid == 0) __hip_atomic_store(epochs + tile, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!ring(k)) {
      leave();
      return;
    }
    // Results [pixel][48] in MID (73728 bytes), rounded through f16 as the
    // last layer's map between separate launches holds them, so that the
    // chain's output is bit for bit that of the separate launches.
    float *res = (float *)(lds + MID);
    auto r16 = [](float v) { return h2f(f2h(v)); };
    three_blocks(std::integral_constant<int, HROW>{}, par, MID,
                 [&](int q) { return (1 + q / OTC) * HROW + (1 + q % OTC) * PB + 16 * (lane >> 5); },
                 [&](int j, const floatx16 &acc) {
      const int q = 32 * (grp + 4 * j) + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int ch = 32 * hf + 8 * g + 4 * (lane >> 5);
        if (ch < 48)
          *(float4v *)(res + q * 48 + ch) = float4v{r16(acc[4 * g]), r16(acc[4 * g + 1]),
                                                    r16(acc[4 * g + 2]), r16(acc[4 * g + 3])};
      }
    });
    __syncthreads();
    // Output row 4 r + i (r < 16) of the tile holds 96 pixels x RGB: 72
    // chunks of 4 floats, three per input pixel; float f of chunk q is
    // output pixel 4 x + j (x = f / 12, j = f / 3 % 4), colour c = f % 3:
    // channel 16 c + 4 i + j of input pixel (r, x) plus the image's colour c.
    const long ow = 4L * a.W;
    for (int v = tid; v < 4 * OTR * 72; v += THREADS) {
      const int row = v / 72, q = v - row * 72;
      const int r = row >> 2, i = row & 3, x = q / 3;
      const int gy = y0 + r, gx = x0 + x;
      if (gy >= a.H || gx >= a.W) continue;
      const float *px = res + (r * OTC + x) * 48;
      const float *im = img + (r * OTC + x) * 3;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int f = 4 * q + e - 12 * x, j = f / 3, c = f - 3 * j;
        o[e] = px[16 * c + 4 * i + j] + im[c];
      }
      *(float4v *)(a.out + ((4L * gy + i) * ow + 4L * x0) * 3 + 4 * q) = float4v{o[0], o[1], o[2], o[3]};
    }
    leave();
  }
}

bool layer_ok(const ien_matrix *m, const float *slope) {
  return m && m->k == 9 * C && m->n == C && m->kb == STEPS && m->nb >= 2 && m->d_packed &&
         m->d_bias && slope;
}

bool maps_ok(const uint16_t *x, const uint16_t *y, int H, int W) {
  const long bytes = (long)H * W * C * 2;
  const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
  return H > 0 && W > 0 && bytes <= 0x7fff0000L && ((xa | ya) & 15) == 0 &&
         (xa + bytes <= ya || ya + bytes <= xa);
}

void fill_layers(PairArgs &a, const ien_matrix *const *w, const float *const *s, int layers) {
  for (int i = 0; i < layers; i++) {
    a.w[i] = w[i]->d_packed;
    a.b[i] = w[i]->d_bias;
    a.s[i] = s[i];
  }
  a.KB = w[0]->kb;
}

}  // namespace

bool pair_supported(const PairCall &p) {
  return layer_ok(p.w1, p.s1) && layer_ok(p.w2, p.s2) && maps_ok(p.x, p.y, p.H, p.W);
}

ien_status launch_pair(ien_ctx *ctx, const PairCall &p) {
  IEN_CHECK(pair_supported(p), IEN_ERR_INPUT, "not a pair of 3x3 64-channel PReLU layers");
  PairArgs a = {};
  a.x = p.x;
  a.y = p.y;
  a.H = p.H;
  a.W = p.W;
  a.tiles_x = (p.W + OTC - 1) / OTC;
  a.tiles_y = (p.H + OTR - 1) / OTR;
  a.pairs = 1;
  const ien_matrix *w[2] = {p.w1, p.w2};
  const float *s[2] = {p.s1, p.s2};
  fill_layers(a, w, s, 2);
  const long tiles = (long)a.tiles_x * a.tiles_y;
  IEN_CHECK(tiles > 0 && tiles < (1L << 31), IEN_ERR_INPUT, "grid of %ld", tiles);
  hipLaunchKernelGGL(conv_pair<false>, dim3((unsigned)tiles), dim3(THREADS), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

bool chain_supported(ien_ctx *ctx, const ChainCall &c) {
  if (!ctx->chain_flags || c.pairs < 1 || c.pairs > MAXPAIRS || !maps_ok(c.a, c.b, c.H, c.W))
    return false;
  for (int i = 0; i < 2 * c.pairs; i++)
    if (!layer_ok(c.w[i], c.s[i])) return false;
  if (c.first) {
    const ien_matrix *m = c.first;
    if (m->k != 36 || m->n != C || m->kb != 3 || m->nb < 2 || !m->d_packed || !m->d_bias ||
        !c.first_slope || !c.image)
      return false;
  }
  if (c.last) {
    const ien_matrix *m = c.last;
    if (m->k != 9 * C || m->n != 48 || m->kb != STEPS || m->nb < 2 || !m->d_packed || !m->d_bias ||
        !c.image || !c.out || ((uintptr_t)c.out & 15) != 0 ||
        (long)c.H * c.W * 48 > 0x7fff0000L)
      return false;
  }
  // Every tile's workgroup resident at once: one per CU at most.
  if (ctx->chain_per_cu < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, conv_pair<true>, THREADS, 0) != hipSuccess)
      n = 0;
    ctx->chain_per_cu = n;
  }
  const long tiles = (long)((c.W + OTC - 1) / OTC) * ((c.H + OTR - 1) / OTR);
  return ctx->chain_per_cu >= 1 && tiles <= (long)ctx->cus && tiles <= ctx->chain_tiles;
}

ien_status launch_chain(ien_ctx *ctx, const ChainCall &c, uint16_t **out) {
  IEN_CHECK(chain_supported(ctx, c), IEN_ERR_INPUT, "not a chain this device runs at once");
  PairArgs a = {};
  a.x = c.a;
  a.border[0] = c.b;
  a.border[1] = c.a;
  a.y = a.border[(c.pairs - 1) & 1];
  a.H = c.H;
  a.W = c.W;
  a.tiles_x = (c.W + OTC - 1) / OTC;
  a.tiles_y = (c.H + OTR - 1) / OTR;
  a.pairs = c.pairs;
  fill_layers(a, c.w, c.s, 2 * c.pairs);
  a.flags = ctx->chain_flags;
  a.seq = ++ctx->chain_seq;
  a.spin_limit = ctx->chain_spin;
  if (c.first) {
    a.w0 = c.first->d_packed;
    a.b0 = c.first->d_bias;
    a.s0 = c.first_slope;
    a.image = c.image;
  }
  if (c.last) {
    a.wl = c.last->d_packed;
    a.bl = c.last->d_bias;
    a.image = c.image;
    a.out = c.out;
  }
  const int tiles = a.tiles_x * a.tiles_y;
  hipLaunchKernelGGL(conv_pair<true>, dim3((unsigned)tiles), dim3(THREADS), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  *out = c.last ? nullptr : a.y;
  return IEN_OK;
}

ien_status chain_status(ien_ctx *ctx, int first) {
  int word = 0;
  IEN_HIP(hipMemcpyAsync(&word, ctx->chain_flags + 1, 4, hipMemcpyDeviceToHost, ctx->stream));
  IEN_HIP(hipStreamSynchronize(ctx->stream));
  if (word < first || word <= ctx->chain_reported) return IEN_OK;
  ctx->chain_reported = word;
  return fail(IEN_ERR_GPU, "body chain: a tile's wait for its neighbours timed out");
}

}  // namespace ien

using namespace ien;

extern "C" ien_status ien_conv3_pair(ien_ctx *ctx, const uint16_t *d_x, uint16_t *d_y,
                                     size_t height, size_t width, const ien_matrix *w1,
                                     const float *d_slope1, const ien_matrix *w2,
                                     const float *d_slope2) {
  IEN_CHECK(ctx && d_x && d_y && w1 && w2 && d_slope1 && d_slope2, IEN_ERR_INPUT,
            "null argument");
  IEN_CHECK(height > 0 && width > 0 && height < (1u << 20) && width < (1u << 20), IEN_ERR_INPUT,
            "map of %zu x %zu", height, width);
  for (const ien_matrix *m : {w1, w2})
    IEN_CHECK(m->k == 9 * C && m->n == C, IEN_ERR_INPUT,
              "pair layers are 3x3 64->64 (k 576, n 64), not k %zu, n %zu", m->k, m->n);
  const size_t bytes = height * width * C * 2;
  IEN_CHECK(bytes <= 0x7fff0000UL, IEN_ERR_INPUT, "map of %zu bytes over 2 GiB", bytes);
  IEN_CHECK((((uintptr_t)d_x | (uintptr_t)d_y) & 15) == 0, IEN_ERR_INPUT,
            "maps must be 16-byte aligned");
  const uintptr_t x = (uintptr_t)d_x, y = (uintptr_t)d_y;
  IEN_CHECK(x + bytes <= y || y + bytes <= x, IEN_ERR_INPUT, "input and output maps overlap");
  PairCall p;
  p.x = d_x;
  p.y = d_y;
  p.H = (int)height;
  p.W = (int)width;
  p.w1 = w1;
  p.s1 = d_slope1;
  p.w2 = w2;
  p.s2 = d_slope2;
  return launch_pair(ctx, p);
}

extern "C" ien_status ien_conv3_chain(ien_ctx *ctx, uint16_t *d_a, uint16_t *d_b, size_t height,
                                      size_t width, size_t pairs, const ien_matrix *const *w,
                                      const float *const *d_slopes, uint16_t **d_out) {
  IEN_CHECK(ctx && d_a && d_b && w && d_slopes && d_out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(pairs >= 1 && pairs <= MAXPAIRS, IEN_ERR_INPUT, "%zu pairs (1 to %d)", pairs, MAXPAIRS);
  IEN_CHECK(height > 0 && width > 0 && height < (1u << 20) && width < (1u << 20), IEN_ERR_INPUT,
            "map of %zu x %zu", height, width);
  ChainCall c;
  c.a = d_a;
  c.b = d_b;
  c.H = (int)height;
  c.W = (int)width;
  c.pairs = (int)pairs;
  for (size_t i = 0; i < 2 * pairs; i++) {
    IEN_CHECK(w[i] && d_slopes[i], IEN_ERR_INPUT, "layer %zu: null argument", i);
    IEN_CHECK(w[i]->k == 9 * C && w[i]->n == C, IEN_ERR_INPUT,
              "layer %zu: chain layers are 3x3 64->64 (k 576, n 64), not k %zu, n %zu", i, w[i]->k,
              w[i]->n);
    c.w[i] = w[i];
    c.s[i] = d_slopes[i];
  }
  const size_t bytes = height * width * C * 2;
  IEN_CHECK(bytes <= 0x7fff0000UL, IEN_ERR_INPUT, "map of %zu bytes over 2 GiB", bytes);
  IEN_CHECK((((uintptr_t)d_a | (uintptr_t)d_b) & 15) == 0, IEN_ERR_INPUT,
            "maps must be 16-byte aligned");
  const uintptr_t a = (uintptr_t)d_a, b = (uintptr_t)d_b;
  IEN_CHECK(a + bytes <= b || b + bytes <= a, IEN_ERR_INPUT, "the two maps overlap");
  IEN_CHECK(chain_supported(ctx, c), IEN_ERR_INPUT,
            "a %zu x %zu map has more 16 x 24 tiles than this device holds at once", height, width);
  return launch_chain(ctx, c, d_out);
}

extern "C" ien_status ien_conv3_chain_status(ien_ctx *ctx) {
  IEN_CHECK(ctx, IEN_ERR_INPUT, "null argument");
  IEN_HIP(hipSetDevice(ctx->device));
  return chain_status(ctx, 1);
}

