// conv_pair.hip -- two consecutive 3x3 64 -> 64 convolutions, each with
// bias and PReLU, in one launch: a pair of Real-ESRGAN's body layers
// (crates/realesrgan-native/src/network.rs:96-109; gemm.rs multiply order).
//
// A launch of one such layer at 256 x 384 spends about as long on fixed
// costs (the gap after the previous kernel, the weights landing, the last
// stores draining) as on its products; a pair pays them once.
//
// One workgroup of 8 waves (two per SIMD) computes a 16 x 24 tile of the
// second layer's outputs:
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
//  - Phase 2: the second layer on the 16 x 24 output pixels (12 blocks),
//    each wave storing its own results as they are finished.
// Wave w takes the 32 output channels of half w / 4 and the blocks w % 4,
// w % 4 + 4, ...; it holds that half of one layer's packed weights in
// registers (36 fragments, the A operand of v_mfma_f32_32x32x16_f16, so the
// product is C^T = W^T X^T): the first layer's loaded once per workgroup
// into LDS beside the halo, the second's straight from memory, each
// fragment as soon as the first layer's last product with it has been
// issued.  Every
// accumulator is seeded with the bias and sums the 36 steps (9 taps x 16
// channels, taps first) in the order of the one-layer resident kernel, so
// a pair gives the same bits as two launches of it.

#include "conv_common.h"

namespace ien {
namespace {

constexpr int C = 64;                      // channels in, between and out
constexpr int OTR = 16, OTC = 24;          // output tile
constexpr int MR = OTR + 2, MC = OTC + 2;  // first layer's pixels: 18 x 26
constexpr int IR = OTR + 4, IC = OTC + 4;  // input halo: 20 x 28
constexpr int PB = 2 * C + 16;             // bytes of a staged pixel
// Staged rows end with 224 bytes of padding: 144-byte pixels put 16
// consecutive pixels on disjoint banks, and with the padding a block's step
// from the last pixel of a row to the first of the next (3 pixels on in the
// staged row) lands on the banks of a one-pixel step, so no B-fragment read
// conflicts even where a block spans rows.
constexpr int RPAD = 224;
constexpr int HROW = IC * PB + RPAD, MROW = MC * PB + RPAD;  // bytes a staged row
constexpr int MPIX = MR * MC, OPIX = OTR * OTC;
constexpr int HALO = IR * HROW;
constexpr int MID = HALO;  // first layer's results; its weights before them
constexpr int WBYTES = 2 * (9 * C / 16) * 1024;  // both halves of a layer
constexpr int MIDSZ = std::max(MR * MROW, WBYTES);
constexpr int PARAM = MID + MIDSZ;
constexpr int LDS = PARAM + 4 * C * 4;                  // bias 1, slope 1, bias 2, slope 2
constexpr int STEPS = 9 * C / 16;
constexpr int MBLK = (MPIX + 31) / 32, OBLK = OPIX / 32;
constexpr int WAVES = 8, THREADS = 64 * WAVES;
constexpr int HLOADS = (HALO + 1024 * WAVES - 1) / (1024 * WAVES);  // 1 KiB halo loads per wave
constexpr int WLOADS = WBYTES / (1024 * WAVES);  // 1 KiB weight loads per wave
static_assert(LDS <= 160 * 1024, "LDS budget");
static_assert(HALO % 16 == 0 && (RPAD + 2 * PB) % 256 == 0, "row padding");
static_assert(MBLK <= 16 && OBLK == 12, "block split over the waves");
static_assert(HLOADS + WLOADS < 64 && WLOADS * 1024 * WAVES == WBYTES, "load split");
static_assert((WAVES - 1 + WAVES * (HLOADS - 2)) * 1024 + 1024 <= HALO, "halo loads before the last");

struct PairArgs {
  const uint16_t *x;  // H x W x 64 f16 (pixels 64 halves apart)
  uint16_t *y;        // the same shape; must not overlap x
  int H, W, tiles_x;
  const uint16_t *w1, *w2;  // packed weights (fragment (kb, nb) at (nb KB + kb) 512 halves)
  int KB;
  const float *b1, *s1, *b2, *s2;  // biases and PReLU slopes (64 each)
};

constexpr int OOB = 0x7ffffff0;

__global__ __launch_bounds__(THREADS) void conv_pair(PairArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS];
  float *par = (float *)(lds + PARAM);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = wave >> 2, grp = wave & 3;  // channel half, block group
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int y0 = (tile / a.tiles_x) * OTR, x0 = (tile % a.tiles_x) * OTC;
  const unsigned lds0 = lds_addr(lds);

  // Lane l's 16 bytes of fragment (step s, channel half hf): rows 16 s +
  // 8 (l / 32) .. + 7 of output channel 32 hf + l % 32.
  half8 w[STEPS];
  {
    // KiB g of the halo: lane l's 16 bytes belong to halo row hy, pixel hx,
    // chunk ch (chunk 8 and the row padding read zeros, as do offsets past
    // the input); lanes past the halo's end load nothing.
    const int4v xr = buffer_rsrc(a.x, (long)a.H * a.W * C * 2);
#pragma unroll
    for (int i = 0; i < HLOADS; i++) {
      const int g = wave + WAVES * i, byte = g * 1024 + lane * 16;
      const int hy = byte / HROW, within = byte - hy * HROW;
      const int hx = within / PB, ch = (within - hx * PB) >> 4;
      const int gy = y0 - 2 + hy, gx = x0 - 2 + hx;
      const bool ok = hx < IC && ch < 8 && (unsigned)gy < (unsigned)a.H &&
                      (unsigned)gx < (unsigned)a.W;
      if (i < HLOADS - 1 || byte < HALO)  // only the last KiB runs past the halo
        dma_lds(xr, __builtin_amdgcn_readfirstlane(lds0 + g * 1024),
                ok ? ((gy * a.W + gx) * C + 8 * ch) * 2 : OOB);
    }
    // The first layer's fragments of both halves, (hf 36 + s) KiB, once per
    // workgroup, where the first layer's results will go.
    const int4v wr = buffer_rsrc(a.w1, WBYTES);
#pragma unroll
    for (int i = 0; i < WLOADS; i++) {
      const int f = wave + WAVES * i;
      dma_lds(wr, __builtin_amdgcn_readfirstlane(lds0 + MID + f * 1024), f * 1024 + lane * 16);
    }
  }
  if (tid < C) {
    par[tid] = a.b1[tid];
    par[C + tid] = a.s1[tid];
    par[2 * C + tid] = a.b2[tid];
    par[3 * C + tid] = a.s2[tid];
  }
  wait_vm<0>();
  __syncthreads();
#pragma unroll
  for (int s = 0; s < STEPS; s++) w[s] = *(const half8 *)(lds + MID + (hf * STEPS + s) * 1024 + lane * 16);
  __syncthreads();  // every wave holds its weights: the first results may overwrite them

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
  // base[j] in a staged map of rows ROW bytes apart.
  auto products = [&](auto nblocks, auto row, const int *base, floatx16 *acc) {
    constexpr int NB = decltype(nblocks)::value, ROW = decltype(row)::value;
    constexpr int DEPTH = NB > 2 ? 2 : 3;  // B fragment prefetch
    auto frag = [&](int j, int s) {
      const int tap = s / 4, kc = s % 4;
      return *(const half8 *)(lds + base[j] + (tap / 3) * ROW + (tap % 3) * PB + 32 * kc);
    };
    half8 xv[NB][DEPTH + 1];
#pragma unroll
    for (int s = 0; s < DEPTH; s++)
#pragma unroll
      for (int j = 0; j < NB; j++) xv[j][s] = frag(j, s);
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      if (s + DEPTH < STEPS)
#pragma unroll
        for (int j = 0; j < NB; j++) xv[j][(s + DEPTH) % (DEPTH + 1)] = frag(j, s + DEPTH);
#pragma unroll
      for (int j = 0; j < NB; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s], xv[j][s % (DEPTH + 1)], acc[j], 0, 0, 0);
    }
  };
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

  // ---- phase 1: the first layer on the 18 x 26 pixels, blocks grp +
  // 4 i (i < 4) in two passes of two; blocks past the last are computed on
  // its final pixel and dropped ----
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
    int base[2], pix[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int p = 32 * (grp + 4 * (2 * pass + j)) + (lane & 31);
      pix[j] = p;
      const int pc = p < MPIX ? p : MPIX - 1;
      base[j] = (pc / MC) * HROW + (pc % MC) * PB + 16 * (lane >> 5);
    }
    floatx16 acc[2] = {seed(par), seed(par)};
    products(std::integral_constant<int, 2>{}, std::integral_constant<int, HROW>{}, base, acc);
    __builtin_amdgcn_sched_barrier(0);
    float4v s4[4];
    slopes(par + C, s4);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int p = pix[j];
      if (p >= MPIX) continue;
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
  }
  __syncthreads();  // the first layer's results complete; the halo is free

  // ---- the second layer's weights, staged where the halo was ----
  {
    const int4v wr = buffer_rsrc(a.w2, WBYTES);
#pragma unroll
    for (int i = 0; i < WLOADS; i++) {
      const int f = wave + WAVES * i;
      dma_lds(wr, __builtin_amdgcn_readfirstlane(lds0 + f * 1024), f * 1024 + lane * 16);
    }
  }
  wait_vm<0>();
  __syncthreads();
#pragma unroll
  for (int s = 0; s < STEPS; s++) w[s] = *(const half8 *)(lds + (hf * STEPS + s) * 1024 + lane * 16);
  __syncthreads();  // every wave holds its weights: the staging below may overwrite them

  // ---- phase 2: the second layer on the 16 x 24 outputs, blocks grp,
  // grp + 4, grp + 8 ----
  int base[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const int q = 32 * (grp + 4 * j) + (lane & 31);
    base[j] = MID + (q / OTC) * MROW + (q % OTC) * PB + 16 * (lane >> 5);
  }
  floatx16 acc[3] = {seed(par + 2 * C), seed(par + 2 * C), seed(par + 2 * C)};
  products(std::integral_constant<int, 3>{}, std::integral_constant<int, MROW>{}, base, acc);

  // Each wave's 96 pixels of its 32 channels go out through LDS (its own
  // 6 KiB where the halo was), so that a lane stores 16 bytes and 4 lanes
  // a pixel's 64 contiguous bytes.  Staged pixel wp = 32 j + l % 32 holds
  // its 4 chunks of 8 channels at chunk c ^ (wp / 4 % 4), which keeps both
  // the writes (16 pixels, one chunk) and the reads (4 pixels, 4 chunks)
  // free of bank conflicts.
  unsigned char *stage = lds + wave * (OBLK / 4) * 32 * 64;
  float4v s4[4];
  slopes(par + 3 * C, s4);
#pragma unroll
  for (int j = 0; j < 3; j++) {
    uint2 o[4];
    finish(acc[j], s4, ~0u, o);
    const int wp = 32 * j + (lane & 31);
#pragma unroll
    for (int pr = 0; pr < 2; pr++) {
      // Lanes < 32 hold channels 16 pr + 0..3 (o[2 pr]) and 16 pr + 8..11
      // (o[2 pr + 1]), lanes >= 32 the runs 4 above; swapping the upper
      // half's o[2 pr] with the lower half's o[2 pr + 1] gives lane l < 32
      // channels 16 pr + 0..7 and lane l + 32 channels 16 pr + 8..15.
      const auto sx = __builtin_amdgcn_permlane32_swap(o[2 * pr].x, o[2 * pr + 1].x, false, false);
      const auto sy = __builtin_amdgcn_permlane32_swap(o[2 * pr].y, o[2 * pr + 1].y, false, false);
      const uint4 v = {sx[0], sy[0], sx[1], sy[1]};
      const int c = 2 * pr + (lane >> 5);
      *(uint4 *)(stage + wp * 64 + 16 * (c ^ ((wp >> 2) & 3))) = v;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(a.y, 0, (int)((long)a.H * a.W * C * 2), 0x00020000);
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
}

}  // namespace

bool pair_supported(const PairCall &p) {
  auto layer = [](const ien_matrix *m, const float *slope) {
    return m && m->k == 9 * C && m->n == C && m->kb == STEPS && m->nb >= 2 && slope;
  };
  const long bytes = (long)p.H * p.W * C * 2;
  const uintptr_t x = (uintptr_t)p.x, y = (uintptr_t)p.y;
  return layer(p.w1, p.s1) && layer(p.w2, p.s2) && p.H > 0 && p.W > 0 && bytes <= 0x7fff0000L &&
         ((x | y) & 15) == 0 && (x + bytes <= y || y + bytes <= x);
}

ien_status launch_pair(ien_ctx *ctx, const PairCall &p) {
  IEN_CHECK(pair_supported(p), IEN_ERR_INPUT, "not a pair of 3x3 64-channel PReLU layers");
  PairArgs a;
  a.x = p.x;
  a.y = p.y;
  a.H = p.H;
  a.W = p.W;
  a.tiles_x = (p.W + OTC - 1) / OTC;
  a.w1 = p.w1->d_packed;
  a.w2 = p.w2->d_packed;
  a.KB = p.w1->kb;
  a.b1 = p.w1->d_bias;
  a.s1 = p.s1;
  a.b2 = p.w2->d_bias;
  a.s2 = p.s2;
  const long tiles = (long)a.tiles_x * ((p.H + OTR - 1) / OTR);
  IEN_CHECK(tiles > 0 && tiles < (1L << 31), IEN_ERR_INPUT, "grid of %ld", tiles);
  hipLaunchKernelGGL(conv_pair, dim3((unsigned)tiles), dim3(THREADS), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
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
