// conv_small.hip -- convolutions whose channel counts leave most of an MFMA
// tile empty in the general kernel (conv.hip), which pads the input to
// 16-channel steps and the output to 64-channel tiles.
//
// conv_narrow: NHWC inputs of 4 channels (LaMa's masked image,
// lama-native network.rs:46-58 first conv, 7x7 reflect; SCUNet's image
// with a zero fourth channel, scunet-native network.rs:113-140 head, 3x3).
// K = taps x 4 is dense: one v_mfma_f32_32x32x16_f16 step covers 4 taps of
// 4 channels, lane half h reading taps 4s + 2h and 4s + 2h + 1 (two 8-byte
// LDS reads).  The product is C^T = W^T X^T: the packed weight fragments
// are the A operand and stay in VGPRs for the whole launch (64 output
// channels, 2 x ceil(taps / 4) fragments), the pixels are the B operand.
// Persistent workgroups of 8 waves walk 8 x 32-pixel tiles (wave w: tile
// row w).  Halos (8 bytes a pixel) are loaded straight into LDS as 4-byte
// items by buffer loads the compiler does not see, two tiles ahead into
// three buffers; the range check of the buffer loads supplies the zero
// padding.  Each iteration issues the previous tile's stores first, then
// the loads, so the end-of-tile vmcnt wait for the next halo rarely waits
// for stores.  Each wave stages its 32 pixels x 64 channels in LDS and
// writes whole 16-byte chunks of pixel rows.  The activation is a template
// parameter (no branch per value).
//
// conv_few: NHWC inputs of 64 channels into N outputs with N x KS <= 32
// (LaMa's last conv 64 -> 3 7x7 reflect + sigmoid, network.rs:415-489;
// SCUNet's tail 64 -> 3 3x3, network.rs:113-140).  The MFMA rows are the
// (output, kx) pairs and K = (ky, channel): for an output row y and 64
// consecutive padded input columns q,
//   Z[(n, kx)][q] = sum_ky sum_c W[ky][kx][c][n] in[y + ky - P][q][c],
// then out[n][x] = bias[n] + sum_kx Z[(n, kx)][x + kx]: 64 - 2P outputs per
// 64 columns, the kx sum read back from LDS.  A workgroup of 4 waves (one
// output row each) stages the item's KS + 3 input rows x 64 columns in LDS
// (a ring: going down a column tile, an item loads only its 4 new rows)
// with whole 128-byte pixels, loaded into registers while the previous
// item computes; the A operand stays in LDS too.  Padding is applied to the
// input row and column indices (reflect, or zero for rows and columns
// outside the image: those read the context's zero buffer).
// Both: bias, old output when accumulating, activation -- the order of
// gemm.rs:583-666.

#include "conv_common.h"

namespace ien {

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Input row or column i of an n-pixel axis: reflected (valid) or zero
// padded (valid only inside).  Indices far outside (pixels that only feed
// outputs past the edge) are clamped so that every address stays inside.
__device__ __forceinline__ int pad_index(int i, int n, bool reflect, bool &ok) {
  ok = reflect || (unsigned)i < (unsigned)n;
  if (reflect) i = reflect_idx(i, n);
  return min(max(i, 0), n - 1);
}

template <int KS>
struct Narrow {
  static constexpr int P = KS / 2, TAPS = KS * KS;
  static constexpr int STEPS = (TAPS * 4 + 15) / 16;  // 4 taps of 4 channels a step
  static constexpr int WAVES = 8, TR = WAVES, TC = 32;
  static constexpr int HR = TR + KS - 1, HC = TC + KS - 1, HPIX = HR * HC;
  // The halo (HPIX pixels x 8 bytes) as dwords, half a pixel each, loaded
  // straight into LDS: HL 256-byte loads per wave, whole rounds of 8 waves.
  static constexpr int HL = (HPIX * 2 + WAVES * 64 - 1) / (WAVES * 64);
  static constexpr int HALO = HL * WAVES * 256;  // bytes a buffer
  static constexpr int SPX = 64 + 8;             // staged halves a pixel
  static constexpr int STAGE = 32 * SPX * 2;     // bytes a wave
  static constexpr int PARAM = 3 * HALO;         // 64 biases and 64 slopes (512 bytes)
  static constexpr int STG = PARAM + 512;
  static constexpr int LDS = STG + WAVES * STAGE;
  static_assert(2 * STEPS * 1024 <= WAVES * STAGE, "the prologue's weights fit the staging");
  static_assert(HL < 16, "vmcnt range");
  static_assert(LDS <= 64 * 1024, "LDS budget");
};

// Byte offset of tap t's pixel from the tap-(0, 0) pixel of a halo row of
// HC pixels; the padding taps past KS x KS (zero weights) read tap 0.
template <int KS>
__device__ __forceinline__ constexpr int tap_off(int t) {
  return t < KS * KS ? ((t / KS) * Narrow<KS>::HC + t % KS) * 8 : 0;
}

template <int KS, int ACT>
__global__ __launch_bounds__(512) void conv_narrow(ConvArgs a) {
  using R = Narrow<KS>;
  constexpr int STEPS = R::STEPS, P = R::P, HL = R::HL;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[R::LDS];
  float *bias_l = (float *)(lds + R::PARAM), *slope_l = bias_l + 64;

  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tn = blockIdx.x % a.tiles_n;            // this block's 64 output channels
  const int per_n = gridDim.x / a.tiles_n;          // blocks sharing them
  const int tiles_x = (a.OW + R::TC - 1) / R::TC;
  const int tiles_m = tiles_x * ((a.OH + R::TR - 1) / R::TR);
  const bool reflect = a.pad_reflect != 0;
  const unsigned lds0 = lds_addr(lds);

  auto origin = [&](int mt, int &oy0, int &ox0) {
    oy0 = (mt / tiles_x) * R::TR;
    ox0 = (mt % tiles_x) * R::TC;
  };
  // The halo of tile mt into LDS buffer `buf`: load i of this wave carries
  // dwords d = 64 (wave + 8 i) + lane, i.e. channels 2 (d % 2), +1 of halo
  // pixel d / 2.  Zero padding and the dwords past the halo read the
  // buffer's range check (zeros); reflect padding reads the mirrored pixel.
  constexpr int OOB = 0x7ffffff0;
  const int4v xr = buffer_rsrc(a.x, (long)a.H * a.W * a.xs * 2);
  auto load_halo = [&](int mt, int buf) {
    int oy0, ox0;
    origin(mt, oy0, ox0);
#pragma unroll
    for (int i = 0; i < HL; i++) {
      const int d = 64 * (wave + R::WAVES * i) + lane, hp = d >> 1;
      const int hy = hp / R::HC, hx = hp - hy * R::HC;
      bool oky, okx;
      const int iy = pad_index(oy0 + hy - P, a.H, reflect, oky);
      const int ix = pad_index(ox0 + hx - P, a.W, reflect, okx);
      const int off = hp < R::HPIX && oky && okx ? ((iy * a.W + ix) * a.xs + 2 * (d & 1)) * 2 : OOB;
      dma_lds4(xr, __builtin_amdgcn_readfirstlane(lds0 + buf * R::HALO + 256 * (wave + R::WAVES * i)),
               off);
    }
  };

  // ---- prologue: weights (fragments (2 tn + j, s)) through the staging
  // area into VGPRs, biases and slopes into LDS, the first two halos ----
  for (int f = wave; f < 2 * STEPS; f += R::WAVES) {
    const int j = f / STEPS, s = f - j * STEPS;
    *(u32x4 *)(lds + R::STG + f * 1024 + lane * 16) =
        *(const u32x4 *)(a.wp + ((long)(2 * tn + j) * a.KB + s) * 512 + lane * 8);
  }
  if (tid < 64) {
    const int n = tn * 64 + tid;
    bias_l[tid] = a.bias[n];  // padded to whole 128-column tiles
    slope_l[tid] = ACT == IEN_ACT_PRELU && n < a.N ? a.slope[n] : 0.0f;
  }
  int mt = blockIdx.x / a.tiles_n;
  const bool any = mt < tiles_m, second = mt + per_n < tiles_m;
  if (any) load_halo(mt, 0);
  if (second) load_halo(mt + per_n, 1);
  if (second)
    wait_vm<HL>();  // the first halo (the second may be in flight)
  else
    wait_vm<0>();
  __syncthreads();
  half8 wr[2][STEPS];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int s = 0; s < STEPS; s++)
      wr[j][s] = *(const half8 *)(lds + R::STG + (j * STEPS + s) * 1024 + lane * 16);
  __syncthreads();  // every wave has its weights before the staging is written

  unsigned char *stage = lds + R::STG + wave * R::STAGE;
  uint16_t *yh = (uint16_t *)a.y;
  // The staged tile ending at (oy0, ox0): 32 pixels x 8 chunks of 16 bytes,
  // item v = lane + 64 q.
  auto store_tile = [&](int oy0, int ox0) {
    const int oy = oy0 + wave;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int v = lane + 64 * q, px = v >> 3, chunk = v & 7;
      const u32x4 val = *(const u32x4 *)(stage + (px * R::SPX + 8 * chunk) * 2);
      const int sx = ox0 + px, n = tn * 64 + 8 * chunk;
      if (oy < a.OH && sx < a.OW && n < a.N)
        *(u32x4 *)(yh + ((long)oy * a.OW + sx) * a.ys + n) = val;
    }
  };

  // Iteration t: buffer t % 3 holds tile t's halo, t + 1's is in flight;
  // the stores of tile t - 1 go out first, then the loads of tile t + 2's
  // halo, then tile t's steps and epilogue into this wave's stage.
  auto run = [&](auto accum) {
    constexpr bool ACC = decltype(accum)::value;
    int prev_oy0 = -1, prev_ox0 = 0, buf = 0;
    while (mt < tiles_m) {
      if (prev_oy0 >= 0) store_tile(prev_oy0, prev_ox0);
      const int far = mt + 2 * per_n;
      const bool dma = far < tiles_m;  // uniform
      if (dma) load_halo(far, buf == 0 ? 2 : buf - 1);
      int oy0, ox0;
      origin(mt, oy0, ox0);
      const int oy = oy0 + wave, ox = ox0 + l32;
      const bool in_out = oy < a.OH && ox < a.OW;
      const long pix = (long)oy * a.OW + ox;

      // Old outputs (when accumulating): the lane's 4 channels of each group.
      u32x2 old[2][4];
      if constexpr (ACC) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const int n = tn * 64 + 32 * j + 8 * g + 4 * hf;
            old[j][g] = in_out && n < a.N ? *(const u32x2 *)(yh + pix * a.ys + n) : u32x2{0u, 0u};
          }
      }

      floatx16 acc[2];
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4v b4 = *(const float4v *)(bias_l + 32 * j + 8 * g + 4 * hf);
#pragma unroll
          for (int e = 0; e < 4; e++) acc[j][4 * g + e] = b4[e];
        }
      const unsigned char *hb = lds + buf * R::HALO + (wave * R::HC + l32) * 8;
#pragma unroll
      for (int s = 0; s < STEPS; s++) {
        const int o0 = hf ? tap_off<KS>(4 * s + 2) : tap_off<KS>(4 * s);
        const int o1 = hf ? tap_off<KS>(4 * s + 3) : tap_off<KS>(4 * s + 1);
        const u32x2 p0 = *(const u32x2 *)(hb + o0), p1 = *(const u32x2 *)(hb + o1);
        const u32x4 raw = {p0[0], p0[1], p1[0], p1[1]};
        half8 xb;
        __builtin_memcpy(&xb, &raw, 16);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wr[0][s], xb, acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wr[1][s], xb, acc[1], 0, 0, 0);
      }

      // C^T: lane pixel l32, register 4 g + e = channel 32 j + 8 g + 4 hf + e.
      __builtin_amdgcn_wave_barrier();  // tile t - 1's stage was read above
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int ch = 32 * j + 8 * g + 4 * hf;
          const float4v s4 = *(const float4v *)(slope_l + ch);
          uint16_t oh[4], h[4];
          if constexpr (ACC) __builtin_memcpy(oh, &old[j][g], 8);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float v = acc[j][4 * g + e];
            if constexpr (ACC) v += h2f(oh[e]);
            h[e] = f2h(act_c<ACT>(v, s4[e]));
          }
          u32x2 o;
          __builtin_memcpy(&o, h, 8);
          *(u32x2 *)(stage + (l32 * R::SPX + ch) * 2) = o;
        }
      __builtin_amdgcn_wave_barrier();
      prev_oy0 = oy0;
      prev_ox0 = ox0;
      mt += per_n;
      buf = buf == 2 ? 0 : buf + 1;
      // Tile t + 1's halo (loaded before this iteration's HL loads, which
      // may be in flight; stores in between could be counted in their
      // place, so without them wait for everything).
      if (dma)
        wait_vm<HL>();
      else
        wait_vm<0>();
      __syncthreads();  // ... of every wave; buffer t % 3 is free for tile t + 3
    }
    if (prev_oy0 >= 0) store_tile(prev_oy0, prev_ox0);
  };
  if (a.accumulate)
    run(std::true_type{});
  else
    run(std::false_type{});
}

template <int KS>
struct Few {
  static constexpr int P = KS / 2, C = 64;
  static constexpr int STEPS = KS * C / 16;   // K = (ky, channel)
  static constexpr int TW = 64 - 2 * P;       // outputs of a 64-column item
  static constexpr int WAVES = 4, RB = WAVES;  // output rows of an item, one a wave
  static constexpr int IR = RB + KS - 1;      // staged input rows
  static constexpr int PXB = C * 2 + 16;      // bytes a staged pixel (one pad chunk)
  static constexpr int IN = IR * 64 * PXB;    // staged input bytes
  static constexpr int ZP = 64 + 4;           // floats a staged Z row
  static constexpr int ABYTES = STEPS * 1024;
  static constexpr int ZBYTES = 32 * ZP * 4;
  static constexpr int LDS = IN + ABYTES + WAVES * ZBYTES + 64 * 4;  // + bias, slope
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int KS>
__global__ __launch_bounds__(256) void conv_few(ConvArgs a) {
  using R = Few<KS>;
  constexpr int STEPS = R::STEPS, P = R::P, C = R::C, ZP = R::ZP, PXB = R::PXB;
  __shared__ __attribute__((aligned(16))) unsigned char lds[R::LDS];
  unsigned char *in_l = lds, *a_l = lds + R::IN;
  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float *zs = (float *)(lds + R::IN + R::ABYTES) + wave * (32 * ZP);
  const int rows_used = a.N * KS;
  const bool reflect = a.pad_reflect != 0;

  // ---- prologue: the A operand of step s (W^T rows m = (n, kx), k = 16 s +
  // 8 h + i = (ky, channel)), kept in LDS, gathered from the packed
  // fragments: W[k'][n] for k' = (ky KS + kx) C + c sits in fragment
  // k' / 16, lane n + 32 ((k' % 16) / 8) ----
  for (int s = wave; s < STEPS; s += R::WAVES) {
    const int m = l32, n = m / KS, kx = m - n * KS;
    const int k0 = 16 * s + 8 * hf, ky = k0 / C, c0 = k0 - ky * C;
    const int kk = (ky * KS + kx) * C + c0;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < rows_used) v = *(const u32x4 *)(a.wp + (long)(kk >> 4) * 512 + (n + 32 * ((kk & 15) >> 3)) * 8);
    *(u32x4 *)(a_l + s * 1024 + lane * 16) = v;
  }

  float *bs = (float *)(lds + R::IN + R::ABYTES + R::WAVES * R::ZBYTES);  // bias, slope
  if (tid < a.N) {
    bs[tid] = a.bias[tid];
    bs[32 + tid] = a.act == IEN_ACT_PRELU ? a.slope[tid] : 0.0f;
  }

  // Items are (column tile, group of RB output rows), numbered down each
  // column tile; a workgroup takes a contiguous run of them.  The staged
  // input rows form a ring of IR rows in LDS (input row y0 - P + r of item
  // y0 sits in slot (y0 + r) % IR), so an item that continues the previous
  // one down its tile loads only its RB new rows.
  const int tiles_x = (a.OW + R::TW - 1) / R::TW, groups = (a.OH + R::RB - 1) / R::RB;
  const long items = (long)groups * tiles_x;
  const long per = (items + gridDim.x - 1) / gridDim.x;
  const long first = blockIdx.x * per, last = min(items, first + per);
  uint16_t *yh = (uint16_t *)a.y;
  float *yf = (float *)a.y;
  // Whole 128-byte pixels as 16-byte pieces (padding pixels read the zero
  // buffer), up to PER of them a thread, loaded into registers while the
  // previous item computes.
  constexpr int PER = R::IR * 64 * 8 / 256, NEW = R::RB * 64 * 8 / 256;
  static_assert(PER * 256 == R::IR * 64 * 8 && NEW * 256 == R::RB * 64 * 8, "whole pieces a thread");
  u32x4 pre[PER];
  auto load_item = [&](long item, bool full) {
    const int y0 = (int)(item % groups) * R::RB, x0 = (int)(item / groups) * R::TW;
    const int r0 = full ? 0 : KS - 1, n = full ? PER : NEW;
#pragma unroll
    for (int b = 0; b < PER; b++) {
      if (b < n) {
        const int e = tid + 256 * b, r = r0 + (e >> 9), j = (e >> 3) & 63, ch = e & 7;
        bool oky, okx;
        const int iy = pad_index(y0 - P + r, a.H, reflect, oky);
        const int ix = pad_index(x0 - P + j, a.W, reflect, okx);
        const uint16_t *src = oky && okx ? a.x + ((long)iy * a.W + ix) * a.xs + 8 * ch : a.zeros;
        pre[b] = *(const u32x4 *)src;
      }
    }
  };
  auto continues = [&](long item) { return item != first && item % groups != 0; };
  if (first < last) load_item(first, true);
  for (long item = first; item < last; item++) {  // uniform in the block
    const int y0 = (int)(item % groups) * R::RB, x0 = (int)(item / groups) * R::TW;
    {
      const bool full = !continues(item);
      const int r0 = full ? 0 : KS - 1, n = full ? PER : NEW;
#pragma unroll
      for (int b = 0; b < PER; b++) {
        if (b < n) {
          const int e = tid + 256 * b, r = r0 + (e >> 9), j = (e >> 3) & 63, ch = e & 7;
          *(u32x4 *)(in_l + (((y0 + r) % R::IR) * 64 + j) * PXB + 16 * ch) = pre[b];
        }
      }
    }
    __syncthreads();  // the rows (and, the first time, the A operand and bias) are in
    if (item + 1 < last) load_item(item + 1, !continues(item + 1));
    const int y = y0 + wave;
    floatx16 acc[2] = {};  // the two 32-column blocks: independent chains
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      const int k0 = 16 * s, ky = k0 / C, c0 = k0 - ky * C + 8 * hf;
      const half8 wa = *(const half8 *)(a_l + s * 1024 + lane * 16);
#pragma unroll
      for (int cb = 0; cb < 2; cb++) {
        const half8 xb = *(const half8 *)(in_l + (((y0 + wave + ky) % R::IR) * 64 + 32 * cb + l32) * PXB + c0 * 2);
        acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wa, xb, acc[cb], 0, 0, 0);
      }
    }
    // C: row 8 (r / 4) + 4 hf + r % 4 = (n, kx), column 32 cb + l32.
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        zs[(8 * (r >> 2) + 4 * hf + (r & 3)) * ZP + 32 * cb + l32] = acc[cb][r];
    __builtin_amdgcn_wave_barrier();
    const int x = x0 + lane;
    if (y < a.OH && lane < R::TW && x < a.OW) {
      const long pix = (long)y * a.OW + x;
      for (int n = 0; n < a.N; n++) {
        float v = bs[n];
#pragma unroll
        for (int kx = 0; kx < KS; kx++) v += zs[(n * KS + kx) * ZP + lane + kx];
        const long at = pix * a.ys + n;
        const float sl = bs[32 + n];
        if (a.out_f32) {
          if (a.accumulate) v += yf[at];
          yf[at] = activate(v, a.act, sl);
        } else {
          if (a.accumulate) v += h2f(yh[at]);
          yh[at] = f2h(activate(v, a.act, sl));
        }
      }
    }
    __syncthreads();  // every wave is done with the rows and its Z before the next item
  }
}

int cus_of(ien_ctx *ctx) { return ctx->cus > 0 ? ctx->cus : 256; }

template <int KS>
ien_status narrow_act(ien_ctx *ctx, const ConvArgs &a, dim3 grid) {
  switch (a.act) {
    case IEN_ACT_RELU:
      hipLaunchKernelGGL((conv_narrow<KS, IEN_ACT_RELU>), grid, dim3(512), 0, ctx->stream, a);
      break;
    case IEN_ACT_PRELU:
      hipLaunchKernelGGL((conv_narrow<KS, IEN_ACT_PRELU>), grid, dim3(512), 0, ctx->stream, a);
      break;
    case IEN_ACT_GELU:
      hipLaunchKernelGGL((conv_narrow<KS, IEN_ACT_GELU>), grid, dim3(512), 0, ctx->stream, a);
      break;
    case IEN_ACT_SIGMOID:
      hipLaunchKernelGGL((conv_narrow<KS, IEN_ACT_SIGMOID>), grid, dim3(512), 0, ctx->stream, a);
      break;
    default:
      hipLaunchKernelGGL((conv_narrow<KS, IEN_ACT_NONE>), grid, dim3(512), 0, ctx->stream, a);
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace

bool narrow_supported(const ConvArgs &a, int ks, int stride, int nchw, int noff, int rows_mode) {
  // The halo loads take 32-bit byte offsets: inputs below 2 GiB.
  return !nchw && !noff && !rows_mode && stride == 1 && a.C == 4 &&
         (long)a.H * a.W * a.xs * 2 <= 0x7fff0000L &&
         (ks == 3 || ks == 5 || ks == 7) && a.xs % 4 == 0 && ((uintptr_t)a.x & 7) == 0 &&
         a.p_begin == 0 && a.p_end == a.OH * a.OW && a.OH == a.H && a.OW == a.W &&
         !a.out_f32 && !a.out_nchw && a.N % 8 == 0 && a.ys % 8 == 0 &&
         ((uintptr_t)a.y & 15) == 0;
}

ien_status launch_narrow(ien_ctx *ctx, ConvArgs a, int ks) {
  const int tiles_m = ((a.OW + 31) / 32) * ((a.OH + 7) / 8);
  a.tiles_n = (a.N + 63) / 64;
  // One workgroup per CU at 7 x 7 (its weights fill the VGPRs), two at
  // 3 x 3 and 5 x 5.
  const int per_cu = ks == 7 ? 1 : 2;
  const int per_n = std::max(1, std::min(tiles_m, per_cu * cus_of(ctx) / a.tiles_n));
  const dim3 grid(per_n * a.tiles_n);
  if (ks == 3) return narrow_act<3>(ctx, a, grid);
  if (ks == 5) return narrow_act<5>(ctx, a, grid);
  return narrow_act<7>(ctx, a, grid);
}

bool few_supported(const ConvArgs &a, int ks, int stride, int nchw, int noff, int rows_mode) {
  return !nchw && !noff && !rows_mode && stride == 1 && a.C == 64 && (ks == 3 || ks == 7) &&
         a.N * ks <= 32 && a.xs % 8 == 0 && ((uintptr_t)a.x & 15) == 0 && a.p_begin == 0 &&
         a.p_end == a.OH * a.OW && a.OH == a.H && a.OW == a.W && !a.out_nchw;
}

ien_status launch_few(ien_ctx *ctx, ConvArgs a, int ks) {
  const int tw = ks == 3 ? Few<3>::TW : Few<7>::TW;
  // One workgroup a CU (its staged rows fill the LDS), each over a run of
  // `per` items of 4 output rows x tw columns; no workgroup's run is empty.
  const long items = (long)((a.OH + 3) / 4) * ((a.OW + tw - 1) / tw);
  const long per = (items + cus_of(ctx) - 1) / cus_of(ctx);
  const int blocks = (int)std::max(1L, (items + per - 1) / per);
  if (ks == 3) hipLaunchKernelGGL(conv_few<3>, dim3(blocks), dim3(256), 0, ctx->stream, a);
  else hipLaunchKernelGGL(conv_few<7>, dim3(blocks), dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien
