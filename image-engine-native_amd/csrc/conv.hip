// conv.hip -- convolution and dense products as implicit GEMM on gfx950
// f16 MFMA (v_mfma_f32_32x32x16_f16) with f32 accumulation.
//
// Replaces the reference's matrix product (crates/native-engine/src/gemm.rs
// multiply, every conv and linear layer of the CPU path) and its Vulkan
// shaders (realesrgan-native shaders/conv_*.comp, scunet-native
// shaders/conv3.comp and gemm*.comp, lama-native shaders/conv*.comp,
// birefnet-native shaders/gemm*.comp).
//
// Shape of the GEMM: M = output pixels (row-major), N = output channels,
// K = taps x input channels, taps outer and channels inner (gemm.rs:
// "the reduction runs over taps in order, channels within each").
//
// One workgroup = 4 wave64s computes a TR x TC tile of output pixels for
// BN = 32 * NBW * NSPLIT output channels.  Per chunk of CK input channels it
// stages in LDS
//   - the tile's input halo, ((TR-1) S + KS) x ((TC-1) S + KS) pixels,
//     NHWC with a padded pixel stride (CK + 8 halves, so the 32 lanes of an
//     A-fragment read -- 16 bytes each, 32 consecutive pixels -- hit
//     distinct banks), and
//   - the chunk's weights, already packed as MFMA B fragments,
// with every thread keeping 8 independent 16-byte loads in flight (a
// workgroup fills its CU's LDS, so one wave per SIMD has to hide its own
// latency).  Then it walks taps x 16-channel steps fully unrolled: the LDS
// offset of every fragment is a compile-time constant from one base
// address, fragments are double-buffered in registers, and each step issues
// MBW x NBW MFMAs.  The epilogue adds the bias and applies the activation in
// the accumulators (bias, old output when accumulating, activation: the
// order of gemm.rs:583-666), stages f32 results per wave in LDS and writes
// 16-byte vectors.
//
// Launches whose workgroups fill the CUs at most once (counting the
// double-buffered workgroups that fit a CU) keep two chunk buffers (DB):
// chunk i + 1 is loaded while chunk i is multiplied -- NHWC halo and
// fragments by buffer loads straight into LDS that the compiler does not
// see (waited for with vmcnt(loads per wave)), NCHW halo groups through
// registers written after the products.  No other workgroup would hide the
// load latency there.
//
// Block ids are remapped so that each XCD (blocks are dealt round-robin to
// the 8 XCDs) gets a contiguous band of tiles: neighbouring tiles share halo
// rows, which then stay in that XCD's L2.

#include "conv_common.h"
#include "lanes.h"

namespace ien {

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW,
          bool DB = false, int NBUF = 2>
struct ConvCfg {
  static constexpr int NSPLIT = 4 / MSPLIT;
  static constexpr int BN = 32 * NBW * NSPLIT;
  static constexpr int NBT = BN / 32;           // 32-channel blocks per tile
  static constexpr int MB = TR * TC / 32;       // M-blocks per tile
  static constexpr int MBW = MB / MSPLIT;       // M-blocks per wave
  static constexpr int EXT = KS == 0 ? 2 : KS;  // offset taps read one pixel on
  static constexpr int TMAX = KS == 0 ? 4 : KS * KS;
  static constexpr int HR = (TR - 1) * S + EXT;
  static constexpr int HC = (TC - 1) * S + EXT;
  // NHWC 16-channel inputs are staged by direct-to-LDS loads into an
  // unpadded halo whose 16-byte chunks are XOR-swizzled per pixel (SWZ);
  // the other layouts are written through registers into a halo whose
  // pixel stride is padded by 8 halves.  Either way the 32 lanes of an
  // A-fragment read hit distinct banks.
  static constexpr bool DMA = VEC && !IN_NCHW;
  static constexpr int CKP = DMA ? CK : (VEC ? CK + 8 : CK);  // halves per halo pixel
  static constexpr int PB = CK * 2;                           // bytes per DMA halo pixel
  static constexpr int NCH = PB / 16;                         // 16-byte chunks per pixel
  static constexpr int RPB = PB >= 256 ? 1 : 256 / PB;        // pixels per 256-byte bank row
  // Double-buffered chunks (DB): whole rounds of the 4 waves' 1 KiB loads.
  static constexpr int HALO_ROUND = DB ? 4096 : 1024;
  static constexpr int HALO_BYTES =
      DMA ? (HR * HC * PB + HALO_ROUND - 1) / HALO_ROUND * HALO_ROUND : HR * HC * CKP * 2;
  // 16-deep k steps of one chunk: VEC walks taps x CK/16; otherwise K is
  // flattened over (tap, channel) and rounded up to 16.
  static constexpr int KSTEPS = VEC ? TMAX * (CK / 16) : (TMAX * CK + 15) / 16;
  static constexpr int BFRAGS = DB ? (NBT * KSTEPS + 3) / 4 * 4 : NBT * KSTEPS;
  static constexpr int B_BYTES = BFRAGS * 1024;  // B fragments of the chunk
  // Epilogue staging per wave: NHWC [px][NBW*32 + 8] or NCHW [NBW*32][px + 4] floats.
  static constexpr int STAGE_NHWC = MBW * 32 * (NBW * 32 + 8);
  static constexpr int STAGE_NCHW = NBW * 32 * (MBW * 32 + 4);
  static constexpr int STAGE = STAGE_NHWC > STAGE_NCHW ? STAGE_NHWC : STAGE_NCHW;
  static constexpr int MAIN_BYTES = HALO_BYTES + B_BYTES;
  static constexpr int BUFS = DB ? NBUF : 1;
  static constexpr int LDS_BYTES =
      BUFS * MAIN_BYTES > 4 * STAGE * 4 ? BUFS * MAIN_BYTES : 4 * STAGE * 4;
  // Direct-to-LDS loads per wave and chunk (DB): the halo's KiBs (NHWC)
  // and the fragments.
  static constexpr int DW = DB ? (DMA ? HALO_BYTES / 4096 : 0) + BFRAGS / 4 : 0;
  // NCHW (DB): 16-byte groups of 8 pixels of one channel row a chunk's halo
  // spans, and per thread.
  static constexpr int NGROUPS = CK * HR * ((HC + 14) / 8);
  static constexpr int NITEMS = (NGROUPS + 255) / 256;
  // (Double buffering takes 16-channel steps: NHWC through direct-to-LDS
  // loads, NCHW through registers.)
  static constexpr bool FITS = (!DB || VEC) && (NBUF == 2 || DMA) && LDS_BYTES <= 160 * 1024 &&
                               (NBUF - 1) * DW < 64;
  static_assert(MB % MSPLIT == 0, "M-blocks must split evenly over waves");
  static_assert(TC % 32 == 0, "tile columns are whole M-blocks");
  static_assert(!VEC || CK % 16 == 0, "16-channel steps");
  static_assert(HALO_BYTES % 16 == 0, "B fragments start 16-byte aligned");
  static_assert(DB || LDS_BYTES <= 160 * 1024, "LDS budget");
};

// Offset tap t (< 4; offsets of 0 or 1 pixel, as launch_conv checks) from
// bit masks built with constant indices: indexing the argument arrays at
// run time (or selects the compiler turns back into such indexing) copies
// the whole argument block to scratch memory.
__device__ __forceinline__ void offset_tap(const ConvArgs &a, int t, int &dy, int &dx) {
  const int ybits = a.offy[0] | a.offy[1] << 1 | a.offy[2] << 2 | a.offy[3] << 3;
  const int xbits = a.offx[0] | a.offx[1] << 1 | a.offx[2] << 2 | a.offx[3] << 3;
  dy = (ybits >> t) & 1;
  dx = (xbits >> t) & 1;
}

// Swizzled chunk slot of 16-byte chunk c of DMA halo pixel p.
template <class Cfg>
__device__ __forceinline__ int swz_slot(int p, int c) {
  return c ^ ((p / Cfg::RPB) & (Cfg::NCH - 1));
}

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW,
          bool DB = false, int NBUF = 2>
__global__ __launch_bounds__(256) void conv_mfma(ConvArgs a) {
  using Cfg = ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, DB, NBUF>;
  constexpr int HR = Cfg::HR, HC = Cfg::HC, CKP = Cfg::CKP, MBW = Cfg::MBW, NBT = Cfg::NBT;
  constexpr int KSTEPS = Cfg::KSTEPS;
  constexpr int P = KS == 0 ? 0 : KS / 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[Cfg::LDS_BYTES];
  uint16_t *halo = (uint16_t *)lds_raw;
  uint16_t *bl = (uint16_t *)(lds_raw + Cfg::HALO_BYTES);

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tpix = a.tiles_x * a.tiles_y;
  const int tn = a.n_major ? bid / tpix : bid % a.tiles_n;
  const int t = a.n_major ? bid % tpix : bid / a.tiles_n;
  const int tx = t % a.tiles_x;
  const int ty = t / a.tiles_x + a.ty_begin;
  const int oy0 = ty * TR, ox0 = tx * TC;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int mg = wave % MSPLIT, ng = wave / MSPLIT;
  const int nblk_tile = tn * NBT;          // first 32-channel block of the tile
  const int nblk0 = nblk_tile + ng * NBW;  // first 32-channel block of this wave
  const int T = KS == 0 ? a.noff : KS * KS;

  // Bias and PReLU slope of this lane's accumulator column, per N-block:
  // loaded now, used after the products.
  float bias_r[NBW], slope_r[NBW];
  const bool raw_split = a.ksplit > 1 && !a.part;  // raw sums for a finishing pass
  if (raw_split) a.y = (float *)a.y + (long)blockIdx.y * (a.p_end - a.p_begin) * a.ys;
#pragma unroll
  for (int j = 0; j < NBW; j++) {
    const int n = (nblk0 + j) * 32 + (lane & 31);  // < NB * 32: the bias is padded
    bias_r[j] = raw_split ? 0.0f : a.bias[n];
    slope_r[j] = a.act == IEN_ACT_PRELU ? a.slope[min(n, a.N - 1)] : 0.0f;
  }

  floatx16 acc[MBW][NBW];
#pragma unroll
  for (int i = 0; i < MBW; i++)
#pragma unroll
    for (int j = 0; j < NBW; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  // Halo origin in input pixels.
  const int iy0 = oy0 * S - P, ix0 = ox0 * S - P;

  // Offset of input pixel (iy, ix), or -1 for a zero (padding, outside).
  auto resolve = [&](int iy, int ix) -> int {
    if (a.rows_mode) {
      const int r = iy * a.W + ix;
      if (iy < 0 || ix < 0 || ix >= a.W || r >= a.M) return -1;
      return r * a.xs;
    }
    if (iy < 0 || iy >= a.H || ix < 0 || ix >= a.W) {
      if (!a.pad_reflect || KS == 0) return -1;
      // Clamped as well: halo pixels that feed no stored output may lie
      // further out than one reflection reaches, and must stay in bounds.
      iy = min(max(reflect_idx(iy, a.H), 0), a.H - 1);
      ix = min(max(reflect_idx(ix, a.W), 0), a.W - 1);
    }
    const int p = iy * a.W + ix;
    return IN_NCHW ? p : p * a.xs;
  };

  // This wave's A-fragment base per M-block: halo pixel of tap (0, 0) for
  // the lane's pixel, plus the lane's 8-channel half of a 16-channel step.
  int abase[MBW], apix[MBW];
#pragma unroll
  for (int i = 0; i < MBW; i++) {
    const int mb = mg * MBW + i;
    const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (lane & 31);
    apix[i] = (r * S) * HC + cx * S;
    abase[i] = apix[i] * CKP + (VEC ? 8 * (lane >> 5) : 0);
  }

  const int c_begin = (int)blockIdx.y * a.kchunks * CK;
  const int c_end = min(a.C, c_begin + a.kchunks * CK);
  // The products of one staged channel chunk (its halo and B fragments at
  // `base`; cc channels).
  auto compute = [&](const unsigned char *base, int cc) {
    const uint16_t *halo = (const uint16_t *)base;
    const uint16_t *bw =
        (const uint16_t *)(base + Cfg::HALO_BYTES) + ng * NBW * KSTEPS * 512 + lane * 8;
    auto mma = [&](const half8 *av, const half8 *bv) {
#pragma unroll
      for (int i = 0; i < MBW; i++)
#pragma unroll
        for (int j = 0; j < NBW; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
    };
    if constexpr (VEC && KS > 0) {
      // ---- taps x 16-channel steps, unrolled: constant LDS offsets ----
      auto frag = [&](int s, half8 *av, half8 *bv) {
        const int tap = s / (CK / 16), kc = s % (CK / 16);
        const int dy = tap / KS, dx = tap % KS;
        if constexpr (Cfg::DMA) {
          const int c = 2 * kc + (lane >> 5);
#pragma unroll
          for (int i = 0; i < MBW; i++) {
            const int p = apix[i] + dy * HC + dx;
            av[i] = *(const half8 *)(base + p * Cfg::PB + 16 * swz_slot<Cfg>(p, c));
          }
        } else {
          const int off = (dy * HC + dx) * CKP + kc * 16;
#pragma unroll
          for (int i = 0; i < MBW; i++) av[i] = *(const half8 *)(halo + abase[i] + off);
        }
#pragma unroll
        for (int j = 0; j < NBW; j++) bv[j] = *(const half8 *)(bw + (j * KSTEPS + s) * 512);
      };
      // The scheduler barriers keep step s+1's fragment reads ahead of
      // step s's MFMAs; left alone, the compiler sinks each read next to
      // its use and every MFMA pair then waits out an LDS round trip.
      half8 av[2][MBW], bv[2][NBW];
      frag(0, av[0], bv[0]);
#pragma unroll
      for (int s = 0; s < KSTEPS; s++) {
        if (s + 1 < KSTEPS) frag(s + 1, av[(s + 1) & 1], bv[(s + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        mma(av[s & 1], bv[s & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (VEC) {
      // Offset taps (transposed-conv phases): at most 4, known at run time.
      const int steps = T * (CK / 16);
      for (int s = 0; s < steps; s++) {
        const int tap = s / (CK / 16), kc = s % (CK / 16);
        half8 av[MBW], bv[NBW];
        const int c = 2 * kc + (lane >> 5);
#pragma unroll
        for (int i = 0; i < MBW; i++) {
          int ody, odx;
          offset_tap(a, tap, ody, odx);
          const int p = apix[i] + ody * HC + odx;
          av[i] = *(const half8 *)(base + p * Cfg::PB + 16 * swz_slot<Cfg>(p, c));
        }
#pragma unroll
        for (int j = 0; j < NBW; j++) bv[j] = *(const half8 *)(bw + (j * KSTEPS + s) * 512);
        mma(av, bv);
      }
    } else {
      // Few channels (one chunk holds them all): K flattened over
      // (tap, channel) as the reference orders it, 16 at a time.
      const int K = T * cc;
      const int kbs = (K + 15) / 16;
      for (int kb = 0; kb < kbs; kb++) {
        half8 av[MBW], bv[NBW];
#pragma unroll
        for (int j = 0; j < NBW; j++) bv[j] = *(const half8 *)(bw + (j * KSTEPS + kb) * 512);
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const int k = kb * 16 + 8 * (lane >> 5) + q;
          const int kk = k < K ? k : 0;
          const int tap = kk / cc, c = kk - tap * cc;
          int dy, dx;
          if constexpr (KS == 0) {
            offset_tap(a, tap, dy, dx);
          } else {
            dy = tap / KS;
            dx = tap - dy * KS;
          }
          const int off = (dy * HC + dx) * CKP + c;
#pragma unroll
          for (int i = 0; i < MBW; i++) {
            uint16_t hv = k < K ? halo[abase[i] + off] : (uint16_t)0;
            _Float16 f;
            __builtin_memcpy(&f, &hv, 2);
            av[i][q] = f;
          }
        }
        mma(av, bv);
      }
    }
  };

  if constexpr (DB && !Cfg::DMA) {
    // Double-buffered NCHW chunks (zero padding, rows of whole 16-byte
    // groups): chunk i + 1's halo groups are loaded into registers and its
    // fragments straight into the other LDS buffer while chunk i is
    // multiplied; the groups are written (transposed to pixel-major) after
    // the products, then one barrier.
    constexpr int OOB = 0x7ffffff0;
    const int4v wrs = uniform_rsrc(a.wp, (long)a.NB * a.KB * 1024);
    const unsigned lds0 = lds_addr(lds_raw);
    auto floor8 = [](int v) { return v >= 0 ? v / 8 : -((7 - v) / 8); };
    const int g0 = floor8(ix0);
    const int groups = floor8(ix0 + HC - 1) + 1 - g0;
    const int items = CK * HR * groups;  // <= Cfg::NGROUPS
    auto where = [&](int e, int &hy, int &c, int &gx) {
      const int g = e % groups, rest = e / groups;
      hy = rest % HR;
      c = rest / HR;
      gx = (g0 + g) * 8;
      const int iy = iy0 + hy;
      return e < items && iy >= 0 && iy < a.H && gx >= 0 && gx < a.W;
    };
    u32x4 hv[Cfg::NITEMS];
    auto load_groups = [&](int c0) {
#pragma unroll
      for (int j = 0; j < Cfg::NITEMS; j++) {
        int hy, c, gx;
        const bool ok = where(tid + 256 * j, hy, c, gx);
        hv[j] = *(const u32x4 *)(a.x + (ok ? (c0 + c) * a.xs + (iy0 + hy) * a.W + gx : 0));
      }
    };
    auto store_groups = [&](unsigned char *base) {
      uint16_t *hl = (uint16_t *)base;
#pragma unroll
      for (int j = 0; j < Cfg::NITEMS; j++) {
        const int e = tid + 256 * j;
        if (e >= items) break;
        int hy, c, gx;
        const bool ok = where(e, hy, c, gx);
        uint16_t v8[8];
        const u32x4 val = ok ? hv[j] : u32x4{0u, 0u, 0u, 0u};
        __builtin_memcpy(v8, &val, 16);
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const int hx = gx + q - ix0;
          if (hx >= 0 && hx < HC) hl[(hy * HC + hx) * CKP + c] = v8[q];
        }
      }
    };
    auto issue_weights = [&](int c0, int buf) {
      const unsigned bb = lds0 + buf * Cfg::MAIN_BYTES + Cfg::HALO_BYTES;
#pragma unroll
      for (int fi = 0; fi < Cfg::BFRAGS / 4; fi++) {
        const int f = wave + 4 * fi;
        const int jn = f / KSTEPS, st = f - jn * KSTEPS;
        int off = OOB;
        if (jn < NBT) {
          const int tap = st / (CK / 16), kc = st % (CK / 16);
          const int kb = tap * (a.C / 16) + c0 / 16 + kc;
          off = (((nblk_tile + jn) * a.KB + kb) * 512 + lane * 8) * 2;
        }
        dma_lds(wrs, __builtin_amdgcn_readfirstlane(bb + f * 1024), off);
      }
    };
    if (c_begin < c_end) {
      load_groups(c_begin);
      issue_weights(c_begin, 0);
      store_groups(lds_raw);
      wait_vm<0>();
      __syncthreads();
    }
    int i = 0;
    for (int c0 = c_begin; c0 < c_end; c0 += CK, i++) {
      const bool next = c0 + CK < c_end;  // uniform
      if (next) {
        load_groups(c0 + CK);
        issue_weights(c0 + CK, (i + 1) & 1);
      }
      compute(lds_raw + (i & 1) * Cfg::MAIN_BYTES, CK);
      if (next) store_groups(lds_raw + ((i + 1) & 1) * Cfg::MAIN_BYTES);
      wait_vm<0>();     // chunk i + 1's fragments
      __syncthreads();  // chunk i + 1 is in; every wave is done with buffer i % 2
    }
  } else if constexpr (DB) {
    // Double-buffered chunks: chunk i + 1's halo and fragments are loaded
    // (straight into the other LDS buffer, by loads the compiler does not
    // see) while chunk i is multiplied; a wait for the chunk's own loads
    // (all but the DW loads issued after them) and one barrier on each side.
    // The buffer range checks give the zero padding.
    constexpr int OOB = 0x7ffffff0;
    const long in_halves = a.rows_mode ? (long)a.M * a.xs : (long)a.H * a.W * a.xs;
    const int4v xr = uniform_rsrc(a.x, in_halves * 2);
    const int4v wrs = uniform_rsrc(a.wp, (long)a.NB * a.KB * 1024);
    const unsigned lds0 = lds_addr(lds_raw);
    const int steps = T * (CK / 16);
    auto issue = [&](int c0, int buf) {
      const unsigned bb = lds0 + buf * Cfg::MAIN_BYTES;
#pragma unroll
      for (int gi = 0; gi < Cfg::HALO_BYTES / 4096; gi++) {
        const int g = wave + 4 * gi;
        const int byte = g * 1024 + lane * 16;
        const int hp = byte / Cfg::PB, slot = (byte % Cfg::PB) / 16;
        int off = OOB;
        if (hp < HR * HC) {
          const int hy = hp / HC, hx = hp - hy * HC;
          const int o = resolve(iy0 + hy, ix0 + hx);
          if (o >= 0) off = (o + c0 + 8 * swz_slot<Cfg>(hp, slot)) * 2;
        }
        dma_lds(xr, __builtin_amdgcn_readfirstlane(bb + g * 1024), off);
      }
#pragma unroll
      for (int fi = 0; fi < Cfg::BFRAGS / 4; fi++) {
        const int f = wave + 4 * fi;
        const int jn = f / KSTEPS, st = f - jn * KSTEPS;
        int off = OOB;
        if (jn < NBT && st < steps) {
          const int tap = st / (CK / 16), kc = st % (CK / 16);
          const int kb = tap * (a.C / 16) + c0 / 16 + kc;
          off = (((nblk_tile + jn) * a.KB + kb) * 512 + lane * 8) * 2;
        }
        dma_lds(wrs, __builtin_amdgcn_readfirstlane(bb + Cfg::HALO_BYTES + f * 1024), off);
      }
    };
    // NBUF buffers: NBUF - 1 chunks in flight while one is multiplied.
    const int nchunks = (c_end - c_begin + CK - 1) / CK;
#pragma unroll
    for (int q = 0; q < NBUF - 1; q++)
      if (q < nchunks) issue(c_begin + q * CK, q);
    for (int i = 0; i < nchunks; i++) {
      if (i + NBUF - 1 < nchunks) issue(c_begin + (i + NBUF - 1) * CK, (i + NBUF - 1) % NBUF);
      // Loads complete in order: chunk i is in once at most the later
      // chunks' loads are outstanding.
      const int ahead = min(NBUF - 1, nchunks - 1 - i);  // uniform
      if (NBUF > 2 && ahead >= 2)
        wait_vm<(NBUF > 2 ? 2 * Cfg::DW : 0)>();
      else if (ahead == 1)
        wait_vm<Cfg::DW>();
      else
        wait_vm<0>();
      __syncthreads();  // chunk i is in every wave's view
      compute(lds_raw + (i % NBUF) * Cfg::MAIN_BYTES, CK);
      __syncthreads();  // every wave is done with buffer i % NBUF before chunk i + NBUF fills it
    }
  } else {
    for (int c0 = c_begin; c0 < c_end; c0 += CK) {
      const int cc = min(CK, a.C - c0);  // == CK when VEC
      __syncthreads();
      // ---- global -> LDS: the halo of this channel chunk ----
      if constexpr (Cfg::DMA) {
        // One KiB per wave instruction: lane l fills byte 16 l of it, which
        // is chunk slot s of halo pixel p, holding input chunk
        // s ^ swizzle(p); padding pixels read the zero page.
        constexpr int G = Cfg::HALO_BYTES / 1024;
        for (int g = wave; g < G; g += 4) {
          const int byte = g * 1024 + lane * 16;
          const int hp = byte / Cfg::PB, slot = (byte % Cfg::PB) / 16;
          const uint16_t *src = a.zeros;
          if (hp < HR * HC) {
            const int hy = hp / HC, hx = hp - hy * HC;
            const int off = resolve(iy0 + hy, ix0 + hx);
            if (off >= 0) src = a.x + off + c0 + 8 * swz_slot<Cfg>(hp, slot);
          }
          dma16(src, lds_raw + g * 1024);
        }
      } else if constexpr (!IN_NCHW) {
        // Few channels: one half per element.
        auto where = [&](int e, int &hp, int &c) {
          hp = e / cc;
          c = e - hp * cc;
          const int hy = hp / HC, hx = hp - hy * HC;
          return resolve(iy0 + hy, ix0 + hx);
        };
        staged_copy<8>(
            HR * HC * cc, tid,
            [&](int e) -> u32x4 {
              int hp, c;
              const int off = where(e, hp, c);
              return u32x4{(uint32_t)a.x[(off >= 0 ? off : 0) + c0 + c], 0u, 0u, 0u};
            },
            [&](int e, u32x4 val) {
              int hp, c;
              const int off = where(e, hp, c);
              halo[hp * CKP + c] = off >= 0 ? (uint16_t)val[0] : (uint16_t)0;
            });
      } else {
        // NCHW.  Fast path (rows of whole 16-byte groups, zero padding): 8
        // neighbouring pixels of one channel row per load; a group lies wholly
        // inside or wholly outside the image.  Otherwise one half per element.
        const bool fast = !a.rows_mode && !a.pad_reflect && (a.W & 7) == 0 && (a.xs & 7) == 0 &&
                          (((uintptr_t)a.x) & 15) == 0;
        if (fast) {
          auto floor8 = [](int v) { return v >= 0 ? v / 8 : -((7 - v) / 8); };
          const int g0 = floor8(ix0);
          const int groups = floor8(ix0 + HC - 1) + 1 - g0;
          auto where = [&](int e, int &hy, int &c, int &gx) {
            const int g = e % groups, rest = e / groups;
            hy = rest % HR;
            c = rest / HR;
            gx = (g0 + g) * 8;
            const int iy = iy0 + hy;
            return iy >= 0 && iy < a.H && gx >= 0 && gx < a.W;
          };
          staged_copy<8>(
              cc * HR * groups, tid,
              [&](int e) -> u32x4 {
                int hy, c, gx;
                const bool ok = where(e, hy, c, gx);
                const int off = ok ? (c0 + c) * a.xs + (iy0 + hy) * a.W + gx : 0;
                return *(const u32x4 *)(a.x + off);
              },
              [&](int e, u32x4 val) {
                int hy, c, gx;
                if (!where(e, hy, c, gx)) val = u32x4{0u, 0u, 0u, 0u};
                uint16_t v8[8];
                __builtin_memcpy(v8, &val, 16);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                  const int hx = gx + q - ix0;
                  if (hx >= 0 && hx < HC) halo[(hy * HC + hx) * CKP + c] = v8[q];
                }
              });
        } else {
          auto where = [&](int e, int &hp, int &c) {
            c = e / (HR * HC);
            hp = e - c * (HR * HC);
            const int hy = hp / HC, hx = hp - hy * HC;
            return resolve(iy0 + hy, ix0 + hx);
          };
          staged_copy<8>(
              cc * HR * HC, tid,
              [&](int e) -> u32x4 {
                int hp, c;
                const int off = where(e, hp, c);
                return u32x4{(uint32_t)a.x[(c0 + c) * a.xs + (off >= 0 ? off : 0)], 0u, 0u, 0u};
              },
              [&](int e, u32x4 val) {
                int hp, c;
                const int off = where(e, hp, c);
                halo[hp * CKP + c] = off >= 0 ? (uint16_t)val[0] : (uint16_t)0;
              });
        }
      }

      // ---- global -> LDS: this chunk's weight fragments, [block][step], ----
      // one KiB fragment per wave instruction.
      {
        const int steps = VEC ? T * (CK / 16) : (T * cc + 15) / 16;
        for (int f = wave; f < NBT * steps; f += 4) {
          const int jn = f / steps, s = f - jn * steps;
          int kb = s;  // one chunk holds all channels: fragments in order
          if (VEC) {
            const int tap = s / (CK / 16), kc = s % (CK / 16);
            kb = tap * (a.C / 16) + c0 / 16 + kc;
          }
          dma16(a.wp + ((nblk_tile + jn) * a.KB + kb) * 512 + lane * 8,
                bl + (jn * KSTEPS + s) * 512);
        }
      }
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the direct-to-LDS loads have landed
      __syncthreads();

      compute(lds_raw, cc);
    }
  }

  // ---- split-K counted in per tile: this split's sums go out (16 bytes a
  // lane per accumulator quarter, in register order, at device scope so
  // that a split on another XCD reads them from memory), then the tile's
  // counter; the split that brings it to ksplit returns it to zero, adds
  // the tile's sums in split order and carries on with the epilogue ----
  if (a.ksplit > 1 && a.part) {
    int *last = (int *)lds_raw;  // (written after the barrier below: every wave is past its products)
    constexpr int G = MBW * NBW * 4;  // 16-byte groups a thread
    constexpr int SC1 = 16;           // cache policy bits of a device-scope access
    const int z = blockIdx.y;
    const long first = (long)blockIdx.x * a.ksplit;  // the tile's first split block
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        a.part, (short)0, (int)((long)gridDim.x * a.ksplit * G * 4096), 0x00020000);
    auto at = [&](int s, int g) { return (int)((((first + s) * G + g) * 256 + tid) * 16); };
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int j = 0; j < NBW; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4v v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                             acc[i][j][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(*(const u32x4 *)&v, pr, at(z, (i * NBW + j) * 4 + q),
                                                 0, SC1);
        }
    wait_vm<0>();  // this thread's sums are out
    __syncthreads();
    if (tid == 0) {
      const int done =
          __hip_atomic_fetch_add(a.tile_count + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = done == a.ksplit - 1;
      if (*last) __hip_atomic_store(a.tile_count + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last) return;
    // The sums in split order, this split's own read back too (the order,
    // and so the result, must not depend on which split came last).
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int j = 0; j < NBW; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    for (int s = 0; s < a.ksplit; s++) {
#pragma unroll
      for (int i = 0; i < MBW; i++)
#pragma unroll
        for (int j = 0; j < NBW; j++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const u32x4 raw =
                __builtin_amdgcn_raw_buffer_load_b128(pr, at(s, (i * NBW + j) * 4 + q), 0, SC1);
            const float4v v = *(const float4v *)&raw;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][j][4 * q + e] += v[e];
          }
    }
  }

  // ---- epilogue -----------------------------------------------------------
  // Bias (and, when not accumulating, the activation) in the accumulators;
  // then a per-wave f32 staging in LDS and 8 outputs per lane per store.
  __syncthreads();  // every wave is done with the halo and the weights
  float *stage = (float *)lds_raw + wave * Cfg::STAGE;
  auto finish = [&](auto f) {
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int j = 0; j < NBW; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = f(acc[i][j][r] + bias_r[j], slope_r[j]);
  };
  // One loop per activation (uniform per launch), not a switch per value.
  const int act_now = a.accumulate ? IEN_ACT_NONE : a.act;
  if (act_now == IEN_ACT_RELU)
    finish([](float v, float) { return v > 0.0f ? v : 0.0f; });
  else if (act_now == IEN_ACT_PRELU)
    finish([](float v, float sl) { return v < 0.0f ? v * sl : v; });
  else if (act_now == IEN_ACT_GELU)
    finish([](float v, float) { return gelu_f(v); });
  else if (act_now == IEN_ACT_SIGMOID)
    finish([](float v, float) { return sigmoid_f(v); });
  else
    finish([](float v, float) { return v; });
  // C fragment: lane holds column n = lane % 32 and rows
  // 8 (r / 4) + 4 (lane / 32) + r % 4 of each 32 x 32 block.
  if (!a.out_nchw) {
    constexpr int SP = NBW * 32 + 8;  // floats per staged pixel
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int j = 0; j < NBW; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int m = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          stage[(i * 32 + m) * SP + j * 32 + (lane & 31)] = acc[i][j][r];
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_wave_barrier();
    constexpr int GROUPS = NBW * 4;  // 8-channel groups per staged pixel
    constexpr int ITEMS = MBW * 32 * GROUPS / 64;  // per lane
    // Item t of this lane: its output offset, or -1 outside the output.
    auto item_at = [&](int t, int &g) -> long {
      const int item = lane + 64 * t;
      const int q = item / GROUPS;
      g = item % GROUPS;
      const int mb = mg * MBW + q / 32;
      const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (q & 31);
      const int oy = oy0 + r, ox = ox0 + cx;
      const int p = oy * a.OW + ox;
      const int n = nblk0 * 32 + 8 * g;
      if (oy >= a.OH || ox >= a.OW || p < a.p_begin || p >= a.p_end || n >= a.N) return -1;
      if (a.phase) {
        const int q = a.phase - 1;
        return ((long)(2 * oy + (q >> 1)) * (2 * a.OW) + 2 * ox + (q & 1)) * a.ys + n;
      }
      return (long)(p - a.p_begin) * a.ys + n;
    };
    // f16 outputs in whole 16-byte groups: the old values (when
    // accumulating) are all loaded first, unconditionally, so one memory
    // latency covers them; then one loop per activation (picked once).
    const bool groups16 = !a.out_f32 && (a.ys & 7) == 0 && (a.N & 7) == 0 &&
                          (((uintptr_t)a.y) & 15) == 0;
    if (groups16) {
      uint16_t *yh = (uint16_t *)a.y;
      u32x4 old[ITEMS], add[ITEMS];
      if (a.accumulate) {
#pragma unroll
        for (int t = 0; t < ITEMS; t++) {
          int g;
          const long at = item_at(t, g);
          old[t] = *(const u32x4 *)(yh + (at >= 0 ? at : 0));
        }
      }
      if (a.add2) {
#pragma unroll
        for (int t = 0; t < ITEMS; t++) {
          int g;
          const long at = item_at(t, g);
          add[t] = *(const u32x4 *)(a.add2 + (at >= 0 ? at : 0));
        }
      }
      auto store = [&](auto actf) {
#pragma unroll
        for (int t = 0; t < ITEMS; t++) {
          int g;
          const long at = item_at(t, g);
          if (at < 0) continue;
          const int q = (lane + 64 * t) / GROUPS;
          const float4v s0 = *(const float4v *)(stage + q * SP + 8 * g);
          const float4v s1 = *(const float4v *)(stage + q * SP + 8 * g + 4);
          float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
          uint16_t o[8];
          if (a.accumulate) {
            uint16_t oh[8];
            __builtin_memcpy(oh, &old[t], 16);
            const int n = nblk0 * 32 + 8 * g;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = f2h(actf(v[e] + h2f(oh[e]), n + e));
          } else {
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = f2h(v[e]);  // activated in the accumulators
          }
          if (a.add2) {
            uint16_t ah[8];
            __builtin_memcpy(ah, &add[t], 16);
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = f2h(h2f(o[e]) + h2f(ah[e]));
          }
          u32x4 ov;
          __builtin_memcpy(&ov, o, 16);
          *(u32x4 *)(yh + at) = ov;
        }
      };
      const int act = a.accumulate ? a.act : IEN_ACT_NONE;
      if (act == IEN_ACT_RELU)
        store([](float v, int) { return v > 0.0f ? v : 0.0f; });
      else if (act == IEN_ACT_GELU)
        store([](float v, int) { return gelu_f(v); });
      else if (act == IEN_ACT_SIGMOID)
        store([](float v, int) { return sigmoid_f(v); });
      else if (act == IEN_ACT_PRELU) {
        const float *sl = a.slope;
        store([sl](float v, int n) { return v < 0.0f ? v * sl[n] : v; });
      } else {
        store([](float v, int) { return v; });
      }
      return;
    }
    for (int item = lane; item < MBW * 32 * GROUPS; item += 64) {
      const int q = item / GROUPS, g = item % GROUPS;
      const int mb = mg * MBW + q / 32;
      const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (q & 31);
      const int oy = oy0 + r, ox = ox0 + cx;
      const int p = oy * a.OW + ox;
      const int n = nblk0 * 32 + 8 * g;
      if (oy >= a.OH || ox >= a.OW || p < a.p_begin || p >= a.p_end || n >= a.N) continue;
      const float4v s0 = *(const float4v *)(stage + q * SP + 8 * g);
      const float4v s1 = *(const float4v *)(stage + q * SP + 8 * g + 4);
      float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      const int nv = min(8, a.N - n);
      const long base = (long)(p - a.p_begin) * a.ys + n;
      if (a.out_f32) {
        float *yo = (float *)a.y + base;
        if (nv == 8 && !a.accumulate && (((uintptr_t)yo) & 15) == 0) {
          // Two 16-byte stores (split-K partial sums take this path).
          *(float4v *)yo = float4v{v[0], v[1], v[2], v[3]};
          *(float4v *)(yo + 4) = float4v{v[4], v[5], v[6], v[7]};
          continue;
        }
        for (int e = 0; e < nv; e++) {
          float o = v[e];
          if (a.accumulate)
            o = activate(o + yo[e], a.act, a.act == IEN_ACT_PRELU ? a.slope[n + e] : 0.0f);
          yo[e] = o;
        }
      } else {
        uint16_t *yo = (uint16_t *)a.y + base;
        const bool vec = nv == 8 && (((uintptr_t)yo & 15) == 0);
        if (a.accumulate) {
          uint16_t old[8];
          if (vec) {
            u32x4 ov = *(const u32x4 *)yo;
            __builtin_memcpy(old, &ov, 16);
          } else {
            for (int e = 0; e < nv; e++) old[e] = yo[e];
          }
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const int ne = min(n + e, a.N - 1);
            v[e] = activate(v[e] + (e < nv ? h2f(old[e]) : 0.0f), a.act,
                            a.act == IEN_ACT_PRELU ? a.slope[ne] : 0.0f);
          }
        }
        uint16_t outv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) outv[e] = f2h(v[e]);
        if (vec) {
          u32x4 ov;
          __builtin_memcpy(&ov, outv, 16);
          *(u32x4 *)yo = ov;
        } else {
          for (int e = 0; e < nv; e++) yo[e] = outv[e];
        }
      }
    }
  } else {
    constexpr int PXS = MBW * 32 + 4;  // floats per staged channel row
#pragma unroll
    for (int i = 0; i < MBW; i++)
#pragma unroll
      for (int j = 0; j < NBW; j++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
          const int m = 8 * r4 + 4 * (lane >> 5);
          float4v v4 = {acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2],
                        acc[i][j][4 * r4 + 3]};
          *(float4v *)(stage + (j * 32 + (lane & 31)) * PXS + i * 32 + m) = v4;
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // 8 consecutive pixels of one channel per item: a 16-byte store where
    // they share an output row.
    constexpr int PG = MBW * 4;  // 8-pixel groups per staged channel row
    for (int item = lane; item < NBW * 32 * PG; item += 64) {
      const int ch = item / PG, pg = item % PG;
      const int n = nblk0 * 32 + ch;
      if (n >= a.N) continue;
      const int q0 = pg * 8;
      const int mb = mg * MBW + q0 / 32;
      const int r = mb / (TC / 32), cx = (mb % (TC / 32)) * 32 + (q0 & 31);
      const int oy = oy0 + r, ox = ox0 + cx;
      const int p = oy * a.OW + ox;
      const float4v s0 = *(const float4v *)(stage + ch * PXS + q0);
      const float4v s1 = *(const float4v *)(stage + ch * PXS + q0 + 4);
      float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      const float sl = a.act == IEN_ACT_PRELU ? a.slope[n] : 0.0f;
      const bool whole = oy < a.OH && ox + 8 <= a.OW && p >= a.p_begin && p + 8 <= a.p_end;
      const long at = (long)n * a.ys + (p - a.p_begin);
      if (!a.out_f32 && !a.accumulate && whole && ((((uintptr_t)((uint16_t *)a.y + at)) & 15) == 0)) {
        uint16_t outv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) outv[e] = f2h(v[e]);
        u32x4 ov;
        __builtin_memcpy(&ov, outv, 16);
        *(u32x4 *)((uint16_t *)a.y + at) = ov;
        continue;
      }
      for (int e = 0; e < 8; e++) {
        const int pe = p + e;
        if (oy >= a.OH || ox + e >= a.OW || pe < a.p_begin || pe >= a.p_end) continue;
        const long ae = (long)n * a.ys + (pe - a.p_begin);
        float o = v[e];
        if (a.out_f32) {
          float *yo = (float *)a.y + ae;
          if (a.accumulate) o = activate(o + *yo, a.act, sl);
          *yo = o;
        } else {
          uint16_t *yo = (uint16_t *)a.y + ae;
          if (a.accumulate) o = activate(o + h2f(*yo), a.act, sl);
          *yo = f2h(o);
        }
      }
    }
  }
}

// Split-K finish: out(p, n) = act((acc ? out : 0) + bias[n] + sum over the
// ksplit partial sums in order), the epilogue's order.
__global__ __launch_bounds__(256) void k_splitk_finish(const float *__restrict__ part, int ksplit,
                                                       long rows, int pitch, int N,
                                                       const float *__restrict__ bias,
                                                       const float *__restrict__ slope, int act,
                                                       int accumulate, void *y, long ys,
                                                       int out_f32, int out_nchw) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * N) return;
  const long p = i / N;
  const int n = (int)(i % N);
  float s = 0.0f;
  for (int z = 0; z < ksplit; z++) s += part[((long)z * rows + p) * pitch + n];
  float v = s + bias[n];
  const float sl = act == IEN_ACT_PRELU ? slope[n] : 0.0f;
  const long at = out_nchw ? (long)n * ys + p : p * ys + n;
  if (out_f32) {
    float *yo = (float *)y + at;
    *yo = accumulate ? activate(v + *yo, act, sl) : activate(v, act, sl);
  } else {
    uint16_t *yo = (uint16_t *)y + at;
    *yo = f2h(accumulate ? activate(v + h2f(*yo), act, sl) : activate(v, act, sl));
  }
}

// The same for NCHW outputs: a workgroup sums 32 pixels x 32 channels
// (reading the partial sums along channels, the 4 loads of a split issued
// together from valid addresses), transposes them through LDS and writes 4
// consecutive pixels of one channel per thread (8 or 16 bytes when
// aligned).
__global__ __launch_bounds__(256) void k_splitk_finish_nchw(const float *__restrict__ part,
                                                            int ksplit, long rows, int pitch, int N,
                                                            const float *__restrict__ bias,
                                                            const float *__restrict__ slope,
                                                            int act, int accumulate, void *y,
                                                            long ys, int out_f32) {
  __shared__ float tile[32][32 + 1];
  const long p0 = (long)blockIdx.x * 32;
  const int n0 = blockIdx.y * 32, tid = threadIdx.x;
  // Sum: thread (pixel group pg, channel nn): pixels pg + 8 k, channel n0 + nn.
  const int nn = tid & 31, pg = tid >> 5;
  long at_in[4];
  bool ok[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const long p = p0 + pg + 8 * k;
    ok[k] = p < rows && n0 + nn < N;
    at_in[k] = ok[k] ? p * pitch + n0 + nn : 0;
  }
  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int z = 0; z < ksplit; z++) {
    const float *pz = part + (long)z * rows * pitch;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = pz[at_in[k]];
#pragma unroll
    for (int k = 0; k < 4; k++) sum[k] += v[k];
  }
#pragma unroll
  for (int k = 0; k < 4; k++) tile[nn][pg + 8 * k] = ok[k] ? sum[k] : 0.0f;
  __syncthreads();
  // Write: thread (channel row r, 4-pixel chunk q).
  const int r = tid >> 3, q = (tid & 7) * 4, n = n0 + r;
  if (n >= N) return;
  const float b = bias[n], sl = act == IEN_ACT_PRELU ? slope[n] : 0.0f;
  const long at = (long)n * ys + p0 + q;
  const bool whole = p0 + q + 4 <= rows;
  float v[4], old[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int e = 0; e < 4; e++) v[e] = tile[r][q + e] + b;
  if (out_f32) {
    float *yo = (float *)y + at;
    const bool vec = whole && ((((uintptr_t)yo) & 15) == 0);
    if (accumulate) {
      if (vec) {
        const float4v o = *(const float4v *)yo;
#pragma unroll
        for (int e = 0; e < 4; e++) old[e] = o[e];
      } else {
        for (int e = 0; e < 4; e++) old[e] = p0 + q + e < rows ? yo[e] : 0.0f;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = activate(accumulate ? v[e] + old[e] : v[e], act, sl);
    if (vec) {
      *(float4v *)yo = float4v{v[0], v[1], v[2], v[3]};
    } else {
      for (int e = 0; e < 4; e++)
        if (p0 + q + e < rows) yo[e] = v[e];
    }
  } else {
    uint16_t *yo = (uint16_t *)y + at;
    const bool vec = whole && ((((uintptr_t)yo) & 7) == 0);
    uint16_t h[4];
    if (accumulate) {
      if (vec) {
        const uint2 o = *(const uint2 *)yo;
        __builtin_memcpy(h, &o, 8);
      } else {
        for (int e = 0; e < 4; e++) h[e] = p0 + q + e < rows ? yo[e] : (uint16_t)0;
      }
#pragma unroll
      for (int e = 0; e < 4; e++) old[e] = h2f(h[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) h[e] = f2h(activate(accumulate ? v[e] + old[e] : v[e], act, sl));
    if (vec) {
      uint2 o;
      __builtin_memcpy(&o, h, 8);
      *(uint2 *)yo = o;
    } else {
      for (int e = 0; e < 4; e++)
        if (p0 + q + e < rows) yo[e] = h[e];
    }
  }
}

// o[e] = f16(o[e] + add[e]) for 8 halves: the map added after the
// activation and rounding, as ien_add adds it.
__device__ __forceinline__ void add_after(uint16_t *o, const uint16_t *add) {
  uint16_t h[8];
  *(u32x4 *)h = *(const u32x4 *)add;
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = f2h(h2f(o[e]) + h2f(h[e]));
}

// The same for f16 NHWC outputs with 8-aligned widths and strides: 8
// channels per thread, 16-byte loads and stores, one loop per activation.
__global__ __launch_bounds__(256) void k_splitk_finish8(const float *__restrict__ part, int ksplit,
                                                        long rows, int pitch, int N,
                                                        const float *__restrict__ bias,
                                                        const float *__restrict__ slope, int act,
                                                        int accumulate, uint16_t *y, long ys,
                                                        const uint16_t *add2) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int groups = N >> 3;
  if (i >= rows * groups) return;
  const long p = i / groups;
  const int n = (int)(i - p * groups) * 8;
  float4v s0 = *(const float4v *)(bias + n), s1 = *(const float4v *)(bias + n + 4);
  for (int z = 0; z < ksplit; z++) {
    const float *q = part + ((long)z * rows + p) * pitch + n;
    s0 += *(const float4v *)q;
    s1 += *(const float4v *)(q + 4);
  }
  float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  uint16_t *yo = y + p * ys + n;
  if (accumulate) {
    uint16_t h[8];
    *(u32x4 *)h = *(const u32x4 *)yo;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] += h2f(h[e]);
  }
  uint16_t o[8];
  auto out = [&](auto actf) {
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = f2h(actf(v[e], e));
  };
  switch (act) {
    case IEN_ACT_RELU: out([&](float x, int) { return act_c<IEN_ACT_RELU>(x, 0.0f); }); break;
    case IEN_ACT_GELU: out([&](float x, int) { return act_c<IEN_ACT_GELU>(x, 0.0f); }); break;
    case IEN_ACT_SIGMOID: out([&](float x, int) { return act_c<IEN_ACT_SIGMOID>(x, 0.0f); }); break;
    case IEN_ACT_PRELU: out([&](float x, int e) { return act_c<IEN_ACT_PRELU>(x, slope[n + e]); }); break;
    default: out([&](float x, int) { return x; }); break;
  }
  if (add2) add_after(o, add2 + p * ys + n);
  *(u32x4 *)yo = *(const u32x4 *)o;
}

// The same for outputs too few to fill the CUs (deep splits of small
// maps): T lanes an 8-channel item, lane t adding splits t, t + T, ... in
// order, then the group's sum (a fixed order, so repeated launches agree);
// the group's first lane finishes the item.
template <int T>
__global__ __launch_bounds__(256) void k_splitk_finish8_lanes(const float *__restrict__ part,
                                                              int ksplit, long rows, int pitch, int N,
                                                              const float *__restrict__ bias,
                                                              const float *__restrict__ slope, int act,
                                                              int accumulate, uint16_t *y, long ys,
                                                              const uint16_t *add2) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) / T;
  const int t = threadIdx.x & (T - 1);
  const int groups = N >> 3;
  if (i >= rows * groups) return;  // (whole lane groups)
  const long p = i / groups;
  const int n = (int)(i - p * groups) * 8;
  float4v s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
  for (int z = t; z < ksplit; z += T) {
    const float *q = part + ((long)z * rows + p) * pitch + n;
    s0 += *(const float4v *)q;
    s1 += *(const float4v *)(q + 4);
  }
  float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = group_sum<T>(v[e]);
  if (t != 0) return;
  const float4v b0 = *(const float4v *)(bias + n), b1 = *(const float4v *)(bias + n + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    v[e] += b0[e];
    v[4 + e] += b1[e];
  }
  uint16_t *yo = y + p * ys + n;
  if (accumulate) {
    uint16_t h[8];
    *(u32x4 *)h = *(const u32x4 *)yo;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] += h2f(h[e]);
  }
  uint16_t o[8];
  auto out = [&](auto actf) {
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = f2h(actf(v[e], e));
  };
  switch (act) {
    case IEN_ACT_RELU: out([&](float x, int) { return act_c<IEN_ACT_RELU>(x, 0.0f); }); break;
    case IEN_ACT_GELU: out([&](float x, int) { return act_c<IEN_ACT_GELU>(x, 0.0f); }); break;
    case IEN_ACT_SIGMOID: out([&](float x, int) { return act_c<IEN_ACT_SIGMOID>(x, 0.0f); }); break;
    case IEN_ACT_PRELU: out([&](float x, int e) { return act_c<IEN_ACT_PRELU>(x, slope[n + e]); }); break;
    default: out([&](float x, int) { return x; }); break;
  }
  if (add2) add_after(o, add2 + p * ys + n);
  *(u32x4 *)yo = *(const u32x4 *)o;
}

ien_status splitk_finish(ien_ctx *ctx, int ksplit, long rows, int pitch, const ConvArgs &a) {
  IEN_CHECK(!a.add2 || (!a.out_f32 && !a.out_nchw && a.N % 8 == 0 && pitch % 8 == 0 &&
                        a.ys % 8 == 0 && (((uintptr_t)a.y | (uintptr_t)a.add2) & 15) == 0),
            IEN_ERR_INPUT, "an added map needs whole 16-byte f16 groups");
  if (!a.out_f32 && !a.out_nchw && a.N % 8 == 0 && pitch % 8 == 0 && a.ys % 8 == 0 &&
      (((uintptr_t)a.y) & 15) == 0) {
    const long items = rows * (a.N / 8);
    // Fewer items than 64 Ki threads: up to 8 lanes an item (no more than
    // the splits).
    int lanes = 1;
    while (lanes < 8 && 2 * lanes <= ksplit && items * lanes < 65536) lanes *= 2;
    if (lanes > 1) {
      auto k = lanes == 2 ? k_splitk_finish8_lanes<2> : lanes == 4 ? k_splitk_finish8_lanes<4>
                                                                    : k_splitk_finish8_lanes<8>;
      hipLaunchKernelGGL(k, dim3((unsigned)((items * lanes + 255) / 256)), dim3(256), 0, ctx->stream,
                         (const float *)ctx->splitk, ksplit, rows, pitch, a.N, a.bias, a.slope, a.act,
                         a.accumulate, (uint16_t *)a.y, (long)a.ys, a.add2);
      IEN_HIP(hipGetLastError());
      return IEN_OK;
    }
    hipLaunchKernelGGL(k_splitk_finish8, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       ctx->stream, (const float *)ctx->splitk, ksplit, rows, pitch, a.N, a.bias,
                       a.slope, a.act, a.accumulate, (uint16_t *)a.y, (long)a.ys, a.add2);
  } else if (a.out_nchw) {
    const dim3 grid((unsigned)((rows + 31) / 32), (unsigned)((a.N + 31) / 32));
    hipLaunchKernelGGL(k_splitk_finish_nchw, grid, dim3(256), 0, ctx->stream,
                       (const float *)ctx->splitk, ksplit, rows, pitch, a.N, a.bias, a.slope, a.act,
                       a.accumulate, a.y, (long)a.ys, a.out_f32);
  } else {
    const long items = rows * a.N;
    hipLaunchKernelGGL(k_splitk_finish, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       ctx->stream, (const float *)ctx->splitk, ksplit, rows, pitch, a.N, a.bias,
                       a.slope, a.act, a.accumulate, a.y, (long)a.ys, a.out_f32, a.out_nchw);
  }
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

// ---------------------------------------------------------------------------
// Host dispatch.

template <int KS, int S, int TR, int TC, int MSPLIT, int NBW, int CK, bool VEC, bool IN_NCHW>
static ien_status run_cfg(ien_ctx *ctx, ConvArgs a) {
  using Cfg = ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW>;
  // Tile grid over the requested pixel range.
  const int first_row = a.p_begin / a.OW, last_row = (a.p_end - 1) / a.OW;
  a.ty_begin = first_row / TR;
  a.tiles_y = last_row / TR + 1 - a.ty_begin;
  a.tiles_x = (a.OW + TC - 1) / TC;
  a.tiles_n = (a.N + Cfg::BN - 1) / Cfg::BN;
  const long blocks = (long)a.tiles_y * a.tiles_x * a.tiles_n;
  IEN_CHECK(blocks > 0 && blocks < (1L << 31), IEN_ERR_INPUT, "grid of %ld tiles", blocks);
  // The packed weights must cover every fragment the tiles touch.
  IEN_CHECK(a.tiles_n * Cfg::NBT <= a.NB, IEN_ERR_INPUT, "weights narrower than the tile");
  // Split-K when the tiles leave three quarters of the CUs idle, or any CU
  // idle for a 1 x 1 product at least 1536 deep: about two workgroups per
  // CU, each split at least 512 deep in K (the partial sums cost an f32
  // write and read of the output per split), partial sums in the context's
  // workspace, then the finishing pass.
  const int chunks = (a.C + CK - 1) / CK;
  const long rows = a.p_end - a.p_begin;
  const int pitch = a.tiles_n * Cfg::BN;
  const int T = KS == 0 ? a.noff : KS * KS;
  const int min_chunks = (512 + T * CK - 1) / (T * CK);
  // Double-buffered chunks when the tiles (and their splits) fill the CUs
  // at most once: then no other workgroup hides a chunk's load latency.
  // Each split keeps at least two chunks to overlap; the buffer loads take
  // 32-bit byte offsets.  Not for offset taps (LaMa's transposed phases:
  // no gain, 3.25 against 3.23 ms per image), nor when the context asks for
  // compact launches.
  bool db = false;
  if constexpr (VEC && KS > 0) {
    if constexpr (ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true>::FITS) {
      const long in_bytes = (a.rows_mode ? (long)a.M : (long)a.H * a.W) * a.xs * 2;
      // NCHW: the fast halo path only (zero padding, whole 16-byte groups).
      const bool layout_ok =
          !IN_NCHW || (!a.rows_mode && !a.pad_reflect && (a.W & 7) == 0 && (a.xs & 7) == 0 &&
                       (((uintptr_t)a.x) & 15) == 0);
      constexpr int FIT =
          160 * 1024 / ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true>::LDS_BYTES;
      // Buffer ranges stay below the padding loads' out-of-range offset
      // (0x7ffffff0), so a padding load never lands inside the buffer.
      db = layout_ok && !ctx->compact && blocks <= (long)ctx->cus * FIT && chunks >= 2 &&
           (IN_NCHW || in_bytes <= 0x7fff0000L) && (long)a.NB * a.KB * 1024 <= 0x7fff0000L;
    }
  }
  // Each XCD takes a contiguous band of blocks.  Channels fastest, every
  // band reads all the weights and its share of the input halos; pixels
  // fastest, the reverse.  Take the order that fetches fewer bytes.
  {
    const long tpix = (long)a.tiles_y * a.tiles_x;
    const double wb = (double)a.tiles_n * Cfg::NBT * a.KB * 1024.0;
    const double xb = (double)tpix * Cfg::HR * Cfg::HC * a.C * 2.0;
    const double by_n = xb * std::max(1.0, 8.0 / tpix) + wb * std::min(8L, tpix);
    const double by_pix = wb * std::max(1.0, 8.0 / a.tiles_n) + xb * std::min(8, a.tiles_n);
    a.n_major = a.tiles_n > 1 && (blocks & 7) == 0 && by_pix < by_n;
  }
  int ksplit = 1;
  const bool idle = 4 * blocks <= ctx->cus || (KS == 1 && T * a.C >= 1536 && blocks < ctx->cus);
  if (VEC && chunks >= 2 * min_chunks && idle && !a.phase) {
    ksplit = (int)std::min<long>(chunks / min_chunks, (2L * ctx->cus + blocks - 1) / blocks);
    if (db) ksplit = (int)std::min<long>({(long)ksplit, ctx->cus / blocks, chunks / 2L});
    ksplit = std::max(ksplit, 1);
    while (ksplit > 1 && (size_t)ksplit * rows * pitch > ctx->splitk_floats) ksplit--;
  }
  a.kchunks = (chunks + ksplit - 1) / ksplit;
  a.ksplit = (chunks + a.kchunks - 1) / a.kchunks;
  // Three chunk buffers (two chunks in flight) where a workgroup runs at
  // least three chunks and as many workgroups still fit a CU.
  bool db3 = false;
  if constexpr (VEC && KS > 0 && ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true, 3>::FITS) {
    constexpr int FIT3 =
        160 * 1024 / ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true, 3>::LDS_BYTES;
    db3 = db && a.kchunks >= 3 && blocks * a.ksplit <= (long)ctx->cus * FIT3;
  }
  auto launch = [&](const ConvArgs &la, dim3 grid) -> ien_status {
    if constexpr (VEC && KS > 0 &&
                  ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true, 3>::FITS) {
      if (db3) {
        hipLaunchKernelGGL((conv_mfma<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true, 3>), grid,
                           dim3(256), 0, ctx->stream, la);
        IEN_HIP(hipGetLastError());
        return IEN_OK;
      }
    }
    if constexpr (VEC && KS > 0 &&
                  ConvCfg<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true>::FITS) {
      if (db) {
        hipLaunchKernelGGL((conv_mfma<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW, true>), grid,
                           dim3(256), 0, ctx->stream, la);
        IEN_HIP(hipGetLastError());
        return IEN_OK;
      }
    }
    hipLaunchKernelGGL((conv_mfma<KS, S, TR, TC, MSPLIT, NBW, CK, VEC, IN_NCHW>), grid, dim3(256),
                       0, ctx->stream, la);
    IEN_HIP(hipGetLastError());
    return IEN_OK;
  };
  if (a.ksplit <= 1) {
    a.ksplit = 1;
    a.kchunks = chunks;
    return launch(a, dim3((unsigned)blocks));
  }
  // Double-buffered launches of up to 4 splits, each tile's splits counted
  // in: its last split adds them and finishes the tile (the sums of a split
  // block: 256 threads x MBW NBW accumulators).  Deeper splits keep the
  // finishing pass, which spreads the additions over every CU rather than
  // one split a tile (BiRefNet's 8-tile, 32-split decoder products: 3.11
  // -> 3.18 ms an image counted in), and so do the single-buffered launches
  // (BiRefNet's 7 x 7 products in 4 splits: 3.16 -> 3.19 ms).
  const long split_floats = 256L * Cfg::MBW * NBW * 16;
  if (db && a.ksplit <= 4 && blocks <= ien_ctx::SPLITK_TILES &&
      blocks * a.ksplit * split_floats <= (long)ctx->splitk_floats) {
    a.part = ctx->splitk;
    a.tile_count = (int *)(ctx->splitk + ctx->splitk_floats);
    return launch(a, dim3((unsigned)blocks, (unsigned)a.ksplit));
  }
  ConvArgs pa = a;
  pa.part = nullptr;
  pa.tile_count = nullptr;
  pa.y = ctx->splitk;
  pa.ys = pitch;
  pa.out_f32 = 1;
  pa.out_nchw = 0;
  pa.act = IEN_ACT_NONE;
  pa.accumulate = 0;
  pa.add2 = nullptr;
  const ien_status st = launch(pa, dim3((unsigned)blocks, (unsigned)a.ksplit));
  if (st != IEN_OK) return st;
  return splitk_finish(ctx, a.ksplit, rows, pitch, a);
}

// Channel chunk of the 16-channel-step kernels: the largest of 64, 32, 16
// that divides the channel count.
static int pick_ck(int c) { return c % 64 == 0 ? 64 : c % 32 == 0 ? 32 : 16; }

ien_status launch_conv(ien_ctx *ctx, const ConvCall &c) {
  const ien_matrix *w = c.w;
  IEN_CHECK(w && w->d_packed, IEN_ERR_INPUT, "no weights");
  const int T = c.noff ? c.noff : c.ks * c.ks;
  IEN_CHECK((size_t)T * c.C == w->k, IEN_ERR_INPUT,
            "input does not match the weights: %d taps x %d channels, k = %zu", T, c.C, w->k);
  IEN_CHECK(c.rows > 0, IEN_ERR_INPUT, "no rows");
  IEN_CHECK(c.act != IEN_ACT_PRELU || c.slope, IEN_ERR_INPUT, "PReLU without slopes");
  const bool nchw = c.in_nchw != 0;
  // The kernels index with 32-bit offsets.
  const long in_extent = c.rows_mode ? (c.row0 + c.rows) * c.xs
                         : nchw     ? (long)c.C * c.xs
                                    : (long)c.H * c.W * c.xs;
  const long out_extent = c.out_nchw ? (long)w->n * c.ys : c.rows * c.ys;
  IEN_CHECK(in_extent < (1L << 31) && out_extent < (1L << 31) && c.row0 + c.rows < (1L << 31),
            IEN_ERR_INPUT, "tensors over 2^31 elements");
  ConvArgs a{};
  std::memset(&a, 0, sizeof a);
  a.x = c.x;
  a.H = c.H;
  a.W = c.W;
  a.C = c.C;
  a.xs = (int)c.xs;
  a.rows_mode = c.rows_mode;
  a.pad_reflect = c.pad_reflect;
  a.noff = c.noff;
  for (int i = 0; i < 4; i++) {
    a.offy[i] = c.offy[i];
    a.offx[i] = c.offx[i];
  }
  a.OH = c.OH;
  a.OW = c.OW;
  a.p_begin = (int)c.row0;
  a.p_end = (int)(c.row0 + c.rows);
  a.wp = w->d_packed;
  a.zeros = ctx->zeros;
  a.KB = w->kb;
  a.NB = w->nb;
  a.N = (int)w->n;
  a.bias = c.bias ? c.bias : w->d_bias;
  a.slope = c.slope;
  a.y = c.y;
  a.ys = (int)c.ys;
  a.out_nchw = c.out_nchw;
  a.out_f32 = c.out_f32;
  a.act = c.act;
  a.accumulate = c.accumulate;
  a.add2 = c.add2;
  a.phase = c.phase;

  // 16-channel MFMA steps; NHWC halo loads of 16 bytes need aligned pixels.
  const bool vec = c.C % 16 == 0 && (nchw || (c.xs % 8 == 0 && ((uintptr_t)c.x & 15) == 0));
  const int ck = pick_ck(c.C);
#define IEN_CK(KS, S, TR, TC, L)                                                   \
  return ck == 64 ? run_cfg<KS, S, TR, TC, 4, 2, 64, true, L>(ctx, a)              \
         : ck == 32 ? run_cfg<KS, S, TR, TC, 4, 2, 32, true, L>(ctx, a)            \
                    : run_cfg<KS, S, TR, TC, 4, 2, 16, true, L>(ctx, a)
  // An added map: the general kernel's 16-byte f16 group epilogue (and its
  // split-K finishing passes) only; the special kernels below are skipped.
  IEN_CHECK(!c.add2 || (!nchw && !c.rows_mode && c.noff == 0 && c.ks == 3 && c.stride == 1 &&
                        vec && !c.out_nchw && !c.out_f32 && c.ys % 8 == 0 && w->n % 8 == 0 &&
                        (((uintptr_t)c.y | (uintptr_t)c.add2) & 15) == 0),
            IEN_ERR_INPUT, "an added map needs an NHWC 3x3 product with whole 16-byte f16 groups");
  IEN_CHECK(c.phase == 0 ||
                (c.phase >= 1 && c.phase <= 4 && !nchw && !c.rows_mode && vec && c.stride == 1 &&
                 !c.out_nchw && !c.out_f32 && c.row0 == 0 && c.rows == (long)c.OH * c.OW &&
                 c.ys % 8 == 0 && w->n % 8 == 0 && ((uintptr_t)c.y & 15) == 0 &&
                 (c.ks == 3 || c.noff > 0)),
            IEN_ERR_INPUT, "a phase-scattered output needs a whole NHWC product in 16-byte f16 groups");
  const bool special = !c.add2 && !c.phase;
  if (c.rows_mode) {
    // Input::Rows: a virtual image 32 pixels wide, rows in order.
    IEN_CHECK(!nchw && c.ks == 1 && c.noff == 0, IEN_ERR_INPUT, "rows are NHWC, one tap");
    a.W = a.OW = 32;
    a.M = a.p_end;
    a.H = a.OH = (a.M + 31) / 32;
    if (vec && rows_supported(a, c.rows)) return launch_rows(ctx, a);
    if (vec) IEN_CK(1, 1, 4, 32, false);
    IEN_CHECK(c.C <= 64, IEN_ERR_INPUT, "rows of %d values (not a multiple of 16, over 64)", c.C);
    return run_cfg<1, 1, 4, 32, 4, 2, 64, false, false>(ctx, a);
  }
  IEN_CHECK(vec || c.C <= 16, IEN_ERR_INPUT, "%d channels: a multiple of 16, or at most 16", c.C);
  if (c.noff) {
    IEN_CHECK(!nchw, IEN_ERR_INPUT, "offset taps read NHWC");
    for (int i = 0; i < c.noff; i++)
      IEN_CHECK(c.offy[i] >= 0 && c.offy[i] <= 1 && c.offx[i] >= 0 && c.offx[i] <= 1,
                IEN_ERR_INPUT, "offsets past one pixel");
    if (vec) IEN_CK(0, 1, 4, 32, false);
    return run_cfg<0, 1, 4, 32, 4, 2, 16, false, false>(ctx, a);
  }
  // Four input channels (the models' image inputs) and few outputs (their
  // last convolutions): the general kernel would pad these to 16-channel
  // steps and 64-channel tiles.
  if (special && narrow_supported(a, c.ks, c.stride, nchw, c.noff, c.rows_mode))
    return launch_narrow(ctx, a, c.ks);
  if (special && few_supported(a, c.ks, c.stride, nchw, c.noff, c.rows_mode))
    return launch_few(ctx, a, c.ks);
  // Resident weights: NHWC, zero padding, 16, 32 or 64 channels, K <= 640.
  // Its results are staged as f16: f32 outputs take the general kernel, and
  // so do compact launches of 64 channels (beside another branch's kernels,
  // whose workgroups the resident one's 158 KiB of LDS would shut out).
  if (special && vec && !c.out_f32 && !(ctx->compact && c.C == 64) &&
      resident_supported(c.ks, c.stride, c.C, nchw, c.pad_reflect, c.noff, c.rows_mode,
                         (long)c.H * c.W * c.xs * 2))
    return launch_resident(ctx, a, c.ks);
  // NCHW 1x1 products of whole planes: the register-transposing kernel.
  if (nchw && nchw1_supported(a, c.ks, c.stride, c.rows)) return launch_nchw1(ctx, a);
  // NCHW 3x3 64 -> 64: the whole layer's weights and a 4 x 96 tile a CU.
  if (nchw && nchw3_supported(a, c.ks, c.stride, c.rows)) return launch_nchw3(ctx, a);
  // NCHW 3x3 128 -> 128: 2 x 96 tiles a channel half, K in double-buffered quarters.
  if (nchw && nchw3q_supported(a, c.ks, c.stride, c.rows)) return launch_nchw3q(ctx, a);
  if (c.ks == 3 && c.stride == 1) {
    if (!vec) {
      if (nchw) return run_cfg<3, 1, 4, 32, 4, 2, 16, false, true>(ctx, a);
      return run_cfg<3, 1, 4, 32, 4, 2, 16, false, false>(ctx, a);
    }
    // NHWC: 4 x 32 tiles and 32-channel chunks, so that the halo and weight
    // stages of three workgroups fit a CU's LDS and hide each other's load
    // latency (same-box A/B against 64-channel chunks and 4 x 96 tiles:
    // SCUNet 4.49 -> 4.30, LaMa 4.08 -> 4.01 ms).
    // NCHW likewise (the conv sweep: 3x3 64 at 256 x 384 25.4 -> 22.5 us,
    // 128 at 128 x 192 38.1 -> 27.1 us, 512 at 32 x 32 35.7 -> 25.9 us).
    if (ck == 64) {
      // Between one and two tiles a CU: 16-channel chunks, double-buffered
      // two workgroups a CU.
      const long tiles = (long)((c.OH + 3) / 4) * ((c.OW + 31) / 32) * ((w->n + 63) / 64);
      if (tiles > ctx->cus && tiles <= 2L * ctx->cus && !ctx->compact) {
        if (nchw) return run_cfg<3, 1, 4, 32, 4, 2, 16, true, true>(ctx, a);
        return run_cfg<3, 1, 4, 32, 4, 2, 16, true, false>(ctx, a);
      }
      if (nchw) return run_cfg<3, 1, 4, 32, 4, 2, 32, true, true>(ctx, a);
      return run_cfg<3, 1, 4, 32, 4, 2, 32, true, false>(ctx, a);
    }
    if (nchw) IEN_CK(3, 1, 4, 32, true);
    IEN_CK(3, 1, 4, 32, false);
  }
  if (c.ks == 3 && c.stride == 2) {
    IEN_CHECK(!nchw, IEN_ERR_INPUT, "strided convolutions read NHWC");
    if (!vec) return run_cfg<3, 2, 4, 32, 4, 2, 16, false, false>(ctx, a);
    if (ck >= 32) return run_cfg<3, 2, 4, 32, 4, 2, 32, true, false>(ctx, a);
    return run_cfg<3, 2, 4, 32, 4, 2, 16, true, false>(ctx, a);
  }
  if (c.ks == 1 && c.stride == 1) {
    IEN_CHECK(vec, IEN_ERR_INPUT, "1x1 products over %d channels", c.C);
    if (!nchw && !c.pad_reflect && rows_supported(a, c.rows)) return launch_rows(ctx, a);
    if (nchw) IEN_CK(1, 1, 4, 32, true);
    IEN_CK(1, 1, 4, 32, false);
  }
  if (c.ks == 7 && c.stride == 1) {
    IEN_CHECK(!nchw, IEN_ERR_INPUT, "7x7 convolutions read NHWC");
    if (!vec) return run_cfg<7, 1, 4, 32, 4, 2, 16, false, false>(ctx, a);
    // 8 x 32 tiles (two M-blocks a wave): each chunk's 49-tap fragments
    // (98 KiB at 64 output channels) are staged for twice the pixels; 16 x 32
    // tiles (four a wave) where those still make two rounds of the CUs.
    const long tall = (long)((c.OH + 15) / 16) * ((c.OW + 31) / 32) * ((a.N + 63) / 64);
    if (tall >= 2L * ctx->cus) return run_cfg<7, 1, 16, 32, 4, 2, 16, true, false>(ctx, a);
    return run_cfg<7, 1, 8, 32, 4, 2, 16, true, false>(ctx, a);
  }
#undef IEN_CK
  return fail(IEN_ERR_INPUT, "no kernel for %dx%d stride %d convolutions", c.ks, c.ks, c.stride);
}

// Fill a ConvCall from the op-level descriptors.
static ien_status describe(const ien_input *in, size_t row0, size_t rows, const ien_matrix *w,
                           ConvCall *c) {
  IEN_CHECK(in && w, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(in->data, IEN_ERR_INPUT, "null input data");
  c->x = (const uint16_t *)in->data;
  c->w = w;
  c->row0 = (long)row0;
  c->rows = (long)rows;
  if (in->kind == IEN_INPUT_ROWS) {
    IEN_CHECK(in->stride >= w->k, IEN_ERR_INPUT, "row stride %zu under k = %zu", in->stride, w->k);
    c->rows_mode = 1;
    c->C = (int)w->k;
    c->xs = (long)in->stride;
    c->ks = 1;
    c->stride = 1;
    return IEN_OK;
  }
  IEN_CHECK(in->kind == IEN_INPUT_IMAGE, IEN_ERR_INPUT, "input kind %d", (int)in->kind);
  IEN_CHECK(in->height > 0 && in->width > 0 && in->height < (1u << 20) && in->width < (1u << 20),
            IEN_ERR_INPUT, "%zu x %zu image", in->width, in->height);
  c->H = (int)in->height;
  c->W = (int)in->width;
  c->C = (int)in->channels;
  c->xs = (long)in->stride;
  c->in_nchw = in->layout == IEN_LAYOUT_NCHW;
  if (c->in_nchw)
    IEN_CHECK(in->stride >= in->height * in->width, IEN_ERR_INPUT, "plane stride under h x w");
  else
    IEN_CHECK(in->stride >= in->channels, IEN_ERR_INPUT, "pixel stride under channels");
  c->pad_reflect = in->pad == IEN_PAD_REFLECT;
  if (in->taps == IEN_TAPS_CONV) {
    IEN_CHECK(in->size % 2 == 1 && in->step > 0, IEN_ERR_INPUT, "size %zu step %zu", in->size,
              in->step);
    IEN_CHECK(!c->pad_reflect || (in->size / 2 < in->height && in->size / 2 < in->width),
              IEN_ERR_INPUT, "reflect padding past a %zu x %zu image", in->width, in->height);
    c->ks = (int)in->size;
    c->stride = (int)in->step;
    c->OH = (int)((in->height - 1) / in->step + 1);
    c->OW = (int)((in->width - 1) / in->step + 1);
  } else {
    IEN_CHECK(in->count >= 1 && in->count <= 4, IEN_ERR_INPUT, "%zu offsets", in->count);
    c->noff = (int)in->count;
    for (size_t i = 0; i < in->count; i++) {
      c->offy[i] = (int)in->offsets[i][0];
      c->offx[i] = (int)in->offsets[i][1];
    }
    c->ks = 0;
    c->stride = 1;
    c->OH = (int)in->height;
    c->OW = (int)in->width;
  }
  IEN_CHECK(row0 + rows <= (size_t)c->OH * c->OW, IEN_ERR_INPUT, "rows %zu..%zu past %d pixels",
            row0, row0 + rows, c->OH * c->OW);
  return IEN_OK;
}

}  // namespace ien

using namespace ien;

extern "C" {

ien_status ien_multiply_ex(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                           const ien_matrix *w, const ien_output *out, ien_act act,
                           const float *d_slope, int accumulate) {
  IEN_CHECK(ctx && out && out->data, IEN_ERR_INPUT, "null argument");
  if (rows == 0) return IEN_OK;
  ConvCall c;
  ien_status s = describe(input, row0, rows, w, &c);
  if (s != IEN_OK) return s;
  c.y = out->data;
  c.ys = (long)out->stride;
  c.out_nchw = out->layout == IEN_LAYOUT_NCHW;
  c.out_f32 = out->type == IEN_OUT_F32;
  if (c.out_nchw)
    IEN_CHECK(out->stride >= rows, IEN_ERR_INPUT, "plane stride under the rows");
  else
    IEN_CHECK(out->stride >= w->n, IEN_ERR_INPUT, "output stride %zu under n = %zu", out->stride,
              w->n);
  c.act = act;
  c.slope = d_slope;
  c.accumulate = accumulate;
  return launch_conv(ctx, c);
}

ien_status ien_multiply(ien_ctx *ctx, const ien_input *input, size_t row0, size_t rows,
                        const ien_matrix *w, void *d_out, size_t stride, ien_act act,
                        int accumulate) {
  IEN_CHECK(act == IEN_ACT_NONE || act == IEN_ACT_RELU || act == IEN_ACT_GELU, IEN_ERR_INPUT,
            "multiply takes Act::{None, Relu, Gelu}");
  ien_output out = {d_out, stride, IEN_LAYOUT_NHWC, IEN_OUT_F16};
  return ien_multiply_ex(ctx, input, row0, rows, w, &out, act, nullptr, accumulate);
}

ien_status ien_conv3(ien_ctx *ctx, const ien_input *input, const ien_matrix *w, void *d_out,
                     size_t stride, int accumulate, ien_act finish, const float *d_slope) {
  IEN_CHECK(input && input->kind == IEN_INPUT_IMAGE && input->taps == IEN_TAPS_CONV &&
                input->size == 3 && input->step == 1,
            IEN_ERR_INPUT, "conv3 needs a 3x3 stride-1 convolution");
  IEN_CHECK(finish == IEN_ACT_NONE || finish == IEN_ACT_RELU || finish == IEN_ACT_PRELU,
            IEN_ERR_INPUT, "finish %d", (int)finish);
  ien_output out = {d_out, stride, IEN_LAYOUT_NHWC, IEN_OUT_F16};
  return ien_multiply_ex(ctx, input, 0, input->height * input->width, w, &out, finish, d_slope,
                         accumulate);
}

}  // extern "C"
