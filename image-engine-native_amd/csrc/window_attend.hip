// window_attend.hip -- the first half of Swin window attention in one pass
// per window and head: the rolled window gather, LayerNorm 1, the head's
// q, k, v and the attention with position bias and shift mask
// (crates/birefnet-native/src/swin.rs:219-296 Block::attend up to the
// projection; crates/scunet-native/src/swin.rs:131-220), for any width
// that is a multiple of 32 up to 256 and windows of up to 64 or 160 tokens
// (BiRefNet's 7 x 7 and 12 x 12, SCUNet's 8 x 8 beyond the widths its
// whole-window kernel takes).  The projection, added straight back onto the
// map, stays a row product.
//
// One workgroup per (window, head), one wave per block of 32 window
// tokens (NP / 32 waves; tokens past the window's N, and tokens the roll
// puts past the map's edge, are zero rows after the LayerNorm, so their
// q, k, v are the biases -- swin.rs:238-254):
//  - Wave t loads its tokens as MFMA fragments (lane l: token 32 t + l %
//    32, channels 16 s + 8 (l / 32) .. + 7), normalises them (mean, then
//    the mean square deviation, eps 1e-5: math.rs:95-116) and rounds them
//    to f16 as the window rows hold them.  Those registers are the B
//    operand of K^T = Wk^T x^T and Q^T = Wq^T x^T and the A operand of
//    V = x Wv on v_mfma_f32_32x32x16_f16, whose other operands are the
//    packed qkv fragments as they are (a B fragment of W is an A fragment
//    of W^T).  The raw rows stay in registers between the sum and the
//    square deviation, and up to 96 channels until the products.
//  - Accumulator registers 8 s .. 8 s + 7 of K^T, Q^T and V read as an f16
//    operand hold the 16-wide k step 16 s + 4 (l / 32) + {0..3, 8..11}: the
//    same permutation of the head's dims on both sides of S^T = K Q^T and
//    of the keys on both sides of O^T = V^T P^T.  Each wave leaves its K
//    and V blocks in LDS as those operands; after one barrier wave t
//    computes S^T for its 32 queries against every key block, each tile
//    starting from its bias (the bias tables are packed in the accumulator
//    layout, keys past N at -inf; q is scaled by 1 / sqrt(32) before it is
//    rounded, as attention.rs scales it), the softmax (keys in registers
//    plus one exchange with lane l ^ 32), and O^T.
//  - O^T's lane l holds query l % 32, dims 8 (r / 4) + 4 (l / 32) + r % 4:
//    written to the window row as 8-byte runs.
// Normalised x, q, k, v and the output are f16 and products accumulate in
// f32, as in the unfused path; the probabilities enter O^T as f16 before
// the division by their sum, which scales O^T (the unfused kernel rounds
// them after it).

#include "conv_common.h"
#include "window_geo.h"

namespace ien {
namespace {

struct QkvAttnArgs {
  WinGeo g;
  const uint16_t *map;
  long stride;
  int c, heads;
  const float *gamma, *beta;  // LayerNorm 1 (c each, 16-byte aligned)
  const uint16_t *wqkv;       // packed c x 3c fragments, n-block major
  const float *bqkv;          // 3c
  const float *tables;        // [class][head][query block][key block][4][64][4]
  uint16_t *out;              // windows x N rows of c: the heads' outputs
};

__device__ __forceinline__ half8 wfrag(const uint16_t *p, int idx, int lane) {
  return *(const half8 *)(p + (size_t)idx * 512 + lane * 8);
}

__device__ __forceinline__ half8 acc_operand(const floatx16 &t, int s, float scale) {
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; i++) h[i] = (_Float16)(t[8 * s + i] * scale);
  return h;
}

// Lane's 8 f16 values of a raw 16-byte row chunk as floats.
__device__ __forceinline__ void unpack_chunk(const u32x4 &raw, float *v) {
  uint16_t h[8];
  __builtin_memcpy(h, &raw, 16);
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = h2f(h[e]);
}

// Channels 16 s + 8 hf .. + 7 normalised: (v - mean) inv gamma + beta, times
// keep (0 for a zero row).
__device__ __forceinline__ half8 norm_chunk(const QkvAttnArgs &a, const u32x4 &raw, int s, int hf,
                                            float mean, float inv, float keep) {
  float v[8];
  unpack_chunk(raw, v);
  const float4 g0 = *(const float4 *)(a.gamma + 16 * s + 8 * hf);
  const float4 g1 = *(const float4 *)(a.gamma + 16 * s + 8 * hf + 4);
  const float4 b0 = *(const float4 *)(a.beta + 16 * s + 8 * hf);
  const float4 b1 = *(const float4 *)(a.beta + 16 * s + 8 * hf + 4);
  const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
  half8 x;
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = (_Float16)(((v[e] - mean) * inv * gg[e] + bb[e]) * keep);
  return x;
}

// KB key (and query) blocks of 32; KS_ = c / 16 steps of 16 channels.
template <int KB, int KS_>
__global__ __launch_bounds__(64 * KB) __attribute__((amdgpu_waves_per_eu(KS_ == 8 || KS_ == 12 ? 3 : 4))) void
k_window_qkv_attention(QkvAttnArgs a) {
  __shared__ half8 kshare[KB * 2 * 64], vshare[KB * 2 * 64];  // [block][s][lane]
  const int tb = threadIdx.x >> 6, lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
  // Blocks are dealt to the 8 XCDs in turn: XCD x takes a contiguous band
  // of (window, head) items, so the heads of a window read its rows from
  // one L2.
  const int nb = (int)gridDim.x, xcd = (int)blockIdx.x & 7;
  const int item = xcd * (nb >> 3) + min(xcd, nb & 7) + ((int)blockIdx.x >> 3);
  const int w = item / a.heads, h = item - w * a.heads;
  constexpr int KS = KS_;
  const int CB = a.c >> 5;
  const int t = 32 * tb + l32;
  const int src = t < a.g.n ? win_source(a.g, w, t) : -1;
  const float keep = src < 0 ? 0.0f : 1.0f;
  const uint16_t *row = a.map + (long)(src < 0 ? 0 : src) * a.stride + 8 * hf;
  const float inv_c = 1.0f / (float)a.c;

  floatx16 qt = {}, kt = {}, vv = {};
  auto step = [&](int s, const half8 &xn) {
    const half8 wq = wfrag(a.wqkv, h * KS + s, lane);
    const half8 wk = wfrag(a.wqkv, (CB + h) * KS + s, lane);
    const half8 wv = wfrag(a.wqkv, (2 * CB + h) * KS + s, lane);
    qt = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq, xn, qt, 0, 0, 0);
    kt = __builtin_amdgcn_mfma_f32_32x32x16_f16(wk, xn, kt, 0, 0, 0);
    vv = __builtin_amdgcn_mfma_f32_32x32x16_f16(xn, wv, vv, 0, 0, 0);
  };
  {
    u32x4 xr[KS_];
#pragma unroll
    for (int s = 0; s < KS_; s++) xr[s] = *(const u32x4 *)(row + 16 * s);
    float sum = 0.0f;
#pragma unroll
    for (int s = 0; s < KS_; s++) {
      float v[8];
      unpack_chunk(xr[s], v);
#pragma unroll
      for (int e = 0; e < 8; e++) sum += v[e];
    }
    sum += __shfl_xor(sum, 32);
    const float mean = sum * inv_c;
    float sq = 0.0f;
#pragma unroll
    for (int s = 0; s < KS_; s++) {
      float v[8];
      unpack_chunk(xr[s], v);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = v[e] - mean;
        sq += d * d;
      }
    }
    sq += __shfl_xor(sq, 32);
    const float inv = 1.0f / sqrtf(sq * inv_c + 1e-5f);
    if constexpr (KS_ > 6) {
      // Past 96 channels the rows are read again (from the cache) for the
      // products rather than kept: 48 more live registers had cost a wave
      // a SIMD.
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int s = 0; s < KS_; s++)
        step(s, norm_chunk(a, *(const u32x4 *)(row + 16 * s), s, hf, mean, inv, keep));
    } else {
#pragma unroll
      for (int s = 0; s < KS_; s++) step(s, norm_chunk(a, xr[s], s, hf, mean, inv, keep));
    }
  }

  // Biases: Q^T and K^T rows are dims 8 (r / 4) + 4 hf + r % 4, V's columns
  // dims l32.
  const float bv = a.bqkv[2 * a.c + 32 * h + l32];
#pragma unroll
  for (int q4 = 0; q4 < 4; q4++) {
    const float4 bq = *(const float4 *)(a.bqkv + 32 * h + 8 * q4 + 4 * hf);
    const float4 bk = *(const float4 *)(a.bqkv + a.c + 32 * h + 8 * q4 + 4 * hf);
    const float bqa[4] = {bq.x, bq.y, bq.z, bq.w}, bka[4] = {bk.x, bk.y, bk.z, bk.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      qt[4 * q4 + e] += bqa[e];
      kt[4 * q4 + e] += bka[e];
      vv[4 * q4 + e] += bv;
    }
  }
  // q / sqrt(32) (attention.rs scales q before the products).
  const float scale = 0.17677669529663688f;
  half8 qo[2];
#pragma unroll
  for (int s = 0; s < 2; s++) {
    qo[s] = acc_operand(qt, s, scale);
    kshare[(tb * 2 + s) * 64 + lane] = acc_operand(kt, s, 1.0f);
    vshare[(tb * 2 + s) * 64 + lane] = acc_operand(vv, s, 1.0f);
  }
  __syncthreads();

  // S^T for this wave's queries: key 32 kb + 8 (r / 4) + 4 hf + r % 4 in
  // register r of st[kb], query l32.  The bias tables are packed in that
  // accumulator layout, so each tile starts from its bias.
  const int cls = win_class(a.g, w);
  const float *tp =
      a.tables + ((long)(cls * a.heads + h) * KB + tb) * KB * 1024 + lane * 4;
  floatx16 st[KB];
  float mx = -__builtin_inff();
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    floatx16 bt;
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
      const float4 b4 = *(const float4 *)(tp + (kb * 4 + q4) * 256);
      bt[4 * q4] = b4.x;
      bt[4 * q4 + 1] = b4.y;
      bt[4 * q4 + 2] = b4.z;
      bt[4 * q4 + 3] = b4.w;
    }
    st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kshare[(kb * 2) * 64 + lane], qo[0], bt, 0, 0, 0);
    st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kshare[(kb * 2 + 1) * 64 + lane], qo[1], st[kb],
                                                    0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; r++) mx = fmaxf(mx, st[kb][r]);
  }
  // p = e^(s - max) as 2^(s log2 e - max log2 e): one fused multiply-add
  // before the exponential.  The probabilities enter O^T unnormalised (f16,
  // in (0, 1]); O^T is divided by their sum once.
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  constexpr float LOG2E = 1.4426950408889634f;
  const float mxl = -mx * LOG2E;
  float sum = 0.0f;
#pragma unroll
  for (int kb = 0; kb < KB; kb++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r], LOG2E, mxl));
      st[kb][r] = p;
      sum += p;
    }
  sum += __shfl_xor(sum, 32);
  const float inv = 1.0f / sum;
  floatx16 o = {};
#pragma unroll
  for (int kb = 0; kb < KB; kb++)
#pragma unroll
    for (int s = 0; s < 2; s++)
      o = __builtin_amdgcn_mfma_f32_32x32x16_f16(vshare[(kb * 2 + s) * 64 + lane],
                                                 acc_operand(st[kb], s, 1.0f), o, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; r++) o[r] *= inv;
  if (t < a.g.n) {
    uint16_t *op = a.out + ((long)w * a.g.n + t) * a.c + 32 * h + 4 * hf;
#pragma unroll
    for (int gq = 0; gq < 4; gq++) {
      uint16_t hv[4];
#pragma unroll
      for (int e = 0; e < 4; e++) hv[e] = f2h(o[4 * gq + e]);
      uint2 v;
      __builtin_memcpy(&v, hv, 8);
      *(uint2 *)(op + 8 * gq) = v;
    }
  }
}

template <int KB>
void *qkv_attention_kernel(int ks) {
  switch (ks) {
    case 2: return (void *)k_window_qkv_attention<KB, 2>;
    case 4: return (void *)k_window_qkv_attention<KB, 4>;
    case 6: return (void *)k_window_qkv_attention<KB, 6>;
    case 8: return (void *)k_window_qkv_attention<KB, 8>;
    case 12: return (void *)k_window_qkv_attention<KB, 12>;
    default: return (void *)k_window_qkv_attention<KB, 16>;
  }
}

}  // namespace

// Up to 256 channels.  Wider blocks (BiRefNet stages 3 and 4: 36 and 9
// windows) keep the unfused launches: with the rows read three times and
// one head a workgroup, the pass took 54 and 57 us per block at 1024 x 1024
// against 31 and 28 us for the gather, q k v product and attention.
bool window_qkv_attention_supported(int c, int window) {
  const int n = window * window, np = (n + 31) / 32 * 32;
  return c >= 32 && c <= 256 && c % 32 == 0 && (np == 64 || np == 160);
}

ien_status window_qkv_attention(ien_ctx *ctx, const ien_windows *win, const uint16_t *d_map,
                                size_t stride, int c, const float *gamma, const float *beta,
                                const ien_matrix *qkv, const float *d_tables, uint16_t *d_out) {
  IEN_CHECK(ctx && win && d_map && gamma && beta && qkv && d_tables && d_out, IEN_ERR_INPUT,
            "null argument");
  WinGeo g;
  ien_status st = geometry(win, &g);
  if (st != IEN_OK) return st;
  IEN_CHECK(window_qkv_attention_supported(c, g.window), IEN_ERR_INPUT,
            "%d channels, window %d", c, g.window);
  IEN_CHECK(stride >= (size_t)c && stride % 8 == 0 && aligned16(d_map) && aligned16(gamma) &&
                aligned16(beta) && ((uintptr_t)d_out & 7) == 0,
            IEN_ERR_INPUT, "map stride %zu / alignment", stride);
  IEN_CHECK(qkv->k == (size_t)c && qkv->n == 3 * (size_t)c && qkv->kb == c / 16 &&
                qkv->nb >= 3 * c / 32,
            IEN_ERR_INPUT, "qkv weights %zu x %zu for %d channels", qkv->k, qkv->n, c);
  const long tokens = (long)g.height * g.width;
  IEN_CHECK(tokens * (long)stride < (1L << 31) && g.windows * g.n * (long)c < (1L << 31),
            IEN_ERR_INPUT, "map of %ld tokens", tokens);
  const int heads = c / 32;
  const long blocks = g.windows * heads;
  IEN_CHECK(blocks < (1L << 31), IEN_ERR_INPUT, "%ld windows x heads", blocks);
  QkvAttnArgs a{g, d_map, (long)stride, c, heads, gamma, beta, qkv->d_packed, qkv->d_bias,
                d_tables, d_out};
  const int kb = (g.n + 31) / 32;
  void *k = kb == 2 ? qkv_attention_kernel<2>(c / 16) : qkv_attention_kernel<5>(c / 16);
  hipLaunchKernelGGL((void (*)(QkvAttnArgs))k, dim3((unsigned)blocks), dim3(64 * kb), 0,
                     ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace ien
