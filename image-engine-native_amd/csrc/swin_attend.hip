// swin_attend.hip -- the attention half of a Swin block in one pass per
// window (crates/scunet-native/src/swin.rs:131-232 Transformer::attend):
// gather of the rolled window, LayerNorm, q k v, attention with the
// position bias and shift mask, projection and residual, written back to
// the window's own tokens.  Window 8 (64 tokens), c = 32, 64 or 128
// (heads of 32).
//
// Everything between the load of x and the store stays in registers (but
// for the exchange of head outputs):
//  - x is loaded as MFMA fragments (lane l: token l % 32 of a 32-token
//    block, channels 16 s + 8 (l / 32) + 0..7) and normalised in place;
//    those registers are both the B operand of K^T = Wk^T x^T, Q^T = Wq^T
//    x^T and the A operand of V = x Wv (v_mfma_f32_32x32x16_f16).  The
//    packed qkv weights serve as A (for W^T) and B fragments unchanged.
//  - An accumulator tile holds row 8 (r / 4) + 4 (l / 32) + r % 4 in
//    register r and column l % 32.  Read in pairs of registers 8 s .. 8 s
//    + 7 it is an operand whose 16-wide k step holds rows 16 s + 4 (l / 32)
//    + {0..3, 8..11}: a fixed permutation of that step's k.  K^T and Q^T
//    tiles are then the A and B operands of S^T = K Q^T (same dims on both
//    sides), V and S^T tiles those of O^T = V^T P^T (same keys), and O^T
//    the B operand of Y^T = Wp^T O^T, whose A fragments are packed on the
//    host with the head dims in that permuted order.
//  - S^T has keys in rows and queries in columns: the softmax over keys is
//    in-register plus one exchange with lane l ^ 32.  The bias tables
//    (position bias plus the shift mask of the window's class) are packed
//    on the host in the accumulator layout, so a lane reads 16-byte runs.
//  - Y^T's rows are output channels: the residual is read and the result
//    written 4 channels (8 bytes) at a time per token.
// Rounding points are the unfused path's: normalised x, q, k, v, the
// probabilities and the attention output are f16; products accumulate in
// f32; the result is rounded once after bias and residual.
// One wave per window and head of 32 dims; with several heads the waves of
// a window exchange their outputs through LDS before the projection.
//
// At c = 32 the block's MLP half (swin.rs:236-275) can follow in the same
// wave: the result rounded to f16 (as the map would hold it) is
// normalised per token (each lane holds 16 of its token's channels, the
// lane l ^ 32 the other 16), and its registers are the permuted-k B
// operand of H^T = W1^T x^T.  The fc1 accumulators, GELU'd and rounded to
// f16, are in turn the permuted-k B operand of Z^T = W2^T H^T; both A
// operands are packed on the host in those permuted orders.  The MLP is
// per token and every token of the map lies in one window, so the fused
// order gives the separate passes' results.

#include "conv_common.h"
#include "window_geo.h"

namespace ien {
namespace {

struct AttendArgs {
  WinGeo g;
  uint16_t *map;
  long stride;
  const float *gamma, *beta;  // LayerNorm 1 (c each, 16-byte aligned)
  const uint16_t *wqkv;       // packed fragments of the c x 3c qkv weights
  const float *bqkv;          // 3c
  const uint16_t *wproj;      // Wp^T A fragments [c / 32][heads][2][512]
  const float *bproj;         // c
  const float *bias;          // [class][head][query block][key block][4][64][4]
  // The MLP half (c = 32): LayerNorm 2, permuted fc1 / fc2 A fragments
  // [4 unit blocks][2 k steps][64 lanes][8], biases (4c, c).
  const float *gamma2, *beta2;
  const uint16_t *w1, *w2;
  const float *b1, *b2;
};

__device__ __forceinline__ half8 frag(const uint16_t *p, int idx, int lane) {
  return *(const half8 *)(p + (size_t)idx * 512 + lane * 8);
}

// Registers 8 s .. 8 s + 7 of an accumulator tile (+ per-register add) as
// an f16 operand.
__device__ __forceinline__ half8 operand(const floatx16 &t, int s, float scale) {
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; i++) h[i] = (_Float16)(t[8 * s + i] * scale);
  return h;
}

// x of window w's 64 tokens as normalised fragments (LayerNorm: mean, then
// the mean square deviation, eps 1e-5: math.rs:95-116); tokens past the
// map's edge are zero rows.
template <int C>
__device__ __forceinline__ void load_norm(const AttendArgs &a, const long (&src)[2],
                                          half8 (&xn)[2][C / 16]) {
  constexpr int KS = C / 16;
  const int hf = (threadIdx.x & 63) >> 5;
  u32x4 xr[2][KS];
#pragma unroll
  for (int tb = 0; tb < 2; tb++)
#pragma unroll
    for (int s = 0; s < KS; s++)
      xr[tb][s] = *(const u32x4 *)(a.map + (src[tb] < 0 ? 0 : src[tb]) * a.stride + 16 * s + 8 * hf);
#pragma unroll
  for (int tb = 0; tb < 2; tb++) {
    float v[KS][8];
    float sum = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      uint16_t h[8];
      __builtin_memcpy(h, &xr[tb][s], 16);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        v[s][e] = h2f(h[e]);
        sum += v[s][e];
      }
    }
    sum += __shfl_xor(sum, 32);
    const float mean = sum / (float)C;
    float sq = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = v[s][e] - mean;
        sq += d * d;
      }
    sq += __shfl_xor(sq, 32);
    const float inv = 1.0f / sqrtf(sq / (float)C + 1e-5f);
    const float keep = src[tb] < 0 ? 0.0f : 1.0f;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const float4 g0 = *(const float4 *)(a.gamma + 16 * s + 8 * hf);
      const float4 g1 = *(const float4 *)(a.gamma + 16 * s + 8 * hf + 4);
      const float4 b0 = *(const float4 *)(a.beta + 16 * s + 8 * hf);
      const float4 b1 = *(const float4 *)(a.beta + 16 * s + 8 * hf + 4);
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int e = 0; e < 8; e++)
        xn[tb][s][e] = (_Float16)(((v[s][e] - mean) * inv * gg[e] + bb[e]) * keep);
    }
  }
}

// Head h of the window: q, k, v of all 64 tokens, S^T, softmax, O^T; the
// result as the B operands of the projection, ob[query block][k step]
// (head dims 16 s + 4 hf + {0..3, 8..11}).
template <int C>
__device__ __forceinline__ void head_attention(const AttendArgs &a, const half8 (&xn)[2][C / 16],
                                               int cls, int h, half8 (&ob)[2][2]) {
  constexpr int H = C / 32, KS = C / 16, CB = C / 32;
  const int lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
  const float scale = 0.17677669529663688f;  // 1 / sqrt(32)
  // K and V first, then Q: fewer accumulators live at once.
  half8 ka[2][2], qo[2][2], va[2][2];
  {
    floatx16 kt[2] = {}, vv[2] = {};
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const half8 wk = frag(a.wqkv, (CB + h) * KS + s, lane);
      const half8 wv = frag(a.wqkv, (2 * CB + h) * KS + s, lane);
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        kt[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wk, xn[tb][s], kt[tb], 0, 0, 0);
        vv[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xn[tb][s], wv, vv[tb], 0, 0, 0);
      }
    }
    // Biases: K^T rows are dims 8 (r / 4) + 4 hf + r % 4; V columns are
    // dims l32.
    const float bv = a.bqkv[2 * C + 32 * h + l32];
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
      const float4 bk = *(const float4 *)(a.bqkv + C + 32 * h + 8 * q4 + 4 * hf);
      const float bka[4] = {bk.x, bk.y, bk.z, bk.w};
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
          kt[tb][4 * q4 + e] += bka[e];
          vv[tb][4 * q4 + e] += bv;
        }
    }
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        ka[tb][s] = operand(kt[tb], s, 1.0f);
        va[tb][s] = operand(vv[tb], s, 1.0f);
      }
  }
  {
    floatx16 qt[2] = {};
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const half8 wq = frag(a.wqkv, h * KS + s, lane);
#pragma unroll
      for (int tb = 0; tb < 2; tb++)
        qt[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq, xn[tb][s], qt[tb], 0, 0, 0);
    }
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
      const float4 bq = *(const float4 *)(a.bqkv + 32 * h + 8 * q4 + 4 * hf);
      const float bqa[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int tb = 0; tb < 2; tb++) qt[tb][4 * q4 + e] += bqa[e];
    }
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int tb = 0; tb < 2; tb++) qo[tb][s] = operand(qt[tb], s, 1.0f);
  }
  const float *tbl = a.bias + (size_t)(cls * H + h) * 4 * 4 * 256;
#pragma unroll
  for (int qb = 0; qb < 2; qb++) {
    floatx16 st[2];
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kb][0], qo[qb][0], floatx16{}, 0, 0, 0);
      st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kb][1], qo[qb][1], st[kb], 0, 0, 0);
      const float *tq = tbl + ((qb * 2 + kb) * 4) * 256 + lane * 4;
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const float4 bt = *(const float4 *)(tq + q4 * 256);
        const float bta[4] = {bt.x, bt.y, bt.z, bt.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float v = st[kb][4 * q4 + e] * scale + bta[e];
          st[kb][4 * q4 + e] = v;
          mx = fmaxf(mx, v);
        }
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float p = __expf(st[kb][r] - mx);
        st[kb][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 32);
    const float inv = 1.0f / sum;
    floatx16 o = {};
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int s = 0; s < 2; s++)
        o = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[kb][s], operand(st[kb], s, inv), o, 0, 0, 0);
    ob[qb][0] = operand(o, 0, 1.0f);
    ob[qb][1] = operand(o, 1, 1.0f);
  }
}

// One wave per window and head (H = c / 32 waves per window, 4 / H windows
// per workgroup).  With several heads the waves of a window leave their
// heads' outputs in LDS (as the operands they are), meet at a barrier, and
// wave h projects all heads onto output channels 32 h .. 32 h + 31; the
// barrier also orders every read of the window before the first write.
template <int C, bool MLP>
__global__ __launch_bounds__(256, C <= 64 ? 2 : 1) void k_swin_attend(AttendArgs a) {
  static_assert(!MLP || C == 32, "the fused MLP takes one head");
  constexpr int H = C / 32, KS = C / 16, WPG = 4 / H;
  __shared__ half8 xo[H > 1 ? WPG * 2 * H * 2 * 64 : 1];  // [window][query block][head][s][lane]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  const int wl = wave / H, h = wave % H;
  const long wr = (long)blockIdx.x * WPG + wl;
  const bool live = wr < a.g.windows;
  const long w = live ? wr : a.g.windows - 1;
  long src[2];
#pragma unroll
  for (int tb = 0; tb < 2; tb++) src[tb] = win_source(a.g, w, 32 * tb + l32);
  half8 xn[2][KS];
  load_norm<C>(a, src, xn);
  half8 ob[2][2];
  head_attention<C>(a, xn, win_class(a.g, w), h, ob);

  // Y^T (output channels 32 h + rows, tokens of query block qb).
  floatx16 y[2] = {};
  if constexpr (H == 1) {
#pragma unroll
    for (int qb = 0; qb < 2; qb++)
#pragma unroll
      for (int s = 0; s < 2; s++)
        y[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag(a.wproj, s, lane), ob[qb][s], y[qb], 0, 0, 0);
  } else {
#pragma unroll
    for (int qb = 0; qb < 2; qb++)
#pragma unroll
      for (int s = 0; s < 2; s++) xo[(((wl * 2 + qb) * H + h) * 2 + s) * 64 + lane] = ob[qb][s];
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < H; hh++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const half8 wp = frag(a.wproj, (h * H + hh) * 2 + s, lane);
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
          y[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              wp, xo[(((wl * 2 + qb) * H + hh) * 2 + s) * 64 + lane], y[qb], 0, 0, 0);
      }
  }

  if constexpr (MLP) {
    // x1 = the attention half's result, rounded as the map would hold it.
    float x1[2][16];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      const long t = src[qb];
      const bool real = live && t >= 0;
      const uint16_t *row = a.map + (real ? t : 0) * a.stride;
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const int ch = 8 * q4 + 4 * hf;
        const float4 bp = *(const float4 *)(a.bproj + ch);
        const float bpa[4] = {bp.x, bp.y, bp.z, bp.w};
        const uint2 old = real ? *(const uint2 *)(row + ch) : uint2{0u, 0u};
        uint16_t hv[4];
        __builtin_memcpy(hv, &old, 8);
#pragma unroll
        for (int e = 0; e < 4; e++) x1[qb][4 * q4 + e] = h2f(f2h(y[qb][4 * q4 + e] + bpa[e] + h2f(hv[e])));
      }
    }
    // LayerNorm 2 per token; register 8 s + i is channel 16 s + 4 hf +
    // (i & 3) + 8 (i >> 2): the permuted-k operand of fc1.
    half8 xn[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      float sum = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r++) sum += x1[qb][r];
      sum += __shfl_xor(sum, 32);
      const float mean = sum / 32.0f;
      float sq = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float d = x1[qb][r] - mean;
        sq += d * d;
      }
      sq += __shfl_xor(sq, 32);
      const float inv = 1.0f / sqrtf(sq / 32.0f + 1e-5f);
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const int ch = 8 * q4 + 4 * hf;
        const float4 g = *(const float4 *)(a.gamma2 + ch);
        const float4 b = *(const float4 *)(a.beta2 + ch);
        const float ga[4] = {g.x, g.y, g.z, g.w}, ba[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int r = 4 * q4 + e;
          xn[qb][r >> 3][r & 7] = (_Float16)((x1[qb][r] - mean) * inv * ga[e] + ba[e]);
        }
      }
    }
    // fc1 + GELU + fc2, 32 hidden units at a time.
    floatx16 z[2] = {};
#pragma unroll
    for (int ub = 0; ub < 4; ub++) {
      floatx16 hacc[2] = {};
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const half8 w1 = frag(a.w1, ub * 2 + s, lane);
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
          hacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, xn[qb][s], hacc[qb], 0, 0, 0);
      }
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const float4 bu = *(const float4 *)(a.b1 + 32 * ub + 8 * q4 + 4 * hf);
        const float bua[4] = {bu.x, bu.y, bu.z, bu.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int qb = 0; qb < 2; qb++)
            hacc[qb][4 * q4 + e] = gelu_f(hacc[qb][4 * q4 + e] + bua[e]);
      }
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const half8 w2 = frag(a.w2, ub * 2 + s, lane);
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
          z[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w2, operand(hacc[qb], s, 1.0f), z[qb], 0, 0, 0);
      }
    }
    // x1 + fc2 + bias, rounded once.
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      const long t = src[qb];
      if (!live || t < 0) continue;
      uint16_t *row = a.map + t * a.stride;
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const int ch = 8 * q4 + 4 * hf;
        const float4 bz = *(const float4 *)(a.b2 + ch);
        const float bza[4] = {bz.x, bz.y, bz.z, bz.w};
        uint16_t hv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) hv[e] = f2h(x1[qb][4 * q4 + e] + (z[qb][4 * q4 + e] + bza[e]));
        uint2 o;
        __builtin_memcpy(&o, hv, 8);
        *(uint2 *)(row + ch) = o;
      }
    }
    return;
  }

  // Bias, old token, rounded once; rows of Y^T are output channels.
#pragma unroll
  for (int qb = 0; qb < 2; qb++) {
    const long t = src[qb];
    if (!live || t < 0) continue;
    uint16_t *row = a.map + t * a.stride;
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
      const int ch = 32 * h + 8 * q4 + 4 * hf;
      const float4 bp = *(const float4 *)(a.bproj + ch);
      const float bpa[4] = {bp.x, bp.y, bp.z, bp.w};
      uint2 old = *(const uint2 *)(row + ch);
      uint16_t hv[4];
      __builtin_memcpy(hv, &old, 8);
#pragma unroll
      for (int e = 0; e < 4; e++) hv[e] = f2h(y[qb][4 * q4 + e] + bpa[e] + h2f(hv[e]));
      __builtin_memcpy(&old, hv, 8);
      *(uint2 *)(row + ch) = old;
    }
  }
}

template <int C, bool MLP = false>
ien_status launch(ien_ctx *ctx, const AttendArgs &a) {
  constexpr int WPG = 4 / (C / 32);
  const long blocks = (a.g.windows + WPG - 1) / WPG;
  IEN_CHECK(blocks < (1L << 31), IEN_ERR_INPUT, "%ld windows", a.g.windows);
  hipLaunchKernelGGL((k_swin_attend<C, MLP>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace

bool swin_attend_supported(int c, int window) {
  return window == 8 && (c == 32 || c == 64 || c == 128);
}

std::vector<uint16_t> swin_attend_proj(const float *proj_w, int c) {
  // Fragment (cb, head, s): lane l, slot i -> output channel 32 cb + l % 32,
  // head dim 16 s + 4 (l / 32) + (i & 3) + 8 (i >> 2).
  const int heads = c / 32;
  std::vector<uint16_t> out((size_t)c * c);
  for (int cb = 0; cb < c / 32; cb++)
    for (int h = 0; h < heads; h++)
      for (int s = 0; s < 2; s++)
        for (int l = 0; l < 64; l++)
          for (int i = 0; i < 8; i++) {
            const int o = 32 * cb + l % 32;
            const int j = 32 * h + 16 * s + 4 * (l / 32) + (i & 3) + 8 * (i >> 2);
            out[(((size_t)(cb * heads + h) * 2 + s) * 64 + l) * 8 + i] =
                f32_to_half(proj_w[(size_t)j * c + o]);
          }
  return out;
}

std::vector<uint16_t> swin_attend_mlp(const float *fc1_w, const float *fc2_w) {
  // c = 32.  fc1 fragment (ub, s): lane l, slot i -> hidden unit 32 ub + l % 32,
  // channel 16 s + 4 (l / 32) + (i & 3) + 8 (i >> 2); then fc2 fragment
  // (ub, s): output channel l % 32, unit 32 ub + 16 s + 4 (l / 32) + (i & 3)
  // + 8 (i >> 2).
  constexpr int c = 32, units = 4 * c;
  std::vector<uint16_t> out((size_t)2 * 8 * 512);
  for (int ub = 0; ub < 4; ub++)
    for (int s = 0; s < 2; s++)
      for (int l = 0; l < 64; l++)
        for (int i = 0; i < 8; i++) {
          const int perm = 16 * s + 4 * (l / 32) + (i & 3) + 8 * (i >> 2);
          const size_t at = (((size_t)(ub * 2 + s)) * 64 + l) * 8 + i;
          const int unit1 = 32 * ub + l % 32, ch1 = perm;
          out[at] = f32_to_half(fc1_w[(size_t)ch1 * units + unit1]);
          const int ch2 = l % 32, unit2 = 32 * ub + perm;
          out[8 * 512 + at] = f32_to_half(fc2_w[(size_t)unit2 * c + ch2]);
        }
  return out;
}

ien_status swin_attend(ien_ctx *ctx, const ien_windows *win, uint16_t *d_map, size_t stride,
                       int c, const float *gamma, const float *beta, const ien_matrix *qkv,
                       const uint16_t *d_proj, const float *bproj, const float *d_tables,
                       const AttendMlp *mlp) {
  IEN_CHECK(ctx && win && d_map && gamma && beta && qkv && d_proj && bproj && d_tables,
            IEN_ERR_INPUT, "null argument");
  WinGeo g;
  ien_status st = geometry(win, &g);
  if (st != IEN_OK) return st;
  IEN_CHECK(swin_attend_supported(c, g.window), IEN_ERR_INPUT, "%d channels, window %d", c,
            g.window);
  IEN_CHECK(stride >= (size_t)c && stride % 8 == 0 && aligned16(d_map) && aligned16(gamma) &&
                aligned16(beta),
            IEN_ERR_INPUT, "map stride %zu / alignment", stride);
  IEN_CHECK(qkv->k == (size_t)c && qkv->n == 3 * (size_t)c && qkv->kb == c / 16, IEN_ERR_INPUT,
            "qkv weights %zu x %zu for %d channels", qkv->k, qkv->n, c);
  AttendArgs a{g,      d_map,   (long)stride, gamma,   beta,    qkv->d_packed, qkv->d_bias,
               d_proj, bproj,   d_tables,     nullptr, nullptr, nullptr,       nullptr,
               nullptr, nullptr};
  if (mlp) {
    IEN_CHECK(c == 32 && mlp->gamma && mlp->beta && mlp->w && mlp->b1 && mlp->b2 &&
                  aligned16(mlp->gamma) && aligned16(mlp->beta) && aligned16(mlp->b1) &&
                  aligned16(mlp->b2),
              IEN_ERR_INPUT, "fused MLP: 32 channels, aligned parameters");
    a.gamma2 = mlp->gamma;
    a.beta2 = mlp->beta;
    a.w1 = mlp->w;
    a.w2 = mlp->w + 8 * 512;
    a.b1 = mlp->b1;
    a.b2 = mlp->b2;
    return launch<32, true>(ctx, a);
  }
  switch (c) {
    case 32: return launch<32>(ctx, a);
    case 64: return launch<64>(ctx, a);
    default: return launch<128>(ctx, a);
  }
}

}  // namespace ien
