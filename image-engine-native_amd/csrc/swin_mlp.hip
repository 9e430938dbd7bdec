// swin_mlp.hip -- the Swin block's MLP half in one pass over the token rows
// (crates/scunet-native/src/swin.rs:236-275, crates/birefnet-native/src/
// swin.rs Mlp): x += fc2(GELU(fc1(LayerNorm(x)))), for c = 32, 64 and 96.
//
// One workgroup of 4 waves per 64 token rows:
//  - LayerNorm (mean, then the mean square deviation, eps 1e-5: math.rs:
//    95-116) of the 64 rows into LDS as f16, the A operand of fc1.
//  - The hidden layer in chunks of 128 units: wave w computes the chunk's
//    32 units 32 w .. 32 w + 31 for all 64 rows (fc1 on v_mfma_f32_32x32x16
//    _f16, B fragments straight from the packed weights), adds the bias,
//    applies GELU and writes the chunk to LDS as f16 (double-buffered: one
//    barrier per chunk).  The chunk is then the A operand of fc2, whose
//    64 x c output stays in accumulators across all chunks.
//  - fc2's bias, then the old row, rounded once to f16 and stored in place
//    (the order of gemm.rs:583-666 with accumulate), through an f32 staging
//    tile so that every global access is a 16-byte vector.
// The rounding points are the unfused path's: the normalised rows and the
// GELU outputs are f16, every product accumulates in f32.  Rows past the
// end are computed from a clamped copy of the last row and never stored.

#include "conv_common.h"

namespace ien {
namespace {

constexpr int MLP_ROWS = 64;   // token rows per workgroup
constexpr int MLP_CHUNK = 128; // hidden units per chunk

struct MlpArgs {
  uint16_t *map;  // row r at map + r stride, c channels, updated in place
  long stride;
  long rows;
  const float *gamma, *beta;        // LayerNorm (c each, 16-byte aligned)
  const uint16_t *w1, *w2;          // packed fragments: c x 4c, 4c x c
  int kb1, kb2;                     // k fragments of w1, w2
  const float *b1, *b2;
};

template <int C>
struct Mlp {
  static constexpr int XP = C + 8;                  // halves per normalised row
  static constexpr int HP = MLP_CHUNK + 8;          // halves per hidden row
  static constexpr int CHUNKS = 4 * C / MLP_CHUNK;  // = C / 32
  static constexpr int KS1 = C / 16;                // fc1 k steps
  static constexpr int KS2 = MLP_CHUNK / 16;        // fc2 k steps per chunk
  static constexpr int TILES = 2 * (C / 32);        // 32 x 32 output tiles
  static constexpr int TW = (TILES + 3) / 4;        // output tiles per wave
  static constexpr int L = C / 8 <= 4 ? 4 : C / 8 <= 8 ? 8 : C / 8 <= 16 ? 16 : 32;  // LN lanes per row
  static constexpr int PASSES = MLP_ROWS * L / 256;
  static constexpr int X_HALVES = MLP_ROWS * XP;
  static constexpr int H_HALVES = 2 * MLP_ROWS * HP;
  static constexpr int STAGE_FLOATS = MLP_ROWS * C;
  static constexpr size_t LDS_BYTES =
      (size_t)(X_HALVES + H_HALVES) * 2 > (size_t)STAGE_FLOATS * 4 ? (size_t)(X_HALVES + H_HALVES) * 2
                                                                   : (size_t)STAGE_FLOATS * 4;
  static_assert(C % 32 == 0 && C >= 32 && C <= 256, "c");
};

template <int C>
__global__ __launch_bounds__(256) void k_swin_mlp(MlpArgs a) {
  using S = Mlp<C>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[S::LDS_BYTES];
  uint16_t *xa = (uint16_t *)lds;
  uint16_t *hb = xa + S::X_HALVES;
  float *stage = (float *)lds;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  const long row0 = (long)blockIdx.x * MLP_ROWS;
  const long last = a.rows - 1;

  // LayerNorm: L lanes per row, one 8-channel chunk per lane.  When every
  // lane holds a chunk (L = c / 8), thread tid's chunk of pass p is its
  // output item p, so the rows stay in registers for the residual.
  constexpr bool KEEP = S::L == C / 8;
  u32x4 raw[S::PASSES];
  {
    const int sub = tid & (S::L - 1), chunks = C / 8;
    const int k = sub < chunks ? sub : chunks - 1;
#pragma unroll
    for (int p = 0; p < S::PASSES; p++) {
      const long r = min(row0 + p * (256 / S::L) + tid / S::L, last);
      raw[p] = *(const u32x4 *)(a.map + r * a.stride + 8 * k);
    }
    const float4 g0 = *(const float4 *)(a.gamma + 8 * k), g1 = *(const float4 *)(a.gamma + 8 * k + 4);
    const float4 e0 = *(const float4 *)(a.beta + 8 * k), e1 = *(const float4 *)(a.beta + 8 * k + 4);
    const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float bb[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
#pragma unroll
    for (int p = 0; p < S::PASSES; p++) {
      uint16_t h[8];
      __builtin_memcpy(h, &raw[p], 16);
      float v[8];
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        v[e] = h2f(h[e]);
        sum += v[e];
      }
      if (sub >= chunks) sum = 0.0f;
#pragma unroll
      for (int off = S::L / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      const float mean = sum / (float)C;
      float sq = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = v[e] - mean;
        sq += d * d;
      }
      if (sub >= chunks) sq = 0.0f;
#pragma unroll
      for (int off = S::L / 2; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
      const float inv = 1.0f / sqrtf(sq / (float)C + 1e-5f);
      if (sub < chunks) {
        uint16_t o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = f2h((v[e] - mean) * inv * gg[e] + bb[e]);
        const int r = p * (256 / S::L) + tid / S::L;
        __builtin_memcpy(xa + r * S::XP + 8 * k, o, 16);
      }
    }
  }
  __syncthreads();

  // Output tiles of this wave: t = wave + 4 j, rows 32 (t % 2), channels
  // 32 (t / 2); t % 2 = wave % 2 for every j.
  const int rb = wave & 1;
  floatx16 z[S::TW];
#pragma unroll
  for (int j = 0; j < S::TW; j++) z[j] = floatx16{};

  for (int ch = 0; ch < S::CHUNKS; ch++) {
    // fc1: the chunk's units 32 wave .. + 31 for rows 0..63.
    half8 w1f[S::KS1];
    const uint16_t *w1 = a.w1 + ((size_t)(ch * 4 + wave) * a.kb1) * 512 + lane * 8;
#pragma unroll
    for (int s = 0; s < S::KS1; s++) w1f[s] = *(const half8 *)(w1 + s * 512);
    floatx16 h0 = {}, h1 = {};
#pragma unroll
    for (int s = 0; s < S::KS1; s++) {
      const half8 x0 = *(const half8 *)(xa + l32 * S::XP + 16 * s + 8 * hf);
      const half8 x1 = *(const half8 *)(xa + (32 + l32) * S::XP + 16 * s + 8 * hf);
      h0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0, w1f[s], h0, 0, 0, 0);
      h1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1, w1f[s], h1, 0, 0, 0);
    }
    // fc2's fragments for this chunk, in flight during the GELU.
    half8 w2f[S::TW][S::KS2];
#pragma unroll
    for (int j = 0; j < S::TW; j++) {
      const int t = wave + 4 * j;
      const int cb = t < S::TILES ? t >> 1 : 0;
      const uint16_t *w2 = a.w2 + ((size_t)cb * a.kb2 + ch * S::KS2) * 512 + lane * 8;
#pragma unroll
      for (int s = 0; s < S::KS2; s++) w2f[j][s] = *(const half8 *)(w2 + s * 512);
    }
    const int unit = ch * MLP_CHUNK + wave * 32 + l32;
    const float bias1 = a.b1[unit];
    uint16_t *hbuf = hb + (ch & 1) * MLP_ROWS * S::HP;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = 8 * (r >> 2) + 4 * hf + (r & 3);
      hbuf[row * S::HP + wave * 32 + l32] = f2h(gelu_f(h0[r] + bias1));
      hbuf[(32 + row) * S::HP + wave * 32 + l32] = f2h(gelu_f(h1[r] + bias1));
    }
    __syncthreads();
    // fc2: rows 32 rb .. + 31 of the chunk against this wave's tiles.
#pragma unroll
    for (int s = 0; s < S::KS2; s++) {
      const half8 hx = *(const half8 *)(hbuf + (32 * rb + l32) * S::HP + 16 * s + 8 * hf);
#pragma unroll
      for (int j = 0; j < S::TW; j++)
        if (wave + 4 * j < S::TILES) z[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hx, w2f[j][s], z[j], 0, 0, 0);
    }
  }
  __syncthreads();  // every read of the normalised rows and hidden chunks done

  // Stage acc + bias as f32 rows, then old row + it, rounded once.
#pragma unroll
  for (int j = 0; j < S::TW; j++) {
    const int t = wave + 4 * j;
    if (t < S::TILES) {
      const int col = (t >> 1) * 32 + l32;
      const float bias2 = a.b2[col];
#pragma unroll
      for (int r = 0; r < 16; r++)
        stage[(32 * rb + 8 * (r >> 2) + 4 * hf + (r & 3)) * C + col] = z[j][r] + bias2;
    }
  }
  __syncthreads();
  constexpr int ITEMS = MLP_ROWS * C / 8 / 256;  // 16-byte items per thread
  u32x4 old[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; i++) {
    const int item = tid + 256 * i, r = item / (C / 8), k = item % (C / 8);
    if constexpr (KEEP)
      old[i] = raw[i];
    else
      old[i] = *(const u32x4 *)(a.map + min(row0 + r, last) * a.stride + 8 * k);
  }
#pragma unroll
  for (int i = 0; i < ITEMS; i++) {
    const int item = tid + 256 * i, r = item / (C / 8), k = item % (C / 8);
    if (row0 + r > last) continue;
    const float4v s0 = *(const float4v *)(stage + r * C + 8 * k);
    const float4v s1 = *(const float4v *)(stage + r * C + 8 * k + 4);
    uint16_t h[8];
    __builtin_memcpy(h, &old[i], 16);
    const float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = f2h(v[e] + h2f(h[e]));
    __builtin_memcpy(a.map + (row0 + r) * a.stride + 8 * k, h, 16);
  }
}

template <int C>
ien_status launch(ien_ctx *ctx, const MlpArgs &a) {
  const long blocks = (a.rows + MLP_ROWS - 1) / MLP_ROWS;
  hipLaunchKernelGGL(k_swin_mlp<C>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace

// Up to 96 channels: wider blocks have too few rows per token map at the
// networks' sizes to fill the chip with 64-row workgroups, and their
// weights no longer stay close; the row products serve them better.
bool swin_mlp_supported(int c) { return c == 32 || c == 64 || c == 96; }

ien_status swin_mlp(ien_ctx *ctx, uint16_t *d_map, size_t stride, long rows, int c,
                    const float *gamma, const float *beta, const ien_matrix *fc1,
                    const ien_matrix *fc2) {
  IEN_CHECK(ctx && d_map && gamma && beta && fc1 && fc2, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(swin_mlp_supported(c), IEN_ERR_INPUT, "%d channels", c);
  IEN_CHECK(rows > 0, IEN_ERR_INPUT, "%ld rows", rows);
  IEN_CHECK(stride >= (size_t)c && stride % 8 == 0 && ((uintptr_t)d_map & 15) == 0 &&
                ((uintptr_t)gamma & 15) == 0 && ((uintptr_t)beta & 15) == 0,
            IEN_ERR_INPUT, "map stride %zu / alignment", stride);
  IEN_CHECK(fc1->k == (size_t)c && fc1->n == 4 * (size_t)c && fc2->k == 4 * (size_t)c &&
                fc2->n == (size_t)c && fc1->kb == c / 16 && fc2->kb == c / 4 &&
                fc1->nb >= c / 8 && fc2->nb >= c / 32,
            IEN_ERR_INPUT, "mlp weights %zu x %zu, %zu x %zu for %d channels", fc1->k, fc1->n,
            fc2->k, fc2->n, c);
  MlpArgs a{d_map, (long)stride, rows, gamma, beta, fc1->d_packed, fc2->d_packed,
            fc1->kb, fc2->kb, fc1->d_bias, fc2->d_bias};
  switch (c) {
    case 32: return launch<32>(ctx, a);
    case 64: return launch<64>(ctx, a);
    default: return launch<96>(ctx, a);
  }
}

}  // namespace ien
