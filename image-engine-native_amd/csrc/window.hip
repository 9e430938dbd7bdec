// window.hip -- Swin window attention on gfx950: the rolled window gather
// with its LayerNorm, attention over every window and head on MFMA, the
// residual scatter, and the host-side position-bias and mask tables
// (crates/scunet-native/src/swin.rs, crates/birefnet-native/src/swin.rs,
// crates/native-engine/src/attention.rs).

#include "conv_common.h"
#include "lanes.h"
#include "window_geo.h"

namespace ien {
namespace {

__device__ __forceinline__ void unpack8(const u32x4 &raw, float *v) {
  uint16_t h[8];
  __builtin_memcpy(h, &raw, 16);
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = h2f(h[e]);
}

__device__ __forceinline__ u32x4 pack8(const float *v) {
  uint16_t h[8];
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = f2h(v[e]);
  u32x4 raw;
  __builtin_memcpy(&raw, h, 16);
  return raw;
}

// L lanes per window row (the row's 8-channel chunks rounded up to a power
// of two, at most 64), 64 / L rows per wave instruction, R such rows per
// lane group: gather, LayerNorm (mean, then the mean square deviation, eps
// 1e-5: math.rs:95-116), or a zero row past the edge.  A lane holds one
// 8-channel chunk, two when L = 64 and c > 512 (c <= 1024).  The R rows'
// loads and the lane's gamma and beta are all requested first; wave v's
// instruction j covers rows (R v + j) 64 / L .. + 64 / L - 1, whole runs of
// consecutive rows.  The reductions stay inside the row's aligned lane
// group (DPP moves up to 16 lanes); row and window arithmetic in 32 bits
// (the host checks the thread count).
template <int L, int R>
__global__ __launch_bounds__(256) void k_window_gather(WinGeo g, const uint16_t *__restrict__ map,
                                                       long stride, int c,
                                                       const float *__restrict__ gamma,
                                                       const float *__restrict__ beta,
                                                       uint16_t *__restrict__ tokens) {
  constexpr int Q = L == 64 ? 2 : 1, RPW = 64 / L;
  const int sub = threadIdx.x & (L - 1);
  const int wave = (int)((blockIdx.x * 256 + threadIdx.x) >> 6);
  const int row0 = wave * R * RPW + (int)((threadIdx.x & 63) / L);
  const int rows = (int)g.windows * g.n, chunks = c >> 3;
  int src[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int row = row0 + j * RPW;
    const int w = row / g.n;
    src[j] = row < rows ? win_source(g, w, row - w * g.n) : -1;
  }
  u32x4 raw[R][Q];
  float4 gb[4 * Q];
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int k = min(sub + L * q, chunks - 1);  // (lanes past the row repeat its last chunk)
#pragma unroll
    for (int j = 0; j < R; j++)
      if (src[j] >= 0) raw[j][q] = *(const u32x4 *)(map + (long)src[j] * stride + 8 * k);
    gb[4 * q] = *(const float4 *)(gamma + 8 * k);
    gb[4 * q + 1] = *(const float4 *)(gamma + 8 * k + 4);
    gb[4 * q + 2] = *(const float4 *)(beta + 8 * k);
    gb[4 * q + 3] = *(const float4 *)(beta + 8 * k + 4);
  }
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int row = row0 + j * RPW;
    if (row >= rows) continue;  // (whole lane groups)
    uint16_t *dst = tokens + (long)row * c;
    if (src[j] < 0) {
      const u32x4 zero = {0u, 0u, 0u, 0u};
      for (int k = sub; k < chunks; k += L) *(u32x4 *)(dst + 8 * k) = zero;
      continue;
    }
    float v[8 * Q];
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const int k = sub + L * q;
      if (k < chunks) {
        unpack8(raw[j][q], v + 8 * q);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[8 * q + e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; e++) sum += v[8 * q + e];
    }
    sum = group_sum<L>(sum);
    const float mean = sum / (float)c;
    float sq = 0.0f;
#pragma unroll
    for (int q = 0; q < Q; q++) {
      if (sub + L * q < chunks) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float d = v[8 * q + e] - mean;
          sq += d * d;
        }
      }
    }
    sq = group_sum<L>(sq);
    const float inv = 1.0f / sqrtf(sq / (float)c + 1e-5f);
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const int k = sub + L * q;
      if (k < chunks) {
        const float4 g0 = gb[4 * q], g1 = gb[4 * q + 1], b0 = gb[4 * q + 2], b1 = gb[4 * q + 3];
        const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (v[8 * q + e] - mean) * inv * gg[e] + bb[e];
        *(u32x4 *)(dst + 8 * k) = pack8(o);
      }
    }
  }
}

// Attention of one window and head per workgroup; wave q computes queries
// 32 q .. 32 q + 31 of the window (NP: the tokens rounded up to 32).
//  - S^T = K Q^T on v_mfma_f32_32x32x16_f16 (A: keys x dims, B: dims x
//    queries, both 16-byte loads of qkv rows), so lane l holds query l % 32
//    and, in register r of key block b, key 32 b + 8 (r / 4) + 4 (l / 32) +
//    r % 4: the softmax over keys is in-register plus one exchange with
//    lane l ^ 32.
//  - The probabilities (already divided by the sum) are the B operand of
//    O^T = V^T P^T as they lie: for the 16 keys of step (b, s) lane half h
//    holds keys 32 b + 16 s + 4 h + {0..3, 8..11}, and the A operand (V^T,
//    staged in LDS as [dim][key]) reads the same keys for its dim.
//  - Keys past N get -inf; V rows past N are zero in LDS.
//  - PACKED: the bias tables come in the accumulator layout of
//    pack_bias_tables (keys past N already -inf), read as 16-byte runs;
//    otherwise as [class][head][query][key] rows, a strided read per lane.
// Scores are (q . k) / sqrt(32) + bias, the reference's (q / sqrt(32)) . k
// up to rounding (attention.rs:66-111).
template <int NP, bool PACKED>
__global__ __launch_bounds__(NP * 2) void k_window_attention(WinGeo g, const uint16_t *__restrict__ qkv,
                                                             int c, int heads,
                                                             const float *__restrict__ tables,
                                                             uint16_t *__restrict__ out) {
  constexpr int KB = NP / 32;
  constexpr int PITCH = NP + 4;  // halves: 32 dims' rows on distinct banks
  __shared__ __attribute__((aligned(16))) uint16_t vt[32 * PITCH];
  const long w = blockIdx.x / heads;
  const int head = (int)(blockIdx.x - w * heads);
  const int n = g.n;
  const long row3 = 3L * c;
  const uint16_t *base = qkv + w * n * row3;

  // V^T: item (key j, 8-dim chunk q).
  for (int it = threadIdx.x; it < NP * 4; it += NP * 2) {
    const int j = it >> 2, q = it & 3;
    // Unconditional load from a row inside the window, zero past N.
    u32x4 raw = *(const u32x4 *)(base + min(j, n - 1) * row3 + 2 * c + head * 32 + 8 * q);
    if (j >= n) raw = u32x4{0u, 0u, 0u, 0u};
    uint16_t h[8];
    __builtin_memcpy(h, &raw, 16);
#pragma unroll
    for (int e = 0; e < 8; e++) vt[(8 * q + e) * PITCH + j] = h[e];
  }

  const int lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
  const int qi = (threadIdx.x >> 6) * 32 + l32;
  const int qc = qi < n ? qi : n - 1;
  const half8 q0 = *(const half8 *)(base + qc * row3 + head * 32 + 8 * hf);
  const half8 q1 = *(const half8 *)(base + qc * row3 + head * 32 + 16 + 8 * hf);
  floatx16 st[KB];
#pragma unroll
  for (int b = 0; b < KB; b++) {
    const int kj = min(32 * b + l32, n - 1);
    const half8 k0 = *(const half8 *)(base + kj * row3 + c + head * 32 + 8 * hf);
    const half8 k1 = *(const half8 *)(base + kj * row3 + c + head * 32 + 16 + 8 * hf);
    floatx16 z = {};
    z = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, q0, z, 0, 0, 0);
    st[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(k1, q1, z, 0, 0, 0);
  }

  const float scale = 0.17677669529663688f;  // 1 / sqrt(32)
  const int cls = win_class(g, w);
  float mx = -__builtin_inff();
  if constexpr (PACKED) {
    const float *tp = tables + ((long)(cls * heads + head) * KB + (threadIdx.x >> 6)) * KB * 1024 + lane * 4;
#pragma unroll
    for (int b = 0; b < KB; b++)
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const float4 bt = *(const float4 *)(tp + (b * 4 + q4) * 256);
        const float bta[4] = {bt.x, bt.y, bt.z, bt.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float s = st[b][4 * q4 + e] * scale + bta[e];
          st[b][4 * q4 + e] = s;
          mx = fmaxf(mx, s);
        }
      }
  } else {
    const float *tb = tables + ((long)(cls * heads + head) * n + qc) * n;
#pragma unroll
    for (int b = 0; b < KB; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int j = 32 * b + 8 * (r >> 2) + 4 * hf + (r & 3);
        const float bj = tb[min(j, n - 1)];  // in bounds for every j
        const float s = j < n ? st[b][r] * scale + bj : -__builtin_inff();
        st[b][r] = s;
        mx = fmaxf(mx, s);
      }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.0f;
#pragma unroll
  for (int b = 0; b < KB; b++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = __expf(st[b][r] - mx);
      st[b][r] = p;
      sum += p;
    }
  sum += __shfl_xor(sum, 32);
  const float inv = 1.0f / sum;

  __syncthreads();  // V^T staged
  floatx16 ot = {};
#pragma unroll
  for (int b = 0; b < KB; b++)
#pragma unroll
    for (int s = 0; s < 2; s++) {
      half8 pb;
#pragma unroll
      for (int e = 0; e < 8; e++) pb[e] = (_Float16)(st[b][8 * s + e] * inv);
      const int kb0 = 32 * b + 16 * s + 4 * hf;
      const uint2 lo = *(const uint2 *)(vt + l32 * PITCH + kb0);
      const uint2 hi = *(const uint2 *)(vt + l32 * PITCH + kb0 + 8);
      u32x4 raw = {lo.x, lo.y, hi.x, hi.y};
      half8 va;
      __builtin_memcpy(&va, &raw, 16);
      ot = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, ot, 0, 0, 0);
    }
  if (qi < n) {
    uint16_t *o = out + (w * n + qi) * (long)c + head * 32 + 4 * hf;
#pragma unroll
    for (int gq = 0; gq < 4; gq++) {
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; e++) h[e] = f2h(ot[4 * gq + e]);
      uint2 v;
      __builtin_memcpy(&v, h, 8);
      *(uint2 *)(o + 8 * gq) = v;
    }
  }
}

// One thread per 8-channel chunk of a window row: map[source] += row.
__global__ __launch_bounds__(256) void k_window_scatter_add(WinGeo g, const uint16_t *__restrict__ rows,
                                                            int c, uint16_t *__restrict__ map,
                                                            long stride) {
  const int chunks = c >> 3;
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  if (item >= g.windows * g.n * chunks) return;
  const long row = item / chunks;
  const int k = (int)(item - row * chunks);
  const long src = win_source(g, row / g.n, (int)(row % g.n));
  if (src < 0) return;
  float a[8], b[8];
  unpack8(*(const u32x4 *)(rows + row * c + 8 * k), a);
  uint16_t *m = map + src * stride + 8 * k;
  unpack8(*(const u32x4 *)m, b);
#pragma unroll
  for (int e = 0; e < 8; e++) b[e] += a[e];
  *(u32x4 *)m = pack8(b);
}


}  // namespace

namespace {

ien_status launch_attention(ien_ctx *ctx, const WinGeo &g, const uint16_t *d_qkv, int c,
                            const float *d_tables, bool packed, uint16_t *d_out) {
  const int heads = c / 32;
  const long blocks = g.windows * heads;
  IEN_CHECK(blocks < (1L << 31), IEN_ERR_INPUT, "%ld windows x heads", blocks);
  const int np = (g.n + 31) / 32 * 32;
  void (*k)(WinGeo, const uint16_t *, int, int, const float *, uint16_t *) = nullptr;
#define IEN_ATT(NP)                                                                \
  k = packed ? k_window_attention<NP, true> : k_window_attention<NP, false>;      \
  break
  switch (np) {
    case 32: IEN_ATT(32);
    case 64: IEN_ATT(64);
    case 96: IEN_ATT(96);
    case 128: IEN_ATT(128);
    case 160: IEN_ATT(160);
    case 192: IEN_ATT(192);
    case 224: IEN_ATT(224);
    default: IEN_ATT(256);
  }
#undef IEN_ATT
  hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(np * 2), 0, ctx->stream, g, d_qkv, c, heads,
                     d_tables, d_out);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // namespace

std::vector<float> pack_bias_tables(const float *tables, int classes, int heads, int n) {
  // [class][head][query block][key block][q4][lane][e] = table[query
  // 32 qb + lane % 32][key 32 kb + 8 q4 + 4 (lane / 32) + e]; keys past n
  // are -inf, queries past n 0.
  const int kbs = (n + 31) / 32;
  std::vector<float> out((size_t)classes * heads * kbs * kbs * 1024);
  for (int cls = 0; cls < classes; cls++)
    for (int h = 0; h < heads; h++) {
      const float *t = tables + (size_t)(cls * heads + h) * n * n;
      for (int qb = 0; qb < kbs; qb++)
        for (int kb = 0; kb < kbs; kb++)
          for (int q4 = 0; q4 < 4; q4++)
            for (int l = 0; l < 64; l++)
              for (int e = 0; e < 4; e++) {
                const int i = 32 * qb + l % 32, j = 32 * kb + 8 * q4 + 4 * (l / 32) + e;
                const float v = j >= n ? -__builtin_inff() : i >= n ? 0.0f : t[(size_t)i * n + j];
                out[((((size_t)(cls * heads + h) * kbs + qb) * kbs + kb) * 4 + q4) * 256 + l * 4 + e] = v;
              }
    }
  return out;
}

ien_status window_attention(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_qkv, int c,
                            const float *d_tables, bool packed, uint16_t *d_out) {
  IEN_CHECK(ctx && d_qkv && d_tables && d_out, IEN_ERR_INPUT, "null argument");
  WinGeo g;
  ien_status st = geometry(w, &g);
  if (st != IEN_OK) return st;
  IEN_CHECK(c >= 32 && c % 32 == 0, IEN_ERR_INPUT, "%d channels (heads of 32)", c);
  IEN_CHECK(aligned16(d_qkv) && ((uintptr_t)d_out & 7) == 0, IEN_ERR_INPUT, "alignment");
  return launch_attention(ctx, g, d_qkv, c, d_tables, packed, d_out);
}

}  // namespace ien

using namespace ien;

extern "C" {

long ien_window_count(const ien_windows *w) {
  WinGeo g;
  if (geometry(w, &g) != IEN_OK) return -1;
  return g.windows;
}

ien_status ien_position_bias(const float *table, int heads, int window,
                             ien_position_layout layout, float *out) {
  IEN_CHECK(table && out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(heads >= 1 && window >= 1 && window <= 16, IEN_ERR_INPUT, "%d heads, window %d", heads,
            window);
  IEN_CHECK(layout == IEN_POS_SCUNET || layout == IEN_POS_SWIN, IEN_ERR_INPUT, "layout %d",
            (int)layout);
  const int n = window * window, side = 2 * window - 1;
  for (int h = 0; h < heads; h++)
    for (int i = 0; i < n; i++)
      for (int j = 0; j < n; j++) {
        // Offsets (yi - yj, xi - xj), each shifted into 0 .. 2W - 2.
        const int cell = (i / window - j / window + window - 1) * side +
                         (i % window - j % window + window - 1);
        out[((size_t)h * n + i) * n + j] =
            layout == IEN_POS_SCUNET ? table[(size_t)h * side * side + cell]
                                     : table[(size_t)cell * heads + h];
      }
  return IEN_OK;
}

int ien_bias_tables(const float *position, int heads, int window, int shift, float masked,
                    float *out) {
  if (!position || !out || heads < 1 || window < 1 || window > 16 || shift < 0 ||
      shift >= window) {
    set_error("input: bias tables of %d heads, window %d, shift %d", heads, window, shift);
    return -1;
  }
  const size_t n = (size_t)window * window, per = (size_t)heads * n * n;
  if (shift == 0) {
    std::memcpy(out, position, sizeof(float) * per);
    return 1;
  }
  for (int cls = 0; cls < 4; cls++) {
    // Region of a token in a window of this class: its row (last-column
    // class: column) in the part the roll brought from the far side.
    auto region = [&](size_t t) {
      const bool row = (cls & 2) && (int)(t / window) >= window - shift;
      const bool col = (cls & 1) && (int)(t % window) >= window - shift;
      return 2 * (int)row + (int)col;
    };
    for (int h = 0; h < heads; h++)
      for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) {
          const size_t at = ((size_t)h * n + i) * n + j;
          out[cls * per + at] = position[at] + (region(i) == region(j) ? 0.0f : masked);
        }
  }
  return 4;
}

ien_status ien_window_gather(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_map,
                             size_t stride, int c, const float *d_gamma, const float *d_beta,
                             uint16_t *d_tokens) {
  IEN_CHECK(ctx && d_map && d_gamma && d_beta && d_tokens, IEN_ERR_INPUT, "null argument");
  WinGeo g;
  ien_status st = geometry(w, &g);
  if (st != IEN_OK) return st;
  IEN_CHECK(c >= 8 && c <= 1024 && c % 8 == 0, IEN_ERR_INPUT, "%d channels (8 .. 1024, by 8)", c);
  IEN_CHECK(stride >= (size_t)c && stride % 8 == 0 && aligned16(d_map) && aligned16(d_tokens),
            IEN_ERR_INPUT, "map stride %zu / alignment (16-byte rows)", stride);
  IEN_CHECK(((uintptr_t)d_gamma & 15) == 0 && ((uintptr_t)d_beta & 15) == 0, IEN_ERR_INPUT,
            "LayerNorm parameters must be 16-byte aligned");
  const long rows = g.windows * g.n;
  const int chunks = c / 8;
  int lanes = 1;
  while (lanes < chunks && lanes < 64) lanes *= 2;
  // One row a lane group (2 and 4 measured no faster at SCUNet's level 1):
  // waves of 64 / lanes rows, whole workgroups.
  constexpr int R = 1;
  const long per_block = 4L * R * (64 / lanes);
  const long blocks = (rows + per_block - 1) / per_block;
  IEN_CHECK(blocks * per_block < (1L << 31) && blocks * 256 < (1L << 31), IEN_ERR_INPUT, "%ld rows",
            rows);
  void (*k)(WinGeo, const uint16_t *, long, int, const float *, const float *, uint16_t *) =
      nullptr;
  switch (lanes) {
    case 1: k = k_window_gather<1, R>; break;
    case 2: k = k_window_gather<2, R>; break;
    case 4: k = k_window_gather<4, R>; break;
    case 8: k = k_window_gather<8, R>; break;
    case 16: k = k_window_gather<16, R>; break;
    case 32: k = k_window_gather<32, R>; break;
    default: k = k_window_gather<64, R>; break;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, g, d_map, (long)stride, c,
                     d_gamma, d_beta, d_tokens);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

ien_status ien_window_attention(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_qkv, int c,
                                const float *d_tables, uint16_t *d_out) {
  return window_attention(ctx, w, d_qkv, c, d_tables, false, d_out);
}

ien_status ien_window_scatter_add(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_rows,
                                  int c, uint16_t *d_map, size_t stride) {
  IEN_CHECK(ctx && d_rows && d_map, IEN_ERR_INPUT, "null argument");
  WinGeo g;
  ien_status st = geometry(w, &g);
  if (st != IEN_OK) return st;
  IEN_CHECK(c >= 8 && c % 8 == 0, IEN_ERR_INPUT, "%d channels (by 8)", c);
  IEN_CHECK(stride >= (size_t)c && stride % 8 == 0 && aligned16(d_map) && aligned16(d_rows),
            IEN_ERR_INPUT, "map stride %zu / alignment (16-byte rows)", stride);
  const long items = g.windows * g.n * (c / 8);
  hipLaunchKernelGGL(k_window_scatter_add, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     ctx->stream, g, d_rows, c, d_map, (long)stride);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

}  // extern "C"
