// birefnet.hip -- BiRefNet-lite on the GPU (crates/birefnet-native/src/
// lib.rs:144-171 run_normalized, swin.rs, decoder.rs): f16 NHWC maps.
//  - Backbone: the 4x4 patch embedding as rows (ky, kx, c) through a
//    product and a LayerNorm; the Swin blocks through ien_swin (windows of
//    7 or 12, shift window / 2, -100 between regions, zero rows past the
//    edge); stage outputs normalised into the decoder's level maps; 2x2
//    merges as column-major gathers, LayerNorm over 4c and a product.
//  - Decoder: 3x3 convolutions through the implicit-GEMM kernels; the ASPP's
//    pooling branch as a two-pass column mean and a one-workgroup pass of
//    its two small products (a bias for conv1), its four branches as k x k
//    convolutions into the columns of one 1024-channel map (the network is
//    deformable-free: all-zero offset and modulator convolutions sample the
//    integer taps with modulator 2 sigmoid(0) = 1, decoder.rs:254-313) or,
//    where a branch's offsets are not zero, its offset convolution, the
//    bilinear samples and their product in chunks of rows; and
//    conv1 with that bias; the gate as a 3x3 convolution to 16
//    channels and a per-pixel sigmoid scale; the image-to-patches stacks;
//    the head before the final resize; the full-resolution branch in 32 x 32
//    tiles, its composed 5x5 convolution off the edge ring and, in the
//    border tiles, both convolutions on the ring (decoder.rs:594-757).
// One event is recorded after each of 14 steps (the 2 x 4 backbone stages,
// the squeeze and the four decoder blocks, the head) for progress reports.

#include <cmath>
#include <string>

#include "birefnet.h"
#include "conv_common.h"

namespace ien {

namespace {

constexpr int INTER = 64, BRANCH = 256;
constexpr int STAGE_C[4] = {96, 192, 384, 768};
constexpr int STAGE_DEPTH[4] = {2, 2, 6, 2};
constexpr int ASPP_SIZES[4] = {1, 1, 3, 7};
constexpr int LEVEL_CIN[4] = {1728, 960, 480, 240};   // decoder.rs:776
constexpr int LEVEL_COUT[4] = {768, 384, 192, 96};
constexpr int PATCH_CIN[4] = {3072, 768, 192, 48};   // patches5..2
constexpr int PATCH_COUT[4] = {192, 192, 96, 48};
constexpr int SQUEEZE_CIN = 2880, SQUEEZE_COUT = 1536;
constexpr float MASKED = -100.0f;  // swin.rs:21-23
constexpr int POOL_PARTS = 256;    // partial sums of the ASPP's column mean
// Bilinear samples of a deformable branch are built this many bytes of rows
// at a time (the 7 x 7 branch: about 10k pixels of 49 x 64 halves).
constexpr size_t SAMPLE_BYTES = (size_t)64 << 20;

unsigned blocks_for(long items, int per) { return (unsigned)((items + per - 1) / per); }

// swin.rs:190-196: token r's row of 48 values, (ky, kx, c) over its 4 x 4
// patch of the f16 image; one thread per (token, ky): 12 halves.
__global__ __launch_bounds__(256) void k_patch_rows(const uint16_t *__restrict__ img, int side,
                                                    uint16_t *__restrict__ rows) {
  const int grid = side / 4;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)grid * grid * 4) return;
  const long r = i / 4;
  const int ky = (int)(i % 4);
  const int ty = (int)(r / grid), tx = (int)(r % grid);
  const uint16_t *s = img + ((long)(ty * 4 + ky) * side + tx * 4) * 3;
  uint16_t *d = rows + r * 48 + ky * 12;
#pragma unroll
  for (int e = 0; e < 12; e++) d[e] = s[e];
}

// Columns 0..c of `rows` rows, src rows `ss` halves apart, into dst rows
// `ds` apart (decoder.rs:523-533 place); 8 halves per thread.
__global__ __launch_bounds__(256) void k_copy_cols(const uint16_t *__restrict__ src, long rows,
                                                   int c, long ss, uint16_t *__restrict__ dst,
                                                   long ds) {
  const int chunks = c / 8;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * chunks) return;
  const long r = i / chunks;
  const int k = (int)(i % chunks);
  *(u32x4 *)(dst + r * ds + 8 * k) = *(const u32x4 *)(src + r * ss + 8 * k);
}

// ASPP pooling, pass 1 (decoder.rs:140-150): part b of POOL_PARTS sums the
// 64 channels over its rows in f32 (4 row groups of 64 lanes, combined in
// a fixed order: the result does not depend on timing).
__global__ __launch_bounds__(256) void k_pool_partial(const uint16_t *__restrict__ t, long rows,
                                                      float *__restrict__ partial) {
  __shared__ float part[4][INTER];
  const int ch = threadIdx.x % INTER, g = threadIdx.x / INTER;
  const long per = (rows + POOL_PARTS - 1) / POOL_PARTS;
  const long r0 = (long)blockIdx.x * per, r1 = r0 + per < rows ? r0 + per : rows;
  float s = 0.0f;
  for (long r = r0 + g; r < r1; r += 4) s += h2f(t[r * INTER + ch]);
  part[g][ch] = s;
  __syncthreads();
  if (g == 0) partial[blockIdx.x * INTER + ch] = ((part[0][ch] + part[1][ch]) + part[2][ch]) + part[3][ch];
}

// Pass 2, one workgroup: the mean, the pooling product (64 -> 256) + ReLU,
// and its share of conv1 (256 -> 64) plus conv1's bias: the bias every
// pixel of conv1 gets (decoder.rs:150-170).  pool: [64][256] weight, [256]
// bias, [256][64] conv1 rows, [64] conv1 bias.  The 64-wide sums are split
// over the 4 lane groups (parts g, g + 4, ...; conv1 rows 64 g ..) and
// combined in a fixed order, the loops unrolled so that loads go out in
// batches.
__global__ __launch_bounds__(256) void k_pool_finish(const float *__restrict__ partial, long rows,
                                                     const float *__restrict__ pool,
                                                     float *__restrict__ bias) {
  static_assert(INTER == 64 && BRANCH == 256 && POOL_PARTS % 4 == 0, "pool shapes");
  __shared__ double msum[4][INTER];
  __shared__ float mean[INTER];
  __shared__ float pooled[BRANCH];
  __shared__ float bsum[4][INTER];
  const int tid = threadIdx.x, ch = tid % INTER, g = tid / INTER;
  {
    double s = 0.0;
#pragma unroll 16
    for (int b = g; b < POOL_PARTS; b += 4) s += (double)partial[b * INTER + ch];
    msum[g][ch] = s;
  }
  __syncthreads();
  if (tid < INTER)
    mean[tid] = (float)((((msum[0][tid] + msum[1][tid]) + msum[2][tid]) + msum[3][tid]) / (double)rows);
  __syncthreads();
  const float *pw = pool, *pb = pool + INTER * BRANCH, *cw = pb + BRANCH, *cb = cw + BRANCH * INTER;
  {
    float p = pb[tid];
#pragma unroll 16
    for (int c = 0; c < INTER; c++) p += mean[c] * pw[c * BRANCH + tid];
    pooled[tid] = p > 0.0f ? p : 0.0f;
  }
  __syncthreads();
  {
    float b = 0.0f;
#pragma unroll 16
    for (int j = INTER * g; j < INTER * g + INTER; j++) b += pooled[j] * cw[j * INTER + ch];
    bsum[g][ch] = b;
  }
  __syncthreads();
  if (tid < INTER) bias[tid] = cb[tid] + (((bsum[0][tid] + bsum[1][tid]) + bsum[2][tid]) + bsum[3][tid]);
}

// decoder.rs:378-401 the gate: out[p] *= sigmoid(b + sum_k g[p][k] w[k]),
// one thread per 8 channels of a pixel.
struct GateW {
  float w[16];
  float b;
};
__global__ __launch_bounds__(256) void k_gate(uint16_t *__restrict__ out, long rows, int c,
                                              const uint16_t *__restrict__ g, GateW gw) {
  const int chunks = c / 8;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * chunks) return;
  const long p = i / chunks;
  const int k = (int)(i % chunks);
  float s = gw.b;
#pragma unroll
  for (int j = 0; j < 16; j++) s = s + h2f(g[p * 16 + j]) * gw.w[j];
  s = sigmoid_f(s);
  u32x4 *o = (u32x4 *)(out + p * c + 8 * k);
  u32x4 v = *o;
  uint16_t h[8];
  __builtin_memcpy(h, &v, 16);
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = f2h(h2f(h[e]) * s);
  __builtin_memcpy(&v, h, 16);
  *o = v;
}

// decoder.rs:546-577 image2patches: pixel (y, x) of the size x size stack,
// channel (c grid + gy) grid + gx = image pixel (gy size + y, gx size + x),
// colour c.  One thread per output element (any grid), or for grids of 4,
// 8, 16 and 32 one thread per (gy, c, output pixel), pixels fastest: it reads
// the GRID image pixels of its run (neighbouring threads read neighbouring
// pixels) and writes the run's GRID consecutive channels as 16-byte (8 when
// GRID is 4) stores.
__global__ __launch_bounds__(256) void k_image_patches_any(const uint16_t *__restrict__ img,
                                                           int side, int size,
                                                           uint16_t *__restrict__ out) {
  const int grid = side / size, channels = 3 * grid * grid;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)size * size * channels) return;
  const long p = i / channels;
  const int ch = (int)(i % channels);
  const int y = (int)(p / size), x = (int)(p % size);
  const int c = ch / (grid * grid), gy = (ch / grid) % grid, gx = ch % grid;
  out[i] = img[((long)(gy * size + y) * side + gx * size + x) * 3 + c];
}

template <int GRID>
__global__ __launch_bounds__(256) void k_image_patches(const uint16_t *__restrict__ img, int side,
                                                       uint16_t *__restrict__ out) {
  const int size = side / GRID, channels = 3 * GRID * GRID;
  const long pixels = (long)size * size;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= pixels * 3 * GRID) return;
  const long p = i % pixels;
  const int run = (int)(i / pixels), c = run / GRID, gy = run % GRID;
  const int y = (int)(p / size), x = (int)(p % size);
  const uint16_t *src = img + ((long)(gy * size + y) * side + x) * 3 + c;
  uint16_t v[GRID];
#pragma unroll
  for (int gx = 0; gx < GRID; gx++) v[gx] = src[(long)gx * size * 3];
  uint16_t *dst = out + p * channels + (c * GRID + gy) * GRID;
  if constexpr (GRID % 8 == 0) {
#pragma unroll
    for (int q = 0; q < GRID / 8; q++) {
      u32x4 o;
      __builtin_memcpy(&o, v + 8 * q, 16);
      *(u32x4 *)(dst + 8 * q) = o;
    }
  } else {
    static_assert(GRID == 4, "runs of 4 or a multiple of 8");
    uint2 o;
    __builtin_memcpy(&o, v, 8);
    *(uint2 *)dst = o;
  }
}

// The full-resolution branch's weights (decoder.rs:604-635 FullResolution):
// the composed 5x5 weights [25][3] with their bias after them, and the two
// convolutions it composes (conv1 [27][64] + bias1, conv_out [9][64] +
// bias_out), all device f32.
struct FullParams {
  const float *composed, *conv1, *bias1, *conv_out;
  float bias_out, head_bias;
};

// decoder.rs:637-757 FullResolution::add with the head bias.  One
// workgroup per 32 x 32 pixel tile; the tile's image patch with two pixels
// around it (zeros outside the image) staged in LDS as three planes.
//  - Pixels off the image's edge ring: the composed 5x5 convolution
//    (composed_row: the bias, then each tap's three products in order),
//    four neighbouring pixels a thread, which share each tap row's reads.
//  - The edge ring's pixels are computed exactly (decoder.rs:700-734: conv1
//    + bias1 at each in-image neighbour, the intermediate map's zero
//    padding reached, then conv_out), dealt over all workgroups, four at a
//    time (one a wave): lane k takes intermediate channel k over the
//    neighbours, and a 64-lane sum adds the channels.  (The ring left to
//    the border tiles alone had made them take 80 us against a few for
//    the others.)
constexpr int FT = 32, FP = FT + 4;
__global__ __launch_bounds__(256) void k_full_res(const float *__restrict__ image, int side,
                                                  FullParams f, float *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) float patch[3][FP][FP];
  __shared__ float rpatch[4][3][5][5];  // each wave's ring pixel's 5 x 5 window
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int tiles = side / FT;
  const int y0 = (int)(blockIdx.x / tiles) * FT, x0 = (int)(blockIdx.x % tiles) * FT;
  // Ring pixels r of this workgroup: per = ceil(ring / workgroups), taken
  // four at a time; ring order: the top row left to right, the right
  // column down, the bottom row right to left, the left column up.
  const int ring = 4 * (side - 1), per = (ring + (int)gridDim.x - 1) / (int)gridDim.x;
  auto ring_pos = [&](int r, int &ry, int &rx) {
    const int e = side - 1;
    if (r < e) {
      ry = 0;
      rx = r;
    } else if (r < 2 * e) {
      ry = r - e;
      rx = e;
    } else if (r < 3 * e) {
      ry = e;
      rx = e - (r - 2 * e);
    } else {
      ry = e - (r - 3 * e);
      rx = 0;
    }
  };
  for (int i = t; i < FP * FP; i += 256) {
    const int py = y0 - 2 + i / FP, px = x0 - 2 + i % FP;
    const bool in = py >= 0 && px >= 0 && py < side && px < side;
    const float *p = image + ((long)(in ? py : 0) * side + (in ? px : 0)) * 3;
#pragma unroll
    for (int c = 0; c < 3; c++) patch[c][i / FP][i % FP] = in ? p[c] : 0.0f;
  }
  __syncthreads();

  // ---- off the ring: thread t, row t / 8, pixels 4 (t % 8) .. + 3 ----
  {
    const int ly = t >> 3, lx = (t & 7) * 4;
    const int y = y0 + ly;
    float s[4];
#pragma unroll
    for (int q = 0; q < 4; q++) s[q] = f.composed[75];
#pragma unroll
    for (int dy = 0; dy < 5; dy++) {
      float row[3][8];
#pragma unroll
      for (int c = 0; c < 3; c++) {
        const float4 a = *(const float4 *)&patch[c][ly + dy][lx];
        const float4 b = *(const float4 *)&patch[c][ly + dy][lx + 4];
        row[c][0] = a.x; row[c][1] = a.y; row[c][2] = a.z; row[c][3] = a.w;
        row[c][4] = b.x; row[c][5] = b.y; row[c][6] = b.z; row[c][7] = b.w;
      }
#pragma unroll
      for (int dx = 0; dx < 5; dx++) {
        const int e = dy * 5 + dx;
#pragma unroll
        for (int q = 0; q < 4; q++)
          s[q] += f.composed[3 * e] * row[0][q + dx] + f.composed[3 * e + 1] * row[1][q + dx] +
                  f.composed[3 * e + 2] * row[2][q + dx];
      }
    }
    float *o = out + (long)y * side + x0 + lx;
    const bool edge_row = y == 0 || y == side - 1;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int x = x0 + lx + q;
      if (!edge_row && x != 0 && x != side - 1) o[q] = f.head_bias + s[q];
    }
  }

  // ---- the ring: wave w takes pixel r = blockIdx.x per + 4 i + w ----
  for (int i = 0; i < per; i += 4) {
    const int r = (int)blockIdx.x * per + i + wave;
    const bool live = i + wave < per && r < ring;  // uniform per wave
    int ry = 0, rx = 0;
    if (live) ring_pos(r, ry, rx);
    __syncthreads();  // (the previous round's windows are read)
    if (live)
      for (int j = lane; j < 75; j += 64) {  // 3 x 25 values over the wave's 64 lanes
        const int c = j / 25, e = j % 25;
        const int py = ry - 2 + e / 5, px = rx - 2 + e % 5;
        const bool in = py >= 0 && px >= 0 && py < side && px < side;
        rpatch[wave][c][e / 5][e % 5] = in ? image[((long)py * side + px) * 3 + c] : 0.0f;
      }
    __syncthreads();
    if (!live) continue;
    const int k = lane;
    float v = 0.0f;
    for (int d = 0; d < 9; d++) {
      const int qy = ry + d / 3 - 1, qx = rx + d % 3 - 1;
      if (qy < 0 || qx < 0 || qy >= side || qx >= side) continue;
      float m = f.bias1[k];
#pragma unroll
      for (int e = 0; e < 9; e++) {
        const int sy = d / 3 + e / 3, sx = d % 3 + e % 3;
#pragma unroll
        for (int c = 0; c < 3; c++) m += rpatch[wave][c][sy][sx] * f.conv1[(e * 3 + c) * INTER + k];
      }
      v += m * f.conv_out[d * INTER + k];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) out[(long)ry * side + rx] = f.head_bias + (f.bias_out + v);
  }
}

ien_status matrix(ien_ctx *ctx, const TensorSource &take, const std::string &name, size_t k,
                  size_t n, bool bias, ien_matrix **out) {
  std::vector<float> w, b;
  ien_status st = take(name + ".weight", {k, n}, &w);
  if (st == IEN_OK && bias) st = take(name + ".bias", {n}, &b);
  if (st != IEN_OK) return st;
  return ien_matrix_new(ctx, w.data(), IEN_W_F32, k, n, bias ? b.data() : nullptr, out);
}

ien_status upload(const std::vector<float> &v, float **d) {
  IEN_HIP(hipMalloc((void **)d, v.size() * 4));
  IEN_HIP(hipMemcpy(*d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
  return IEN_OK;
}

// gamma then beta of a LayerNorm over c, onto the device.
ien_status norm(const TensorSource &take, const std::string &name, size_t c, float **d) {
  std::vector<float> g, b;
  ien_status st = take(name + ".weight", {c}, &g);
  if (st == IEN_OK) st = take(name + ".bias", {c}, &b);
  if (st != IEN_OK) return st;
  g.insert(g.end(), b.begin(), b.end());
  return upload(g, d);
}

// decoder.rs:316-343 Block::load and :102-136 Aspp::load.
ien_status load_block(ien_ctx *ctx, const TensorSource &take, const std::string &q, int cin,
                      int cout, bool gate, BirefnetBlock *B) {
  B->cin = cin;
  B->cout = cout;
  B->gate = gate;
  ien_status st = matrix(ctx, take, q + ".conv_in", 9 * (size_t)cin, INTER, true, &B->conv_in);
  if (st == IEN_OK) st = matrix(ctx, take, q + ".conv_out", 9 * INTER, cout, true, &B->conv_out);
  if (st == IEN_OK && gate) {
    st = matrix(ctx, take, q + ".gdt", 9 * (size_t)cout, 16, true, &B->gdt);
    std::vector<float> w, b;
    if (st == IEN_OK) st = take(q + ".gdt_attn.weight", {16, 1}, &w);
    if (st == IEN_OK) st = take(q + ".gdt_attn.bias", {1}, &b);
    if (st == IEN_OK) {
      for (int j = 0; j < 16; j++) B->gdt_w[j] = w[j];
      B->gdt_b = b[0];
    }
  }
  for (int i = 0; i < 4 && st == IEN_OK; i++) {
    const size_t taps = (size_t)ASPP_SIZES[i] * ASPP_SIZES[i];
    const std::string p = q + ".aspp.branch" + std::to_string(i);
    std::vector<float> ow, ob;
    st = take(p + ".offset.weight", {taps * INTER, 3 * taps}, &ow);
    if (st == IEN_OK) st = take(p + ".offset.bias", {3 * taps}, &ob);
    if (st != IEN_OK) break;
    // All-zero offsets and modulator logits sample the integer taps with
    // modulator 2 sigmoid(0) = 1: the branch is then a plain convolution.
    bool zero = true;
    for (float v : ow) zero = zero && v == 0.0f;
    for (float v : ob) zero = zero && v == 0.0f;
    if (!zero)
      st = ien_matrix_new(ctx, ow.data(), IEN_W_F32, taps * INTER, 3 * taps, ob.data(),
                          &B->offset[i]);
    if (st == IEN_OK) st = matrix(ctx, take, p, taps * INTER, BRANCH, true, &B->branch[i]);
  }
  if (st != IEN_OK) return st;
  std::vector<float> pw, pb, cw, cb;
  st = take(q + ".aspp.pool.weight", {INTER, BRANCH}, &pw);
  if (st == IEN_OK) st = take(q + ".aspp.pool.bias", {BRANCH}, &pb);
  if (st == IEN_OK) st = take(q + ".aspp.conv1.weight", {5 * BRANCH, INTER}, &cw);
  if (st == IEN_OK) st = take(q + ".aspp.conv1.bias", {INTER}, &cb);
  if (st != IEN_OK) return st;
  // conv1's first 4 x 256 rows read the branches; its last 256 the pooling.
  st = ien_matrix_new(ctx, cw.data(), IEN_W_F32, 4 * BRANCH, INTER, nullptr, &B->conv1);
  if (st != IEN_OK) return st;
  std::vector<float> pool(pw);
  pool.insert(pool.end(), pb.begin(), pb.end());
  pool.insert(pool.end(), cw.begin() + 4 * BRANCH * INTER, cw.end());
  pool.insert(pool.end(), cb.begin(), cb.end());
  return upload(pool, &B->d_pool);
}

void free_block(BirefnetBlock &B) {
  ien_matrix_free(B.conv_in);
  ien_matrix_free(B.conv_out);
  ien_matrix_free(B.conv1);
  ien_matrix_free(B.gdt);
  for (auto *m : B.branch) ien_matrix_free(m);
  for (auto *m : B.offset) ien_matrix_free(m);
  (void)hipFree(B.d_pool);
}

void free_maps(Birefnet &b) {
  for (uint16_t **p : {&b.img16, &b.half16, &b.prow, &b.x, &b.mrows, &b.level[0], &b.level[1],
                       &b.level[2], &b.level[3], &b.tmp, &b.x4, &b.in, &b.t, &b.a, &b.cat, &b.g,
                       &b.prev, &b.stacked, &b.mid, &b.low, &b.hprow, &b.hx, &b.hmrows,
                       &b.hscratch}) {
    (void)hipFree(*p);
    *p = nullptr;
  }
  (void)hipFree(b.partial);
  (void)hipFree(b.d_bias);
  (void)hipFree(b.offs);
  (void)hipFree(b.samples);
  b.partial = b.d_bias = b.offs = nullptr;
  b.samples = nullptr;
  b.hscratch_halves = 0;
  b.side = 0;
}

// A size x size stride-1 convolution (zero padding) of an h x w f16 map.
ien_status conv(ien_ctx *ctx, const uint16_t *x, int h, int w, int c, long xs, int size,
                const ien_matrix *m, uint16_t *y, long ys, ien_act act, int accumulate) {
  ConvCall cc;
  cc.x = x;
  cc.H = h;
  cc.W = w;
  cc.C = c;
  cc.xs = xs;
  cc.ks = size;
  cc.stride = 1;
  cc.OH = h;
  cc.OW = w;
  cc.row0 = 0;
  cc.rows = (long)h * w;
  cc.w = m;
  cc.y = y;
  cc.ys = ys;
  cc.act = act;
  cc.accumulate = accumulate;
  return launch_conv(ctx, cc);
}

ien_status rows_product(ien_ctx *ctx, const uint16_t *in, size_t k, long xs, size_t rows,
                        const ien_matrix *m, uint16_t *out, long ys, ien_act act, int accumulate,
                        const float *bias = nullptr) {
  ConvCall cc;
  cc.bias = bias;
  cc.x = in;
  cc.rows_mode = 1;
  cc.C = (int)k;
  cc.xs = xs;
  cc.ks = 1;
  cc.stride = 1;
  cc.row0 = 0;
  cc.rows = (long)rows;
  cc.w = m;
  cc.y = out;
  cc.ys = ys;
  cc.act = act;
  cc.accumulate = accumulate;
  return launch_conv(ctx, cc);
}

ien_status copy_cols(ien_ctx *ctx, const uint16_t *src, long rows, int c, long ss, uint16_t *dst,
                     long ds) {
  IEN_CHECK(c % 8 == 0 && ss % 8 == 0 && ds % 8 == 0 && ((uintptr_t)src & 15) == 0 &&
                ((uintptr_t)dst & 15) == 0,
            IEN_ERR_INPUT, "column copy of %d of %ld / %ld", c, ss, ds);
  hipLaunchKernelGGL(k_copy_cols, dim3(blocks_for(rows * (c / 8), 256)), dim3(256), 0,
                     ctx->stream, src, rows, c, ss, dst, ds);
  IEN_HIP(hipGetLastError());
  return IEN_OK;
}

// decoder.rs:239-313 sample_rows / sample: the deformable input of rows
// row0 .. row0 + rows of an h x w map t (f16, 64 channels): for each tap of
// a size x size kernel, the 64 channels bilinearly sampled at the tap moved
// by its offset, times twice the sigmoid of its modulator logit; a point
// more than a pixel outside the map reads zero and corners outside it count
// as zero (torchvision's deform_conv2d).  offs: 3 taps f32 a pixel (y, x
// offsets per tap, then the logits).  One thread per (row, tap, 8-channel
// group): four 16-byte corner loads, blended in f32 in the reference's
// corner order, one 16-byte store into row r's taps x 64 halves.
__global__ __launch_bounds__(256) void k_deform_sample(const uint16_t *__restrict__ t, int h, int w,
                                                       const float *__restrict__ offs, int size,
                                                       long row0, long rows,
                                                       uint16_t *__restrict__ samples) {
  const int taps = size * size;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * taps * 8) return;
  const int grp = (int)(i % 8), tap = (int)(i / 8 % taps);
  const long r = i / 8 / taps, p = row0 + r;
  const int y = (int)(p / w), x = (int)(p % w);
  const float *o = offs + p * 3 * taps;
  const float half = (float)(size / 2);
  const float py = ((float)y - half + (float)(tap / size)) + o[2 * tap];
  const float px = ((float)x - half + (float)(tap % size)) + o[2 * tap + 1];
  const float m = 2.0f * sigmoid_f(o[2 * taps + tap]);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (!(py <= -1.0f || py >= (float)h || px <= -1.0f || px >= (float)w)) {
    const float y0f = floorf(py), x0f = floorf(px);
    const float ly = py - y0f, lx = px - x0f, hy = 1.0f - ly, hx = 1.0f - lx;
    const int y0 = (int)y0f, x0 = (int)x0f;
    const float cw[4] = {hy * hx, hy * lx, ly * hx, ly * lx};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int cy = y0 + k / 2, cx = x0 + k % 2;
      if (cy < 0 || cx < 0 || cy >= h || cx >= w) continue;
      const u32x4 v = *(const u32x4 *)(t + ((long)cy * w + cx) * INTER + grp * 8);
      uint16_t hv[8];
      __builtin_memcpy(hv, &v, 16);
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] += cw[k] * h2f(hv[j]);
    }
  }
  uint16_t out[8];
#pragma unroll
  for (int j = 0; j < 8; j++) out[j] = f2h(acc[j] * m);
  u32x4 ov;
  __builtin_memcpy(&ov, out, 16);
  *(u32x4 *)(samples + (r * taps + tap) * INTER + grp * 8) = ov;
}

// One deformable ASPP branch (decoder.rs:176-218): the offset convolution
// into f32, then per chunk of rows the samples and their product with the
// branch weights (ReLU) into columns i x 256 of the concatenated map.
ien_status deformable_branch(Birefnet *b, const BirefnetBlock &B, int i, int h, int w) {
  ien_ctx *ctx = b->ctx;
  const int size = ASPP_SIZES[i], taps = size * size;
  const long pixels = (long)h * w;
  ConvCall cc;
  cc.x = b->t;
  cc.H = h;
  cc.W = w;
  cc.C = INTER;
  cc.xs = INTER;
  cc.ks = size;
  cc.stride = 1;
  cc.OH = h;
  cc.OW = w;
  cc.row0 = 0;
  cc.rows = pixels;
  cc.w = B.offset[i];
  cc.y = b->offs;
  cc.ys = 3 * taps;
  cc.out_f32 = 1;
  ien_status st = launch_conv(ctx, cc);
  const long chunk = std::max<long>(64, (long)(SAMPLE_BYTES / ((size_t)taps * INTER * 2)) / 64 * 64);
  for (long row0 = 0; row0 < pixels && st == IEN_OK; row0 += chunk) {
    const long rows = std::min(chunk, pixels - row0);
    hipLaunchKernelGGL(k_deform_sample, dim3(blocks_for(rows * taps * 8, 256)), dim3(256), 0,
                       ctx->stream, b->t, h, w, b->offs, size, row0, rows, b->samples);
    IEN_HIP(hipGetLastError());
    st = rows_product(ctx, b->samples, (size_t)taps * INTER, (long)taps * INTER, (size_t)rows,
                      B.branch[i], b->cat + row0 * 4 * BRANCH + i * BRANCH, 4 * BRANCH,
                      IEN_ACT_RELU, 0);
  }
  return st;
}

// decoder.rs:346-413 Block::run: in (h x w x cin) -> out (h x w x cout).
ien_status block_run(Birefnet *b, const BirefnetBlock &B, const uint16_t *in, int h, int w,
                     uint16_t *out) {
  ien_ctx *ctx = b->ctx;
  const long pixels = (long)h * w;
  ien_status st = conv(ctx, in, h, w, B.cin, B.cin, 3, B.conv_in, b->t, INTER, IEN_ACT_RELU, 0);
  if (st != IEN_OK) return st;
  // The pooling branch only feeds conv1's bias: it runs on branch stream 1
  // beside the four branch convolutions (one workgroup of its two passes
  // would otherwise hold up the CUs between them).
  st = fork_branches(ctx, 1);
  if (st != IEN_OK) return st;
  {
    Branch br(ctx, 1);
    hipLaunchKernelGGL(k_pool_partial, dim3(POOL_PARTS), dim3(256), 0, ctx->stream, b->t, pixels,
                       b->partial);
    hipLaunchKernelGGL(k_pool_finish, dim3(1), dim3(256), 0, ctx->stream, b->partial, pixels,
                       B.d_pool, b->d_bias);
  }
  if (const hipError_t le = hipGetLastError(); le != hipSuccess)
    st = fail(IEN_ERR_GPU, "pooling launch: %s", hipGetErrorString(le));
  for (int i = 0; i < 4 && st == IEN_OK; i++)
    st = B.offset[i] ? deformable_branch(b, B, i, h, w)
                     : conv(ctx, b->t, h, w, INTER, INTER, ASPP_SIZES[i], B.branch[i],
                            b->cat + i * BRANCH, 4 * BRANCH, IEN_ACT_RELU, 0);
  // (Joined after a failure too, so that nothing on the branch outlives the run.)
  const ien_status js = join_branches(ctx, 1);
  if (st == IEN_OK) st = js;
  if (st != IEN_OK) return st;
  // conv1 over the four branches with the pooling's part (constant over the
  // pixels) and conv1's bias as its bias.
  st = rows_product(ctx, b->cat, 4 * BRANCH, 4 * BRANCH, pixels, B.conv1, b->a, INTER,
                    IEN_ACT_RELU, 0, b->d_bias);
  if (st == IEN_OK)
    st = conv(ctx, b->a, h, w, INTER, INTER, 3, B.conv_out, out, B.cout, IEN_ACT_NONE, 0);
  if (st == IEN_OK && B.gate) {
    st = conv(ctx, out, h, w, B.cout, B.cout, 3, B.gdt, b->g, 16, IEN_ACT_RELU, 0);
    if (st != IEN_OK) return st;
    GateW gw;
    for (int j = 0; j < 16; j++) gw.w[j] = B.gdt_w[j];
    gw.b = B.gdt_b;
    hipLaunchKernelGGL(k_gate, dim3(blocks_for(pixels * (B.cout / 8), 256)), dim3(256), 0,
                       ctx->stream, out, pixels, B.cout, b->g, gw);
    IEN_HIP(hipGetLastError());
  }
  return st;
}

// swin.rs:171-215 Backbone::run on the f16 image `img` (side x side x 3):
// each stage's normalised output into level buffer s (columns `col` of
// rows 2 c wide) directly for the full size, through `tmp` and a resize for
// the half size.
// The buffers one backbone run works in: the full-size run uses the
// model's, the half-size run (on a branch stream) its own.
struct BackboneBufs {
  uint16_t *prow, *x, *mrows, *scratch;
  size_t scratch_halves;  // 0: each block's own scratch
};

// swin.rs:171-215 Backbone::run on the f16 image `img` (side x side x 3):
// the patch embedding, then stage by stage (backbone_stage).
ien_status backbone_embed(Birefnet *b, const BackboneBufs &k, const uint16_t *img, int side) {
  ien_ctx *ctx = b->ctx;
  const int grid = side / 4;
  const long tokens = (long)grid * grid;
  hipLaunchKernelGGL(k_patch_rows, dim3(blocks_for(tokens * 4, 256)), dim3(256), 0, ctx->stream,
                     img, side, k.prow);
  IEN_HIP(hipGetLastError());
  ien_status st = rows_product(ctx, k.prow, 48, 48, tokens, b->embed, k.x, 96, IEN_ACT_NONE, 0);
  if (st == IEN_OK) st = ien_layer_norm(ctx, k.x, tokens, 96, 96, b->d_embed_ln, b->d_embed_ln + 96);
  return st;
}

// Stage s on a grid x grid token map: its blocks, the stage output
// normalised into level buffer s (columns 0 .. c of rows 2 c wide)
// directly for the full size, through `tmp` and a resize into columns
// c .. 2 c for the half size; then the merge (s < 3).
ien_status backbone_stage(Birefnet *b, const BackboneBufs &k, int s, int grid, bool half) {
  ien_ctx *ctx = b->ctx;
  const int c = STAGE_C[s];
  ien_status st = IEN_OK;
  for (ien_swin *blk : b->blocks[s]) {
    st = k.scratch_halves ? swin_run_with(blk, k.x, c, grid, grid, k.scratch, k.scratch_halves)
                          : ien_swin_run(blk, k.x, c, grid, grid);
    if (st != IEN_OK) return st;
  }
  const long n = (long)grid * grid;
  if (!half) {
    st = layer_norm_to(ctx, k.x, c, b->level[s], 2L * c, n, c, b->d_norm[s], b->d_norm[s] + c);
  } else {
    st = layer_norm_to(ctx, k.x, c, b->tmp, c, n, c, b->d_norm[s], b->d_norm[s] + c);
    if (st == IEN_OK)
      st = ien_resize(ctx, b->tmp, grid, grid, c, c, b->level[s] + c, 2 * grid, 2 * grid, 2 * c,
                      IEN_OUT_F16, 0);
  }
  if (st == IEN_OK && s < 3) {
    // swin.rs:377-405 merge: (0,0), (1,0), (0,1), (1,1) by (row, column).
    // The 2 x 2 groups gathered as the LayerNorm over 4c reads them.
    const long half_tokens = n / 4;
    st = layer_norm_to(ctx, k.x, c, k.mrows, 4 * c, half_tokens, 4 * c, b->d_merge_ln[s],
                       b->d_merge_ln[s] + 4 * c, grid / 2);
    if (st == IEN_OK)
      st = rows_product(ctx, k.mrows, 4 * c, 4 * c, half_tokens, b->merge[s], k.x, 2 * c,
                        IEN_ACT_NONE, 0);
  }
  return st;
}

// Both backbones (lib.rs:144-171: the image and its half-size resize), the
// half-size one on branch stream 1, stage by stage beside the full-size
// one: its launches are small and leave most CUs to the other.  The two
// write disjoint columns of the level buffers.
ien_status backbones_run(Birefnet *b, int side, Steps *steps, int *step) {
  ien_ctx *ctx = b->ctx;
  const BackboneBufs full{b->prow, b->x, b->mrows, nullptr, 0};
  const BackboneBufs half{b->hprow, b->hx, b->hmrows, b->hscratch, b->hscratch_halves};
  ien_status st = fork_branches(ctx, 1);
  if (st == IEN_OK) st = backbone_embed(b, full, b->img16, side);
  if (st == IEN_OK) {
    Branch br(ctx, 1);
    st = backbone_embed(b, half, b->half16, side / 2);
  }
  for (int s = 0; s < 4 && st == IEN_OK; s++) {
    st = backbone_stage(b, full, s, side >> (s + 2), false);
    if (st == IEN_OK && steps) st = steps->step(ctx->stream);
    ++*step;
    if (st != IEN_OK) break;
    {
      Branch br(ctx, 1);
      st = backbone_stage(b, half, s, side >> (s + 3), true);
      if (st == IEN_OK && steps) st = steps->step(ctx->stream);
    }
    ++*step;
  }
  // (After a failure or a cancel the branch is joined all the same, so
  // that nothing on it outlives the run.)
  const ien_status js = join_branches(ctx, 1);
  return st != IEN_OK ? st : js;
}

}  // namespace

// swin.rs:110-169 Backbone::load, decoder.rs:779-811 Decoder::load.
ien_status birefnet_load(ien_ctx *ctx, const TensorSource &take, const ShapeOf &shape,
                         Birefnet *b) {
  b->ctx = ctx;
  std::vector<size_t> ps;
  if (!shape("stage0.block0.position_bias", &ps) || ps.size() != 3 || ps[1] != ps[2])
    return fail(IEN_ERR_WEIGHTS, "stage0.block0.position_bias: missing or not [heads][N][N]");
  int window = 1;
  while ((size_t)(window * window) < ps[1]) window++;
  IEN_CHECK((size_t)(window * window) == ps[1] && window >= 2 && window <= 16, IEN_ERR_WEIGHTS,
            "position bias of %zu tokens: not a square window of at most 16", ps[1]);
  b->window = window;
  const size_t N = (size_t)window * window;
  ien_status st = matrix(ctx, take, "patch_embed", 48, 96, true, &b->embed);
  if (st == IEN_OK) st = norm(take, "patch_embed.norm", 96, &b->d_embed_ln);
  for (int s = 0; s < 4 && st == IEN_OK; s++) {
    const size_t c = STAGE_C[s], heads = c / 32;
    for (int k = 0; k < STAGE_DEPTH[s] && st == IEN_OK; k++) {
      const std::string p = "stage" + std::to_string(s) + ".block" + std::to_string(k) + ".";
      std::vector<float> g1, b1, qw, qb, pos, pw, pb, g2, b2, f1w, f1b, f2w, f2b;
      if ((st = take(p + "norm1.weight", {c}, &g1)) != IEN_OK) break;
      if ((st = take(p + "norm1.bias", {c}, &b1)) != IEN_OK) break;
      if ((st = take(p + "qkv.weight", {c, 3 * c}, &qw)) != IEN_OK) break;
      if ((st = take(p + "qkv.bias", {3 * c}, &qb)) != IEN_OK) break;
      if ((st = take(p + "position_bias", {heads, N, N}, &pos)) != IEN_OK) break;
      if ((st = take(p + "proj.weight", {c, c}, &pw)) != IEN_OK) break;
      if ((st = take(p + "proj.bias", {c}, &pb)) != IEN_OK) break;
      if ((st = take(p + "norm2.weight", {c}, &g2)) != IEN_OK) break;
      if ((st = take(p + "norm2.bias", {c}, &b2)) != IEN_OK) break;
      if ((st = take(p + "fc1.weight", {c, 4 * c}, &f1w)) != IEN_OK) break;
      if ((st = take(p + "fc1.bias", {4 * c}, &f1b)) != IEN_OK) break;
      if ((st = take(p + "fc2.weight", {4 * c, c}, &f2w)) != IEN_OK) break;
      if ((st = take(p + "fc2.bias", {c}, &f2b)) != IEN_OK) break;
      ien_swin_weights sw{};
      sw.c = (int)c;
      sw.window = window;
      sw.shift = k % 2 == 1 ? window / 2 : 0;
      sw.masked = MASKED;
      sw.ln1_gamma = g1.data();
      sw.ln1_beta = b1.data();
      sw.qkv_w = qw.data();
      sw.qkv_b = qb.data();
      sw.position = pos.data();
      sw.proj_w = pw.data();
      sw.proj_b = pb.data();
      sw.ln2_gamma = g2.data();
      sw.ln2_beta = b2.data();
      sw.fc1_w = f1w.data();
      sw.fc1_b = f1b.data();
      sw.fc2_w = f2w.data();
      sw.fc2_b = f2b.data();
      ien_swin *blk = nullptr;
      st = ien_swin_new(ctx, &sw, &blk);
      if (st == IEN_OK) b->blocks[s].push_back(blk);
    }
    if (st == IEN_OK && s < 3) {
      const std::string p = "stage" + std::to_string(s) + ".merge";
      st = norm(take, p + ".norm", 4 * c, &b->d_merge_ln[s]);
      if (st == IEN_OK) st = matrix(ctx, take, p, 4 * c, 2 * c, false, &b->merge[s]);
    }
    if (st == IEN_OK) st = norm(take, "stage" + std::to_string(s) + ".norm", c, &b->d_norm[s]);
  }
  if (st == IEN_OK)
    st = load_block(ctx, take, "squeeze", SQUEEZE_CIN, SQUEEZE_COUT, false, &b->dec[0]);
  for (int i = 0; i < 4 && st == IEN_OK; i++)
    st = load_block(ctx, take, "block" + std::to_string(4 - i), LEVEL_CIN[i], LEVEL_COUT[i], i < 3,
                    &b->dec[i + 1]);
  for (const BirefnetBlock &B : b->dec)
    for (ien_matrix *m : B.offset) b->deformable = b->deformable || m != nullptr;
  const int lat_c[3] = {768, 384, 192};
  for (int i = 0; i < 3 && st == IEN_OK; i++)
    st = matrix(ctx, take, "lateral" + std::to_string(4 - i), lat_c[i], lat_c[i], true,
                &b->lateral[i]);
  for (int i = 0; i < 4 && st == IEN_OK; i++) {
    const std::string p = "patches" + std::to_string(5 - i);
    st = matrix(ctx, take, p + ".conv1", 9 * (size_t)PATCH_CIN[i], INTER, true, &b->patch_conv1[i]);
    if (st == IEN_OK)
      st = matrix(ctx, take, p + ".conv_out", 9 * INTER, PATCH_COUT[i], true, &b->patch_out[i]);
  }
  if (st == IEN_OK) st = matrix(ctx, take, "head", 96, 1, false, &b->head);
  if (st == IEN_OK) {
    std::vector<float> hb, c1, b1, co, bo;
    st = take("head.bias", {1}, &hb);
    if (st == IEN_OK) st = take("patches1.conv1.weight", {27, INTER}, &c1);
    if (st == IEN_OK) st = take("patches1.conv1.bias", {INTER}, &b1);
    if (st == IEN_OK) st = take("patches1.conv_out.weight", {9 * INTER, 1}, &co);
    if (st == IEN_OK) st = take("patches1.conv_out.bias", {1}, &bo);
    if (st != IEN_OK) return st;
    b->head_bias = hb[0];
    // decoder.rs:604-630: the composed 5x5 weights and bias, summed in f64.
    double composed[75] = {0};
    double cb = bo[0];
    for (int d = 0; d < 9; d++)
      for (int k = 0; k < INTER; k++) {
        const double w2 = co[d * INTER + k];
        cb += w2 * b1[k];
        for (int e = 0; e < 9; e++) {
          const int ey = d / 3 + e / 3, ex = d % 3 + e % 3;
          for (int c = 0; c < 3; c++) composed[(ey * 5 + ex) * 3 + c] += w2 * c1[(e * 3 + c) * INTER + k];
        }
      }
    std::vector<float> full(76);
    for (int i = 0; i < 75; i++) full[i] = (float)composed[i];
    full[75] = (float)cb;
    full.insert(full.end(), c1.begin(), c1.end());
    full.insert(full.end(), b1.begin(), b1.end());
    full.insert(full.end(), co.begin(), co.end());
    b->bias_out = bo[0];
    st = upload(full, &b->d_full);
  }
  return st;
}

void birefnet_free(Birefnet *b) {
  ien_matrix_free(b->embed);
  (void)hipFree(b->d_embed_ln);
  for (int s = 0; s < 4; s++) {
    for (ien_swin *blk : b->blocks[s]) ien_swin_free(blk);
    b->blocks[s].clear();
    (void)hipFree(b->d_norm[s]);
  }
  for (int s = 0; s < 3; s++) {
    (void)hipFree(b->d_merge_ln[s]);
    ien_matrix_free(b->merge[s]);
    ien_matrix_free(b->lateral[s]);
  }
  for (auto &B : b->dec) free_block(B);
  for (int i = 0; i < 4; i++) {
    ien_matrix_free(b->patch_conv1[i]);
    ien_matrix_free(b->patch_out[i]);
  }
  ien_matrix_free(b->head);
  (void)hipFree(b->d_full);
  free_maps(*b);
  (void)hipFree(b->d_in);
  (void)hipFree(b->d_out);
}

// At side S (P = S^2 pixels): img16 3P, half16 3P/4; patch rows P/16 x 48;
// token map x and merge rows P/16 x 96 (every stage's map holds at most
// that); level s (S/2^(s+2))^2 x 2 c_s; tmp P/64 x 96 (the half run's
// stage maps); x4 (S/32)^2 x 2880; the decoder's input P/16 x 240 (every
// level's g^2 cin is at most that), t and a P/16 x 64, cat P/16 x 1024,
// g P/16 x 16, prev P/16 x 96 (every block's g^2 cout is at most that),
// stacked 3P, mid P/16 x 64, low P/16.
ien_status birefnet_reserve(Birefnet *b, size_t side, bool *grew) {
  *grew = false;
  IEN_CHECK(side >= 64 && side % 64 == 0 && side <= 8192, IEN_ERR_INPUT,
            "side %zu: a multiple of 64 (at most 8192)", side);
  for (int s = 0; s < 4; s++)
    for (ien_swin *blk : b->blocks[s]) {
      ien_status st = swin_reserve(blk, (int)(side >> (s + 2)), (int)(side >> (s + 2)));
      if (st != IEN_OK) return st;
    }
  if (side <= b->side) return IEN_OK;
  IEN_HIP(hipStreamSynchronize(b->ctx->stream));
  free_maps(*b);
  *grew = true;
  const size_t P = side * side, Q = P / 16;
  auto alloc = [](uint16_t **p, size_t halves) { return hipMalloc((void **)p, halves * 2); };
  hipError_t e = alloc(&b->img16, 3 * P);
  if (e == hipSuccess) e = alloc(&b->half16, 3 * P / 4);
  if (e == hipSuccess) e = alloc(&b->prow, Q * 48);
  if (e == hipSuccess) e = alloc(&b->x, Q * 96);
  if (e == hipSuccess) e = alloc(&b->mrows, Q * 96);
  for (int s = 0; s < 4 && e == hipSuccess; s++) {
    const size_t g = side >> (s + 2);
    e = alloc(&b->level[s], g * g * 2 * STAGE_C[s]);
  }
  if (e == hipSuccess) e = alloc(&b->tmp, P / 64 * 96);
  if (e == hipSuccess) e = alloc(&b->x4, (side / 32) * (side / 32) * SQUEEZE_CIN);
  if (e == hipSuccess) e = alloc(&b->in, Q * 240);
  if (e == hipSuccess) e = alloc(&b->t, Q * INTER);
  if (e == hipSuccess) e = alloc(&b->a, Q * INTER);
  if (e == hipSuccess) e = alloc(&b->cat, Q * 4 * BRANCH);
  if (e == hipSuccess) e = alloc(&b->g, Q * 16);
  if (e == hipSuccess) e = alloc(&b->prev, Q * 96);
  if (e == hipSuccess) e = alloc(&b->stacked, 3 * P);
  if (e == hipSuccess) e = alloc(&b->mid, Q * INTER);
  if (e == hipSuccess) e = alloc(&b->low, Q);
  // The half-size backbone: a quarter of the full one's rows, and the
  // largest Swin scratch its blocks take.
  if (e == hipSuccess) e = alloc(&b->hprow, Q / 4 * 48);
  if (e == hipSuccess) e = alloc(&b->hx, Q / 4 * 96);
  if (e == hipSuccess) e = alloc(&b->hmrows, Q / 4 * 96);
  size_t hs = 0;
  for (int s = 0; s < 4; s++)
    for (ien_swin *blk : b->blocks[s]) {
      const int g = (int)(side >> (s + 3));
      hs = std::max(hs, swin_scratch_halves(blk, g, g));
    }
  if (e == hipSuccess) e = alloc(&b->hscratch, std::max<size_t>(hs, 8));
  if (e == hipSuccess) b->hscratch_halves = std::max<size_t>(hs, 8);
  if (e == hipSuccess) e = hipMalloc((void **)&b->partial, POOL_PARTS * INTER * 4);
  // conv1's biases: 64 written per run, padded with zeros to the product's
  // 128-column tiles.
  if (e == hipSuccess) e = hipMalloc((void **)&b->d_bias, 2 * INTER * 4);
  if (e == hipSuccess) e = hipMemset(b->d_bias, 0, 2 * INTER * 4);
  if (e == hipSuccess && b->deformable) {
    e = hipMalloc((void **)&b->offs, Q * 3 * 49 * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&b->samples, SAMPLE_BYTES);
  }
  if (e != hipSuccess) {
    free_maps(*b);
    return fail(IEN_ERR_GPU, "BiRefNet maps for side %zu: %s", side, hipGetErrorString(e));
  }
  b->side = side;
  return IEN_OK;
}

// lib.rs:144-171 run_normalized and decoder.rs:813-926 Decoder::run.
ien_status birefnet_enqueue(Birefnet *b, const float *d_image, size_t side_, float *d_logits,
                            Steps *steps) {
  ien_ctx *ctx = b->ctx;
  IEN_CHECK(b->side >= side_ && side_ % 64 == 0, IEN_ERR_INPUT, "maps not reserved for side %zu",
            side_);
  const int side = (int)side_;
  int step = 0;
  ien_status st = ien_floats_to_halves(ctx, d_image, b->img16, (size_t)side * side * 3);
  if (st == IEN_OK)
    st = ien_resize(ctx, b->img16, side, side, 3, 3, b->half16, side / 2, side / 2, 3, IEN_OUT_F16,
                    0);
  if (st == IEN_OK) st = backbones_run(b, side, steps, &step);
  if (st != IEN_OK) return st;
  // The squeeze block's input: levels 1..3 resized to level 4's grid, then
  // level 4 (decoder.rs:840-859).
  const int g4 = side >> 5;
  int offset = 0;
  for (int s = 0; s < 3 && st == IEN_OK; s++) {
    const int g = side >> (s + 2), c = 2 * STAGE_C[s];
    st = ien_resize(ctx, b->level[s], g, g, c, c, b->x4 + offset, g4, g4, SQUEEZE_CIN, IEN_OUT_F16,
                    0);
    offset += c;
  }
  if (st == IEN_OK)
    st = copy_cols(ctx, b->level[3], (long)g4 * g4, 2 * STAGE_C[3], 2 * STAGE_C[3], b->x4 + offset,
                   SQUEEZE_CIN);
  if (st == IEN_OK) st = block_run(b, b->dec[0], b->x4, g4, g4, b->prev);
  if (st == IEN_OK && steps) st = steps->step(ctx->stream);
  step++;
  int prev_grid = g4;
  for (int i = 0; i < 4 && st == IEN_OK; i++) {
    const int level = 3 - i, cin = LEVEL_CIN[i], g = side >> (level + 2);
    const int main_c = i == 0 ? SQUEEZE_COUT : LEVEL_COUT[i - 1];
    const long pixels = (long)g * g;
    if (i == 0) {
      st = copy_cols(ctx, b->prev, pixels, main_c, main_c, b->in, cin);
    } else {
      const int c = 2 * STAGE_C[level];
      st = rows_product(ctx, b->level[level], c, c, pixels, b->lateral[i - 1], b->in, cin,
                        IEN_ACT_NONE, 0);
      if (st == IEN_OK)
        st = ien_resize(ctx, b->prev, prev_grid, prev_grid, main_c, main_c, b->in, g, g, cin,
                        IEN_OUT_F16, 1);
    }
    // decoder.rs:535-591: the image as patches of g x g, both convolutions.
    if (st == IEN_OK) {
      const int gp = side / g;
      const dim3 grid(blocks_for(pixels * 3 * gp, 256));
      if (gp == 4)
        hipLaunchKernelGGL(k_image_patches<4>, grid, dim3(256), 0, ctx->stream, b->img16, side,
                           b->stacked);
      else if (gp == 8)
        hipLaunchKernelGGL(k_image_patches<8>, grid, dim3(256), 0, ctx->stream, b->img16, side,
                           b->stacked);
      else if (gp == 16)
        hipLaunchKernelGGL(k_image_patches<16>, grid, dim3(256), 0, ctx->stream, b->img16, side,
                           b->stacked);
      else if (gp == 32)
        hipLaunchKernelGGL(k_image_patches<32>, grid, dim3(256), 0, ctx->stream, b->img16, side,
                           b->stacked);
      else
        hipLaunchKernelGGL(k_image_patches_any, dim3(blocks_for(pixels * 3 * gp * gp, 256)),
                           dim3(256), 0, ctx->stream, b->img16, side, g, b->stacked);
      IEN_HIP(hipGetLastError());
      st = conv(ctx, b->stacked, g, g, 3 * gp * gp, 3 * gp * gp, 3, b->patch_conv1[i], b->mid,
                INTER, IEN_ACT_NONE, 0);
    }
    if (st == IEN_OK)
      st = conv(ctx, b->mid, g, g, INTER, INTER, 3, b->patch_out[i], b->in + main_c, cin,
                IEN_ACT_NONE, 0);
    if (st == IEN_OK) st = block_run(b, b->dec[i + 1], b->in, g, g, b->prev);
    if (st == IEN_OK && steps) st = steps->step(ctx->stream);
    step++;
    prev_grid = g;
  }
  if (st != IEN_OK) return st;
  // The head before the final resize, then the full-resolution branch
  // (decoder.rs:885-926).
  const long low_pixels = (long)prev_grid * prev_grid;
  st = rows_product(ctx, b->prev, 96, 96, low_pixels, b->head, b->low, 1, IEN_ACT_NONE, 0);
  if (st != IEN_OK) return st;
  const FullParams fp{b->d_full, b->d_full + 76, b->d_full + 76 + 27 * INTER,
                      b->d_full + 76 + 28 * INTER, b->bias_out, b->head_bias};
  hipLaunchKernelGGL(k_full_res, dim3((unsigned)((side / FT) * (side / FT))), dim3(256), 0,
                     ctx->stream, d_image, side, fp, d_logits);
  IEN_HIP(hipGetLastError());
  st = ien_resize(ctx, b->low, prev_grid, prev_grid, 1, 1, d_logits, side, side, 1, IEN_OUT_F32, 1);
  if (st == IEN_OK && steps) st = steps->step(ctx->stream);
  return st;
}

}  // namespace ien
