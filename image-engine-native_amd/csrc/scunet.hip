// scunet.hip -- the SCUNet U-Net on the GPU (crates/scunet-native/src/
// network.rs:113-354): f16 NHWC maps, the block's 3x3 convolutions and the
// head and tail through the implicit-GEMM kernels, 1x1 products over pixel
// rows (a block's join and the next block's split in one pass at 64 and
// 128 channels), the Swin half through ien_swin, the 2x2 halving and doubling
// convolutions as row products that gather / scatter 2 x 2 pixel groups
// themselves.  One event is
// recorded after each of the 28 blocks for progress reports.

#include <algorithm>
#include <string>

#include "ien_internal.h"
#include "scunet.h"

namespace ien {

namespace {

constexpr int DIM = 64, BLOCKS = 4, WINDOW = 8, MULTIPLE = 64;

// A 3x3 zero-padded convolution of an h x w f16 NHWC map.
ien_status conv3(ien_ctx *ctx, const uint16_t *x, int h, int w, int c, long xs,
                 const ien_matrix *m, void *y, long ys, ien_act act, int accumulate) {
  ConvCall cc;
  cc.x = x;
  cc.H = h;
  cc.W = w;
  cc.C = c;
  cc.xs = xs;
  cc.ks = 3;
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

ien_status matrix(ien_ctx *ctx, const TensorSource &take, const std::string &name, size_t k,
                  size_t n, bool bias, ien_matrix **out) {
  std::vector<float> w, b;
  ien_status st = take(name + ".weight", {k, n}, &w);
  if (st == IEN_OK && bias) st = take(name + ".bias", {n}, &b);
  if (st != IEN_OK) return st;
  return ien_matrix_new(ctx, w.data(), IEN_W_F32, k, n, bias ? b.data() : nullptr, out);
}

// swin.rs:98-120 Transformer::load and network.rs:122-134 Block::load.
ien_status load_block(ien_ctx *ctx, const TensorSource &take, const std::string &name, int c,
                      bool shifted, ScunetBlock *b) {
  const size_t h = (size_t)c / 2;
  b->c = c;
  ien_status st = matrix(ctx, take, name + ".conv1_1", c, c, true, &b->split);
  if (st == IEN_OK) st = matrix(ctx, take, name + ".conv_block.0", 9 * h, h, false, &b->conv1);
  if (st == IEN_OK) st = matrix(ctx, take, name + ".conv_block.2", 9 * h, h, false, &b->conv2);
  if (st == IEN_OK) st = matrix(ctx, take, name + ".conv1_2", c, c, true, &b->join);
  if (st != IEN_OK) return st;
  const std::string t = name + ".trans_block";
  std::vector<float> g1, b1, qw, qb, pos, pw, pb, g2, b2, f1w, f1b, f2w, f2b;
  const size_t heads = h / 32;
  if ((st = take(t + ".ln1.weight", {h}, &g1)) != IEN_OK) return st;
  if ((st = take(t + ".ln1.bias", {h}, &b1)) != IEN_OK) return st;
  if ((st = take(t + ".msa.embedding_layer.weight", {h, 3 * h}, &qw)) != IEN_OK) return st;
  if ((st = take(t + ".msa.embedding_layer.bias", {3 * h}, &qb)) != IEN_OK) return st;
  if ((st = take(t + ".msa.position_bias", {heads, 64, 64}, &pos)) != IEN_OK) return st;
  if ((st = take(t + ".msa.linear.weight", {h, h}, &pw)) != IEN_OK) return st;
  if ((st = take(t + ".msa.linear.bias", {h}, &pb)) != IEN_OK) return st;
  if ((st = take(t + ".ln2.weight", {h}, &g2)) != IEN_OK) return st;
  if ((st = take(t + ".ln2.bias", {h}, &b2)) != IEN_OK) return st;
  if ((st = take(t + ".mlp.0.weight", {h, 4 * h}, &f1w)) != IEN_OK) return st;
  if ((st = take(t + ".mlp.0.bias", {4 * h}, &f1b)) != IEN_OK) return st;
  if ((st = take(t + ".mlp.2.weight", {4 * h, h}, &f2w)) != IEN_OK) return st;
  if ((st = take(t + ".mlp.2.bias", {h}, &f2b)) != IEN_OK) return st;
  ien_swin_weights sw{};
  sw.c = (int)h;
  sw.window = WINDOW;
  sw.shift = shifted ? WINDOW / 2 : 0;
  sw.masked = -__builtin_inff();
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
  return ien_swin_new(ctx, &sw, &b->swin);
}

void free_block(ScunetBlock &b) {
  ien_matrix_free(b.split);
  ien_matrix_free(b.conv1);
  ien_matrix_free(b.conv2);
  ien_matrix_free(b.join);
  ien_swin_free(b.swin);
  b = ScunetBlock();
}

void free_maps(Scunet &s) {
  for (uint16_t **p : {&s.img, &s.x, &s.y, &s.t, &s.skip[0], &s.skip[1], &s.skip[2],
                       &s.out16}) {
    (void)hipFree(*p);
    *p = nullptr;
  }
  s.pixels = 0;
}

// network.rs:158-208 run_level on the h x w map x of c channels (y, t:
// the block's buffers).  The split map y (network.rs:9-13: the convolution
// half in channels 0 .. c/2, the Swin half after it) is kept as two planes
// of c/2 channels, y and y + pixels c/2, so that the two branches, which
// run on two streams, write no common cache line; the split product writes
// both planes and the join reads both, in the channel order of one map.
// `add_after`, when not null, is added onto x after the last block (the
// skip of the level below), in the last join's pass.
ien_status run_level(Scunet &s, ScunetBlock *blocks, int h, int w, int c, Steps *steps,
                     int *step, const uint16_t *add_after = nullptr) {
  ien_ctx *ctx = s.ctx;
  const size_t pixels = (size_t)h * w, half = (size_t)c / 2;
  uint16_t *yc = s.y, *ysw = s.y + pixels * half;
  auto split = [&](const ien_matrix *m) {
    RowsPlanes p;
    p.x = p.x2 = s.x;
    p.xs = p.xs2 = c;
    p.k1 = c;
    p.rows = (long)pixels;
    p.w = m;
    p.y = yc;
    p.y2 = ysw;
    p.ys = p.ys2 = (int)half;
    p.n1 = (int)half;
    return launch_rows_planes(ctx, p);
  };
  auto join = [&](const ien_matrix *m, const uint16_t *add) {
    RowsPlanes p;
    p.x = yc;
    p.x2 = ysw;
    p.xs = p.xs2 = (int)half;
    p.k1 = (int)half;
    p.rows = (long)pixels;
    p.w = m;
    p.y = p.y2 = s.x;
    p.ys = p.ys2 = c;
    p.n1 = c;
    p.accumulate = 1;
    p.add = add;
    return launch_rows_planes(ctx, p);
  };
  ien_status st = split(blocks[0].split);
  for (int b = 0; b < BLOCKS && st == IEN_OK; b++) {
    ScunetBlock &B = blocks[b];
    // The two halves are independent until the join: the convolution half
    // on branch 1, the Swin half (the longer) on the context's stream,
    // enqueued first.
    st = fork_branches(ctx, 1);
    if (st == IEN_OK) st = ien_swin_run(B.swin, ysw, half, h, w);
    if (st == IEN_OK) {
      Branch br(ctx, 1);
      // network.rs:135-153 convolve: conv3 + ReLU into t, conv3 added back.
      // Single-buffered: double-buffered chunks (one workgroup of 104 KiB
      // LDS a CU) crowded out the Swin half's kernels (1% slower per image).
      ctx->compact = true;
      st = conv3(ctx, yc, h, w, (int)half, (long)half, B.conv1, s.t, (long)half, IEN_ACT_RELU, 0);
      if (st == IEN_OK)
        st = conv3(ctx, s.t, h, w, (int)half, (long)half, B.conv2, yc, (long)half, IEN_ACT_NONE, 1);
      ctx->compact = false;
    }
    if (st == IEN_OK) st = join_branches(ctx, 1);
    // The join and the next block's split in one pass where it applies
    // (64 and 128 channels), else as two row products.
    JoinSplit js;
    js.yc = yc;
    js.ysw = ysw;
    js.x = s.x;
    js.rows = (long)pixels;
    js.c = c;
    js.join = B.join;
    js.split = b + 1 < BLOCKS ? blocks[b + 1].split : nullptr;
    if (st == IEN_OK && b + 1 < BLOCKS && join_split_supported(js)) {
      st = launch_join_split(ctx, js);
    } else {
      if (st == IEN_OK) st = join(B.join, b + 1 < BLOCKS ? nullptr : add_after);
      if (st == IEN_OK && b + 1 < BLOCKS) st = split(blocks[b + 1].split);
    }
    if (st == IEN_OK && steps) st = steps->step(ctx->stream);
    ++*step;
  }
  return st;
}

}  // namespace

ien_status scunet_load(ien_ctx *ctx, const TensorSource &take, Scunet *s) {
  s->ctx = ctx;
  // The head reads the image map's 4 channels (the fourth is zero): its
  // 27 x DIM weights with a zero row after each tap's 3, so that K = 9 x 4
  // runs on the four-channel kernel.
  std::vector<float> head;
  ien_status st = take("m_head.0.weight", {27, DIM}, &head);
  if (st == IEN_OK) {
    std::vector<float> head4((size_t)36 * DIM, 0.0f);
    for (int t = 0; t < 9; t++)
      for (int c = 0; c < 3; c++)
        std::copy_n(&head[(size_t)(t * 3 + c) * DIM], DIM, &head4[(size_t)(t * 4 + c) * DIM]);
    st = ien_matrix_new(ctx, head4.data(), IEN_W_F32, 36, DIM, nullptr, &s->head);
  }
  for (int l = 0; l < 3 && st == IEN_OK; l++) {
    const int c = DIM << l;
    const std::string name = "m_down" + std::to_string(l + 1);
    for (int b = 0; b < BLOCKS && st == IEN_OK; b++)
      st = load_block(ctx, take, name + "." + std::to_string(b), c, b % 2 == 1, &s->down[l][b]);
    if (st == IEN_OK)
      st = matrix(ctx, take, name + "." + std::to_string(BLOCKS), 4 * c, 2 * c, false, &s->halve[l]);
  }
  for (int b = 0; b < BLOCKS && st == IEN_OK; b++)
    st = load_block(ctx, take, "m_body." + std::to_string(b), 8 * DIM, b % 2 == 1, &s->body[b]);
  for (int l = 0; l < 3 && st == IEN_OK; l++) {
    const int c = DIM << (2 - l);
    const std::string name = "m_up" + std::to_string(3 - l);
    st = matrix(ctx, take, name + ".0", 2 * c, 4 * c, false, &s->dbl[l]);
    for (int b = 0; b < BLOCKS && st == IEN_OK; b++)
      st = load_block(ctx, take, name + "." + std::to_string(b + 1), c, b % 2 == 1, &s->up[l][b]);
  }
  if (st == IEN_OK) st = matrix(ctx, take, "m_tail.0", 9 * DIM, 3, false, &s->tail);
  return st;
}

void scunet_free(Scunet *s) {
  ien_matrix_free(s->head);
  ien_matrix_free(s->tail);
  for (int l = 0; l < 3; l++) {
    for (int b = 0; b < BLOCKS; b++) {
      free_block(s->down[l][b]);
      free_block(s->up[l][b]);
    }
    ien_matrix_free(s->halve[l]);
    ien_matrix_free(s->dbl[l]);
  }
  for (int b = 0; b < BLOCKS; b++) free_block(s->body[b]);
  free_maps(*s);
  (void)hipFree(s->d_in);
  (void)hipFree(s->d_out);
}

void scunet_padded(size_t width, size_t height, size_t *pw, size_t *ph) {
  *pw = (width + MULTIPLE - 1) / MULTIPLE * MULTIPLE;
  *ph = (height + MULTIPLE - 1) / MULTIPLE * MULTIPLE;
}

// The maps grow on demand (never shrink): at the padded size P pixels, x and
// y hold P x 64 halves (every level's c-channel map has at most that), t
// P x 32, the skips P/4 x 128, P/16 x 256, P/64 x 512.
ien_status scunet_reserve(Scunet *s, size_t pw, size_t ph) {
  // Each level's blocks: down l at 1 / 2^l, the body at 1 / 8, up l at
  // 1 / 2^(2 - l).
  for (int l = 0; l < 3; l++)
    for (int b = 0; b < BLOCKS; b++) {
      ien_status st = swin_reserve(s->down[l][b].swin, (int)(ph >> l), (int)(pw >> l));
      if (st == IEN_OK)
        st = swin_reserve(s->up[l][b].swin, (int)(ph >> (2 - l)), (int)(pw >> (2 - l)));
      if (st != IEN_OK) return st;
    }
  for (int b = 0; b < BLOCKS; b++) {
    ien_status st = swin_reserve(s->body[b].swin, (int)(ph >> 3), (int)(pw >> 3));
    if (st != IEN_OK) return st;
  }
  const size_t padded_pixels = pw * ph;
  if (padded_pixels <= s->pixels) return IEN_OK;
  IEN_HIP(hipStreamSynchronize(s->ctx->stream));
  free_maps(*s);
  const size_t P = padded_pixels;
  auto alloc = [](uint16_t **p, size_t halves) { return hipMalloc((void **)p, halves * 2); };
  hipError_t e = alloc(&s->img, P * 8);
  // Channels 3..7 of the image map stay zero (the head reads channel 3).
  if (e == hipSuccess) e = hipMemsetAsync(s->img, 0, P * 8 * 2, s->ctx->stream);
  if (e == hipSuccess) e = alloc(&s->x, P * DIM);
  if (e == hipSuccess) e = alloc(&s->y, P * DIM);
  if (e == hipSuccess) e = alloc(&s->t, P * DIM / 2);
  for (int l = 0; l < 3 && e == hipSuccess; l++) e = alloc(&s->skip[l], (P >> (2 * l + 2)) * (128 << l));
  if (e == hipSuccess) e = alloc(&s->out16, P * 4);
  if (e != hipSuccess) {
    free_maps(*s);
    return fail(IEN_ERR_GPU, "SCUNet maps for %zu pixels: %s", P, hipGetErrorString(e));
  }
  s->pixels = P;
  return IEN_OK;
}

// network.rs:262-354 run: d_image (f32 height x width x 3) to d_out (the
// same shape); maps reserved for the padded size.
ien_status scunet_enqueue(Scunet *s, const float *d_image, size_t width, size_t height,
                          float *d_out, Steps *steps) {
  ien_ctx *ctx = s->ctx;
  size_t pw, ph;
  scunet_padded(width, height, &pw, &ph);
  ien_status st = ien_pad_image(ctx, IEN_PAD_REPLICATE, d_image, nullptr, width, height,
                                MULTIPLE, s->img, 8);
  if (st != IEN_OK) return st;
  int h = (int)ph, w = (int)pw, c = DIM, step = 0;
  // The head (no bias); computed again at the end as the skip into the tail.
  if ((st = conv3(ctx, s->img, h, w, 4, 8, s->head, s->x, DIM, IEN_ACT_NONE, 0)) != IEN_OK) return st;
  // The halving writes the skip and a working copy in y, which then takes
  // the part of x (y is free between levels); the doubling writes its
  // scattered output into y likewise.  Swapped back after the enqueue.
  bool swapped = false;
  auto unswap = [&]() {
    if (swapped) std::swap(s->x, s->y);
    swapped = false;
  };
  for (int l = 0; l < 3; l++) {
    if ((st = run_level(*s, s->down[l], h, w, c, steps, &step)) != IEN_OK) return unswap(), st;
    // network.rs:403-437 halved, kept as the skip of the level up: a
    // product over the map's 2 x 2 pixel groups.
    const size_t q = (size_t)(h / 2) * (w / 2);
    {
      RowsPlanes p;
      p.x = p.x2 = s->x;
      p.xs = p.xs2 = c;
      p.k1 = 4 * c;
      p.rows = (long)q;
      p.w = s->halve[l];
      p.y = p.y2 = s->skip[l];
      p.ys = p.ys2 = 2 * c;
      p.n1 = 2 * c;
      p.gather_w2 = w / 2;
      p.ydup = s->y;
      if ((st = launch_rows_planes(ctx, p)) != IEN_OK) return unswap(), st;
    }
    std::swap(s->x, s->y);
    swapped = !swapped;
    h /= 2;
    w /= 2;
    c *= 2;
  }
  // Each level up starts from the map plus the skip of its size, added in
  // the last join of the level below it.
  if ((st = run_level(*s, s->body, h, w, c, steps, &step, s->skip[2])) != IEN_OK)
    return unswap(), st;
  for (int l = 0; l < 3; l++) {
    const size_t pixels = (size_t)h * w;
    // network.rs:439-478 doubled: each pixel's product scattered over its 2
    // x 2 output pixels.
    {
      RowsPlanes p;
      p.x = p.x2 = s->x;
      p.xs = p.xs2 = c;
      p.k1 = c;
      p.rows = (long)pixels;
      p.w = s->dbl[l];
      p.y = p.y2 = s->y;
      p.ys = p.ys2 = c / 2;
      p.n1 = 2 * c;
      p.scatter_w = w;
      if ((st = launch_rows_planes(ctx, p)) != IEN_OK) return unswap(), st;
    }
    std::swap(s->x, s->y);
    swapped = !swapped;
    h *= 2;
    w *= 2;
    c /= 2;
    if ((st = run_level(*s, s->up[l], h, w, c, steps, &step, l < 2 ? s->skip[1 - l] : nullptr)) !=
        IEN_OK)
      return unswap(), st;
  }
  if ((st = conv3(ctx, s->img, h, w, 4, 8, s->head, s->x, DIM, IEN_ACT_NONE, 1)) != IEN_OK)
    return unswap(), st;
  st = conv3(ctx, s->x, h, w, DIM, DIM, s->tail, s->out16, 4, IEN_ACT_NONE, 0);
  unswap();
  if (st != IEN_OK) return st;
  return ien_crop(ctx, s->out16, pw, 4, width, height, 3, d_out);
}

}  // namespace ien
