// lama.hip -- Big LaMa's generator on the GPU (crates/lama-native/src/
// network.rs): f16 NHWC maps; every convolution through the implicit-GEMM
// kernels (7x7 and 3x3 reflect-padded, 3x3 stride 2, the transposed
// upsamplings as four output-phase products with offset taps, then a 2 x 2
// scatter); the spectral branch's 1x1 convolutions as products over pixel
// or spectrum rows around the Fourier units of fourier.hip.  One event is
// recorded after each of the 26 steps for progress reports.

#include <string>

#include "lama.h"

namespace ien {

namespace {

constexpr int LOCAL = 128, GLOBAL = 384, CHANNELS = 512, SPECTRAL = 192, BLOCKS = 18;
constexpr int MULTIPLE = 8;

// network.rs:271 PHASE_TAPS: output phase p = 2 py + px reads input offsets
// (dy, dx) over the taps of py times those of px.
constexpr int PHASE_COUNT[2] = {1, 2};
constexpr int PHASE_OFFSET[2][2] = {{0, 0}, {0, 1}};

ien_status matrix(ien_ctx *ctx, const TensorSource &take, const std::string &name, size_t k,
                  size_t n, bool bias, ien_matrix **out) {
  std::vector<float> w, b;
  ien_status st = take(name + ".weight", {k, n}, &w);
  if (st == IEN_OK && bias) st = take(name + ".bias", {n}, &b);
  if (st != IEN_OK) return st;
  return ien_matrix_new(ctx, w.data(), IEN_W_F32, k, n, bias ? b.data() : nullptr, out);
}

// A size x size convolution (reflect padding) of an h x w f16 NHWC map.
ien_status conv(ien_ctx *ctx, const uint16_t *x, int h, int w, int c, long xs, int size,
                int step, const ien_matrix *m, uint16_t *y, long ys, ien_act act,
                int accumulate, const uint16_t *add2 = nullptr) {
  ConvCall cc;
  cc.add2 = add2;
  cc.x = x;
  cc.H = h;
  cc.W = w;
  cc.C = c;
  cc.xs = xs;
  cc.ks = size;
  cc.stride = step;
  cc.pad_reflect = size > 1;
  cc.OH = (h - 1) / step + 1;
  cc.OW = (w - 1) / step + 1;
  cc.row0 = 0;
  cc.rows = (long)cc.OH * cc.OW;
  cc.w = m;
  cc.y = y;
  cc.ys = ys;
  cc.act = act;
  cc.accumulate = accumulate;
  return launch_conv(ctx, cc);
}

// out[r] = act((acc ? out[r] : 0) + in[r] m) over `rows` rows of k values.
ien_status rows_product(ien_ctx *ctx, const uint16_t *in, size_t k, size_t rows,
                        const ien_matrix *m, uint16_t *out, long ys, ien_act act,
                        int accumulate) {
  ConvCall cc;
  cc.x = in;
  cc.rows_mode = 1;
  cc.C = (int)k;
  cc.xs = (long)k;
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

// network.rs:174-249 Ffc::run: out = ffc(x), both h x w maps of 512, with
// the unfused spectral chain (maps of sides over 64; the fused branch runs
// in ffc_pipeline).
ien_status ffc_run(Lama *l, const LamaFfc &f, const uint16_t *x, uint16_t *out, int h, int w) {
  ien_ctx *ctx = l->ctx;
  const size_t pixels = (size_t)h * w, half = (size_t)w / 2 + 1, spix = (size_t)h * half;
  // Unfused: local on the context's stream, cross on branch 1, the spectral
  // chain on branch 2, joined before the accumulation.
  ien_status st = fork_branches(ctx, 2);
  // local: all 512 channels -> 128, ReLU.
  if (st == IEN_OK)
    st = conv(ctx, x, h, w, CHANNELS, CHANNELS, 3, 1, f.local, out, CHANNELS, IEN_ACT_RELU, 0);
  // cross: the local part -> the global part, no activation yet.
  if (st == IEN_OK) {
    Branch b(ctx, 1);
    st = conv(ctx, x, h, w, LOCAL, CHANNELS, 3, 1, f.cross, out + LOCAL, CHANNELS, IEN_ACT_NONE,
              0);
  }
  if (st == IEN_OK) {
    Branch b(ctx, 2);
    // spectral_in: 1x1 of the global part -> 192, ReLU.
    st = conv(ctx, x + LOCAL, h, w, GLOBAL, CHANNELS, 1, 1, f.spectral_in, l->spectral, SPECTRAL,
              IEN_ACT_RELU, 0);
    if (st == IEN_OK)
      st = ien_fourier_forward(l->fourier, l->spectral, SPECTRAL, SPECTRAL, l->work, l->spectrum);
    // fourier: 1x1 over spectrum pixels [re | im] -> the same, ReLU.
    if (st == IEN_OK)
      st = rows_product(ctx, l->spectrum, 2 * SPECTRAL, spix, f.fourier, l->filtered,
                        2 * SPECTRAL, IEN_ACT_RELU, 0);
    // spectral += irfft(filtered).
    if (st == IEN_OK)
      st = ien_fourier_inverse(l->fourier, l->filtered, SPECTRAL, l->work, l->spectral, SPECTRAL);
  }
  if (st == IEN_OK) st = join_branches(ctx, 2);
  // global = ReLU(cross + spectral_out(spectral)).
  if (st == IEN_OK)
    st = rows_product(ctx, l->spectral, SPECTRAL, pixels, f.spectral_out, out + LOCAL, CHANNELS,
                      IEN_ACT_RELU, 1);
  return st;
}

// network.rs:279-335 Up::run: the four phase products, each storing its
// outputs straight to their pixels of the doubled map (phase p = 2 py + px
// to pixel (2 y + py, 2 x + px)).
ien_status up_run(Lama *l, ien_matrix *const *phases, const uint16_t *x, int h, int w, int cin,
                  int cout, uint16_t *y) {
  for (int p = 0; p < 4; p++) {
    const int py = p / 2, px = p % 2;
    ConvCall cc;
    cc.x = x;
    cc.H = h;
    cc.W = w;
    cc.C = cin;
    cc.xs = cin;
    cc.noff = 0;
    for (int a = 0; a < PHASE_COUNT[py]; a++)
      for (int b = 0; b < PHASE_COUNT[px]; b++) {
        cc.offy[cc.noff] = PHASE_OFFSET[py][a];
        cc.offx[cc.noff] = PHASE_OFFSET[px][b];
        cc.noff++;
      }
    cc.ks = 0;
    cc.stride = 1;
    cc.OH = h;
    cc.OW = w;
    cc.row0 = 0;
    cc.rows = (long)h * w;
    cc.w = phases[p];
    cc.y = y;
    cc.ys = cout;
    cc.phase = 1 + p;
    cc.act = IEN_ACT_RELU;
    ien_status st = launch_conv(l->ctx, cc);
    if (st != IEN_OK) return st;
  }
  return IEN_OK;
}

void free_maps(Lama &l) {
  for (uint16_t **p : {&l.in4, &l.m0, &l.m1, &l.m2, &l.a, &l.mid, &l.out, &l.spectral,
                       &l.spectrum, &l.filtered, &l.rgb}) {
    (void)hipFree(*p);
    *p = nullptr;
  }
  (void)hipFree(l.work);
  l.work = nullptr;
  l.pixels = 0;
}

}  // namespace

// network.rs:381-413 Network::load (names as tools/lama/export_weights.py
// writes them).
ien_status lama_load(ien_ctx *ctx, const TensorSource &take, Lama *l) {
  l->ctx = ctx;
  IEN_HIP(hipEventCreateWithFlags(&l->ev_local, hipEventDisableTiming));
  IEN_HIP(hipEventCreateWithFlags(&l->ev_cross, hipEventDisableTiming));
  ien_status st = matrix(ctx, take, "first", 49 * 4, 64, true, &l->first);
  const int dins[3] = {64, 128, 256}, douts[3] = {128, 256, CHANNELS};
  for (int i = 0; i < 3 && st == IEN_OK; i++)
    st = matrix(ctx, take, "down" + std::to_string(i), 9 * (size_t)dins[i], douts[i], true,
                &l->down[i]);
  for (int b = 0; b < BLOCKS && st == IEN_OK; b++)
    for (int f = 0; f < 2 && st == IEN_OK; f++) {
      const std::string n = "block" + std::to_string(b) + ".ffc" + std::to_string(f);
      LamaFfc &F = l->blocks[b][f];
      st = matrix(ctx, take, n + ".local", 9 * CHANNELS, LOCAL, true, &F.local);
      if (st == IEN_OK) st = matrix(ctx, take, n + ".cross", 9 * LOCAL, GLOBAL, true, &F.cross);
      if (st == IEN_OK)
        st = matrix(ctx, take, n + ".spectral_in", GLOBAL, SPECTRAL, true, &F.spectral_in);
      if (st == IEN_OK)
        st = matrix(ctx, take, n + ".fourier", 2 * SPECTRAL, 2 * SPECTRAL, true, &F.fourier);
      if (st == IEN_OK)
        st = matrix(ctx, take, n + ".spectral_out", SPECTRAL, GLOBAL, false, &F.spectral_out);
    }
  const int uins[3] = {CHANNELS, 256, 128}, uouts[3] = {256, 128, 64};
  for (int i = 0; i < 3 && st == IEN_OK; i++)
    for (int p = 0; p < 4 && st == IEN_OK; p++) {
      const size_t taps = (size_t)PHASE_COUNT[p / 2] * PHASE_COUNT[p % 2];
      st = matrix(ctx, take, "up" + std::to_string(i) + ".phase" + std::to_string(p),
                  taps * uins[i], uouts[i], true, &l->up[i][p]);
    }
  if (st == IEN_OK) st = matrix(ctx, take, "last", 49 * 64, 3, true, &l->last);
  return st;
}

void lama_free(Lama *l) {
  ien_matrix_free(l->first);
  ien_matrix_free(l->last);
  for (int i = 0; i < 3; i++) {
    ien_matrix_free(l->down[i]);
    for (int p = 0; p < 4; p++) ien_matrix_free(l->up[i][p]);
  }
  for (auto &pair : l->blocks)
    for (LamaFfc &f : pair) {
      ien_matrix_free(f.local);
      ien_matrix_free(f.cross);
      ien_matrix_free(f.spectral_in);
      ien_matrix_free(f.fourier);
      ien_matrix_free(f.spectral_out);
    }
  ien_fourier_free(l->fourier);
  l->fourier = nullptr;
  ien_spectral_free(l->spectral_plan);
  l->spectral_plan = nullptr;
  free_maps(*l);
  (void)hipFree(l->d_in);
  (void)hipFree(l->d_mask);
  (void)hipFree(l->d_out);
  if (l->ev_local) (void)hipEventDestroy(l->ev_local);
  if (l->ev_cross) (void)hipEventDestroy(l->ev_cross);
  l->ev_local = l->ev_cross = nullptr;
}

// network.rs:337-344 padded: sides to multiples of 8.
void lama_padded(size_t width, size_t height, size_t *pw, size_t *ph) {
  *pw = (width + MULTIPLE - 1) / MULTIPLE * MULTIPLE;
  *ph = (height + MULTIPLE - 1) / MULTIPLE * MULTIPLE;
}

// At P padded pixels: in4 P x 4; m0 P x 64, m1 P/4 x 128, m2 P/16 x 256
// (the downs, then the ups' outputs); a, mid, out P/64 x 512; spectral
// P/64 x 192; spectrum and filtered (h/8)(w/16 + 1) <= P/64 pixels of 384
// values and the f32 work as large; rows P x 64 (the largest phase product, 4 x 64 channels at
// P/4); rgb P x 3.  Maps grow and never shrink; the Fourier plan follows
// the size.
ien_status lama_reserve(Lama *l, size_t pw, size_t ph, bool *grew) {
  *grew = false;
  IEN_CHECK(pw >= 16 && ph >= 16 && pw % MULTIPLE == 0 && ph % MULTIPLE == 0, IEN_ERR_INPUT,
            "padded %zu x %zu", pw, ph);
  const size_t h8 = ph / 8, w8 = pw / 8;
  if (!l->fourier || l->pw != pw || l->ph != ph) {
    IEN_HIP(hipStreamSynchronize(l->ctx->stream));
    ien_fourier_free(l->fourier);
    l->fourier = nullptr;
    ien_spectral_free(l->spectral_plan);
    l->spectral_plan = nullptr;
    ien_status st = ien_fourier_new(l->ctx, h8, w8, &l->fourier);
    // The fused spectral branch takes maps of sides up to 64 (images up to
    // 512 x 512); larger ones run the unfused chain.
    if (st == IEN_OK && h8 <= 64 && w8 <= 64)
      st = ien_spectral_new(l->ctx, h8, w8, &l->spectral_plan);
    if (st != IEN_OK) return st;
    l->pw = pw;
    l->ph = ph;
    *grew = true;
  }
  const size_t P = pw * ph;
  if (P <= l->pixels) return IEN_OK;
  IEN_HIP(hipStreamSynchronize(l->ctx->stream));
  free_maps(*l);
  *grew = true;
  // A spectrum has h8 (w8 / 2 + 1) <= h8 w8 = P / 64 pixels (w8 >= 2).
  const size_t S = P / 64;
  auto alloc = [](uint16_t **p, size_t halves) { return hipMalloc((void **)p, halves * 2); };
  hipError_t e = alloc(&l->in4, P * 4);
  if (e == hipSuccess) e = alloc(&l->m0, P * 64);
  if (e == hipSuccess) e = alloc(&l->m1, P / 4 * 128);
  if (e == hipSuccess) e = alloc(&l->m2, P / 16 * 256);
  if (e == hipSuccess) e = alloc(&l->a, P / 64 * CHANNELS);
  if (e == hipSuccess) e = alloc(&l->mid, P / 64 * CHANNELS);
  if (e == hipSuccess) e = alloc(&l->out, P / 64 * CHANNELS);
  if (e == hipSuccess) e = alloc(&l->spectral, P / 64 * SPECTRAL);
  if (e == hipSuccess) e = alloc(&l->spectrum, S * 2 * SPECTRAL);
  if (e == hipSuccess) e = alloc(&l->filtered, S * 2 * SPECTRAL);
  if (e == hipSuccess) e = alloc(&l->rgb, P * 3);
  if (e == hipSuccess) e = hipMalloc((void **)&l->work, S * 2 * SPECTRAL * 4);
  if (e != hipSuccess) {
    free_maps(*l);
    return fail(IEN_ERR_GPU, "LaMa maps for %zu pixels: %s", P, hipGetErrorString(e));
  }
  l->pixels = P;
  return IEN_OK;
}

// network.rs:415-489 Network::run.
// The 18 blocks' FFCs with the fused spectral branch (network.rs:249-262,
// x += ffc1(ffc0(x)): the second FFC's local convolution and back launch
// add their rounded results onto x in place, the sums ien_add would make),
// as a pipeline over three streams.  FFC k: its spectral rows (192 short
// workgroups) and then its local convolution on the context's stream (the
// local convolution enqueued before the branches' launches, so that its
// workgroups, one a CU, are not held back behind theirs), its spectral
// columns on branch 1, its back launch on the context's stream after both
// (R in the spectrum buffer, U in the work buffer).  Its cross
// convolution reads only the local part of its input, which the previous
// FFC's local convolution has written: it runs on branch 2 from there on,
// beside that FFC's columns and back launch (which leave CUs idle: 192
// workgroups of one a CU each).  What the early cross convolution writes
// (the global part of FFC k's output map) no launch before FFC k's back
// reads: FFC k - 1 reads the other map (or, for the second FFC of a
// block, x, whose global part it only reads in its rows and local launches,
// both before the wait).
template <class Done>
ien_status ffc_pipeline(Lama *l, int h, int w, Done &done) {
  ien_ctx *ctx = l->ctx;
  struct Ffc {
    const LamaFfc *f;
    const uint16_t *x;
    uint16_t *out, *residual;
  };
  Ffc ffcs[2 * BLOCKS];
  for (int b = 0; b < BLOCKS; b++) {
    ffcs[2 * b] = {&l->blocks[b][0], l->a, l->mid, nullptr};
    ffcs[2 * b + 1] = {&l->blocks[b][1], l->mid, l->out, l->a};
  }
  constexpr int N = 2 * BLOCKS;
  auto cross = [&](const Ffc &c) {
    return conv(ctx, c.x, h, w, LOCAL, CHANNELS, 3, 1, c.f->cross, c.out + LOCAL, CHANNELS,
                IEN_ACT_NONE, 0);
  };
  const bool split = !ctx->serial_branches;
  hipStream_t branch2 = ctx->branch[1];
  // The first cross convolution: x's local part is final now.
  ien_status st = IEN_OK;
  if (split) {
    IEN_HIP(hipEventRecord(l->ev_local, ctx->stream));
    IEN_HIP(hipStreamWaitEvent(branch2, l->ev_local, 0));
  }
  {
    Branch br(ctx, 2);
    st = cross(ffcs[0]);
  }
  for (int k = 0; k < N && st == IEN_OK; k++) {
    const Ffc &c = ffcs[k];
    st = spectral_rows(l->spectral_plan, c.x + LOCAL, CHANNELS, c.f->spectral_in, l->spectral,
                       (float *)l->spectrum);
    if (st == IEN_OK) st = fork_branches(ctx, 1);
    if (st == IEN_OK)
      st = conv(ctx, c.x, h, w, CHANNELS, CHANNELS, 3, 1, c.f->local,
                c.residual ? c.residual : c.out, CHANNELS, IEN_ACT_RELU, 0, c.residual);
    if (st != IEN_OK) break;
    if (split) {
      // Branch 2 holds this FFC's cross convolution: mark it, then queue the
      // next FFC's after this local convolution.
      IEN_HIP(hipEventRecord(l->ev_cross, branch2));
      if (k + 1 < N) {
        IEN_HIP(hipEventRecord(l->ev_local, ctx->stream));
        IEN_HIP(hipStreamWaitEvent(branch2, l->ev_local, 0));
      }
    }
    if (k + 1 < N) {
      Branch br(ctx, 2);
      st = cross(ffcs[k + 1]);
    }
    if (st == IEN_OK) {
      Branch br(ctx, 1);
      st = spectral_columns(l->spectral_plan, c.f->fourier, (const float *)l->spectrum, l->work);
    }
    if (st == IEN_OK) st = join_branches(ctx, 1);
    if (st == IEN_OK && split) IEN_HIP(hipStreamWaitEvent(ctx->stream, l->ev_cross, 0));
    if (st == IEN_OK)
      st = spectral_back(l->spectral_plan, c.f->spectral_out, l->spectral, l->work, c.out + LOCAL,
                         CHANNELS, c.residual ? c.residual + LOCAL : nullptr,
                         c.residual ? c.residual + LOCAL : nullptr);
    if (st == IEN_OK && k % 2 == 1) st = done();
  }
  // (After a failure or a cancel: nothing on branch 2 outlives the run.)
  if (split) {
    IEN_HIP(hipEventRecord(l->ev_cross, branch2));
    IEN_HIP(hipStreamWaitEvent(ctx->stream, l->ev_cross, 0));
  }
  return st;
}

ien_status lama_enqueue(Lama *l, const float *d_image, const float *d_mask, size_t width,
                        size_t height, float *d_out, Steps *steps) {
  ien_ctx *ctx = l->ctx;
  size_t pw, ph;
  lama_padded(width, height, &pw, &ph);
  IEN_CHECK(l->fourier && l->pw == pw && l->ph == ph && l->pixels >= pw * ph, IEN_ERR_INPUT,
            "LaMa maps not reserved for %zu x %zu", pw, ph);
  int step = 0;
  auto done = [&]() -> ien_status {
    step++;
    return steps ? steps->step(ctx->stream) : IEN_OK;
  };
  // network.rs:346-370 masked_rows: image (1 - m) | m, mirrored to x 8.
  ien_status st = ien_pad_image(ctx, IEN_PAD_SYMMETRIC_MASKED, d_image, d_mask, width, height,
                                MULTIPLE, l->in4, 4);
  int h = (int)ph, w = (int)pw;
  if (st == IEN_OK)
    st = conv(ctx, l->in4, h, w, 4, 4, 7, 1, l->first, l->m0, 64, IEN_ACT_RELU, 0);
  if (st == IEN_OK) st = done();
  uint16_t *maps[4] = {l->m0, l->m1, l->m2, l->a};
  const int chans[4] = {64, 128, 256, CHANNELS};
  for (int i = 0; i < 3 && st == IEN_OK; i++) {
    st = conv(ctx, maps[i], h, w, chans[i], chans[i], 3, 2, l->down[i], maps[i + 1],
              chans[i + 1], IEN_ACT_RELU, 0);
    h = (h - 1) / 2 + 1;
    w = (w - 1) / 2 + 1;
    if (st == IEN_OK) st = done();
  }
  const size_t eighth = (size_t)h * w;
  if (l->spectral_plan && st == IEN_OK) {
    st = ffc_pipeline(l, h, w, done);
  } else {
    for (int b = 0; b < BLOCKS && st == IEN_OK; b++) {
      st = ffc_run(l, l->blocks[b][0], l->a, l->mid, h, w);
      if (st == IEN_OK) st = ffc_run(l, l->blocks[b][1], l->mid, l->out, h, w);
      if (st == IEN_OK) st = ien_add(ctx, l->a, l->out, eighth * CHANNELS);
      if (st == IEN_OK) st = done();
    }
  }
  // The ups write the quarter, half and full-scale maps again.
  for (int i = 0; i < 3 && st == IEN_OK; i++) {
    st = up_run(l, l->up[i], maps[3 - i], h, w, chans[3 - i], chans[2 - i], maps[2 - i]);
    h *= 2;
    w *= 2;
    if (st == IEN_OK) st = done();
  }
  if (st == IEN_OK)
    st = conv(ctx, l->m0, h, w, 64, 64, 7, 1, l->last, l->rgb, 3, IEN_ACT_SIGMOID, 0);
  if (st == IEN_OK) st = ien_crop(ctx, l->rgb, pw, 3, width, height, 3, d_out);
  if (st == IEN_OK) st = done();
  return st;
}

}  // namespace ien
