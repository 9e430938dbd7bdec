// swin.hip -- the Swin transformer block (crates/scunet-native/src/swin.rs
// Transformer, crates/birefnet-native/src/swin.rs Block) composed from the
// window ops and the row products on the context's stream.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "ien_internal.h"
#include "window_geo.h"

using namespace ien;

// Scratch of ien_swin_run_static: the unfused path's window rows (4c wide
// for qkv and the MLP's hidden layer, then c and c) in device memory the
// library never allocates.  Each device holds its own copy for the life of
// the process.  In host code `scratch` names a host-side stand-in; the
// device address comes from hipGetSymbolAddress (swin_static_setup).
static __device__ __align__(256) uint16_t scratch[IEN_SWIN_STATIC_SCRATCH_BYTES / 2];

struct ien_swin {
  ien_ctx *ctx = nullptr;
  int c = 0, window = 0, shift = 0, heads = 0, classes = 0;
  float *d_ln = nullptr;  // ln1 gamma, beta, ln2 gamma, beta (4 c floats)
  // The bias tables in the attention kernels' layout; the fused attention's
  // projection fragments (when it takes the block's width and window).
  float *d_packed = nullptr;
  uint16_t *d_attn_proj = nullptr;
  // At 32 channels: the fc1 / fc2 fragments of the MLP fused after it.
  uint16_t *d_attn_mlp = nullptr;
  ien_matrix *qkv = nullptr, *proj = nullptr, *fc1 = nullptr, *fc2 = nullptr;
  // Scratch: `rows` window rows (at least the map's tokens) of 4c, c, c.
  uint16_t *d_wide = nullptr, *d_tok = nullptr, *d_att = nullptr;
  size_t rows = 0;
};

namespace {

void release(ien_swin *b) {
  if (!b) return;
  ien_matrix_free(b->qkv);
  ien_matrix_free(b->proj);
  ien_matrix_free(b->fc1);
  ien_matrix_free(b->fc2);
  (void)hipFree(b->d_ln);
  (void)hipFree(b->d_packed);
  (void)hipFree(b->d_attn_proj);
  (void)hipFree(b->d_attn_mlp);
  (void)hipFree(b->d_wide);
  (void)hipFree(b->d_tok);
  (void)hipFree(b->d_att);
  delete b;
}

// Grow the scratch to `rows` rows (the stream drains first: kernels may
// still use the old buffers).
ien_status reserve(ien_swin *b, size_t rows) {
  if (rows <= b->rows) return IEN_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  IEN_HIP(hipStreamIsCapturing(b->ctx->stream, &cap));
  IEN_CHECK(cap == hipStreamCaptureStatusNone, IEN_ERR_INPUT,
            "swin block scratch must grow to %zu rows while the stream is capturing; "
            "reserve it before capture", rows);
  IEN_HIP(hipStreamSynchronize(b->ctx->stream));
  (void)hipFree(b->d_wide);
  (void)hipFree(b->d_tok);
  (void)hipFree(b->d_att);
  b->d_wide = b->d_tok = b->d_att = nullptr;
  b->rows = 0;
  const size_t c = (size_t)b->c;
  IEN_HIP(hipMalloc((void **)&b->d_wide, rows * 4 * c * 2));
  IEN_HIP(hipMalloc((void **)&b->d_tok, rows * c * 2));
  IEN_HIP(hipMalloc((void **)&b->d_att, rows * c * 2));
  b->rows = rows;
  return IEN_OK;
}

// The device address of `scratch`, per device (swin_static_setup).
std::mutex g_scratch_mu;
std::vector<uint16_t *> g_scratch;

uint16_t *static_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return device >= 0 && (size_t)device < g_scratch.size() ? g_scratch[device] : nullptr;
}

ien_status rows_product(ien_ctx *ctx, const uint16_t *in, size_t k, size_t rows,
                        const ien_matrix *m, uint16_t *out, size_t stride, ien_act act,
                        int accumulate) {
  ien_input x{};
  x.kind = IEN_INPUT_ROWS;
  x.data = in;
  x.stride = k;
  ien_output o{};
  o.data = out;
  o.stride = stride;
  o.layout = IEN_LAYOUT_NHWC;
  o.type = IEN_OUT_F16;
  return ien_multiply_ex(ctx, &x, 0, rows, m, &o, act, nullptr, accumulate);
}


bool rows16_map(const uint16_t *d_map, size_t stride) {
  return stride % 8 == 0 && ((uintptr_t)d_map & 15) == 0;
}

// Window rows of a block's scratch for a height x width map (at least the
// map's tokens), or 0 for an invalid map.
size_t block_rows(const ien_swin *b, int height, int width) {
  ien_windows w{b->window, b->shift, height, width};
  const long wins = ien_window_count(&w);
  if (wins <= 0) return 0;
  const size_t rows = (size_t)wins * b->window * b->window, tokens = (size_t)height * width;
  return rows > tokens ? rows : tokens;
}

// Whether run_block touches its scratch: the fused passes do not.
bool needs_scratch(const ien_swin *b, const uint16_t *d_map, size_t stride) {
  const bool rows16 = rows16_map(d_map, stride);
  if (b->d_attn_mlp && rows16) return false;
  const bool attend_fused = b->d_attn_proj && rows16;
  const bool mlp_fused = swin_mlp_supported(b->c) && rows16;
  return !(attend_fused && mlp_fused);
}

// One block (attend, then mlp) with the unfused path's scratch at wide
// (rows x 4c), tok and att (rows x c each).
ien_status run_block(ien_swin *b, uint16_t *d_map, size_t stride, int height, int width,
                     uint16_t *wide, uint16_t *tok, uint16_t *att) {
  ien_ctx *ctx = b->ctx;
  const size_t c = (size_t)b->c;
  ien_windows w{b->window, b->shift, height, width};
  const long wins = ien_window_count(&w);
  IEN_CHECK(wins > 0, IEN_ERR_INPUT, "map %d x %d", height, width);
  const size_t rows = (size_t)wins * b->window * b->window;
  const size_t tokens = (size_t)height * width;
  ien_status st = IEN_OK;
  const float *g1 = b->d_ln, *b1 = b->d_ln + c, *g2 = b->d_ln + 2 * c, *b2 = b->d_ln + 3 * c;
  const bool rows16 = rows16_map(d_map, stride);
  // attend (scunet swin.rs:131-232): one fused pass per window where its
  // kernel takes the width and window, else the window rows, qkv,
  // attention, projection over the token rows, added back onto the map.
  if (b->d_attn_mlp && rows16) {
    // Both halves in one pass per window (32 channels).
    const AttendMlp mlp{g2, b2, b->d_attn_mlp, b->fc1->d_bias, b->fc2->d_bias};
    return swin_attend(ctx, &w, d_map, stride, b->c, g1, b1, b->qkv, b->d_attn_proj,
                       b->proj->d_bias, b->d_packed, &mlp);
  }
  if (b->d_attn_proj && rows16) {
    st = swin_attend(ctx, &w, d_map, stride, b->c, g1, b1, b->qkv, b->d_attn_proj,
                     b->proj->d_bias, b->d_packed);
  } else {
    if (rows16 && window_qkv_attention_supported(b->c, b->window)) {
      // Gather, LayerNorm, q k v and attention in one pass per window and head.
      st = window_qkv_attention(ctx, &w, d_map, stride, b->c, g1, b1, b->qkv, b->d_packed, att);
    } else {
      st = ien_window_gather(ctx, &w, d_map, stride, b->c, g1, b1, tok);
      if (st == IEN_OK)
        st = rows_product(ctx, tok, c, rows, b->qkv, wide, 3 * c, IEN_ACT_NONE, 0);
      if (st == IEN_OK)
        st = window_attention(ctx, &w, wide, b->c, b->d_packed, true, att);
    }
    // The projection added straight back onto the map's pixels.
    WinGeo g;
    if (st == IEN_OK) st = geometry(&w, &g);
    if (st == IEN_OK) {
      RowsPlanes p;
      p.x = p.x2 = att;
      p.xs = p.xs2 = (int)c;
      p.k1 = (int)c;
      p.rows = (long)rows;
      p.w = b->proj;
      p.y = p.y2 = d_map;
      p.ys = p.ys2 = (int)stride;
      p.n1 = (int)c;
      p.windows = &g;
      st = launch_rows_planes(ctx, p);
    }
  }
  if (st != IEN_OK) return st;
  // mlp (scunet swin.rs:236-275): every token normalised, fc1 + GELU, fc2
  // added back; one fused pass where its kernel takes the width, else a
  // 1 x 1 window gather (the copy with its LayerNorm) and two products.
  if (swin_mlp_supported(b->c) && rows16)
    return swin_mlp(ctx, d_map, stride, (long)tokens, b->c, g2, b2, b->fc1, b->fc2);
  ien_windows one{1, 0, height, width};
  if ((st = ien_window_gather(ctx, &one, d_map, stride, b->c, g2, b2, tok)) != IEN_OK)
    return st;
  if ((st = rows_product(ctx, tok, c, tokens, b->fc1, wide, 4 * c, IEN_ACT_GELU, 0)) !=
      IEN_OK)
    return st;
  return rows_product(ctx, wide, 4 * c, tokens, b->fc2, d_map, stride, IEN_ACT_NONE, 1);
}

}  // namespace

namespace ien {

// Scratch for a height x width map ahead of time (outside any graph
// capture: growing drains the stream).
ien_status swin_reserve(ien_swin *b, int height, int width) {
  IEN_CHECK(b, IEN_ERR_INPUT, "no block");
  ien_windows w{b->window, b->shift, height, width};
  const long wins = ien_window_count(&w);
  IEN_CHECK(wins > 0, IEN_ERR_INPUT, "map %d x %d", height, width);
  const size_t rows = (size_t)wins * b->window * b->window, tokens = (size_t)height * width;
  return reserve(b, rows > tokens ? rows : tokens);
}

// Halves of scratch a block's run on a height x width map may use (the
// unfused path's window rows at 6c halves each), or 0 for an invalid map.
size_t swin_scratch_halves(const ien_swin *b, int height, int width) {
  return block_rows(b, height, width) * 6 * (size_t)b->c;
}

// A block's run with the caller's scratch (at least swin_scratch_halves),
// so that runs of one block on different streams do not share the block's
// own scratch.
ien_status swin_run_with(ien_swin *b, uint16_t *d_map, size_t stride, int height, int width,
                         uint16_t *scratch, size_t halves) {
  IEN_CHECK(b && d_map && scratch, IEN_ERR_INPUT, "null argument");
  const size_t rows = block_rows(b, height, width);
  IEN_CHECK(rows > 0, IEN_ERR_INPUT, "map %d x %d", height, width);
  const size_t c = (size_t)b->c;
  IEN_CHECK(rows * 6 * c <= halves, IEN_ERR_INPUT, "scratch of %zu halves for %zu", halves,
            rows * 6 * c);
  uint16_t *wide = scratch, *tok = wide + rows * 4 * c, *att = tok + rows * c;
  return run_block(b, d_map, stride, height, width, wide, tok, att);
}

// Once per device, with that device current (ien_open): the device
// address of `scratch` for ien_swin_run_static.
hipError_t swin_static_setup(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((size_t)device < g_scratch.size() && g_scratch[device]) return hipSuccess;
  void *ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if ((size_t)device >= g_scratch.size()) g_scratch.resize(device + 1, nullptr);
  g_scratch[device] = (uint16_t *)ptr;
  return hipSuccess;
}

}  // namespace ien


extern "C" {

ien_status ien_swin_new(ien_ctx *ctx, const ien_swin_weights *w, ien_swin **out) {
  IEN_CHECK(ctx && w && out, IEN_ERR_INPUT, "null argument");
  *out = nullptr;
  const ien_swin_weights &W = *w;
  IEN_CHECK(W.c >= 32 && W.c % 32 == 0 && W.c <= 1024, IEN_ERR_INPUT,
            "%d channels (heads of 32, at most 1024)", W.c);
  IEN_CHECK(W.window >= 1 && W.window <= 16 && W.shift >= 0 && W.shift < W.window,
            IEN_ERR_INPUT, "window %d, shift %d", W.window, W.shift);
  IEN_CHECK(W.ln1_gamma && W.ln1_beta && W.qkv_w && W.qkv_b && W.position && W.proj_w &&
                W.proj_b && W.ln2_gamma && W.ln2_beta && W.fc1_w && W.fc1_b && W.fc2_w && W.fc2_b,
            IEN_ERR_INPUT, "missing weights");
  ien_swin *b = new ien_swin;
  b->ctx = ctx;
  b->c = W.c;
  b->window = W.window;
  b->shift = W.shift;
  b->heads = W.c / 32;
  const size_t c = (size_t)W.c, n = (size_t)W.window * W.window;
  auto fail_with = [&](ien_status st) {
    release(b);
    return st;
  };
  std::vector<float> tables(4 * (size_t)b->heads * n * n);
  b->classes = ien_bias_tables(W.position, b->heads, W.window, W.shift, W.masked, tables.data());
  if (b->classes < 0) return fail_with(IEN_ERR_INPUT);
  std::vector<float> ln(4 * c);
  std::memcpy(ln.data(), W.ln1_gamma, c * 4);
  std::memcpy(ln.data() + c, W.ln1_beta, c * 4);
  std::memcpy(ln.data() + 2 * c, W.ln2_gamma, c * 4);
  std::memcpy(ln.data() + 3 * c, W.ln2_beta, c * 4);
  hipError_t e = hipMalloc((void **)&b->d_ln, 4 * c * 4);
  if (e == hipSuccess) e = hipMemcpy(b->d_ln, ln.data(), 4 * c * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    const std::vector<float> packed = pack_bias_tables(tables.data(), b->classes, b->heads, (int)n);
    e = hipMalloc((void **)&b->d_packed, packed.size() * 4);
    if (e == hipSuccess)
      e = hipMemcpy(b->d_packed, packed.data(), packed.size() * 4, hipMemcpyHostToDevice);
  }
  if (e == hipSuccess && swin_attend_supported(W.c, W.window)) {
    const std::vector<uint16_t> proj = swin_attend_proj(W.proj_w, W.c);
    e = hipMalloc((void **)&b->d_attn_proj, proj.size() * 2);
    if (e == hipSuccess)
      e = hipMemcpy(b->d_attn_proj, proj.data(), proj.size() * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess && W.c == 32) {
      const std::vector<uint16_t> mlp = swin_attend_mlp(W.fc1_w, W.fc2_w);
      e = hipMalloc((void **)&b->d_attn_mlp, mlp.size() * 2);
      if (e == hipSuccess)
        e = hipMemcpy(b->d_attn_mlp, mlp.data(), mlp.size() * 2, hipMemcpyHostToDevice);
    }
  }
  if (e != hipSuccess) {
    release(b);
    return fail(IEN_ERR_GPU, "swin upload: %s", hipGetErrorString(e));
  }
  ien_status st = ien_matrix_new(ctx, W.qkv_w, IEN_W_F32, c, 3 * c, W.qkv_b, &b->qkv);
  if (st == IEN_OK) st = ien_matrix_new(ctx, W.proj_w, IEN_W_F32, c, c, W.proj_b, &b->proj);
  if (st == IEN_OK) st = ien_matrix_new(ctx, W.fc1_w, IEN_W_F32, c, 4 * c, W.fc1_b, &b->fc1);
  if (st == IEN_OK) st = ien_matrix_new(ctx, W.fc2_w, IEN_W_F32, 4 * c, c, W.fc2_b, &b->fc2);
  if (st != IEN_OK) return fail_with(st);
  *out = b;
  return IEN_OK;
}

void ien_swin_free(ien_swin *block) { release(block); }

ien_status ien_swin_run(ien_swin *b, uint16_t *d_map, size_t stride, int height, int width) {
  IEN_CHECK(b && d_map, IEN_ERR_INPUT, "null argument");
  const size_t rows = block_rows(b, height, width);
  IEN_CHECK(rows > 0, IEN_ERR_INPUT, "map %d x %d", height, width);
  ien_status st = reserve(b, rows);
  if (st != IEN_OK) return st;
  return run_block(b, d_map, stride, height, width, b->d_wide, b->d_tok, b->d_att);
}

ien_status ien_swin_run_static(ien_swin *b, uint16_t *d_map, size_t stride, int height,
                               int width) {
  IEN_CHECK(b && d_map, IEN_ERR_INPUT, "null argument");
  const size_t rows = block_rows(b, height, width);
  IEN_CHECK(rows > 0, IEN_ERR_INPUT, "map %d x %d", height, width);
  uint16_t *wide = nullptr, *tok = nullptr, *att = nullptr;
  if (needs_scratch(b, d_map, stride)) {
    const size_t c = (size_t)b->c, bytes = rows * 6 * c * 2;
    IEN_CHECK(bytes <= IEN_SWIN_STATIC_SCRATCH_BYTES, IEN_ERR_INPUT,
              "a %d x %d map of %d channels needs %zu bytes of scratch; the static scratch "
              "holds %zu",
              height, width, b->c, bytes, (size_t)IEN_SWIN_STATIC_SCRATCH_BYTES);
    uint16_t *base = static_scratch(b->ctx->device);
    IEN_CHECK(base, IEN_ERR_GPU, "no static scratch on device %d", b->ctx->device);
    wide = base;
    tok = wide + rows * 4 * c;
    att = tok + rows * c;
  }
  return run_block(b, d_map, stride, height, width, wide, tok, att);
}

}  // extern "C"
