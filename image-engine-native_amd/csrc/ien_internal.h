// ien_internal.h -- shared internals of libien_hip.so (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/ien_hip.h"

namespace ien {

// Thread-local message behind ien_last_error (crates/native-engine/src/lib.rs:73-83).
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Return `status` after recording a formatted message.
ien_status fail(ien_status status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

#define IEN_HIP(call)                                                                     \
  do {                                                                                    \
    hipError_t e_ = (call);                                                               \
    if (e_ != hipSuccess)                                                                 \
      return ::ien::fail(IEN_ERR_GPU, "%s: %s (%s:%d)", #call, hipGetErrorString(e_),     \
                         __FILE__, __LINE__);                                             \
  } while (0)

#define IEN_CHECK(cond, status, ...)                       \
  do {                                                     \
    if (!(cond)) return ::ien::fail(status, __VA_ARGS__);  \
  } while (0)

}  // namespace ien

struct ien_ctx {
  int device = 0;
  hipStream_t own = nullptr;     // the context's stream
  hipStream_t stream = nullptr;  // where work goes (own, or the caller's)
  std::string name;
  int cus = 0;
  // 4 KiB of zeros in device memory: the source of padding pixels for
  // loads that write LDS directly (they cannot write a constant).
  uint16_t *zeros = nullptr;
  // Split-K partial sums of the convolution kernels (f32), allocated once
  // with the context so that no launch allocates (graph capture):
  // splitk_floats of them, then SPLITK_TILES int tile counters (zero at
  // open; a launch that counts its splits in returns each to zero).
  float *splitk = nullptr;
  size_t splitk_floats = 0;
  static constexpr int SPLITK_TILES = 65536;
  // Branch streams (default priority, non-blocking) with their own split-K
  // workspaces: independent parts of a network run on them between fork()
  // and join(), so that they overlap on the GPU (and in a captured graph).
  static constexpr int BRANCHES = 3;
  hipStream_t branch[BRANCHES] = {};
  float *branch_splitk[BRANCHES] = {};
  hipEvent_t fork_ev = nullptr, join_ev[BRANCHES] = {};
  // Convolutions keep a single chunk buffer in LDS (no double-buffered
  // chunks): set by a driver around work that runs beside LDS-hungry
  // kernels of another branch.
  bool compact = false;
  // Every branch's work stays on the context's stream, one kernel at a time
  // (IEN_SERIAL_BRANCHES=1 at ien_open): for profiles that attribute time
  // to single kernels.
  bool serial_branches = false;
  // Chains of body pairs (conv_pair.hip): an abort word, a failure word, a
  // count of workgroups done and chain_tiles epoch words; the workgroups of the chain kernel one CU
  // holds (-1 until asked); the wall-clock ticks (100 MHz) a tile may wait
  // for a neighbour.
  int *chain_flags = nullptr;
  // Sequence number of the last chain launched on this context, and the
  // highest failed one already reported (chain_status).
  int chain_seq = 0, chain_reported = 0;
  int chain_tiles = 0;
  int chain_per_cu = -1;
  long chain_spin = 100000000;
};

// Packed weights (gemm.rs Matrix): k x n padded to whole 16 x 32 MFMA
// fragments.  Fragment (kb, nb) holds 512 halves: lane l's 8 consecutive
// values are W[16 kb + 8 (l / 32) + i][32 nb + l % 32], the B-operand
// register layout of v_mfma_f32_32x32x16_f16, so a wave loads one fragment
// with one 16-byte load per lane.
struct ien_matrix {
  ien_ctx *ctx = nullptr;
  size_t k = 0, n = 0;
  int kb = 0, nb = 0;          // fragments along k (16) and n (32)
  uint16_t *d_packed = nullptr;  // nb x kb fragments of 512 halves, n-block major
  float *d_bias = nullptr;       // 32 nb floats, zero padded
};

namespace ien {

// fork_branches(ctx, n): branch streams 1..n start after the work already
// on the context's stream; join_branches(ctx, n): the context's stream
// continues after the branches' work.  Between them, a Branch object sends
// the context's launches (and its split-K workspace) to branch i while it
// lives.
ien_status fork_branches(ien_ctx *ctx, int n);
ien_status join_branches(ien_ctx *ctx, int n);
struct Branch {
  ien_ctx *ctx;
  hipStream_t stream;
  float *splitk;
  Branch(ien_ctx *c, int i) : ctx(c), stream(c->stream), splitk(c->splitk) {
    if (ctx->serial_branches) return;
    ctx->stream = ctx->branch[i - 1];
    ctx->splitk = ctx->branch_splitk[i - 1];
  }
  ~Branch() {
    ctx->stream = stream;
    ctx->splitk = splitk;
  }
  Branch(const Branch &) = delete;
  Branch &operator=(const Branch &) = delete;
};

// Progress of a run (realesrgan-native lib.rs:168-188, scunet-native
// lib.rs:205-215): a model driver calls step() after issuing each step's
// work (a layer, block or stage).  step() records an event for that step,
// then waits for the previous step and reports it, so one step stays
// queued on the GPU while the callback runs.  When the callback asks to
// stop, step() returns IEN_ERR_CANCELLED and the driver issues nothing
// more; the run ends after the step already queued.  `total` counts the
// steps of the whole call (tiles x steps per image).
struct Steps {
  ien_progress progress = nullptr;
  void *user = nullptr;
  int total = 0, issued = 0, reported = 0;
  hipEvent_t ev[2] = {nullptr, nullptr};
  Steps(ien_progress p, void *u, int t) : progress(p), user(u), total(t) {}
  ~Steps();
  Steps(const Steps &) = delete;
  Steps &operator=(const Steps &) = delete;
  ien_status step(hipStream_t stream);
  // Wait for the last issued step and report it.
  ien_status drain();

 private:
  ien_status report_through(int done);
};

// Pack row-major k x n weights (as floats) into the fragment layout above.
std::vector<uint16_t> pack_fragments(const float *w, size_t k, size_t n, int *kb, int *nb);

// Host-side round to nearest even (the same map as half.rs:7-40).
uint16_t f32_to_half(float v);

// Launch helpers of conv.hip, shared by the ops and the model drivers.
struct ConvCall {
  // input
  const uint16_t *x = nullptr;
  int H = 0, W = 0, C = 0;
  long xs = 0;  // NHWC: halves between pixels; NCHW: halves between planes
  int in_nchw = 0;
  int rows_mode = 0;  // Input::Rows: M rows of k values, no image grid
  int ks = 1, stride = 1, pad_reflect = 0;
  int noff = 0;  // Taps::Offsets count (0: Conv taps)
  int offy[4] = {0, 0, 0, 0}, offx[4] = {0, 0, 0, 0};
  // output grid and range
  int OH = 0, OW = 0;
  long row0 = 0, rows = 0;
  // weights
  const ien_matrix *w = nullptr;
  // output
  void *y = nullptr;
  long ys = 0;
  int out_nchw = 0, out_f32 = 0;
  int act = IEN_ACT_NONE;
  const float *slope = nullptr;
  int accumulate = 0;
  // Optional: device biases in place of the matrix's (as many as its padded
  // columns, whole 32-column blocks).
  const float *bias = nullptr;
  // Optional, NHWC f16 outputs of 3x3 stride-1 products only: a map (rows
  // ys apart, 16-byte aligned) added to each f16 result after the
  // activation, rounded again (the product followed by ien_add; it may be y).
  const uint16_t *add2 = nullptr;
  // Optional, the same outputs and 3x3 or offset-tap products over whole
  // maps: 1 + 2 py + px writes output pixel (y, x) to pixel (2 y + py,
  // 2 x + px) of y, a map 2 OH x 2 OW with pixels ys apart (a transposed
  // convolution's phase scattered as it is stored); 0 for none.
  int phase = 0;
};

ien_status launch_conv(ien_ctx *ctx, const ConvCall &c);

// conv_pair.hip: two 3x3 64 -> 64 convolutions with bias and PReLU in one
// launch (x -> w1 -> w2 -> y, the intermediate map never stored): NHWC f16
// maps of H x W x 64, 16-byte aligned, x and y not overlapping.
struct PairCall {
  const uint16_t *x = nullptr;
  uint16_t *y = nullptr;
  int H = 0, W = 0;
  const ien_matrix *w1 = nullptr, *w2 = nullptr;
  const float *s1 = nullptr, *s2 = nullptr;  // PReLU slopes
};
// rows.hip: out = x W + bias (+ old out) over `rows` rows whose first k1
// channels come from x (rows xs halves apart) and the rest from x2, the
// first n1 output columns going to y and the rest to y2: the two halves of
// a map kept as separate planes.
struct WinGeo;
struct RowsPlanes {
  const uint16_t *x = nullptr, *x2 = nullptr;
  int xs = 0, xs2 = 0, k1 = 0;
  long rows = 0;
  const ien_matrix *w = nullptr;
  uint16_t *y = nullptr, *y2 = nullptr;
  int ys = 0, ys2 = 0, n1 = 0;
  int accumulate = 0;
  // 2 x 2 regroupings, one plane each way (0: none).  gather_w2: row r is
  // the 2 x 2 pixel group (2 (r / gather_w2) + dy, 2 (r % gather_w2) + dx)
  // of x, a map 2 gather_w2 wide with pixels xs apart, channels in blocks
  // of k / 4 by 2 dy + dx (ien_gather_2x2's row-major order).  scatter_w:
  // rows are the pixels of a map scatter_w wide, and column block q of n / 4
  // goes to pixel (2 (r / scatter_w) + q / 2, 2 (r % scatter_w) + q % 2) of
  // y, a map 2 scatter_w wide with pixels ys apart (ien_scatter_2x2).
  int gather_w2 = 0, scatter_w = 0;
  // With gather_w2: a second copy of the output rows (ys apart), or null.
  uint16_t *ydup = nullptr;
  // A map (rows ys apart) added to the f16 result, rounded again: the
  // product followed by ien_add in one pass; or null.
  const uint16_t *add = nullptr;
  // Rows are the tokens of these windows over y's map (rows ys apart): each
  // row's f16 result is added onto its map pixel and rounded again, tokens
  // past the edge dropped (the product followed by ien_window_scatter_add);
  // or null.
  const WinGeo *windows = nullptr;
};
ien_status launch_rows_planes(ien_ctx *ctx, const RowsPlanes &p);

// elementwise.hip: LayerNorm (math.rs:95-116, eps 1e-5) of `rows` rows of c
// values read from src (sstride apart) into dst (stride apart), in place
// when they are the same rows (ien_layer_norm); other rows need 8-aligned
// channels and strides and 16-byte aligned maps.  With gather_w2 > 0 the
// rows are read as ien_gather_2x2's column-major 2 x 2 groups of src, a map
// 2 gather_w2 wide of c / 4 channels (pixels sstride apart; c a multiple
// of 32).
ien_status layer_norm_to(ien_ctx *ctx, const uint16_t *src, size_t sstride, uint16_t *dst,
                         size_t stride, size_t rows, size_t c, const float *gamma,
                         const float *beta, int gather_w2 = 0);

// join_split.hip: a SCUNet block boundary over `rows` pixels of a c-channel
// map x (rows c apart), c = 64 or 128: x += join([yc | ysw]) + join bias,
// rounded to f16, then [yc | ysw] = split(x) + split bias, the split map as
// two planes of c / 2 channels (rows c / 2 apart), both updated in place.
// The same bits as the two row products (the join accumulating onto x).
struct JoinSplit {
  uint16_t *yc = nullptr, *ysw = nullptr, *x = nullptr;
  long rows = 0;
  int c = 0;
  const ien_matrix *join = nullptr, *split = nullptr;
};
bool join_split_supported(const JoinSplit &p);
ien_status launch_join_split(ien_ctx *ctx, const JoinSplit &p);

bool pair_supported(const PairCall &p);
ien_status launch_pair(ien_ctx *ctx, const PairCall &p);

// A chain of `pairs` such pairs in one launch (layers w[0], w[1], ...,
// slopes s[i]): the input in `a`; `b` and `a` hold the borders the tiles
// exchange, and the output ends in the map launch_chain returns (`a` for an
// even count), or, with a final layer, in `out`.  Supported when every tile's workgroup can be resident at
// once.  Each launch takes the context's next sequence number;
// chain_status(ctx, first) waits for the stream and reports IEN_ERR_GPU
// when a chain numbered `first` or later gave up (a wait for a neighbour
// that timed out aborts its chain) and that failure was not reported
// before.
struct ChainCall {
  uint16_t *a = nullptr, *b = nullptr;
  int H = 0, W = 0, pairs = 0;
  const ien_matrix *w[32] = {};
  const float *s[32] = {};
  // Optional: a final 3x3 64 -> 48 layer (no activation) whose output is
  // pixel-shuffled x4 and added to the f32 RGB image (H x W x 3) into out
  // ((4 H) x (4 W) x 3 f32): realesrgan-native network.rs:110-141.
  const ien_matrix *last = nullptr;
  const float *image = nullptr;
  float *out = nullptr;
  // Optional: a first 3x3 layer over the image's RGB and a zero fourth
  // channel (k = 36, 64 outputs, PReLU) that the first pair computes from
  // `image` instead of reading `a`: network.rs:96-109 with i = 0.
  const ien_matrix *first = nullptr;
  const float *first_slope = nullptr;
};
bool chain_supported(ien_ctx *ctx, const ChainCall &c);
ien_status launch_chain(ien_ctx *ctx, const ChainCall &c, uint16_t **out);
ien_status chain_status(ien_ctx *ctx, int first);

// io.hip: the 8-bit image passes of the models' u8 entry points, on the
// context's stream (to_float, to_byte, LaMa's mask and compositing,
// BiRefNet's normalisation of interleaved RGB).
ien_status bytes_to_floats(ien_ctx *ctx, const uint8_t *src, float *dst, size_t n);
ien_status floats_to_bytes(ien_ctx *ctx, const float *src, uint8_t *dst, size_t n);
ien_status mask_bytes(ien_ctx *ctx, const uint8_t *src, float *dst, size_t n);
ien_status normalize_bytes(ien_ctx *ctx, const uint8_t *src, size_t pixels, const float mean[3],
                           const float deviation[3], float *dst);
ien_status composite_bytes(ien_ctx *ctx, const uint8_t *rgb, const uint8_t *mask,
                           const float *pred, size_t pixels, uint8_t *out);

// swin.hip: a block's scratch grown for a height x width map in advance.
ien_status swin_reserve(ien_swin *b, int height, int width);
// Scratch halves of a block's run on a height x width map, and a run with
// the caller's scratch of that size (runs of one block on two streams).
size_t swin_scratch_halves(const ien_swin *b, int height, int width);
ien_status swin_run_with(ien_swin *b, uint16_t *d_map, size_t stride, int height, int width,
                         uint16_t *scratch, size_t halves);

// swin_mlp.hip: map rows += fc2(GELU(fc1(LayerNorm(rows)))) in one pass,
// for c = 32, 64 and 96 (16-byte aligned rows).
// window.hip: [class][head][query][key] bias tables of n-token windows in
// the attention kernels' accumulator layout, [class][head][query block]
// [key block][4][64 lanes][4] (keys past n -inf); the attention over
// windows with tables in that layout (packed) or the plain one.
std::vector<float> pack_bias_tables(const float *tables, int classes, int heads, int n);
ien_status window_attention(ien_ctx *ctx, const ien_windows *w, const uint16_t *d_qkv, int c,
                            const float *d_tables, bool packed, uint16_t *d_out);

// window_attend.hip: gather, LayerNorm 1, the head's q, k, v and the
// attention in one pass per window and head, into the windows' rows of c
// (what the unfused gather, qkv product and attention give); widths by 32,
// windows of up to 64 or 129 .. 160 tokens, tables packed.
bool window_qkv_attention_supported(int c, int window);
ien_status window_qkv_attention(ien_ctx *ctx, const ien_windows *win, const uint16_t *d_map,
                                size_t stride, int c, const float *gamma, const float *beta,
                                const ien_matrix *qkv, const float *d_tables, uint16_t *d_out);

bool swin_mlp_supported(int c);
// The device address of ien_swin_run_static's static scratch on `device`
// (current), looked up once per device.
hipError_t swin_static_setup(int device);
ien_status swin_mlp(ien_ctx *ctx, uint16_t *d_map, size_t stride, long rows, int c,
                    const float *gamma, const float *beta, const ien_matrix *fc1,
                    const ien_matrix *fc2);

// swin_attend.hip: a Swin block's attention half (gather, LayerNorm, qkv,
// attention, projection, residual) in one pass per window, for window 8
// and 32, 64 or 128 channels; its projection fragments are packed once per
// block by swin_attend_proj, its bias tables by pack_bias_tables.
bool swin_attend_supported(int c, int window);
std::vector<uint16_t> swin_attend_proj(const float *proj_w, int c);
// The MLP half fused after the attention (c = 32): LayerNorm 2, the fc1
// and fc2 A fragments from swin_attend_mlp (fc1's 8 KiB, then fc2's), the
// biases (4c and c floats); all 16-byte aligned.
struct AttendMlp {
  const float *gamma, *beta;
  const uint16_t *w;
  const float *b1, *b2;
};
std::vector<uint16_t> swin_attend_mlp(const float *fc1_w, const float *fc2_w);
ien_status swin_attend(ien_ctx *ctx, const ien_windows *win, uint16_t *d_map, size_t stride,
                       int c, const float *gamma, const float *beta, const ien_matrix *qkv,
                       const uint16_t *d_proj, const float *bproj, const float *d_tables,
                       const AttendMlp *mlp = nullptr);

}  // namespace ien
