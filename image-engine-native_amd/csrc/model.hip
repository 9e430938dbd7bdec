// model.hip -- the model drivers behind ien_model_*: the reference's
// Model::load / run (crates/realesrgan-native/src/lib.rs:111-232) with the
// GPU engine, and its weights-file reader (crates/native-engine/src/
// weight_file.rs).
//
// Real-ESRGAN (SRVGGNetCompact, realesrgan-native network.rs): 34 3x3
// convolutions on two f16 NHWC maps of 64 channels that take turns as input
// and output (as gpu.rs:40-70 keeps them), PReLU fused into each
// convolution's epilogue, then the x4 pixel shuffle plus the repeated input
// into f32.  The whole run is one stream of launches; with graphs enabled it
// is captured once per image size and replayed, so the 36 launches cost one
// submission.
//
// SCUNet, LaMa and BiRefNet are objects of their own (scunet.hip, lama.hip,
// birefnet.hip) that this file loads, sizes and runs the same way.

#include <algorithm>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>

#include "birefnet.h"
#include "ien_internal.h"
#include "lama.h"
#include "scunet.h"

namespace ien {

// ---- weight_file.rs:15-146 ----------------------------------------------
struct Tensor {
  std::vector<size_t> shape;
  std::vector<float> values;
};

// Whether `s` is well-formed UTF-8 (as str::from_utf8 accepts it: no
// overlong forms, no surrogates, nothing past U+10FFFF).
static bool utf8(const std::string &s) {
  const unsigned char *p = (const unsigned char *)s.data(), *end = p + s.size();
  while (p < end) {
    const unsigned c = *p;
    if (c < 0x80) {
      p++;
      continue;
    }
    const int n = (c & 0xe0) == 0xc0 ? 1 : (c & 0xf0) == 0xe0 ? 2 : (c & 0xf8) == 0xf0 ? 3 : -1;
    if (n < 0 || end - p <= n) return false;
    unsigned cp = c & (0x3f >> n);
    for (int i = 1; i <= n; i++) {
      if ((p[i] & 0xc0) != 0x80) return false;
      cp = (cp << 6) | (p[i] & 0x3f);
    }
    static const unsigned least[4] = {0, 0x80, 0x800, 0x10000};
    if (cp < least[n] || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
    p += n + 1;
  }
  return true;
}

class WeightFile {
 public:
  std::map<std::string, Tensor> tensors;

  // weight_file.rs:40-117: every length checked against what is left before
  // anything is allocated for it.
  ien_status read(const char *path, const char magic[8]) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(IEN_ERR_IO, "%s: cannot open", path);
    f.seekg(0, std::ios::end);
    unsigned long long left = (unsigned long long)f.tellg();
    f.seekg(0);
    auto take = [&](void *dst, size_t n) -> bool {
      if (n > left) return false;
      left -= n;
      f.read((char *)dst, (std::streamsize)n);
      return (bool)f;
    };
    char m[8];
    if (!take(m, 8)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
    if (std::memcmp(m, magic, 8) != 0) {
      std::string kind(magic, 8);
      while (!kind.empty() && kind.back() == '\0') kind.pop_back();
      return fail(IEN_ERR_WEIGHTS, "not a %s weights file", kind.c_str());
    }
    uint32_t version = 0, count = 0;
    if (!take(&version, 4)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
    if (version != 1)
      return fail(IEN_ERR_WEIGHTS, "weights file version %u, expected 1", version);
    if (!take(&count, 4)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
    for (uint32_t t = 0; t < count; t++) {
      uint16_t name_len = 0;
      if (!take(&name_len, 2)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
      std::string name(name_len, '\0');
      if (!take(name.data(), name_len)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
      if (!utf8(name)) return fail(IEN_ERR_WEIGHTS, "tensor name is not UTF-8");
      uint8_t dr[2];
      if (!take(dr, 2)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
      size_t width = dr[0] == 0 ? 4 : dr[0] == 1 ? 2 : 0;
      if (!width) return fail(IEN_ERR_WEIGHTS, "%s: unknown type %u", name.c_str(), dr[0]);
      Tensor tensor;
      unsigned long long elems = 1;
      for (int d = 0; d < dr[1]; d++) {
        uint32_t dim = 0;
        if (!take(&dim, 4)) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
        if (dim && elems > (~0ull) / dim) return fail(IEN_ERR_WEIGHTS, "%s: too large", name.c_str());
        elems *= dim;
        tensor.shape.push_back(dim);
      }
      if (elems > left / width) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
      std::vector<unsigned char> bytes(elems * width);
      if (!take(bytes.data(), bytes.size())) return fail(IEN_ERR_WEIGHTS, "weights file is truncated");
      tensor.values.resize(elems);
      if (width == 4) {
        std::memcpy(tensor.values.data(), bytes.data(), bytes.size());
      } else {
        for (size_t i = 0; i < elems; i++) {
          _Float16 h;
          std::memcpy(&h, bytes.data() + 2 * i, 2);
          tensor.values[i] = (float)h;
        }
      }
      if (!tensors.emplace(name, std::move(tensor)).second)
        return fail(IEN_ERR_WEIGHTS, "%s: stored twice", name.c_str());
    }
    if (left != 0) return fail(IEN_ERR_WEIGHTS, "trailing bytes after the last tensor");
    return IEN_OK;
  }

  // weight_file.rs:119-137 take
  ien_status take(const std::string &name, std::vector<size_t> shape, std::vector<float> *out) {
    auto it = tensors.find(name);
    if (it == tensors.end()) return fail(IEN_ERR_WEIGHTS, "%s: missing", name.c_str());
    if (it->second.shape != shape) {
      std::string got, want;
      for (size_t d : it->second.shape) got += std::to_string(d) + ",";
      for (size_t d : shape) want += std::to_string(d) + ",";
      return fail(IEN_ERR_WEIGHTS, "%s: shape [%s], expected [%s]", name.c_str(), got.c_str(),
                  want.c_str());
    }
    *out = std::move(it->second.values);
    tensors.erase(it);
    return IEN_OK;
  }

  // The shape of a stored tensor, without taking it.
  bool shape_of(const std::string &name, std::vector<size_t> *shape) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) return false;
    *shape = it->second.shape;
    return true;
  }

  // weight_file.rs:139-145 finish
  ien_status finish() {
    if (!tensors.empty())
      return fail(IEN_ERR_WEIGHTS, "%s: not used by this model", tensors.begin()->first.c_str());
    return IEN_OK;
  }
};

// ---- Real-ESRGAN ---------------------------------------------------------
struct EsrganLayer {
  ien_matrix *conv = nullptr;
  float *d_slope = nullptr;  // PReLU slopes; null on the last layer
  int cin = 0, cout = 0;
};

struct Maps {
  size_t pixels = 0;
  uint16_t *image = nullptr;  // f16 copy of the input, 3 channels
  uint16_t *a = nullptr, *b = nullptr;  // 64-channel maps
  float *d_in = nullptr, *d_out = nullptr;  // host-API staging
};

}  // namespace ien

struct ien_model {
  ien_ctx *ctx = nullptr;
  ien_model_kind kind = IEN_MODEL_REALESRGAN;
  std::vector<ien::EsrganLayer> layers;
  std::unique_ptr<ien::Scunet> scunet;  // IEN_MODEL_SCUNET
  std::unique_ptr<ien::Lama> lama;      // IEN_MODEL_LAMA
  std::unique_ptr<ien::Birefnet> birefnet;  // IEN_MODEL_BIREFNET
  ien::Maps maps;
  bool use_graph = false;
  hipGraphExec_t graph = nullptr;
  // The capture held one launch: replaying it from a graph saves no host
  // work and costs a few microseconds a replay, so runs launch it directly.
  bool graph_direct = false;
  const float *graph_in = nullptr, *graph_mask = nullptr;
  float *graph_out = nullptr;
  size_t graph_w = 0, graph_h = 0;
  // 8-bit images of the u8 entry point on the device (ien_model_run_u8).
  uint8_t *d_bytes = nullptr;
  size_t bytes_cap = 0;
  // A run launched a chain of body pairs (checked when the run ends), the
  // sequence number of its first chain, and whether one of them gave up; a
  // run repeated after such a failure takes the pair path (no_chain).
  bool chained = false, chain_fell = false, no_chain = false;
  int chain_first = 0;
};

namespace ien {

static constexpr int FEATURES = 64, STEPS = 34, SCALE = 4;
// realesrgan-native lib.rs:34-41 GPU_TILE, MARGIN (= network::REACH, the 34
// layers' reach); scunet-native lib.rs:33-38 TILE, MARGIN.
static constexpr size_t ESRGAN_GPU_TILE = 768, ESRGAN_MARGIN = 34;
static constexpr size_t SCUNET_TILE = 896, SCUNET_MARGIN = 64;

static void free_maps(Maps &m) {
  (void)hipFree(m.image);
  (void)hipFree(m.a);
  (void)hipFree(m.b);
  (void)hipFree(m.d_in);
  (void)hipFree(m.d_out);
  m = Maps();
}

static void drop_graph(ien_model *model) {
  if (model->graph) (void)hipGraphExecDestroy(model->graph);
  model->graph = nullptr;
  model->graph_direct = false;
}

// gpu.rs:131-136: maps grow on demand and are never shrunk.
static ien_status ensure_maps(ien_model *model, size_t pixels, bool host_staging) {
  Maps &m = model->maps;
  if (m.pixels < pixels) {
    drop_graph(model);
    free_maps(m);
    // The f16 image, 4 halves a pixel: the fourth stays zero (the first
    // layer reads 4 channels).
    IEN_HIP(hipMalloc(&m.image, pixels * 4 * 2));
    IEN_HIP(hipMemsetAsync(m.image, 0, pixels * 4 * 2, model->ctx->stream));
    IEN_HIP(hipMalloc(&m.a, pixels * FEATURES * 2));
    IEN_HIP(hipMalloc(&m.b, pixels * FEATURES * 2));
    m.pixels = pixels;
  }
  if (host_staging && !m.d_in) {
    IEN_HIP(hipMalloc(&m.d_in, m.pixels * 3 * 4));
    IEN_HIP(hipMalloc(&m.d_out, m.pixels * 3 * SCALE * SCALE * 4));
  }
  return IEN_OK;
}

// realesrgan-native network.rs:54-74 Network::load
static ien_status load_esrgan(ien_model *model, const TensorSource &take) {
  for (int i = 0; i < STEPS; i++) {
    int cin = i == 0 ? 3 : FEATURES;
    bool last = i == STEPS - 1;
    int cout = last ? 3 * SCALE * SCALE : FEATURES;
    std::string name = "body." + std::to_string(2 * i);
    std::vector<float> w, b, s;
    ien_status st = take(name + ".weight", {(size_t)9 * cin, (size_t)cout}, &w);
    if (st != IEN_OK) return st;
    st = take(name + ".bias", {(size_t)cout}, &b);
    if (st != IEN_OK) return st;
    EsrganLayer layer;
    layer.cin = cin;
    layer.cout = cout;
    if (i == 0) {
      // The image map has 4 channels (the fourth zero): a zero weight row
      // after each tap's 3, so that K = 9 x 4 runs on the four-channel kernel.
      std::vector<float> w4((size_t)36 * cout, 0.0f);
      for (int t = 0; t < 9; t++)
        for (int c = 0; c < 3; c++)
          std::copy_n(&w[(size_t)(t * 3 + c) * cout], cout, &w4[(size_t)(t * 4 + c) * cout]);
      w.swap(w4);
      layer.cin = 4;
    }
    st = ien_matrix_new(model->ctx, w.data(), IEN_W_F32, 9 * layer.cin, cout, b.data(),
                        &layer.conv);
    if (st != IEN_OK) return st;
    model->layers.push_back(layer);
    if (!last) {
      st = take("body." + std::to_string(2 * i + 1) + ".weight", {(size_t)FEATURES}, &s);
      if (st != IEN_OK) return st;
      IEN_HIP(hipMalloc(&model->layers.back().d_slope, FEATURES * 4));
      IEN_HIP(hipMemcpy(model->layers.back().d_slope, s.data(), FEATURES * 4,
                        hipMemcpyHostToDevice));
    }
  }
  return IEN_OK;
}

// The launches of one run: input to f16, 34 convolutions, shuffle.  With
// `steps`, progress is reported after each layer; without, the whole
// network runs as one chain of pairs where the device holds every tile at
// once.
static ien_status enqueue_esrgan(ien_model *model, const float *d_image, size_t width,
                                 size_t height, float *d_out, Steps *steps) {
  ien_ctx *ctx = model->ctx;
  Maps &m = model->maps;
  const size_t pixels = width * height;
  ChainCall chain;
  chain.a = m.a;
  chain.b = m.b;
  chain.H = (int)height;
  chain.W = (int)width;
  chain.pairs = (STEPS - 2) / 2;
  for (int i = 0; i < 2 * chain.pairs; i++) {
    chain.w[i] = model->layers[1 + i].conv;
    chain.s[i] = model->layers[1 + i].d_slope;
  }
  chain.first = model->layers[0].conv;
  chain.first_slope = model->layers[0].d_slope;
  chain.last = model->layers[STEPS - 1].conv;
  chain.image = d_image;
  chain.out = d_out;
  if (!steps && !model->no_chain && chain_supported(ctx, chain)) {
    // The whole network, image to shuffled output, in one launch.
    uint16_t *out = nullptr;
    if (!model->chained) model->chain_first = ctx->chain_seq + 1;
    ien_status st = launch_chain(ctx, chain, &out);
    if (st == IEN_OK) model->chained = true;
    return st;
  }
  ien_status st = ien_pad_image(ctx, IEN_PAD_REPLICATE, d_image, nullptr, width, height, 1,
                                m.image, 4);
  if (st != IEN_OK) return st;
  // Layer i writes `a` when i is even, `b` when odd (gpu.rs:163-169); two
  // body layers in one launch where the pair kernel takes them, from one
  // map to the other (so that a pair of layers 2k - 1, 2k also ends in `a`).
  uint16_t *ma = m.a, *mb = m.b;
  for (int i = 0; i < STEPS; i++) {
    const EsrganLayer &l = model->layers[i];
    const uint16_t *src = i == 0 ? m.image : (i % 2 == 1 ? ma : mb);
    uint16_t *dst = i % 2 == 0 ? ma : mb;
    if (i % 2 == 1 && i + 1 < STEPS - 1) {
      PairCall pc;
      pc.x = ma;
      pc.y = mb;
      pc.H = (int)height;
      pc.W = (int)width;
      pc.w1 = l.conv;
      pc.s1 = l.d_slope;
      pc.w2 = model->layers[i + 1].conv;
      pc.s2 = model->layers[i + 1].d_slope;
      if (pair_supported(pc)) {
        // Layers i and i + 1 from `a` into `b`, then the roles swap back:
        // the next layer reads what this pair wrote.
        if ((st = launch_pair(ctx, pc)) != IEN_OK) return st;
        std::swap(ma, mb);
        for (int k = 0; k < 2; k++)
          if (steps && (st = steps->step(ctx->stream)) != IEN_OK) return st;
        i++;
        continue;
      }
    }
    ConvCall c;
    c.x = src;
    c.H = (int)height;
    c.W = (int)width;
    c.C = l.cin;
    c.xs = l.cin;
    c.ks = 3;
    c.stride = 1;
    c.OH = (int)height;
    c.OW = (int)width;
    c.row0 = 0;
    c.rows = (long)pixels;
    c.w = l.conv;
    c.y = dst;
    c.ys = l.cout;
    c.act = l.d_slope ? IEN_ACT_PRELU : IEN_ACT_NONE;
    c.slope = l.d_slope;
    st = launch_conv(ctx, c);
    if (st != IEN_OK) return st;
    if (i == STEPS - 1) {
      st = ien_pixel_shuffle_add(ctx, dst, (size_t)l.cout, d_image, width, height, d_out);
      if (st != IEN_OK) return st;
    }
    if (steps && (st = steps->step(ctx->stream)) != IEN_OK) return st;
  }
  return IEN_OK;
}

// Steps of a run (progress reports) and output floats per input pixel.
static int model_steps(const ien_model *m) {
  switch (m->kind) {
    case IEN_MODEL_SCUNET: return SCUNET_STEPS;
    case IEN_MODEL_LAMA: return LAMA_STEPS;
    case IEN_MODEL_BIREFNET: return BIREFNET_STEPS;
    default: return STEPS;
  }
}
static size_t out_per_pixel(const ien_model *m) {
  return m->kind == IEN_MODEL_REALESRGAN ? 3 * SCALE * SCALE
         : m->kind == IEN_MODEL_BIREFNET ? 1
                                         : 3;
}

// Maps for an image of this size, then its launches.
static ien_status prepare(ien_model *model, size_t width, size_t height) {
  if (model->kind == IEN_MODEL_SCUNET) {
    size_t pw, ph;
    scunet_padded(width, height, &pw, &ph);
    const size_t before = model->scunet->pixels;
    ien_status st = scunet_reserve(model->scunet.get(), pw, ph);
    if (st == IEN_OK && model->scunet->pixels != before) drop_graph(model);
    return st;
  }
  if (model->kind == IEN_MODEL_BIREFNET) {
    bool grew = false;
    ien_status st = birefnet_reserve(model->birefnet.get(), width, &grew);
    if (grew) drop_graph(model);
    return st;
  }
  if (model->kind == IEN_MODEL_LAMA) {
    size_t pw, ph;
    lama_padded(width, height, &pw, &ph);
    bool grew = false;
    ien_status st = lama_reserve(model->lama.get(), pw, ph, &grew);
    if (grew) drop_graph(model);
    return st;
  }
  return ensure_maps(model, width * height, false);
}

static ien_status enqueue(ien_model *model, const float *d_image, const float *d_mask,
                          size_t width, size_t height, float *d_out, Steps *steps) {
  if (model->kind == IEN_MODEL_LAMA)
    return lama_enqueue(model->lama.get(), d_image, d_mask, width, height, d_out, steps);
  if (model->kind == IEN_MODEL_BIREFNET)
    return birefnet_enqueue(model->birefnet.get(), d_image, width, d_out, steps);
  if (model->kind == IEN_MODEL_SCUNET)
    return scunet_enqueue(model->scunet.get(), d_image, width, height, d_out, steps);
  return enqueue_esrgan(model, d_image, width, height, d_out, steps);
}

static ien_status check_size(const ien_model *model, size_t width, size_t height) {
  // realesrgan-native lib.rs:302-316
  if (width == 0 || height == 0) return fail(IEN_ERR_INPUT, "empty %zu x %zu image", width, height);
  // birefnet-native lib.rs:175-187: a square side x side image, side a
  // positive multiple of 64.
  if (model->kind == IEN_MODEL_BIREFNET && (width != height || width % 64 != 0))
    return fail(IEN_ERR_INPUT, "%zu x %zu image: BiRefNet takes a square side, a multiple of 64",
                width, height);
  // lama-native lib.rs:180-187: sides of at least 9.
  if (model->kind == IEN_MODEL_LAMA && (width < LAMA_MIN_SIDE || height < LAMA_MIN_SIDE))
    return fail(IEN_ERR_INPUT, "%zu x %zu image: sides of at least %zu pixels", width, height,
                LAMA_MIN_SIDE);
  if (width > (1u << 15) || height > (1u << 15) || width * height > (1ull << 28))
    return fail(IEN_ERR_INPUT, "%zu x %zu image is too large", width, height);
  return IEN_OK;
}

static ien_status check_mask(const ien_model *model, bool has_mask) {
  if (model->kind == IEN_MODEL_LAMA)
    IEN_CHECK(has_mask, IEN_ERR_INPUT, "LaMa needs a mask");
  else
    IEN_CHECK(!has_mask, IEN_ERR_INPUT, "this model takes no mask");
  return IEN_OK;
}

// Device buffers of a run through host buffers: the f32 input, mask and
// output of a width x height image, grown on demand and never shrunk, with
// the model's maps reserved for that size.
struct Staging {
  float *in = nullptr, *mask = nullptr, *out = nullptr;
};

static ien_status grow(float **p, size_t floats) {
  (void)hipFree(*p);
  *p = nullptr;
  IEN_HIP(hipMalloc((void **)p, floats * 4));
  return IEN_OK;
}

static ien_status stage(ien_model *model, size_t width, size_t height, Staging *io) {
  ien_ctx *ctx = model->ctx;
  const size_t pixels = width * height;
  ien_status st = prepare(model, width, height);
  if (st != IEN_OK) return st;
  size_t *staged = nullptr;
  float **in = nullptr, **mask = nullptr, **out = nullptr;
  if (model->kind == IEN_MODEL_LAMA) {
    Lama &l = *model->lama;
    staged = &l.staged;
    in = &l.d_in, mask = &l.d_mask, out = &l.d_out;
  } else if (model->kind == IEN_MODEL_BIREFNET) {
    Birefnet &b = *model->birefnet;
    staged = &b.staged;
    in = &b.d_in, out = &b.d_out;
  } else if (model->kind == IEN_MODEL_SCUNET) {
    Scunet &s = *model->scunet;
    staged = &s.staged;
    in = &s.d_in, out = &s.d_out;
  } else {
    if ((st = ensure_maps(model, pixels, true)) != IEN_OK) return st;
    io->in = model->maps.d_in;
    io->out = model->maps.d_out;
    return IEN_OK;
  }
  if (*staged < pixels) {
    IEN_HIP(hipStreamSynchronize(ctx->stream));
    *staged = 0;
    if ((st = grow(in, pixels * 3)) != IEN_OK) return st;
    if (mask && (st = grow(mask, pixels)) != IEN_OK) return st;
    if ((st = grow(out, pixels * out_per_pixel(model))) != IEN_OK) return st;
    *staged = pixels;
  }
  io->in = *in;
  io->mask = mask ? *mask : nullptr;
  io->out = *out;
  return IEN_OK;
}

// Device copies of 8-bit images (input, mask, output), 256-byte aligned
// parts of one buffer grown on demand.
struct Bytes {
  uint8_t *in = nullptr, *mask = nullptr, *out = nullptr;
};

static size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

static ien_status stage_bytes(ien_model *model, size_t in, size_t mask, size_t out, Bytes *b) {
  const size_t need = round256(in) + round256(mask) + round256(out);
  if (model->bytes_cap < need) {
    IEN_HIP(hipStreamSynchronize(model->ctx->stream));
    (void)hipFree(model->d_bytes);
    model->d_bytes = nullptr;
    model->bytes_cap = 0;
    IEN_HIP(hipMalloc((void **)&model->d_bytes, need));
    model->bytes_cap = need;
  }
  b->in = model->d_bytes;
  b->mask = b->in + round256(in);
  b->out = b->mask + round256(mask);
  return IEN_OK;
}

// After a run's launches: the last step reported, then the stream drained
// (a cancelled run still finishes the work already queued, and the model
// stays usable).
static ien_status finish_run(ien_model *model, ien_status st, Steps *steps) {
  if (st == IEN_OK && steps) st = steps->drain();
  const hipError_t e = hipStreamSynchronize(model->ctx->stream);
  const bool chained = model->chained;
  model->chained = false;
  if (st != IEN_OK) return st;
  if (e != hipSuccess) return fail(IEN_ERR_GPU, "run: %s", hipGetErrorString(e));
  if (chained && (st = chain_status(model->ctx, model->chain_first)) != IEN_OK) {
    model->chain_fell = true;
    return st;
  }
  return IEN_OK;
}

// A host-buffer run whose chain gave up (a neighbour's workgroup was not
// resident in time: another stream or process holding CUs) is issued once
// more through the pair path, which gives the same bits and needs no
// workgroups resident together.
template <class Run>
static ien_status with_pair_fallback(ien_model *model, Run run) {
  model->chain_fell = false;
  ien_status st = run();
  if (st != IEN_ERR_GPU || !model->chain_fell) return st;
  model->chain_fell = false;
  model->no_chain = true;
  st = run();
  model->no_chain = false;
  return st;
}

// realesrgan-native lib.rs:230-289 / scunet-native lib.rs:192-247 tiled:
// a grid of equal tiles at most `tile` pixels on a side, each run with up
// to `margin` pixels of its surroundings, only the tile's own output kept.
// T is float (run_float_tiled) or uint8_t (Model::run: to_float on the way
// in, to_byte on the way out, both on the device).
template <typename T>
static ien_status run_tiled_once(ien_model *model, const T *image, size_t width, size_t height,
                                 size_t tile, size_t margin, T *out, ien_progress progress,
                                 void *user) {
  IEN_CHECK(model->kind == IEN_MODEL_REALESRGAN || model->kind == IEN_MODEL_SCUNET,
            IEN_ERR_INPUT, "only Real-ESRGAN and SCUNet run in tiles");
  ien_status st = check_size(model, width, height);
  if (st != IEN_OK) return st;
  IEN_CHECK(tile > 0, IEN_ERR_INPUT, "tile size 0");
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  constexpr bool bytes = sizeof(T) == 1;
  const size_t scale = model->kind == IEN_MODEL_REALESRGAN ? SCALE : 1, ow = width * scale;
  const size_t cols = (width + tile - 1) / tile, rows = (height + tile - 1) / tile;
  auto region = [&](size_t j, size_t i, size_t r[8]) {
    const size_t y0 = j * height / rows, y1 = (j + 1) * height / rows;
    const size_t x0 = i * width / cols, x1 = (i + 1) * width / cols;
    const size_t rx0 = x0 > margin ? x0 - margin : 0, ry0 = y0 > margin ? y0 - margin : 0;
    const size_t rx1 = std::min(x1 + margin, width), ry1 = std::min(y1 + margin, height);
    const size_t v[8] = {x0, x1, y0, y1, rx0, rx1, ry0, ry1};
    std::copy_n(v, 8, r);
  };
  // The largest region first, so that the buffers grow once.
  size_t big_w = 0, big_h = 0;
  for (size_t j = 0; j < rows; j++)
    for (size_t i = 0; i < cols; i++) {
      size_t r[8];
      region(j, i, r);
      if ((r[5] - r[4]) * (r[7] - r[6]) > big_w * big_h) big_w = r[5] - r[4], big_h = r[7] - r[6];
    }
  Staging io;
  if ((st = stage(model, big_w, big_h, &io)) != IEN_OK) return st;
  Bytes b;
  if (bytes && (st = stage_bytes(model, big_w * big_h * 3, 0,
                                 big_w * big_h * 3 * scale * scale, &b)) != IEN_OK)
    return st;
  const int per_tile = model_steps(model);
  Steps steps(progress, user, (int)(cols * rows) * per_tile);
  Steps *sp = progress ? &steps : nullptr;
  for (size_t j = 0; j < rows && st == IEN_OK; j++) {
    for (size_t i = 0; i < cols && st == IEN_OK; i++) {
      size_t r[8];
      region(j, i, r);
      const size_t x0 = r[0], x1 = r[1], y0 = r[2], y1 = r[3], rx0 = r[4], ry0 = r[6];
      const size_t rw = r[5] - r[4], rh = r[7] - r[6];
      if ((st = stage(model, rw, rh, &io)) != IEN_OK) break;
      const T *src = image + (ry0 * width + rx0) * 3;
      if (bytes) {
        IEN_HIP(hipMemcpy2DAsync(b.in, rw * 3, src, width * 3, rw * 3, rh, hipMemcpyHostToDevice,
                                 ctx->stream));
        if ((st = bytes_to_floats(ctx, b.in, io.in, rw * rh * 3)) != IEN_OK) break;
      } else {
        IEN_HIP(hipMemcpy2DAsync(io.in, rw * 3 * 4, src, width * 3 * 4, rw * 3 * 4, rh,
                                 hipMemcpyHostToDevice, ctx->stream));
      }
      if ((st = enqueue(model, io.in, nullptr, rw, rh, io.out, sp)) != IEN_OK) break;
      // The tile's own output: rows y0 .. y1, columns x0 .. x1 (scaled).
      const size_t rws = rw * scale, cw = (x1 - x0) * scale;
      const size_t from = ((y0 - ry0) * scale * rws + (x0 - rx0) * scale) * 3;
      T *dst = out + (y0 * scale * ow + x0 * scale) * 3;
      if (bytes) {
        if ((st = floats_to_bytes(ctx, io.out, b.out, rws * rh * scale * 3)) != IEN_OK) break;
        IEN_HIP(hipMemcpy2DAsync(dst, ow * 3, b.out + from, rws * 3, cw * 3, (y1 - y0) * scale,
                                 hipMemcpyDeviceToHost, ctx->stream));
      } else {
        IEN_HIP(hipMemcpy2DAsync(dst, ow * 3 * 4, io.out + from, rws * 3 * 4, cw * 3 * 4,
                                 (y1 - y0) * scale, hipMemcpyDeviceToHost, ctx->stream));
      }
    }
  }
  return finish_run(model, st, sp);
}

template <typename T>
static ien_status run_tiled(ien_model *model, const T *image, size_t width, size_t height,
                            size_t tile, size_t margin, T *out, ien_progress progress, void *user) {
  return with_pair_fallback(model, [&]() {
    return run_tiled_once(model, image, width, height, tile, margin, out, progress, user);
  });
}

}  // namespace ien

using namespace ien;

extern "C" {

static ien_status model_new(ien_ctx *ctx, ien_model_kind kind, const TensorSource &take,
                            const ShapeOf &shape, ien_model **out) {
  IEN_CHECK(ctx && out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(kind == IEN_MODEL_REALESRGAN || kind == IEN_MODEL_SCUNET || kind == IEN_MODEL_LAMA ||
                kind == IEN_MODEL_BIREFNET,
            IEN_ERR_INPUT, "model kind %d", (int)kind);
  IEN_HIP(hipSetDevice(ctx->device));
  std::unique_ptr<ien_model> model(new ien_model);
  model->ctx = ctx;
  model->kind = kind;
  ien_status st;
  if (kind == IEN_MODEL_SCUNET) {
    model->scunet.reset(new Scunet);
    st = scunet_load(ctx, take, model->scunet.get());
  } else if (kind == IEN_MODEL_LAMA) {
    model->lama.reset(new Lama);
    st = lama_load(ctx, take, model->lama.get());
  } else if (kind == IEN_MODEL_BIREFNET) {
    model->birefnet.reset(new Birefnet);
    st = birefnet_load(ctx, take, shape, model->birefnet.get());
  } else {
    st = load_esrgan(model.get(), take);
  }
  if (st != IEN_OK) {
    ien_model_free(model.release());
    return st;
  }
  *out = model.release();
  return IEN_OK;
}

ien_status ien_model_load(ien_ctx *ctx, ien_model_kind kind, const char *weights_path,
                          ien_model **out) {
  IEN_CHECK(weights_path, IEN_ERR_INPUT, "no weights path");
  WeightFile file;
  // The weights files' magics (realesrgan-native lib.rs:124, scunet-native
  // lib.rs:101, lama-native lib.rs:96).
  // birefnet-native lib.rs:84
  ien_status st = file.read(weights_path, kind == IEN_MODEL_SCUNET     ? "SCUNET\0\0"
                                          : kind == IEN_MODEL_LAMA     ? "LAMA\0\0\0\0"
                                          : kind == IEN_MODEL_BIREFNET ? "BIREFNET"
                                                                       : "REALESRG");
  if (st != IEN_OK) return st;
  st = model_new(
      ctx, kind,
      [&](const std::string &n, std::vector<size_t> s, std::vector<float> *o) {
        return file.take(n, s, o);
      },
      [&](const std::string &n, std::vector<size_t> *s) { return file.shape_of(n, s); }, out);
  if (st != IEN_OK) return st;
  st = file.finish();
  if (st != IEN_OK) {
    ien_model_free(*out);
    *out = nullptr;
  }
  return st;
}

ien_status ien_model_from_tensors(ien_ctx *ctx, ien_model_kind kind, const ien_tensor *tensors,
                                  size_t count, ien_model **out) {
  IEN_CHECK(tensors || count == 0, IEN_ERR_INPUT, "null tensors");
  WeightFile file;
  for (size_t i = 0; i < count; i++) {
    IEN_CHECK(tensors[i].name && tensors[i].values && tensors[i].rank <= 4, IEN_ERR_INPUT,
              "tensor %zu", i);
    Tensor t;
    size_t elems = 1;
    for (size_t d = 0; d < tensors[i].rank; d++) {
      t.shape.push_back(tensors[i].dims[d]);
      elems *= tensors[i].dims[d];
    }
    t.values.assign(tensors[i].values, tensors[i].values + elems);
    if (!file.tensors.emplace(tensors[i].name, std::move(t)).second)
      return fail(IEN_ERR_WEIGHTS, "%s: stored twice", tensors[i].name);
  }
  ien_status st = model_new(
      ctx, kind,
      [&](const std::string &n, std::vector<size_t> s, std::vector<float> *o) {
        return file.take(n, s, o);
      },
      [&](const std::string &n, std::vector<size_t> *s) { return file.shape_of(n, s); }, out);
  if (st != IEN_OK) return st;
  st = file.finish();
  if (st != IEN_OK) {
    ien_model_free(*out);
    *out = nullptr;
  }
  return st;
}

void ien_model_free(ien_model *model) {
  if (!model) return;
  if (model->ctx) {
    (void)hipSetDevice(model->ctx->device);
    (void)hipStreamSynchronize(model->ctx->stream);
  }
  drop_graph(model);
  for (auto &l : model->layers) {
    ien_matrix_free(l.conv);
    (void)hipFree(l.d_slope);
  }
  if (model->scunet) scunet_free(model->scunet.get());
  if (model->lama) lama_free(model->lama.get());
  if (model->birefnet) birefnet_free(model->birefnet.get());
  free_maps(model->maps);
  (void)hipFree(model->d_bytes);
  delete model;
}

ien_status ien_model_set_graph(ien_model *model, int enabled) {
  IEN_CHECK(model, IEN_ERR_INPUT, "no model");
  model->use_graph = enabled != 0;
  if (!model->use_graph) drop_graph(model);
  return IEN_OK;
}

static ien_status run_device(ien_model *model, const float *d_image, const float *d_mask,
                             size_t width, size_t height, float *d_out) {
  if (model->kind == IEN_MODEL_LAMA)
    IEN_CHECK(d_mask != nullptr, IEN_ERR_INPUT, "LaMa needs a mask");
  else
    IEN_CHECK(d_mask == nullptr, IEN_ERR_INPUT, "this model takes no mask");
  ien_status st = check_size(model, width, height);
  if (st != IEN_OK) return st;
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  st = prepare(model, width, height);
  if (st != IEN_OK) return st;
  if (!model->use_graph) return enqueue(model, d_image, d_mask, width, height, d_out, nullptr);
  const bool same = model->graph_in == d_image && model->graph_mask == d_mask &&
                    model->graph_out == d_out && model->graph_w == width && model->graph_h == height;
  if (same && model->graph_direct)
    return enqueue(model, d_image, d_mask, width, height, d_out, nullptr);
  if (!model->graph || !same) {
    drop_graph(model);
    hipGraph_t graph = nullptr;
    IEN_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    st = enqueue(model, d_image, d_mask, width, height, d_out, nullptr);
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (st != IEN_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return st;
    }
    if (e != hipSuccess) return fail(IEN_ERR_GPU, "graph capture: %s", hipGetErrorString(e));
    size_t nodes = 0;
    e = hipGraphGetNodes(graph, nullptr, &nodes);
    if (e == hipSuccess && nodes == 1) {
      (void)hipGraphDestroy(graph);
      model->graph_direct = true;
    } else {
      if (e == hipSuccess) e = hipGraphInstantiate(&model->graph, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      if (e != hipSuccess) {
        model->graph = nullptr;
        return fail(IEN_ERR_GPU, "graph instantiate: %s", hipGetErrorString(e));
      }
    }
    model->graph_in = d_image;
    model->graph_mask = d_mask;
    model->graph_out = d_out;
    model->graph_w = width;
    model->graph_h = height;
    // (the capture ran nothing)
    if (model->graph_direct) return enqueue(model, d_image, d_mask, width, height, d_out, nullptr);
  }
  IEN_HIP(hipGraphLaunch(model->graph, ctx->stream));
  return IEN_OK;
}

ien_status ien_model_run_device(ien_model *model, const float *d_image, const float *d_mask,
                                size_t width, size_t height, float *d_out) {
  IEN_CHECK(model && d_image && d_out, IEN_ERR_INPUT, "null argument");
  const ien_status st = run_device(model, d_image, d_mask, width, height, d_out);
  // The device path does not wait for its chains: ien_model_status reports
  // them.
  model->chained = false;
  return st;
}

ien_status ien_model_status(ien_model *model) {
  IEN_CHECK(model, IEN_ERR_INPUT, "no model");
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return fail(IEN_ERR_GPU, "run: %s", hipGetErrorString(e));
  return chain_status(ctx, 1);
}

static ien_status run_host(ien_model *model, const float *image, const float *mask, size_t width,
                           size_t height, float *out, ien_progress progress, void *user) {
  ien_status st = check_mask(model, mask != nullptr);
  if (st == IEN_OK) st = check_size(model, width, height);
  if (st != IEN_OK) return st;
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  const size_t pixels = width * height;
  Staging io;
  if ((st = stage(model, width, height, &io)) != IEN_OK) return st;
  if (mask) IEN_HIP(hipMemcpyAsync(io.mask, mask, pixels * 4, hipMemcpyHostToDevice, ctx->stream));
  IEN_HIP(hipMemcpyAsync(io.in, image, pixels * 3 * 4, hipMemcpyHostToDevice, ctx->stream));
  Steps steps(progress, user, model_steps(model));
  Steps *sp = progress ? &steps : nullptr;
  st = enqueue(model, io.in, mask ? io.mask : nullptr, width, height, io.out, sp);
  if ((st = finish_run(model, st, sp)) != IEN_OK) return st;
  IEN_HIP(hipMemcpy(out, io.out, pixels * out_per_pixel(model) * 4, hipMemcpyDeviceToHost));
  return IEN_OK;
}

ien_status ien_model_run(ien_model *model, const float *image, const float *mask, size_t width,
                         size_t height, float *out, ien_progress progress, void *user) {
  IEN_CHECK(model && image && out, IEN_ERR_INPUT, "null argument");
  return with_pair_fallback(model, [&]() {
    return run_host(model, image, mask, width, height, out, progress, user);
  });
}

ien_status ien_model_run_tiled(ien_model *model, const float *image, size_t width,
                               size_t height, size_t tile, size_t margin, float *out,
                               ien_progress progress, void *user) {
  IEN_CHECK(model && image && out, IEN_ERR_INPUT, "null argument");
  return run_tiled(model, image, width, height, tile, margin, out, progress, user);
}

ien_status ien_model_run_u8(ien_model *model, const uint8_t *rgb, const uint8_t *mask,
                            size_t width, size_t height, void *out, ien_progress progress,
                            void *user) {
  IEN_CHECK(model && rgb && out, IEN_ERR_INPUT, "null argument");
  ien_status st = check_mask(model, mask != nullptr);
  if (st != IEN_OK) return st;
  // realesrgan-native lib.rs:164-188 and scunet-native lib.rs:123-148:
  // tiles of the engine's size with the model's margin, bytes in and out.
  if (model->kind == IEN_MODEL_REALESRGAN)
    return run_tiled(model, rgb, width, height, ESRGAN_GPU_TILE, ESRGAN_MARGIN, (uint8_t *)out,
                     progress, user);
  if (model->kind == IEN_MODEL_SCUNET)
    return run_tiled(model, rgb, width, height, SCUNET_TILE, SCUNET_MARGIN, (uint8_t *)out,
                     progress, user);
  if ((st = check_size(model, width, height)) != IEN_OK) return st;
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  const size_t pixels = width * height;
  Staging io;
  if ((st = stage(model, width, height, &io)) != IEN_OK) return st;
  const bool lama = model->kind == IEN_MODEL_LAMA;
  Bytes b;
  if ((st = stage_bytes(model, pixels * 3, lama ? pixels : 0, lama ? pixels * 3 : 0, &b)) != IEN_OK)
    return st;
  IEN_HIP(hipMemcpyAsync(b.in, rgb, pixels * 3, hipMemcpyHostToDevice, ctx->stream));
  if (lama) {
    // lama-native lib.rs:138-142: the image / 255 and the mask as 0 or 1.
    IEN_HIP(hipMemcpyAsync(b.mask, mask, pixels, hipMemcpyHostToDevice, ctx->stream));
    st = bytes_to_floats(ctx, b.in, io.in, pixels * 3);
    if (st == IEN_OK) st = mask_bytes(ctx, b.mask, io.mask, pixels);
  } else {
    // birefnet-native lib.rs:111-116: ImageNet's mean and deviation.
    static const float mean[3] = {0.485f, 0.456f, 0.406f}, deviation[3] = {0.229f, 0.224f, 0.225f};
    st = normalize_bytes(ctx, b.in, pixels, mean, deviation, io.in);
  }
  Steps steps(progress, user, model_steps(model));
  Steps *sp = progress ? &steps : nullptr;
  if (st == IEN_OK) st = enqueue(model, io.in, lama ? io.mask : nullptr, width, height, io.out, sp);
  // lama-native lib.rs:147-155: the holes take the prediction as bytes.
  if (st == IEN_OK && lama) st = composite_bytes(ctx, b.in, b.mask, io.out, pixels, b.out);
  if ((st = finish_run(model, st, sp)) != IEN_OK) return st;
  if (lama)
    IEN_HIP(hipMemcpy(out, b.out, pixels * 3, hipMemcpyDeviceToHost));
  else
    IEN_HIP(hipMemcpy(out, io.out, pixels * 4, hipMemcpyDeviceToHost));
  return IEN_OK;
}

}  // extern "C"
