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
  const float *graph_in = nullptr, *graph_mask = nullptr;
  float *graph_out = nullptr;
  size_t graph_w = 0, graph_h = 0;
};

namespace ien {

static constexpr int FEATURES = 64, STEPS = 34, SCALE = 4;

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
// `events`, one event is recorded after each layer for progress reports.
static ien_status enqueue_esrgan(ien_model *model, const float *d_image, size_t width,
                                 size_t height, float *d_out, hipEvent_t *events) {
  ien_ctx *ctx = model->ctx;
  Maps &m = model->maps;
  const size_t pixels = width * height;
  ien_status st = ien_pad_image(ctx, IEN_PAD_REPLICATE, d_image, nullptr, width, height, 1,
                                m.image, 4);
  if (st != IEN_OK) return st;
  for (int i = 0; i < STEPS; i++) {
    const EsrganLayer &l = model->layers[i];
    // Layer i writes `a` when i is even, `b` when odd (gpu.rs:163-169).
    const uint16_t *src = i == 0 ? m.image : (i % 2 == 1 ? m.a : m.b);
    uint16_t *dst = i % 2 == 0 ? m.a : m.b;
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
    if (events) IEN_HIP(hipEventRecord(events[i], ctx->stream));
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
                          size_t width, size_t height, float *d_out, hipEvent_t *events) {
  if (model->kind == IEN_MODEL_LAMA)
    return lama_enqueue(model->lama.get(), d_image, d_mask, width, height, d_out, events);
  if (model->kind == IEN_MODEL_BIREFNET)
    return birefnet_enqueue(model->birefnet.get(), d_image, width, d_out, events);
  if (model->kind == IEN_MODEL_SCUNET)
    return scunet_enqueue(model->scunet.get(), d_image, width, height, d_out, events);
  return enqueue_esrgan(model, d_image, width, height, d_out, events);
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
  delete model;
}

ien_status ien_model_set_graph(ien_model *model, int enabled) {
  IEN_CHECK(model, IEN_ERR_INPUT, "no model");
  model->use_graph = enabled != 0;
  if (!model->use_graph) drop_graph(model);
  return IEN_OK;
}

ien_status ien_model_run_device(ien_model *model, const float *d_image, const float *d_mask,
                                size_t width, size_t height, float *d_out) {
  IEN_CHECK(model && d_image && d_out, IEN_ERR_INPUT, "null argument");
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
  if (!model->graph || model->graph_in != d_image || model->graph_mask != d_mask ||
      model->graph_out != d_out || model->graph_w != width || model->graph_h != height) {
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
    e = hipGraphInstantiate(&model->graph, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
      model->graph = nullptr;
      return fail(IEN_ERR_GPU, "graph instantiate: %s", hipGetErrorString(e));
    }
    model->graph_in = d_image;
    model->graph_mask = d_mask;
    model->graph_out = d_out;
    model->graph_w = width;
    model->graph_h = height;
  }
  IEN_HIP(hipGraphLaunch(model->graph, ctx->stream));
  return IEN_OK;
}

ien_status ien_model_run(ien_model *model, const float *image, const float *mask, size_t width,
                         size_t height, float *out, ien_progress progress, void *user) {
  IEN_CHECK(model && image && out, IEN_ERR_INPUT, "null argument");
  if (model->kind == IEN_MODEL_LAMA)
    IEN_CHECK(mask != nullptr, IEN_ERR_INPUT, "LaMa needs a mask");
  else
    IEN_CHECK(mask == nullptr, IEN_ERR_INPUT, "this model takes no mask");
  ien_status st = check_size(model, width, height);
  if (st != IEN_OK) return st;
  ien_ctx *ctx = model->ctx;
  IEN_HIP(hipSetDevice(ctx->device));
  const size_t pixels = width * height;
  float *d_in = nullptr, *d_out = nullptr, *d_mask = nullptr;
  if (model->kind == IEN_MODEL_LAMA) {
    Lama &l = *model->lama;
    st = prepare(model, width, height);
    if (st != IEN_OK) return st;
    if (l.staged < pixels) {
      IEN_HIP(hipStreamSynchronize(ctx->stream));
      (void)hipFree(l.d_in);
      (void)hipFree(l.d_mask);
      (void)hipFree(l.d_out);
      l.d_in = l.d_mask = l.d_out = nullptr;
      l.staged = 0;
      IEN_HIP(hipMalloc(&l.d_in, pixels * 3 * 4));
      IEN_HIP(hipMalloc(&l.d_mask, pixels * 4));
      IEN_HIP(hipMalloc(&l.d_out, pixels * 3 * 4));
      l.staged = pixels;
    }
    d_in = l.d_in;
    d_mask = l.d_mask;
    d_out = l.d_out;
    IEN_HIP(hipMemcpyAsync(d_mask, mask, pixels * 4, hipMemcpyHostToDevice, ctx->stream));
  } else if (model->kind == IEN_MODEL_BIREFNET) {
    Birefnet &b = *model->birefnet;
    st = prepare(model, width, height);
    if (st != IEN_OK) return st;
    if (b.staged < pixels) {
      IEN_HIP(hipStreamSynchronize(ctx->stream));
      (void)hipFree(b.d_in);
      (void)hipFree(b.d_out);
      b.d_in = b.d_out = nullptr;
      b.staged = 0;
      IEN_HIP(hipMalloc(&b.d_in, pixels * 3 * 4));
      IEN_HIP(hipMalloc(&b.d_out, pixels * 4));
      b.staged = pixels;
    }
    d_in = b.d_in;
    d_out = b.d_out;
  } else if (model->kind == IEN_MODEL_SCUNET) {
    Scunet &s = *model->scunet;
    st = prepare(model, width, height);
    if (st != IEN_OK) return st;
    if (s.staged < pixels) {
      IEN_HIP(hipStreamSynchronize(ctx->stream));
      (void)hipFree(s.d_in);
      (void)hipFree(s.d_out);
      s.d_in = s.d_out = nullptr;
      s.staged = 0;
      IEN_HIP(hipMalloc(&s.d_in, pixels * 3 * 4));
      IEN_HIP(hipMalloc(&s.d_out, pixels * 3 * 4));
      s.staged = pixels;
    }
    d_in = s.d_in;
    d_out = s.d_out;
  } else {
    st = ensure_maps(model, pixels, true);
    if (st != IEN_OK) return st;
    d_in = model->maps.d_in;
    d_out = model->maps.d_out;
  }
  IEN_HIP(hipMemcpyAsync(d_in, image, pixels * 3 * 4, hipMemcpyHostToDevice, ctx->stream));
  const int steps = model_steps(model);
  std::vector<hipEvent_t> events;
  if (progress) {
    events.resize(steps);
    for (auto &e : events) IEN_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  }
  st = enqueue(model, d_in, d_mask, width, height, d_out, progress ? events.data() : nullptr);
  bool cancelled = false;
  if (st == IEN_OK && progress) {
    // lib.rs:168-188 (SCUNet lib.rs:205-215): progress after each layer or
    // block, in order; a break stops the run with Cancelled and leaves the
    // model usable.
    for (int i = 0; i < steps && !cancelled; i++) {
      hipError_t e = hipEventSynchronize(events[i]);
      if (e != hipSuccess) {
        st = fail(IEN_ERR_GPU, "step %d: %s", i, hipGetErrorString(e));
        break;
      }
      if (progress((float)(i + 1) / steps, user) != 0) cancelled = true;
    }
  }
  hipError_t e = hipStreamSynchronize(ctx->stream);
  for (auto &ev : events) (void)hipEventDestroy(ev);
  if (st != IEN_OK) return st;
  if (e != hipSuccess) return fail(IEN_ERR_GPU, "run: %s", hipGetErrorString(e));
  if (cancelled) return fail(IEN_ERR_CANCELLED, "the progress callback stopped the run");
  IEN_HIP(hipMemcpy(out, d_out, pixels * out_per_pixel(model) * 4, hipMemcpyDeviceToHost));
  return IEN_OK;
}

}  // extern "C"
