// scunet.h -- the SCUNet network object behind ien_model (internal).
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "ien_internal.h"

namespace ien {

// A weights source: take(name, shape, &values) as weight_file.rs:119-137.
using TensorSource = std::function<ien_status(const std::string &, std::vector<size_t>,
                                              std::vector<float> *)>;

struct ScunetBlock {
  int c = 0;
  ien_matrix *split = nullptr, *conv1 = nullptr, *conv2 = nullptr, *join = nullptr;
  ien_swin *swin = nullptr;
};

struct Scunet {
  ien_ctx *ctx = nullptr;
  ien_matrix *head = nullptr, *tail = nullptr, *halve[3] = {}, *dbl[3] = {};
  ScunetBlock down[3][4], body[4], up[3][4];
  size_t pixels = 0;  // padded pixels the maps hold
  uint16_t *img = nullptr, *x = nullptr, *y = nullptr, *t = nullptr,
           *skip[3] = {}, *out16 = nullptr;
  float *d_in = nullptr, *d_out = nullptr;  // host-API staging
  size_t staged = 0;                        // pixels of the staging buffers
};

constexpr int SCUNET_STEPS = 28;  // blocks of a run (network.rs:27-31)

ien_status scunet_load(ien_ctx *ctx, const TensorSource &take, Scunet *s);
void scunet_free(Scunet *s);
void scunet_padded(size_t width, size_t height, size_t *pw, size_t *ph);
// Maps and every block's scratch for a padded pw x ph image (outside graph
// capture).
ien_status scunet_reserve(Scunet *s, size_t pw, size_t ph);
ien_status scunet_enqueue(Scunet *s, const float *d_image, size_t width, size_t height,
                          float *d_out, Steps *steps);

}  // namespace ien
