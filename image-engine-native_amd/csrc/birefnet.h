// birefnet.h -- the BiRefNet-lite network object behind ien_model (internal).
#pragma once

#include "ien_internal.h"
#include "scunet.h"

namespace ien {

// The shape of a stored tensor, without taking it (false when absent).
using ShapeOf = std::function<bool(const std::string &, std::vector<size_t> *)>;

// decoder.rs:56-76 Block: conv_in, the ASPP (deformable-free), conv_out and
// the optional gradient-attention gate.
struct BirefnetBlock {
  int cin = 0, cout = 0;
  ien_matrix *conv_in = nullptr, *conv_out = nullptr, *branch[4] = {}, *conv1 = nullptr,
             *gdt = nullptr;
  // A deformable branch's offset convolution (2 taps offsets, then taps
  // modulator logits); null where they are all zero, which makes the
  // branch a plain size x size convolution.
  ien_matrix *offset[4] = {};
  // pool weight [64][256], pool bias [256], conv1's pooling rows [256][64],
  // conv1's bias [64]: f32 on the device for the pooling kernel.
  float *d_pool = nullptr;
  float gdt_w[16] = {}, gdt_b = 0.0f;
  bool gate = false;
};

struct Birefnet {
  ien_ctx *ctx = nullptr;
  int window = 0;
  ien_matrix *embed = nullptr;
  float *d_embed_ln = nullptr;  // gamma, beta (96 each)
  std::vector<ien_swin *> blocks[4];
  float *d_norm[4] = {};        // stage output norms: gamma, beta
  float *d_merge_ln[3] = {};    // merge norms over 4c: gamma, beta
  ien_matrix *merge[3] = {};
  BirefnetBlock dec[5];         // squeeze, blocks 4..1
  ien_matrix *lateral[3] = {};  // levels 3, 2, 1 (768, 384, 192 channels)
  ien_matrix *patch_conv1[4] = {}, *patch_out[4] = {};  // patches5..2
  ien_matrix *head = nullptr;
  float head_bias = 0.0f;
  // Full-resolution branch (f32, device): the composed 5x5 weights [25][3]
  // and their bias, conv1 [27][64], bias1 [64], conv_out [9][64]; its
  // output bias on the host.
  float *d_full = nullptr;
  float bias_out = 0.0f;
  // Deformable branches: their offsets (f32, 3 taps a pixel) and the
  // bilinear samples of one chunk of rows (f16, taps x 64 a row).
  bool deformable = false;
  float *offs = nullptr;
  uint16_t *samples = nullptr;
  size_t side = 0;  // the side the maps are reserved for
  uint16_t *img16 = nullptr, *half16 = nullptr, *prow = nullptr, *x = nullptr, *mrows = nullptr,
           *level[4] = {}, *tmp = nullptr, *x4 = nullptr, *in = nullptr, *t = nullptr,
           *a = nullptr, *cat = nullptr, *g = nullptr, *prev = nullptr, *stacked = nullptr,
           *mid = nullptr, *low = nullptr;
  float *partial = nullptr, *d_bias = nullptr;
  // The half-size backbone's own patch rows, token map, merge rows and Swin
  // scratch: it runs on a branch stream beside the full-size one.
  uint16_t *hprow = nullptr, *hx = nullptr, *hmrows = nullptr, *hscratch = nullptr;
  size_t hscratch_halves = 0;
  float *d_in = nullptr, *d_out = nullptr;  // host-API staging
  size_t staged = 0;
};

constexpr int BIREFNET_STEPS = 14;  // 2 x 4 backbone stages, 5 decoder blocks, the head

ien_status birefnet_load(ien_ctx *ctx, const TensorSource &take, const ShapeOf &shape,
                         Birefnet *b);
void birefnet_free(Birefnet *b);
// Maps and every Swin block's scratch for a side x side image (outside
// graph capture); *grew is set when buffers were replaced.
ien_status birefnet_reserve(Birefnet *b, size_t side, bool *grew);
ien_status birefnet_enqueue(Birefnet *b, const float *d_image, size_t side, float *d_logits,
                            Steps *steps);

}  // namespace ien
