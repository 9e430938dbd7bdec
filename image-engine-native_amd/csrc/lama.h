// lama.h -- the Big LaMa generator object behind ien_model (internal).
#pragma once

#include "ien_internal.h"
#include "scunet.h"

namespace ien {

// network.rs:140-148 Ffc: one fast Fourier convolution's products.
struct LamaFfc {
  ien_matrix *local = nullptr, *cross = nullptr, *spectral_in = nullptr, *fourier = nullptr,
             *spectral_out = nullptr;
};

struct Lama {
  ien_ctx *ctx = nullptr;
  ien_matrix *first = nullptr, *down[3] = {}, *up[3][4] = {}, *last = nullptr;
  LamaFfc blocks[18][2];
  ien_fourier *fourier = nullptr;  // for the eighth-scale maps of the current size
  size_t pw = 0, ph = 0;           // padded size the maps and the plan are for
  size_t pixels = 0;               // padded pixels the maps hold
  // Full-scale 4-channel input; maps at 1, 1/2, 1/4 (reused by the ups);
  // eighth-scale a, mid, out, spectral; spectra; phase products; RGB.
  uint16_t *in4 = nullptr, *m0 = nullptr, *m1 = nullptr, *m2 = nullptr, *a = nullptr,
           *mid = nullptr, *out = nullptr, *spectral = nullptr, *spectrum = nullptr,
           *filtered = nullptr, *rows = nullptr, *rgb = nullptr;
  float *work = nullptr;
  float *d_in = nullptr, *d_mask = nullptr, *d_out = nullptr;  // host-API staging
  size_t staged = 0;
};

constexpr int LAMA_STEPS = 26;     // network.rs:41-44 STEPS
constexpr size_t LAMA_MIN_SIDE = 9;  // network.rs:38-40 MIN_SIDE

ien_status lama_load(ien_ctx *ctx, const TensorSource &take, Lama *l);
void lama_free(Lama *l);
void lama_padded(size_t width, size_t height, size_t *pw, size_t *ph);
// Maps and the Fourier plan for a padded pw x ph image (outside graph
// capture); *grew is set when buffers or the plan were replaced.
ien_status lama_reserve(Lama *l, size_t pw, size_t ph, bool *grew);
ien_status lama_enqueue(Lama *l, const float *d_image, const float *d_mask, size_t width,
                        size_t height, float *d_out, Steps *steps);

}  // namespace ien
