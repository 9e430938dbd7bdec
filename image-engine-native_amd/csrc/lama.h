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
  ien_spectral *spectral_plan = nullptr;  // the fused spectral branch (sides <= 64), else null
  size_t pw = 0, ph = 0;           // padded size the maps and the plan are for
  size_t pixels = 0;               // padded pixels the maps hold
  // Full-scale 4-channel input; maps at 1, 1/2, 1/4 (reused by the ups);
  // eighth-scale a, mid, out, spectral; spectra; RGB.
  uint16_t *in4 = nullptr, *m0 = nullptr, *m1 = nullptr, *m2 = nullptr, *a = nullptr,
           *mid = nullptr, *out = nullptr, *spectral = nullptr, *spectrum = nullptr,
           *filtered = nullptr, *rgb = nullptr;
  float *work = nullptr;
  // The FFC pipeline's cross-stream points: the context's stream after a
  // local convolution, branch 2 after a cross convolution.
  hipEvent_t ev_local = nullptr, ev_cross = nullptr;
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
// spectral.hip: the spectral branch of an FFC in three launches: the front
// two (spectral_in product and row transform; column transforms around the
// fourier product) write the spectral map, R (h w 192 floats) and U (h half
// 384 floats); the back one (inverse rows, residual, spectral_out product
// accumulated with ReLU onto `out`) runs after the cross convolution.
bool spectral_shapes(const ien_matrix *in, const ien_matrix *f, const ien_matrix *out);
ien_status spectral_front(const ien_spectral *sp, const uint16_t *x, long xs,
                          const ien_matrix *m_in, const ien_matrix *m_f, uint16_t *spectral,
                          float *r, float *u);
// The front's two launches one at a time: the rows (spectral map and R),
// then the columns (U).
ien_status spectral_rows(const ien_spectral *sp, const uint16_t *x, long xs,
                         const ien_matrix *m_in, uint16_t *spectral, float *r);
ien_status spectral_columns(const ien_spectral *sp, const ien_matrix *m_f, const float *r,
                            float *u);
// The result (ReLU(out + spectral_out(spectral + irfft(u)))) goes to dst
// (out when null), with `add` (rows ys apart, or null) added after the
// rounding and rounded again.
ien_status spectral_back(const ien_spectral *sp, const ien_matrix *m_out, const uint16_t *spectral,
                         const float *u, uint16_t *out, long ys, uint16_t *dst = nullptr,
                         const uint16_t *add = nullptr);
size_t spectral_r_floats(const ien_spectral *sp);
size_t spectral_u_floats(const ien_spectral *sp);

ien_status lama_enqueue(Lama *l, const float *d_image, const float *d_mask, size_t width,
                        size_t height, float *d_out, Steps *steps);

}  // namespace ien
