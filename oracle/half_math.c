/*
 * half_math.c -- oracle restatement of native-engine's half.rs and math.rs.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Pins: tests/test_oracle_half.py (all 65536 halves and 2^20 float bit
 * patterns against numpy's round-to-nearest-even float16, plus the known
 * answers of half.rs:194-233), tests/test_oracle_math.py (erf series, libm
 * sigmoid, f64 softmax and LayerNorm, torch fixtures).
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

static inline uint32_t bits_of(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}
static inline float float_of(uint32_t u) {
  float v;
  memcpy(&v, &u, 4);
  return v;
}

/* half.rs:7-40 -- nearest half float, ties to even; NaN stays NaN. */
static inline uint32_t round_te(uint32_t kept, uint32_t low, uint32_t shift) {
  uint32_t half = 1u << (shift - 1);
  return kept + ((low > half || (low == half && (kept & 1u))) ? 1u : 0u);
}

uint16_t or_f32_to_half(float v) {
  uint32_t x = bits_of(v);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t mantissa = x & 0x7fffffu;
  if (((x >> 23) & 0xffu) == 0xffu)
    return sign | 0x7c00u | (mantissa == 0 ? 0 : 0x200u);
  int exponent = (int)((x >> 23) & 0xffu) - 112;
  if (exponent >= 31) return sign | 0x7c00u;
  if (exponent <= 0) {
    if (exponent < -10) return sign;
    uint32_t significand = mantissa | 0x800000u;
    uint32_t shift = (uint32_t)(14 - exponent);
    uint32_t low = significand & ((1u << shift) - 1u);
    return sign | (uint16_t)round_te(significand >> shift, low, shift);
  }
  return sign | (uint16_t)round_te(((uint32_t)exponent << 10) | (mantissa >> 13),
                                   mantissa & 0x1fffu, 13);
}

/* half.rs:125-140 -- exact widening. */
float or_half_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exponent = (h >> 10) & 0x1fu;
  uint32_t mantissa = h & 0x3ffu;
  if (exponent == 0 && mantissa == 0) return float_of(sign);
  if (exponent == 0) {
    float magnitude = (float)mantissa * float_of(0x33800000u);
    return sign ? -magnitude : magnitude;
  }
  if (exponent == 0x1f) return float_of(sign | 0x7f800000u | (mantissa << 13));
  return float_of(sign | ((exponent + 112) << 23) | (mantissa << 13));
}

void or_floats_to_halves(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_half(src[i]);
}

void or_halves_to_f32(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_half_to_f32(src[i]);
}

/* math.rs:9-31 -- exp(z) for z <= 0: 2^n times a degree-5 polynomial, n
 * rounded by a magic bias (XNNPACK's f32 "p5" method, BSD-3-Clause). */
float or_exp_neg(float z) {
  const float magic = float_of(0x4b40007fu), log2e = float_of(0x3fb8aa3bu);
  const float ln2_hi = float_of(0xbf317200u), ln2_lo = float_of(0xb5bfbe8eu);
  const float c5 = float_of(0x3c07cfceu), c4 = float_of(0x3d2b9d0du);
  const float c3 = float_of(0x3e2aad40u), c2 = float_of(0x3efffee3u);
  const float c1 = float_of(0x3f7ffffbu), cutoff = float_of(0xc2aeac4fu);
  float n = z * log2e + magic;
  float s = float_of(bits_of(n) << 23);
  n = n - magic;
  float t = n * ln2_lo + (n * ln2_hi + z);
  float p = (((c5 * t + c4) * t + c3) * t + c2) * t + c1;
  float e = (t * s) * p + s;
  return z < cutoff ? 0.0f : e;
}

/* math.rs:33-39 */
static inline float sigmoid_one(float x) {
  float e = or_exp_neg(-fabsf(x));
  float s = e / (e + 1.0f);
  return x > 0.0f ? 1.0f - s : s;
}

void or_sigmoid(float *x, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] = sigmoid_one(x[i]);
}

/* math.rs:41-75 -- exact GELU through erf(x) = x P(x^2) / Q(x^2) on [-4, 4]
 * (Eigen's generic_fast_erf_float coefficients, MPL-2.0). */
static const float ERF_A[7] = {-2.7261423e-10f, 2.7706814e-08f, -2.101024e-06f,
                               -5.6925064e-05f, -7.3499063e-04f, -2.9546e-03f,
                               -1.6096033e-02f};
static const float ERF_B[5] = {-1.4566072e-05f, -2.1337406e-04f, -1.682827e-03f,
                               -7.373329e-03f, -1.426474e-02f};

static inline float gelu_one(float x) {
  float z = x * 0.70710678118654752440f;
  z = z < -4.0f ? -4.0f : (z > 4.0f ? 4.0f : z);
  float z2 = z * z;
  float p = ERF_A[0];
  for (int i = 1; i < 7; i++) p = p * z2 + ERF_A[i];
  float q = ERF_B[0];
  for (int i = 1; i < 5; i++) q = q * z2 + ERF_B[i];
  return 0.5f * x * (1.0f + z * p / q);
}

void or_gelu(float *x, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] = gelu_one(x[i]);
}

/* math.rs:77-93 -- sum in eight interleaved lanes. */
static float lane_sum(const float *v, size_t n) {
  float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t whole = n / 8 * 8;
  for (size_t i = 0; i < whole; i += 8)
    for (int l = 0; l < 8; l++) lanes[l] += v[i + l];
  float total = ((lanes[0] + lanes[4]) + (lanes[1] + lanes[5])) +
                ((lanes[2] + lanes[6]) + (lanes[3] + lanes[7]));
  for (size_t i = whole; i < n; i++) total += v[i];
  return total;
}

/* math.rs:95-116 -- two-pass LayerNorm of one row, epsilon 1e-5. */
static void layer_norm_row(float *x, size_t c, const float *gamma,
                           const float *beta) {
  float n = (float)c;
  float mean = lane_sum(x, c) / n;
  float squares[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t whole = c / 8 * 8;
  for (size_t i = 0; i < whole; i += 8)
    for (int l = 0; l < 8; l++) {
      float d = x[i + l] - mean;
      squares[l] += d * d;
    }
  float var = lane_sum(squares, 8);
  for (size_t i = whole; i < c; i++) {
    float d = x[i] - mean;
    var += d * d;
  }
  float inv = 1.0f / sqrtf(var / n + 1e-5f);
  for (size_t i = 0; i < c; i++) x[i] = (x[i] - mean) * inv * gamma[i] + beta[i];
}

void or_layer_norm(float *x, size_t len, const float *gamma, const float *beta,
                   size_t c) {
  for (size_t r = 0; r + c <= len; r += c) layer_norm_row(x + r, c, gamma, beta);
}

/* math.rs:118-134 */
void or_softmax(float *x, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; i++) max = x[i] > max ? x[i] : max;
  for (size_t i = 0; i < n; i++) x[i] = or_exp_neg(x[i] - max);
  float inv = 1.0f / lane_sum(x, n);
  for (size_t i = 0; i < n; i++) x[i] *= inv;
}
