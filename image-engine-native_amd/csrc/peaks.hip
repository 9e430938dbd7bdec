// peaks.hip -- a measurement of this device, for reports: the sustained
// f16 MFMA rate (the roofline's achievable ceiling beside the published
// peak).  No counterpart in the reference.
//
// Every SIMD runs back-to-back v_mfma_f32_32x32x16_f16 on register
// operands: one workgroup of 8 waves (two per SIMD) per CU, each wave four
// independent accumulator chains, no memory traffic in the loop.

#include "ien_internal.h"

namespace ien {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(512) void k_mfma_loop(int iters, float *sink) {
  const int lane = threadIdx.x & 63;
  half8 a, b;
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (lane + i));
    b[i] = (_Float16)(0.002f * (lane - i));
  }
  floatx16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; it++) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
  }
  float s = 0.0f;
  for (int i = 0; i < 16; i++) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (s == 12345.678f) sink[threadIdx.x] = s;  // keeps the products live
}

}  // namespace
}  // namespace ien

using namespace ien;

extern "C" ien_status ien_measure_mfma(ien_ctx *ctx, int iters, double *tflops, double *ms) {
  IEN_CHECK(ctx && tflops && ms, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(iters > 0 && iters <= (1 << 24), IEN_ERR_INPUT, "%d iterations", iters);
  IEN_HIP(hipSetDevice(ctx->device));
  float *sink = nullptr;
  IEN_HIP(hipMalloc(&sink, 512 * 4));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  const unsigned blocks = (unsigned)ctx->cus;
  // A warm-up launch, then the timed one.
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_mfma_loop, dim3(blocks), dim3(512), 0, ctx->stream, iters / 8 + 1, sink);
    e = hipEventRecord(e0, ctx->stream);
  }
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_mfma_loop, dim3(blocks), dim3(512), 0, ctx->stream, iters, sink);
    e = hipEventRecord(e1, ctx->stream);
  }
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float elapsed = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&elapsed, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(sink);
  if (e != hipSuccess) return fail(IEN_ERR_GPU, "mfma loop: %s", hipGetErrorString(e));
  const double flops = (double)blocks * 8 * iters * 4 * 2.0 * 32 * 32 * 16;
  *ms = elapsed;
  *tflops = flops / (elapsed * 1e-3) / 1e12;
  return IEN_OK;
}
