// runtime.hip -- contexts, memory, errors and weight packing of libien_hip.so.
//
// The role of crates/native-vulkan (device choice, buffers, one-off weight
// upload, ordered submissions) on HIP: one stream per context, device
// buffers from hipMalloc, weights packed once into MFMA fragment order.

#include <cstdlib>
#include <cstring>
#include <mutex>

#include "ien_internal.h"

namespace ien {

ien_status fork_branches(ien_ctx *ctx, int n) {
  IEN_CHECK(n >= 1 && n <= ien_ctx::BRANCHES, IEN_ERR_INPUT, "%d branches", n);
  IEN_HIP(hipEventRecord(ctx->fork_ev, ctx->stream));
  for (int i = 0; i < n; i++) IEN_HIP(hipStreamWaitEvent(ctx->branch[i], ctx->fork_ev, 0));
  return IEN_OK;
}

ien_status join_branches(ien_ctx *ctx, int n) {
  IEN_CHECK(n >= 1 && n <= ien_ctx::BRANCHES, IEN_ERR_INPUT, "%d branches", n);
  for (int i = 0; i < n; i++) {
    IEN_HIP(hipEventRecord(ctx->join_ev[i], ctx->branch[i]));
    IEN_HIP(hipStreamWaitEvent(ctx->stream, ctx->join_ev[i], 0));
  }
  return IEN_OK;
}

static thread_local std::string g_error;

void set_error(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
}

ien_status fail(ien_status status, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  // crates/native-engine/src/lib.rs:73-83: "weights: ...", "input: ...".
  const char *kind = status == IEN_ERR_IO ? "io" :
                     status == IEN_ERR_WEIGHTS ? "weights" :
                     status == IEN_ERR_INPUT ? "input" :
                     status == IEN_ERR_CANCELLED ? "cancelled" : "GPU";
  g_error = std::string(kind) + ": " + buf;
  return status;
}

// half.rs:7-40, on the host: round to nearest, ties to even.
uint16_t f32_to_half(float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t mant = x & 0x7fffffu;
  if (((x >> 23) & 0xffu) == 0xffu) return sign | 0x7c00u | (mant ? 0x200u : 0);
  int e = (int)((x >> 23) & 0xffu) - 112;
  auto round = [](uint32_t kept, uint32_t low, uint32_t shift) {
    uint32_t half = 1u << (shift - 1);
    return kept + ((low > half || (low == half && (kept & 1u))) ? 1u : 0u);
  };
  if (e >= 31) return sign | 0x7c00u;
  if (e <= 0) {
    if (e < -10) return sign;
    uint32_t sig = mant | 0x800000u, shift = (uint32_t)(14 - e);
    return sign | (uint16_t)round(sig >> shift, sig & ((1u << shift) - 1u), shift);
  }
  return sign | (uint16_t)round(((uint32_t)e << 10) | (mant >> 13), mant & 0x1fffu, 13);
}

std::vector<uint16_t> pack_fragments(const float *w, size_t k, size_t n, int *kb_out,
                                     int *nb_out) {
  // n padded to whole 128-column tiles, so that any tile width reads zeros.
  int kb = (int)((k + 15) / 16), nb = (int)((n + 127) / 128) * 4;
  std::vector<uint16_t> out((size_t)kb * nb * 512, 0);
  for (int b = 0; b < nb; b++)
    for (int a = 0; a < kb; a++) {
      uint16_t *frag = out.data() + ((size_t)b * kb + a) * 512;
      for (int l = 0; l < 64; l++)
        for (int i = 0; i < 8; i++) {
          size_t kk = (size_t)a * 16 + 8 * (l / 32) + i, nn = (size_t)b * 32 + l % 32;
          if (kk < k && nn < n) frag[l * 8 + i] = f32_to_half(w[kk * n + nn]);
        }
    }
  *kb_out = kb;
  *nb_out = nb;
  return out;
}

Steps::~Steps() {
  for (hipEvent_t &e : ev)
    if (e) (void)hipEventDestroy(e);
}

ien_status Steps::report_through(int done) {
  while (reported < done) {
    reported++;
    if (progress((float)reported / (float)total, user) != 0)
      return fail(IEN_ERR_CANCELLED, "the progress callback stopped the run");
  }
  return IEN_OK;
}

ien_status Steps::step(hipStream_t stream) {
  hipEvent_t &mine = ev[issued % 2];
  if (!mine) IEN_HIP(hipEventCreateWithFlags(&mine, hipEventDisableTiming));
  IEN_HIP(hipEventRecord(mine, stream));
  issued++;
  if (issued < 2) return IEN_OK;
  // The previous step: its event is the other one of the pair.
  IEN_HIP(hipEventSynchronize(ev[issued % 2]));
  return report_through(issued - 1);
}

ien_status Steps::drain() {
  if (issued == 0) return IEN_OK;
  IEN_HIP(hipEventSynchronize(ev[(issued - 1) % 2]));
  return report_through(issued);
}

}  // namespace ien

using namespace ien;

extern "C" {

const char *ien_last_error(void) { return g_error.c_str(); }

ien_status ien_open(int device, ien_ctx **out) {
  IEN_CHECK(out, IEN_ERR_INPUT, "no output pointer");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
    return fail(IEN_ERR_GPU, "no HIP device");
  IEN_CHECK(device >= 0 && device < count, IEN_ERR_GPU, "device %d of %d", device, count);
  hipDeviceProp_t prop;
  IEN_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(IEN_ERR_GPU, "device %d is %s, this library is built for gfx950", device,
                prop.gcnArchName);
  IEN_HIP(hipSetDevice(device));
  ien_ctx *ctx = new ien_ctx;
  ctx->device = device;
  ctx->cus = prop.multiProcessorCount;
  ctx->name = prop.name[0] ? prop.name : prop.gcnArchName;
  hipError_t e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(IEN_ERR_GPU, "stream: %s", hipGetErrorString(e));
  }
  ctx->stream = ctx->own;
  e = hipMalloc(&ctx->zeros, 4096);
  if (e == hipSuccess) e = hipMemset(ctx->zeros, 0, 4096);
  // 32 MiB of split-K partial sums, then 256 KiB of tile counters.
  ctx->splitk_floats = (size_t)8 << 20;
  auto workspace = [&](float **p) {
    hipError_t r = hipMalloc((void **)p, (ctx->splitk_floats + ien_ctx::SPLITK_TILES) * 4);
    if (r == hipSuccess) r = hipMemset(*p + ctx->splitk_floats, 0, ien_ctx::SPLITK_TILES * 4);
    return r;
  };
  if (e == hipSuccess) e = workspace(&ctx->splitk);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming);
  if (e == hipSuccess) e = swin_static_setup(device);
  ctx->chain_tiles = ctx->cus;
  if (e == hipSuccess) e = hipMalloc((void **)&ctx->chain_flags, (ctx->chain_tiles + 3) * 4);
  if (e == hipSuccess) e = hipMemset(ctx->chain_flags, 0, (ctx->chain_tiles + 3) * 4);
  if (const char *v = std::getenv("IEN_CHAIN_SPIN_TICKS")) ctx->chain_spin = std::atol(v);
  if (const char *v = std::getenv("IEN_SERIAL_BRANCHES")) ctx->serial_branches = std::atoi(v) != 0;
  for (int i = 0; i < ien_ctx::BRANCHES && e == hipSuccess; i++) {
    e = hipStreamCreateWithFlags(&ctx->branch[i], hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->join_ev[i], hipEventDisableTiming);
    if (e == hipSuccess) e = workspace(&ctx->branch_splitk[i]);
  }
  if (e != hipSuccess) {
    const std::string why = hipGetErrorString(e);
    ien_close(ctx);
    return fail(IEN_ERR_GPU, "context buffers: %s", why.c_str());
  }
  *out = ctx;
  return IEN_OK;
}

void ien_close(ien_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (int i = 0; i < ien_ctx::BRANCHES; i++) {
    if (ctx->branch[i]) {
      (void)hipStreamSynchronize(ctx->branch[i]);
      (void)hipStreamDestroy(ctx->branch[i]);
    }
    if (ctx->join_ev[i]) (void)hipEventDestroy(ctx->join_ev[i]);
    (void)hipFree(ctx->branch_splitk[i]);
  }
  if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
  if (ctx->own) (void)hipStreamDestroy(ctx->own);
  (void)hipFree(ctx->zeros);
  (void)hipFree(ctx->splitk);
  (void)hipFree(ctx->chain_flags);
  delete ctx;
}

const char *ien_device_name(const ien_ctx *ctx) { return ctx ? ctx->name.c_str() : ""; }

void *ien_stream(ien_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

ien_status ien_set_stream(ien_ctx *ctx, void *stream) {
  IEN_CHECK(ctx, IEN_ERR_INPUT, "no context");
  ctx->stream = stream ? (hipStream_t)stream : ctx->own;
  return IEN_OK;
}

ien_status ien_alloc(ien_ctx *ctx, size_t bytes, void **d_out) {
  IEN_CHECK(ctx && d_out, IEN_ERR_INPUT, "no context or output pointer");
  IEN_HIP(hipSetDevice(ctx->device));
  IEN_HIP(hipMalloc(d_out, bytes ? bytes : 1));
  return IEN_OK;
}

ien_status ien_free(ien_ctx *ctx, void *d_ptr) {
  IEN_CHECK(ctx, IEN_ERR_INPUT, "no context");
  if (!d_ptr) return IEN_OK;
  IEN_HIP(hipSetDevice(ctx->device));
  IEN_HIP(hipFree(d_ptr));
  return IEN_OK;
}

ien_status ien_upload(ien_ctx *ctx, void *d_dst, const void *src, size_t bytes) {
  IEN_CHECK(ctx && (bytes == 0 || (d_dst && src)), IEN_ERR_INPUT, "null buffer");
  IEN_HIP(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  IEN_HIP(hipStreamSynchronize(ctx->stream));
  return IEN_OK;
}

ien_status ien_download(ien_ctx *ctx, void *dst, const void *d_src, size_t bytes) {
  IEN_CHECK(ctx && (bytes == 0 || (dst && d_src)), IEN_ERR_INPUT, "null buffer");
  IEN_HIP(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  IEN_HIP(hipStreamSynchronize(ctx->stream));
  return IEN_OK;
}

ien_status ien_sync(ien_ctx *ctx) {
  IEN_CHECK(ctx, IEN_ERR_INPUT, "no context");
  IEN_HIP(hipStreamSynchronize(ctx->stream));
  return IEN_OK;
}

ien_status ien_matrix_new(ien_ctx *ctx, const void *w, ien_wtype wtype, size_t k, size_t n,
                          const float *bias, ien_matrix **out) {
  IEN_CHECK(ctx && w && out, IEN_ERR_INPUT, "null argument");
  IEN_CHECK(k > 0 && n > 0 && k < (1u << 24) && n < (1u << 20), IEN_ERR_INPUT,
            "matrix of %zu x %zu", k, n);
  std::vector<float> wf;
  const float *src = (const float *)w;
  if (wtype == IEN_W_F16) {
    // half.rs:125-140, widened exactly; packing rounds back to the same half.
    wf.resize(k * n);
    const uint16_t *h = (const uint16_t *)w;
    for (size_t i = 0; i < k * n; i++) {
      _Float16 v;
      std::memcpy(&v, &h[i], 2);
      wf[i] = (float)v;
    }
    src = wf.data();
  } else {
    IEN_CHECK(wtype == IEN_W_F32, IEN_ERR_INPUT, "weight type %d", (int)wtype);
  }
  ien_matrix *m = new ien_matrix;
  m->ctx = ctx;
  m->k = k;
  m->n = n;
  std::vector<uint16_t> packed = pack_fragments(src, k, n, &m->kb, &m->nb);
  std::vector<float> b((size_t)m->nb * 32, 0.0f);
  if (bias) std::memcpy(b.data(), bias, n * sizeof(float));
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc(&m->d_packed, packed.size() * 2);
  if (e == hipSuccess) e = hipMalloc(&m->d_bias, b.size() * 4);
  if (e == hipSuccess)
    e = hipMemcpyAsync(m->d_packed, packed.data(), packed.size() * 2, hipMemcpyHostToDevice,
                       ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(m->d_bias, b.data(), b.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    ien_matrix_free(m);
    return fail(IEN_ERR_GPU, "matrix upload: %s", hipGetErrorString(e));
  }
  *out = m;
  return IEN_OK;
}

void ien_matrix_free(ien_matrix *m) {
  if (!m) return;
  if (m->ctx) (void)hipSetDevice(m->ctx->device);
  if (m->d_packed) (void)hipFree(m->d_packed);
  if (m->d_bias) (void)hipFree(m->d_bias);
  delete m;
}

}  // extern "C"
