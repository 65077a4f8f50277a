// Status plumbing, the block-type table, device buffers and the per-thread context of the host-pointer entry points;
// the library's small exports (version, device count, last error, the HBM copy of the counter calibration).
#include "common.h"

#include <cstdlib>
#include <vector>

namespace artlite {

namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

namespace {
constexpr QType TYPES[] = {{ARTLITE_F32, "F32", 1, 4, 4},           {ARTLITE_F16, "F16", 1, 2, 2},
                           {ARTLITE_BF16, "BF16", 1, 2, 2},         {ARTLITE_Q4_0, "Q4_0", 32, 18, 18},
                           {ARTLITE_Q4_1, "Q4_1", 32, 20, 20},      {ARTLITE_Q8_0, "Q8_0", 32, 34, 34},
                           {ARTLITE_Q3_K, "Q3_K", 256, 110, 112},   {ARTLITE_Q4_K, "Q4_K", 256, 144, 144},
                           {ARTLITE_Q5_K, "Q5_K", 256, 176, 176},   {ARTLITE_Q6_K, "Q6_K", 256, 210, 224},
                           {ARTLITE_IQ4_NL, "IQ4_NL", 32, 18, 18},  {ARTLITE_IQ4_XS, "IQ4_XS", 256, 136, 144}};
}

const QType* qtype_by_name(const char* name) {
  if (!name) return nullptr;
  for (const QType& t : TYPES)
    if (std::strcmp(t.name, name) == 0) return &t;
  return nullptr;
}

const QType* qtype_by_id(int id) {
  for (const QType& t : TYPES)
    if (t.id == id) return &t;
  return nullptr;
}

int DevBuf::reserve(size_t bytes) {
  if (bytes <= n && p) return ARTLITE_OK;
  release();
  const size_t want = bytes ? (bytes + 255) / 256 * 256 + 256 : 256;  // (a tail the vector loads may touch)
  void* q = nullptr;
  hipError_t e = hipMalloc(&q, want);
  if (e != hipSuccess) return fail(ARTLITE_ENOMEM, "hipMalloc(%zu): %s", want, hipGetErrorString(e));
  p = q;
  n = want - 256;
  return ARTLITE_OK;
}

void DevBuf::release() {
  if (p) (void)hipFree(p);
  p = nullptr;
  n = 0;
}

namespace {
struct CtxHolder {
  std::vector<HostCtx*> per_device;
  ~CtxHolder() {
    for (HostCtx* c : per_device)
      if (c) {
        if (c->stream) (void)hipStreamDestroy(c->stream);
        delete c;
      }
  }
};
thread_local CtxHolder g_ctx;
}  // namespace

int host_ctx(HostCtx** out) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(ARTLITE_EHIP, "no HIP device (hipGetDeviceCount: %s)", hipGetErrorString(e));
  int dev = 0;
  ART_HIP(hipGetDevice(&dev));
  if (g_ctx.per_device.size() < size_t(n)) g_ctx.per_device.resize(n, nullptr);
  HostCtx*& c = g_ctx.per_device[dev];
  if (!c) {
    c = new HostCtx();
    c->device = dev;
    ART_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  }
  *out = c;
  return ARTLITE_OK;
}

// a plain copy of dwordx4 per lane (the counter calibration's known traffic)
__global__ void k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    dst[i] = src[i];
}

}  // namespace artlite

using namespace artlite;

extern "C" size_t artlite_last_error(char* buf, size_t cap) {
  if (buf && cap) {
    const size_t n = g_error.size() < cap - 1 ? g_error.size() : cap - 1;
    std::memcpy(buf, g_error.data(), n);
    buf[n] = 0;
  }
  return g_error.size();
}

extern "C" const char* artlite_version(void) { return "artlite_moe 0.1 gfx950"; }

extern "C" int artlite_device_count(int* n) {
  if (!n) return fail(ARTLITE_EINVAL, "artlite_device_count: null");
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
  *n = c;
  return ARTLITE_OK;
}

extern "C" int artlite_hbm_copy(size_t nbytes, int iters, double* ms_per_copy) {
  if (!ms_per_copy || iters < 1 || nbytes < 16) return fail(ARTLITE_EINVAL, "artlite_hbm_copy: arguments");
  HostCtx* c;
  ART_TRY(host_ctx(&c));
  const size_t n = nbytes / 16;
  DevBuf a, b;
  ART_TRY(a.reserve(n * 16));
  ART_TRY(b.reserve(n * 16));
  ART_HIP(hipMemsetAsync(a.p, 1, n * 16, c->stream));
  hipEvent_t e0, e1;
  ART_HIP(hipEventCreate(&e0));
  ART_HIP(hipEventCreate(&e1));
  const int grid = 256 * 8;
  k_copy<<<grid, 256, 0, c->stream>>>(a.as<uint4>(), b.as<uint4>(), n);
  ART_HIP(hipGetLastError());
  ART_HIP(hipEventRecord(e0, c->stream));
  for (int i = 0; i < iters; i++) k_copy<<<grid, 256, 0, c->stream>>>(a.as<uint4>(), b.as<uint4>(), n);
  ART_HIP(hipEventRecord(e1, c->stream));
  ART_HIP(hipEventSynchronize(e1));
  float ms = 0;
  ART_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms_per_copy = double(ms) / iters;
  return ARTLITE_OK;
}
