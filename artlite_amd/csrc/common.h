// Shared internals of libartlite_moe: status/error plumbing, the GGUF block table, device buffers, and the small
// device helpers the kernels share (fp16 / bf16 conversions, wave reductions).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/artlite_moe.h"

namespace artlite {

// ---- errors: a thread-local message and a status code
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define ART_HIP(expr)                                                                          \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess) return ::artlite::fail(ARTLITE_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define ART_TRY(expr)          \
  do {                         \
    int s_ = (expr);           \
    if (s_ != ARTLITE_OK) return s_; \
  } while (0)

// ---- GGUF block types (reference src/artlite/gguf_model.py:385-390)
struct QType {
  int id;
  const char* name;
  int per;    // values per block
  int bytes;  // bytes per block (in a GGUF file)
  int dev;    // bytes per block in an uploaded layer: the same, but Q6_K's 210 padded to 224 and IQ4_XS's 136 to
              // 144, its 8-byte header to 16 (16-byte aligned blocks and code runs for the decode GEMV's DMAs)
};
const QType* qtype_by_name(const char* name);
const QType* qtype_by_id(int id);

// ---- device memory that grows on demand
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  int reserve(size_t bytes);  // keeps the contents only when no reallocation happens
  void release();
  template <class T>
  T* as() const { return static_cast<T*>(p); }
  ~DevBuf() { release(); }
};

// A per-thread context of the host-pointer entry points: the current device's stream and scratch buffers.
struct HostCtx {
  int device = -1;
  hipStream_t stream = nullptr;
  DevBuf in, out, out2, out3, out4, out5, tmp, tmp2, flag;
};
int host_ctx(HostCtx** ctx);

// ---- device helpers
// fp16 bits -> fp32, exact for subnormals (the reference's f16(), csrc/artlite/dequant.cpp:21-29)
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  const uint32_t s = (h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  if (e == 31) return __uint_as_float(s | 0x7F800000u | (m << 13));
  if (e) return __uint_as_float(s | ((e + 112) << 23) | (m << 13));
  const float v = float(m) * 0x1p-24f;
  return s ? -v : v;
}

// fp32 -> bf16 bits, rounded to nearest even (NaN kept a quiet NaN)
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// four codes (bytes < 16) -> the bytes of IQ4[code] as int8 (IQ4_NL / IQ4_XS's 16 values, ggml's kvalues_iq4nl):
// two byte permutes over the 16-byte table, one per half, the code's bit 3 choosing between them
__device__ __forceinline__ uint32_t iq4_int8(uint32_t c) {
  constexpr int V[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
  constexpr auto pack = [](const int* v) {
    return uint32_t(v[0] & 0xFF) | uint32_t(v[1] & 0xFF) << 8 | uint32_t(v[2] & 0xFF) << 16 |
           uint32_t(v[3] & 0xFF) << 24;
  };
  constexpr uint32_t T0 = pack(V), T1 = pack(V + 4), T2 = pack(V + 8), T3 = pack(V + 12);
  const uint32_t s = c & 0x07070707u, hi = ((c >> 3) & 0x01010101u) * 0xFFu;
  return (__builtin_amdgcn_perm(T3, T2, s) & hi) | (__builtin_amdgcn_perm(T1, T0, s) & ~hi);
}

constexpr int WAVE = 64;
constexpr int LDS_BYTES = 160 * 1024;  // a gfx950 workgroup's LDS

// bytes past the end of an uploaded weight tensor that the expert kernels' loads may touch (zeros): a K-range's
// 16-byte-aligned cover of a row's last partial run
constexpr int WEIGHT_TAIL = 1024;

}  // namespace artlite
