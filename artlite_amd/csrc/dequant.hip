// GGUF rows dequantized on the GPU to the reference's fp32 values bit for bit (reference
// csrc/artlite/dequant.cpp:21-82, gguf_model.QTensor.dequantize): one thread per block, the reference's fp32
// operations in its order, no fused multiply-add (this file is compiled with -ffp-contract=off, and the Q4_K
// products and difference are explicit round-to-nearest operations as well); the C entry points
// artlite_dequant_supported / artlite_dequant_rows.
#include "common.h"

namespace artlite {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return uint32_t(p[0]) | (uint32_t(p[1]) << 8); }

// Q4_0 (18 B per 32): w = (q - 8) d, values 0..15 the low nibbles of bytes 2.., 16..31 the high nibbles
__device__ __forceinline__ void block_q4_0(const uint8_t* b, float* o) {
  const float d = f16_to_f32(ld_u16(b));
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t c = b[2 + j];
    o[j] = __fmul_rn(float(c & 15u) - 8.0f, d);
    o[j + 16] = __fmul_rn(float(c >> 4) - 8.0f, d);
  }
}

// Q8_0 (34 B per 32): w = d q, q int8
__device__ __forceinline__ void block_q8_0(const uint8_t* b, float* o) {
  const float d = f16_to_f32(ld_u16(b));
#pragma unroll
  for (int j = 0; j < 32; j++) o[j] = __fmul_rn(d, float(int8_t(b[2 + j])));
}

// Q4_K (144 B per 256): w = q (d sc_g) - dmin mn_g, 8 groups of 32 (6-bit sc / mn in the 12 bytes at 4; group g's
// value l at byte 16 + 32 (g / 2) + l, the low nibble for even g)
__device__ __forceinline__ void block_q4_k(const uint8_t* b, float* o) {
  const float d = f16_to_f32(ld_u16(b)), dmin = f16_to_f32(ld_u16(b + 2));
  const uint8_t *lo = b + 4, *hi = b + 8, *top = b + 12, *qs = b + 16;
  for (int g = 0; g < 8; g++) {
    const int sc = g < 4 ? lo[g] & 63 : (top[g - 4] & 15) | ((lo[g - 4] >> 6) << 4);
    const int mn = g < 4 ? hi[g] & 63 : (top[g - 4] >> 4) | ((hi[g - 4] >> 6) << 4);
    const float dsc = __fmul_rn(d, float(sc)), dmn = __fmul_rn(dmin, float(mn));
    for (int l = 0; l < 32; l++) {
      const uint32_t c = qs[32 * (g >> 1) + l];
      const float t = __fmul_rn(float((g & 1) ? c >> 4 : c & 15u), dsc);
      o[32 * g + l] = __fsub_rn(t, dmn);
    }
  }
}

template <int QT>
__global__ void k_dequant(const uint8_t* __restrict__ raw, size_t n, size_t row_bytes, size_t blocks_per_row,
                          float* __restrict__ out, size_t cols) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n * blocks_per_row) return;
  const size_t r = i / blocks_per_row, k = i % blocks_per_row;
  const uint8_t* row = raw + r * row_bytes;
  float* o = out + r * cols;
  if (QT == ARTLITE_Q4_0) {
    float v[32];
    block_q4_0(row + k * 18, v);
    for (int j = 0; j < 32; j++) o[k * 32 + j] = v[j];
  } else if (QT == ARTLITE_Q8_0) {
    float v[32];
    block_q8_0(row + k * 34, v);
    for (int j = 0; j < 32; j++) o[k * 32 + j] = v[j];
  } else if (QT == ARTLITE_Q4_K) {
    block_q4_k(row + k * 144, o + k * 256);
  } else if (QT == ARTLITE_F32) {
    const uint8_t* p = row + 4 * k;
    o[k] = __uint_as_float(uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24);
  } else if (QT == ARTLITE_F16) {
    o[k] = f16_to_f32(ld_u16(row + 2 * k));
  } else {  // BF16: the high half of the fp32 value
    o[k] = bf16_to_f32(ld_u16(row + 2 * k));
  }
}

int launch_dequant(const QType* t, const uint8_t* raw, size_t n, size_t row_bytes, size_t cols, float* out,
                   hipStream_t s) {
  const size_t bpr = cols / t->per, total = n * bpr;
  if (!total) return ARTLITE_OK;
  const dim3 grid(unsigned((total + 255) / 256)), block(256);
  switch (t->id) {
    case ARTLITE_Q4_0: k_dequant<ARTLITE_Q4_0><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
    case ARTLITE_Q8_0: k_dequant<ARTLITE_Q8_0><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
    case ARTLITE_Q4_K: k_dequant<ARTLITE_Q4_K><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
    case ARTLITE_F32: k_dequant<ARTLITE_F32><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
    case ARTLITE_F16: k_dequant<ARTLITE_F16><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
    default: k_dequant<ARTLITE_BF16><<<grid, block, 0, s>>>(raw, n, row_bytes, bpr, out, cols); break;
  }
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace artlite

using namespace artlite;

extern "C" int artlite_dequant_supported(const char* qtype) { return qtype_by_name(qtype) != nullptr; }

extern "C" int artlite_dequant_rows(const char* qtype, const uint8_t* raw, size_t n, size_t row_bytes, size_t cols,
                                    float* out) {
  const QType* t = qtype_by_name(qtype);
  if (!t) return fail(ARTLITE_EINVAL, "dequant_rows: no native %s", qtype ? qtype : "(null)");
  if (cols % t->per || cols / t->per * t->bytes > row_bytes)
    return fail(ARTLITE_EINVAL, "dequant_rows: %zu columns of rows of %zu B", cols, row_bytes);
  if (!n || !cols) return ARTLITE_OK;
  if (!raw || !out) return fail(ARTLITE_EINVAL, "dequant_rows: null array");
  HostCtx* c;
  ART_TRY(host_ctx(&c));
  ART_TRY(c->in.reserve(n * row_bytes));
  ART_TRY(c->out.reserve(n * cols * 4));
  ART_HIP(hipMemcpyAsync(c->in.p, raw, n * row_bytes, hipMemcpyHostToDevice, c->stream));
  ART_TRY(launch_dequant(t, c->in.as<uint8_t>(), n, row_bytes, cols, c->out.as<float>(), c->stream));
  ART_HIP(hipMemcpyAsync(out, c->out.p, n * cols * 4, hipMemcpyDeviceToHost, c->stream));
  ART_HIP(hipStreamSynchronize(c->stream));
  return ARTLITE_OK;
}
