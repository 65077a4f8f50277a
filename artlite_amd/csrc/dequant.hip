// GGUF rows dequantized on the GPU to the reference's fp32 values bit for bit (reference
// csrc/artlite/dequant.cpp:21-160, gguf_model.QTensor.dequantize): the reference's native types (F32, F16, BF16,
// Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS). One thread per output value: the value's fields are
// read from its block (the neighbouring threads read the same block, so the reads stay in L1 / L2) and combined by
// the reference's fp32 operations in its order, each rounded on its own (explicit round-to-nearest operations, and
// this file is compiled with -ffp-contract=off); the writes are coalesced rows of fp32. The C entry points
// artlite_dequant_supported / artlite_dequant_rows.
#include "common.h"
#include "experts.h"

namespace artlite {

namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return uint32_t(p[0]) | (uint32_t(p[1]) << 8); }

// a 32-value group's code j in Q4_0's order: the low nibbles of its 16 bytes are values 0..15, the high nibbles 16..31
__device__ __forceinline__ uint32_t nibble32(const uint8_t* q, int j) {
  return j < 16 ? q[j] & 15u : uint32_t(q[j - 16]) >> 4;
}

// IQ4_NL / IQ4_XS's 16 values (ggml's kvalues_iq4nl; reference dequant.cpp:121)
__constant__ int8_t IQ4_VALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// Q4_K / Q5_K's 6-bit scale and min of group g (of 8) from the 12 bytes at s: groups 0..3 in the low 6 bits of
// bytes 0..3 (scales) and 4..7 (mins); groups 4..7 a nibble of bytes 8..11 plus the top two bits of bytes 0..7
__device__ __forceinline__ void k_scale_min(const uint8_t* s, int g, int& sc, int& mn) {
  if (g < 4) {
    sc = s[g] & 63;
    mn = s[4 + g] & 63;
  } else {
    sc = (s[8 + g - 4] & 15) | ((s[g - 4] >> 6) << 4);
    mn = (s[8 + g - 4] >> 4) | ((s[4 + g - 4] >> 6) << 4);
  }
}

// value j of the block at b, as the reference computes it (dequant.cpp line ranges per format); XS: where IQ4_XS's
// codes start (8 in the file, 16 in the layer's padded block)
template <int QT, int XS = 8>
__device__ __forceinline__ float value(const uint8_t* b, int j) {
  if constexpr (QT == ARTLITE_Q4_0) {  // (q - 8) d (:41-48)
    return __fmul_rn(float(nibble32(b + 2, j)) - 8.0f, f16_to_f32(ld_u16(b)));
  } else if constexpr (QT == ARTLITE_Q4_1) {  // d q + m (:50-57)
    return __fadd_rn(__fmul_rn(f16_to_f32(ld_u16(b)), float(nibble32(b + 4, j))), f16_to_f32(ld_u16(b + 2)));
  } else if constexpr (QT == ARTLITE_Q8_0) {  // d q, q int8 (:59-63)
    return __fmul_rn(f16_to_f32(ld_u16(b)), float(int8_t(b[2 + j])));
  } else if constexpr (QT == ARTLITE_Q4_K || QT == ARTLITE_Q5_K) {  // q (d sc_g) - dmin mn_g (:65-84)
    const int g = j >> 5, l = j & 31;
    int sc, mn;
    k_scale_min(b + 4, g, sc, mn);
    const float dsc = __fmul_rn(f16_to_f32(ld_u16(b)), float(sc));
    const float dmn = __fmul_rn(f16_to_f32(ld_u16(b + 2)), float(mn));
    const uint8_t* qs = b + (QT == ARTLITE_Q5_K ? 48 : 16);
    const uint32_t c = qs[32 * (g >> 1) + l];
    uint32_t q = (g & 1) ? c >> 4 : c & 15u;
    if constexpr (QT == ARTLITE_Q5_K) q |= ((uint32_t(b[16 + l]) >> g) & 1u) << 4;  // (qh at 16)
    return __fsub_rn(__fmul_rn(float(q), dsc), dmn);
  } else if constexpr (QT == ARTLITE_Q6_K) {  // (q - 32) (sc_j d), value 128 h + 32 jj + l (:86-106)
    const int h = j >> 7, jj = (j >> 5) & 3, l = j & 31;
    const uint32_t c = b[64 * h + 32 * (jj & 1) + l], e = b[128 + 32 * h + l];
    const int q = int(((c >> (jj < 2 ? 0 : 4)) & 15u) | (((e >> (2 * jj)) & 3u) << 4)) - 32;
    const float s = __fmul_rn(float(int8_t(b[192 + (j >> 4)])), f16_to_f32(ld_u16(b + 208)));
    return __fmul_rn(float(q), s);
  } else if constexpr (QT == ARTLITE_Q3_K) {  // (d sc_j) (q - 4), value 128 n + 32 jj + 16 h + l (:108-123)
    const int n = j >> 7, jj = (j >> 5) & 3, hl = j & 31, sb = j >> 4;
    const uint8_t* s = b + 96;
    const int lo = sb < 8 ? s[sb] & 15 : s[sb - 8] >> 4, hi = (s[8 + (sb & 3)] >> (2 * (sb >> 2))) & 3;
    const int q = ((b[32 + 32 * n + hl] >> (2 * jj)) & 3) | (((b[hl] >> (4 * n + jj)) & 1) << 2);
    const float a = __fmul_rn(f16_to_f32(ld_u16(b + 108)), float((lo | (hi << 4)) - 32));
    return __fmul_rn(a, float(q) - 4.0f);
  } else if constexpr (QT == ARTLITE_IQ4_NL) {  // d IQ4[q] (:126-130)
    return __fmul_rn(f16_to_f32(ld_u16(b)), float(IQ4_VALUES[nibble32(b + 2, j)]));
  } else if constexpr (QT == ARTLITE_IQ4_XS) {  // (d (ls_g - 32)) IQ4[q] (:132-143)
    const int g = j >> 5;
    const int ls = ((b[4 + g / 2] >> (4 * (g & 1))) & 15) | (((int(ld_u16(b + 2)) >> (2 * g)) & 3) << 4);
    const float dl = __fmul_rn(f16_to_f32(ld_u16(b)), float(ls - 32));
    return __fmul_rn(dl, float(IQ4_VALUES[nibble32(b + XS + 16 * g, j & 31)]));
  } else if constexpr (QT == ARTLITE_F32) {
    return __uint_as_float(uint32_t(b[0]) | uint32_t(b[1]) << 8 | uint32_t(b[2]) << 16 | uint32_t(b[3]) << 24);
  } else if constexpr (QT == ARTLITE_F16) {
    return f16_to_f32(ld_u16(b));
  } else {  // BF16: the high half of the fp32 value
    return bf16_to_f32(ld_u16(b));
  }
}

constexpr int CHUNK = 1024;  // values of a row per workgroup pass

// workgroup pass i takes values [c0, c0 + CHUNK) of row r (i = r chunks_per_row + c0 / CHUNK), a value per thread
template <int QT, int PER, int BYTES>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ raw, size_t n, size_t row_bytes,
                                                 size_t cols, float* __restrict__ out) {
  const size_t cpr = (cols + CHUNK - 1) / CHUNK;
  for (size_t i = blockIdx.x; i < n * cpr; i += gridDim.x) {
    const size_t r = i / cpr, c0 = (i % cpr) * CHUNK;
    const uint8_t* row = raw + r * row_bytes;
    float* o = out + r * cols;
    for (size_t c = c0 + threadIdx.x; c < c0 + CHUNK && c < cols; c += 256)
      o[c] = value<QT>(row + (c / PER) * BYTES, int(c % PER));
  }
}

// the largest L1 norm of the rows (sum |w| of the values as dequantized, in fp32, rounded up by 2^-10 relative: the
// fp32 sum of at most 2^13 terms is within 2^-11 of the exact one), a wave per row, by an atomic max on the float's
// bits (non-negative floats order as their bits). BYTES: the block's stride (the layer's padded Q6_K / Q3_K blocks
// keep the file's bytes first)
template <int QT, int PER, int BYTES>
__global__ __launch_bounds__(256) void k_row_l1(const uint8_t* __restrict__ raw, int64_t rows, size_t row_bytes,
                                                int cols, uint32_t* __restrict__ out) {
  const int64_t r = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
  if (r < rows) {
    const uint8_t* row = raw + r * row_bytes;
    for (int c = lane; c < cols; c += 64) s += fabsf(value<QT, 16>(row + (c / PER) * BYTES, c % PER));
  }
  for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0 && r < rows) atomicMax(out, __float_as_uint(s * (1.0f + 0x1p-10f)));
}

template <int QT, int PER, int BYTES>
int launch_l1(const uint8_t* raw, int64_t rows, size_t row_bytes, int cols, float* out, hipStream_t s) {
  ART_HIP(hipMemsetAsync(out, 0, 4, s));
  if (rows <= 0) return ARTLITE_OK;
  k_row_l1<QT, PER, BYTES><<<unsigned((rows + 3) / 4), 256, 0, s>>>(raw, rows, row_bytes, cols,
                                                                    reinterpret_cast<uint32_t*>(out));
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

template <int QT, int PER, int BYTES>
int launch_t(const uint8_t* raw, size_t n, size_t row_bytes, size_t cols, float* out, hipStream_t s) {
  const size_t passes = n * ((cols + CHUNK - 1) / CHUNK);
  const unsigned grid = unsigned(passes < 65536 ? passes : 65536);
  k_dequant<QT, PER, BYTES><<<grid, 256, 0, s>>>(raw, n, row_bytes, cols, out);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- the prefill layout (experts.h, PREFILL_PQ6): per 64 values of a row, their codes (6 bits: a nibble plane and a
// crumb plane) and the fp32 scales of their sub-blocks, made from a block of the layer's uploaded tensor. The code,
// scale and min of value w of a block, as the file's fields hold them (dequant.cpp lines as in value<>).
template <int QT>
struct Pq6;
template <>
struct Pq6<ARTLITE_Q6_K> {  // (layer block: 224 bytes, the file's 210 first) q = 6 bits, (q - 32) (d sc_16)
  static constexpr int PER = 256, DEV = 224, MODE = 0;
  static __device__ uint32_t code(const uint8_t* b, int w) {
    const int h = w >> 7, jj = (w >> 5) & 3, l = w & 31;
    const uint32_t c = b[64 * h + 32 * (jj & 1) + l], e = b[128 + 32 * h + l];
    return ((c >> (jj < 2 ? 0 : 4)) & 15u) | (((e >> (2 * jj)) & 3u) << 4);
  }
  static __device__ float2 scale(const uint8_t* b, int w) {
    return make_float2(__fmul_rn(float(int8_t(b[192 + (w >> 4)])), f16_to_f32(ld_u16(b + 208))), 0.0f);
  }
};
template <>
struct Pq6<ARTLITE_Q3_K> {  // (layer block: 112 bytes, the file's 110 first) q = 3 bits, (d (sc_16 - 32)) (q - 4)
  static constexpr int PER = 256, DEV = 112, MODE = 0;
  static __device__ uint32_t code(const uint8_t* b, int w) {
    const int n = w >> 7, jj = (w >> 5) & 3, hl = w & 31;
    return uint32_t(((b[32 + 32 * n + hl] >> (2 * jj)) & 3) | (((b[hl] >> (4 * n + jj)) & 1) << 2));
  }
  static __device__ float2 scale(const uint8_t* b, int w) {
    const int sb = w >> 4;
    const uint8_t* s = b + 96;
    const int lo = sb < 8 ? s[sb] & 15 : s[sb - 8] >> 4, hi = (s[8 + (sb & 3)] >> (2 * (sb >> 2))) & 3;
    return make_float2(__fmul_rn(f16_to_f32(ld_u16(b + 108)), float((lo | (hi << 4)) - 32)), 0.0f);
  }
};
template <>
struct Pq6<ARTLITE_Q5_K> {  // q = 5 bits, q (d sc_32) - dmin m_32
  static constexpr int PER = 256, DEV = 176, MODE = 1;
  static __device__ uint32_t code(const uint8_t* b, int w) {
    const int g = w >> 5, l = w & 31;
    const uint32_t c = b[48 + 32 * (g >> 1) + l];
    return ((g & 1) ? c >> 4 : c & 15u) | (((uint32_t(b[16 + l]) >> g) & 1u) << 4);
  }
  static __device__ float2 scale(const uint8_t* b, int w) {
    int sc, mn;
    k_scale_min(b + 4, w >> 5, sc, mn);
    return make_float2(__fmul_rn(f16_to_f32(ld_u16(b)), float(sc)), __fmul_rn(f16_to_f32(ld_u16(b + 2)), float(mn)));
  }
};
template <>
struct Pq6<ARTLITE_Q4_1> {  // q = 4 bits, d q + m
  static constexpr int PER = 32, DEV = 20, MODE = 1;
  static __device__ uint32_t code(const uint8_t* b, int w) { return nibble32(b + 4, w); }
  static __device__ float2 scale(const uint8_t* b, int) {
    return make_float2(f16_to_f32(ld_u16(b)), -f16_to_f32(ld_u16(b + 2)));
  }
};
template <>
struct Pq6<ARTLITE_IQ4_NL> {  // the index of IQ4's value, d IQ4[q]
  static constexpr int PER = 32, DEV = 18, MODE = 2;
  static __device__ uint32_t code(const uint8_t* b, int w) { return nibble32(b + 2, w); }
  static __device__ float2 scale(const uint8_t* b, int) { return make_float2(f16_to_f32(ld_u16(b)), 0.0f); }
};
template <>
struct Pq6<ARTLITE_IQ4_XS> {  // (layer block: 144 bytes, the 8-byte header padded to 16) (d (ls_32 - 32)) IQ4[q]
  static constexpr int PER = 256, DEV = 144, MODE = 2;
  static __device__ uint32_t code(const uint8_t* b, int w) { return nibble32(b + 16 + 16 * (w >> 5), w & 31); }
  static __device__ float2 scale(const uint8_t* b, int w) {
    const int g = w >> 5;
    const int ls = ((b[4 + g / 2] >> (4 * (g & 1))) & 15) | (((int(ld_u16(b + 2)) >> (2 * g)) & 3) << 4);
    return make_float2(__fmul_rn(f16_to_f32(ld_u16(b)), float(ls - 32)), 0.0f);
  }
};

// a thread per (row, 64-value stage): its 64 bytes of the prefill layout
template <int QT>
__global__ __launch_bounds__(256) void k_pq6_pack(const uint8_t* __restrict__ src, int64_t rows, int K,
                                                  size_t row_bytes, uint8_t* __restrict__ dst) {
  using F = Pq6<QT>;
  const int stages = K / 64;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * stages) return;
  const int64_t r = i / stages;
  const int st = int(i % stages);
  const uint8_t* row = src + r * row_bytes;
  auto at = [&](int v) { const int a = 64 * st + v; return row + (a / F::PER) * F::DEV; };
  auto in = [&](int v) { return (64 * st + v) % F::PER; };
  float hdr[4];
  if (F::MODE == 1) {  // (scale and min of each 32 values)
    for (int g = 0; g < 2; g++) {
      const float2 so = F::scale(at(32 * g), in(32 * g));
      hdr[2 * g] = so.x;
      hdr[2 * g + 1] = so.y;
    }
  } else {  // (the scale of each 16 values)
    for (int h = 0; h < 4; h++) hdr[h] = F::scale(at(16 * h), in(16 * h)).x;
  }
  uint32_t nib[8], cr[4];
  for (int d = 0; d < 8; d++) {  // (nibble dword 4 g + l: byte k = value 32 g + 8 l + k | value + 4 in the high nibble)
    nib[d] = 0;
    for (int k = 0; k < 4; k++) {
      const int v = 8 * d + k;
      nib[d] |= ((F::code(at(v), in(v)) & 15u) | ((F::code(at(v + 4), in(v + 4)) & 15u) << 4)) << (8 * k);
    }
  }
  for (int d = 0; d < 4; d++) {  // (crumb dword 2 g + m: lane groups 2 m + 1 (bits 0-3), 2 m (bits 4-7) of group g)
    cr[d] = 0;
    const int g = d >> 1, m = d & 1;
    for (int k = 0; k < 4; k++) {
      uint32_t byte = 0;
      for (int par = 0; par < 2; par++) {
        const int v = 32 * g + 8 * (2 * m + 1 - par) + k;
        byte |= ((F::code(at(v), in(v)) >> 4) | ((F::code(at(v + 4), in(v + 4)) >> 4) << 2)) << (4 * par);
      }
      cr[d] |= byte << (8 * k);
    }
  }
  uint4* o = reinterpret_cast<uint4*>(dst + r * int64_t(K) + 64 * st);
  o[0] = make_uint4(__float_as_uint(hdr[0]), __float_as_uint(hdr[1]), __float_as_uint(hdr[2]), __float_as_uint(hdr[3]));
  o[1] = make_uint4(nib[0], nib[1], nib[2], nib[3]);
  o[2] = make_uint4(nib[4], nib[5], nib[6], nib[7]);
  o[3] = make_uint4(cr[0], cr[1], cr[2], cr[3]);
}

template <int QT>
int launch_pack(const uint8_t* src, int64_t rows, int K, size_t row_bytes, uint8_t* dst, hipStream_t s) {
  if (K % Pq6<QT>::PER) return fail(ARTLITE_EINVAL, "prefill layout: K %d is not a multiple of the block", K);
  const int64_t n = rows * (K / 64);
  if (n <= 0) return ARTLITE_OK;
  k_pq6_pack<QT><<<unsigned((n + 255) / 256), 256, 0, s>>>(src, rows, K, row_bytes, dst);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace

bool pq6_mode(int qtype, int& mode, float& off) {
  switch (qtype) {
    case ARTLITE_Q6_K: mode = 0, off = 32.0f; return true;
    case ARTLITE_Q3_K: mode = 0, off = 4.0f; return true;
    case ARTLITE_Q5_K:
    case ARTLITE_Q4_1: mode = 1, off = 0.0f; return true;
    case ARTLITE_IQ4_NL:
    case ARTLITE_IQ4_XS: mode = 2, off = 128.0f; return true;
    default: return false;
  }
}

int launch_pq6_pack(const uint8_t* src, int qtype, int64_t rows, int K, size_t row_bytes, uint8_t* dst,
                    hipStream_t s) {
  if (K <= 0 || K % 64) return fail(ARTLITE_EINVAL, "prefill layout: K %d is not a multiple of 64", K);
  switch (qtype) {
    case ARTLITE_Q6_K: return launch_pack<ARTLITE_Q6_K>(src, rows, K, row_bytes, dst, s);
    case ARTLITE_Q3_K: return launch_pack<ARTLITE_Q3_K>(src, rows, K, row_bytes, dst, s);
    case ARTLITE_Q5_K: return launch_pack<ARTLITE_Q5_K>(src, rows, K, row_bytes, dst, s);
    case ARTLITE_Q4_1: return launch_pack<ARTLITE_Q4_1>(src, rows, K, row_bytes, dst, s);
    case ARTLITE_IQ4_NL: return launch_pack<ARTLITE_IQ4_NL>(src, rows, K, row_bytes, dst, s);
    case ARTLITE_IQ4_XS: return launch_pack<ARTLITE_IQ4_XS>(src, rows, K, row_bytes, dst, s);
    default: return fail(ARTLITE_EINVAL, "prefill layout: type %d", qtype);
  }
}

int launch_dequant(const QType* t, const uint8_t* raw, size_t n, size_t row_bytes, size_t cols, float* out,
                   hipStream_t s) {
  if (!n || !cols) return ARTLITE_OK;
  switch (t->id) {
    case ARTLITE_F32: return launch_t<ARTLITE_F32, 1, 4>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_F16: return launch_t<ARTLITE_F16, 1, 2>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_BF16: return launch_t<ARTLITE_BF16, 1, 2>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q4_0: return launch_t<ARTLITE_Q4_0, 32, 18>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q4_1: return launch_t<ARTLITE_Q4_1, 32, 20>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q8_0: return launch_t<ARTLITE_Q8_0, 32, 34>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q3_K: return launch_t<ARTLITE_Q3_K, 256, 110>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q4_K: return launch_t<ARTLITE_Q4_K, 256, 144>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q5_K: return launch_t<ARTLITE_Q5_K, 256, 176>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_Q6_K: return launch_t<ARTLITE_Q6_K, 256, 210>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_IQ4_NL: return launch_t<ARTLITE_IQ4_NL, 32, 18>(raw, n, row_bytes, cols, out, s);
    case ARTLITE_IQ4_XS: return launch_t<ARTLITE_IQ4_XS, 256, 136>(raw, n, row_bytes, cols, out, s);
    default: return fail(ARTLITE_EINVAL, "dequant: type %d", t->id);
  }
}

int launch_weight_l1(const uint8_t* w, int qtype, int64_t rows, size_t row_bytes, int cols, float* out, hipStream_t s) {
  if (cols <= 0 || cols > 8192) return fail(ARTLITE_EINVAL, "weight L1: %d columns", cols);
  switch (qtype) {  // (block strides as the layer stores them: Q6_K padded to 224 bytes, Q3_K to 112, IQ4_XS to 144)
    case ARTLITE_Q4_0: return launch_l1<ARTLITE_Q4_0, 32, 18>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q4_1: return launch_l1<ARTLITE_Q4_1, 32, 20>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q8_0: return launch_l1<ARTLITE_Q8_0, 32, 34>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q3_K: return launch_l1<ARTLITE_Q3_K, 256, 112>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q4_K: return launch_l1<ARTLITE_Q4_K, 256, 144>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q5_K: return launch_l1<ARTLITE_Q5_K, 256, 176>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_Q6_K: return launch_l1<ARTLITE_Q6_K, 256, 224>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_IQ4_NL: return launch_l1<ARTLITE_IQ4_NL, 32, 18>(w, rows, row_bytes, cols, out, s);
    case ARTLITE_IQ4_XS: return launch_l1<ARTLITE_IQ4_XS, 256, 144>(w, rows, row_bytes, cols, out, s);
    default: return fail(ARTLITE_EINVAL, "weight L1: type %d", qtype);
  }
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
