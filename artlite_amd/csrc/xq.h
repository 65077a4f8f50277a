// XQ, the decode path's activations (layout in gemv.h): the device side of writing them, shared by the
// quantisation of x (gemv.hip, route.hip) and of h (the gate / up GEMV's epilogue).
#pragma once

#include "gemv.h"

namespace artlite {

// Reductions over the 8 lanes of each aligned group of 8 (every lane gets the result) by DPP: lanes i ^ 1, i ^ 2
// (quad_perm), then the mirror lane 7 - i of the other quad (row_half_mirror).
template <int C>
__device__ __forceinline__ int dpp8(int v) {
  return __builtin_amdgcn_update_dpp(0, v, C, 0xF, 0xF, false);
}
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, __int_as_float(dpp8<0xB1>(__float_as_int(v))));  // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, __int_as_float(dpp8<0x4E>(__float_as_int(v))));  // quad_perm [2, 3, 0, 1]
  return fmaxf(v, __int_as_float(dpp8<0x141>(__float_as_int(v))));  // row_half_mirror
}
__device__ __forceinline__ int sum8(int v) {
  v += dpp8<0xB1>(v);
  v += dpp8<0x4E>(v);
  return v + dpp8<0x141>(v);
}
__device__ __forceinline__ int or8(int v) {
  v |= dpp8<0xB1>(v);
  v |= dpp8<0x4E>(v);
  return v | dpp8<0x141>(v);
}

// Quantise a 32-value group held by 8 consecutive lanes (aligned), 4 values each: this lane's int8 plane values, and
// the group's s / 256, sum of (256 a + b) and dequantised sum (s / 256 times that sum).
__device__ __forceinline__ void quant_group(const float (&x)[4], int (&qa)[4], int (&qb)[4], float& s256, int& sum,
                                            float& xsum) {
  constexpr int V = 4;
  float amax = 0.0f;
  int bad = 0;
#pragma unroll
  for (int i = 0; i < V; i++) {
    amax = fmaxf(amax, fabsf(x[i]));
    bad |= !__builtin_isfinite(x[i]);
  }
  amax = max8(amax);
  bad = or8(bad);
  const float inv = 127.0f / amax;
  const bool skip = bad || !(amax > 0.0f) || !__builtin_isfinite(inv);  // (zero or sub-1e-36 groups: 0)
  sum = 0;
#pragma unroll
  for (int i = 0; i < V; i++) {
    const float y = x[i] * inv;
    const float ra = rintf(y);
    const float rb = fminf(fmaxf(rintf((y - ra) * 256.0f), -127.0f), 127.0f);
    qa[i] = skip ? 0 : int(ra);
    qb[i] = skip ? 0 : int(rb);
    sum += 256 * qa[i] + qb[i];
  }
  sum = sum8(sum);
  s256 = bad ? __builtin_nanf("") : skip ? 0.0f : amax / 32512.0f;  // (127 x 256)
  xsum = s256 * float(sum);
}

// dword of an XQ unit holding block dword i (< 16) of group g
__host__ __device__ inline int xq_block(int g, int i) { return 4 * (16 * (g >> 1) + i) + (g & 1); }

// word k (< 16) of the 16 copies of group g's three words in an XQ unit: k < 4: s / 256, k < 8: the sum, else the
// dequantised sum
__device__ __forceinline__ void xq_put_word(uint32_t* ub, int g, int k, float s256, int sum, float xsum) {
  const int c = 16 * (g >> 1), h = g & 1;
  if (k < 4)
    ub[4 * (c + 2 * h + 4 * k) + 2] = __float_as_uint(s256);
  else if (k < 8)
    ub[4 * (c + 2 * h + 1 + 4 * (k - 4)) + 2] = uint32_t(sum);
  else
    ub[4 * (c + h + 2 * (k - 8)) + 3] = __float_as_uint(xsum);
}

// One unit (256 values) of row `row` of x (T rows of K fp32 / bf16 values; XT its dtype) into XQ, by one wave: lane
// l quantises values 4 l .. 4 l + 3 (group l / 8, plane dword l % 8). w: the wave's (row, unit) index.
template <int XT>
__device__ __forceinline__ void xq_quant_unit(const void* __restrict__ x, int64_t w, int K, uint32_t* __restrict__ xq,
                                              int lane) {
  const int U = K / 256;
  const int64_t row = w / U;
  const int u = int(w - row * U);
  const int64_t i0 = row * K + int64_t(u) * 256 + 4 * lane;
  float v[4];
  if (XT == ARTLITE_X_F32) {
    const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + i0);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  } else {
    const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + i0);
    v[0] = bf16_to_f32(b.x & 0xFFFFu), v[1] = bf16_to_f32(b.x >> 16);
    v[2] = bf16_to_f32(b.y & 0xFFFFu), v[3] = bf16_to_f32(b.y >> 16);
  }
  int qa[4], qb[4], sum;
  float s256, xsum;
  quant_group(v, qa, qb, s256, sum, xsum);
  uint32_t pa = 0, pb = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    pa |= uint32_t(qa[i] & 0xFF) << (8 * i);
    pb |= uint32_t(qb[i] & 0xFF) << (8 * i);
  }
  uint32_t* ub = xq + row * (int64_t(U) * XQ_UNIT) + int64_t(u) * XQ_UNIT;
  const int g = lane >> 3, j = lane & 7;
  ub[xq_block(g, j)] = pa;
  ub[xq_block(g, 8 + j)] = pb;
  xq_put_word(ub, g, j, s256, sum, xsum);
  xq_put_word(ub, g, 8 + j, s256, sum, xsum);
}

}  // namespace artlite
