// Decode expert products on the VALU, and the XQ activations they read.
//
// Persistent workgroups (as many as the device holds) take work items in turn: an item is one tile of at most
// GEMV_BM sorted rows of A (tokens for gate / up, pairs for down) of one expert times a block of 16 RB weight rows
// (SwiGLU: those rows of gate and of up). Plain products: 4 waves, one per 16-row block (RB 4, 64 rows). SwiGLU:
// 8 waves, 4 row blocks (64 rows) x 2 waves that take alternate K-units (so the two read neighbouring units, which
// share cache lines, at about the same time), whose partial sums meet in LDS. Each wave
// streams its own steps (16 rows x one K-unit of 8 groups of 32 values: Q4_0 / Q4_K 144 bytes a row, Q5_K 176,
// Q8_0 272)
// with global_load_lds_dwordx4 into two LDS slots of its own, one step ahead, across item boundaries; the XQ records
// of A's rows for a K-unit come the same way. Every load is a DMA counted as it is issued, so each wait names the
// exact count (the compiler, which cannot order DMAs against register loads, would otherwise wait for all of them).
// Lane (p, r) -- 16-lane row p, lane r in it -- takes row r and groups 2 p, 2 p + 1 of each unit, so four lanes
// share a row. The activations are read once per K-unit into registers, one 16-byte XQ chunk per lane per row of A:
// DPP row_newbcast:j hands every lane of 16-lane row p dword j of its groups' blocks as the broadcast operand of
// v_dot4c_i32_i8, and the per-group words the same way. The four lanes of a row are summed at the end. The SwiGLU
// epilogue has no barrier: the last of the item's waves to deliver its partial sums (an LDS counter per buffer) adds
// them in a fixed order, forms h = silu(gate) up and writes it as XQ for the down product.
//
// Arithmetic of one (row of A, group): A = sum_j dot4(a_j, q_j) and B = C + sum_j dot4(b_j, q_j), exactly in int32,
// with q_j the group's codes as int8 (Q4_0 / Q4_K: nibbles 0..15, Q5_K: 0..31, Q8_0: the signed bytes) and C the code offset's
// correction (Q4_0: -8 sum(256 a + b), else 0); then acc += (d s / 256) float(256 A + B), which is
// d s sum (q - 8)(a + b / 256) for Q4_0. Q4_K and Q5_K add -(dmin mn) times the group's dequantised activation sum.
#include "gemv.h"
#include "xq.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <utility>

namespace artlite {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }

// per format: bytes of a row's unit, dwords a lane reads of it (Q4_0 / Q8_0: its two groups; Q4_K / Q5_K: the
// super-block header, Q5_K's 32 high-bit bytes, and the 32-byte run holding its two groups)
template <int QT>
struct Unit;
template <>
struct Unit<ARTLITE_Q4_0> {
  static constexpr int BYTES = 144, LW = 9;
};
template <>
struct Unit<ARTLITE_Q8_0> {
  static constexpr int BYTES = 272, LW = 17;
};
template <>
struct Unit<ARTLITE_IQ4_NL> {  // (Q4_0's layout)
  static constexpr int BYTES = 144, LW = 9;
};
template <>
struct Unit<ARTLITE_Q4_1> {  // (the lane's two 20-byte blocks)
  static constexpr int BYTES = 160, LW = 10;
};
template <>
struct Unit<ARTLITE_IQ4_XS> {  // (a layer's 144-byte block: the header padded to 16 bytes, and the lane's 32-byte run)
  static constexpr int BYTES = 144, LW = 12;
};
template <>
struct Unit<ARTLITE_Q4_K> {
  static constexpr int BYTES = 144, LW = 12;
};
template <>
struct Unit<ARTLITE_Q5_K> {  // (the header, the 32 high-bit bytes, the lane's 32-byte run)
  static constexpr int BYTES = 176, LW = 20;
};
template <>
struct Unit<ARTLITE_Q3_K> {  // (a layer's 112-byte padded block: the 32 high-bit bytes, the lane's 32 low-bit bytes, and
                             // the 12 bytes of scales with d)
  static constexpr int BYTES = 112, LW = 20;
};
template <>
struct Unit<ARTLITE_Q6_K> {  // (a layer's 224-byte padded block: the lane's 64 low-bit bytes, 32 high-bit bytes, and the
                             // 16 scales with d)
  static constexpr int BYTES = 224, LW = 32;
};

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>)
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// LDS reads by asm, completed before they return: reads the compiler sees in a kernel with LDS DMA in flight make
// it wait for every load in flight first
__device__ __forceinline__ int lds_read_i32(const void* p) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
__device__ __forceinline__ int4 lds_read_i4(const void* p) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return make_int4(int(v[0]), int(v[1]), int(v[2]), int(v[3]));
}
// *p += 1 after every earlier LDS access of the wave has completed; returns the old value (one lane's call)
__device__ __forceinline__ int lds_inc(int* p) {
  int old;
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(old)
               : "v"(lds_addr(p)), "v"(1)
               : "memory");
  return old;
}
// *p = v after every earlier LDS access of the wave has completed
__device__ __forceinline__ void lds_store(int* p, int v) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : : "v"(lds_addr(p)), "v"(v)
               : "memory");
}
__device__ __forceinline__ float4 lds_read_f4(const void* p) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}

// The lane's dwords of a unit (at pw; Q4_K / Q5_K: header, Q5_K high bits, at pw, its run at pr) and (MX > 0) its
// record chunk of each of MX rows of A (at px, 1024 bytes apart), and their completion, in one asm block, after the
// step's wait (wait_vm, an asm block of its own just before it): the compiler would otherwise wait for every load in
// flight before reading LDS (it takes the slots' global_load_lds writes for possible producers), and it must not
// touch the outputs before the final wait.
#define ART_R2(I, J) "ds_read2_b32 %[w" #I "], %[pw] offset0:" #J " offset1:" #J "+1\n\t"
#define ART_R1(I, J) "ds_read_b32 %[w" #I "], %[pw] offset:" #J "*4\n\t"
#define ART_OW2(I) [w##I] "=&v"(w2[I])
#define ART_OW1(I) [w##I] "=&v"(w1)
#define ART_W9 ART_R2(0, 0) ART_R2(1, 2) ART_R2(2, 4) ART_R2(3, 6) ART_R1(4, 8)
#define ART_OW9 ART_OW2(0), ART_OW2(1), ART_OW2(2), ART_OW2(3), ART_OW1(4)
#define ART_W10 ART_R2(0, 0) ART_R2(1, 2) ART_R2(2, 4) ART_R2(3, 6) ART_R2(4, 8)
#define ART_OW10 ART_OW2(0), ART_OW2(1), ART_OW2(2), ART_OW2(3), ART_OW2(4)
#define ART_W17 \
  ART_R2(0, 0) ART_R2(1, 2) ART_R2(2, 4) ART_R2(3, 6) ART_R2(4, 8) ART_R2(5, 10) ART_R2(6, 12) ART_R2(7, 14) ART_R1(8, 16)
#define ART_OW17 \
  ART_OW2(0), ART_OW2(1), ART_OW2(2), ART_OW2(3), ART_OW2(4), ART_OW2(5), ART_OW2(6), ART_OW2(7), ART_OW1(8)
#define ART_W12                    \
  "ds_read_b128 %[w0], %[pw]\n\t"  \
  "ds_read_b128 %[w1], %[pr]\n\t"  \
  "ds_read_b128 %[w2], %[pr] offset:16\n\t"
#define ART_OW12 [w0] "=&v"(w4[0]), [w1] "=&v"(w4[1]), [w2] "=&v"(w4[2])
#define ART_W20                                \
  "ds_read_b128 %[w0], %[pw]\n\t"             \
  "ds_read_b128 %[w1], %[pw] offset:16\n\t"   \
  "ds_read_b128 %[w2], %[pw] offset:32\n\t"   \
  "ds_read_b128 %[w3], %[pr]\n\t"             \
  "ds_read_b128 %[w4], %[pr] offset:16\n\t"
#define ART_OW20 [w0] "=&v"(w4[0]), [w1] "=&v"(w4[1]), [w2] "=&v"(w4[2]), [w3] "=&v"(w4[3]), [w4] "=&v"(w4[4])
#define ART_W20S                               \
  "ds_read_b128 %[w0], %[pw]\n\t"             \
  "ds_read_b128 %[w1], %[pw] offset:16\n\t"   \
  "ds_read_b128 %[w2], %[pr]\n\t"             \
  "ds_read_b128 %[w3], %[pr] offset:16\n\t"   \
  "ds_read_b128 %[w4], %[ps]\n\t"
#define ART_OW20S ART_OW20
#define ART_W32                                \
  "ds_read_b128 %[w0], %[pw]\n\t"             \
  "ds_read_b128 %[w1], %[pw] offset:16\n\t"   \
  "ds_read_b128 %[w2], %[pw] offset:32\n\t"   \
  "ds_read_b128 %[w3], %[pw] offset:48\n\t"   \
  "ds_read_b128 %[w4], %[pr]\n\t"             \
  "ds_read_b128 %[w5], %[pr] offset:16\n\t"   \
  "ds_read_b128 %[w6], %[ps]\n\t"             \
  "ds_read_b128 %[w7], %[ps] offset:16\n\t"
#define ART_OW32                                                                                          \
  [w0] "=&v"(w4[0]), [w1] "=&v"(w4[1]), [w2] "=&v"(w4[2]), [w3] "=&v"(w4[3]), [w4] "=&v"(w4[4]), [w5] "=&v"(w4[5]), \
      [w6] "=&v"(w4[6]), [w7] "=&v"(w4[7])
#define ART_RX(T) "ds_read_b128 %[x" #T "], %[px] offset:" #T "*1024\n\t"
#define ART_X0
#define ART_X1 ART_RX(0)
#define ART_X2 ART_X1 ART_RX(1)
#define ART_X3 ART_X2 ART_RX(2)
#define ART_X4 ART_X3 ART_RX(3)
#define ART_OX0
#define ART_OX1 , [x0] "=&v"(x[0])
#define ART_OX2 ART_OX1, [x1] "=&v"(x[1])
#define ART_OX3 ART_OX2, [x2] "=&v"(x[2])
#define ART_OX4 ART_OX3, [x3] "=&v"(x[3])
#define ART_READ(WN, MN)                                                 \
  asm volatile(ART_W##WN ART_X##MN "s_waitcnt lgkmcnt(0)"                \
               : ART_OW##WN ART_OX##MN                                    \
               : [pw] "v"(pw), [pr] "v"(pr), [ps] "v"(ps), [px] "v"(px) \
               : "memory")
#define ART_READ_M(WN)                   \
  if constexpr (MX == 0) ART_READ(WN, 0); \
  if constexpr (MX == 1) ART_READ(WN, 1); \
  if constexpr (MX == 2) ART_READ(WN, 2); \
  if constexpr (MX == 3) ART_READ(WN, 3); \
  if constexpr (MX == 4) ART_READ(WN, 4);
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" : : "i"(N) : "memory");
}
template <int QT, int MX>
__device__ __forceinline__ void read_unit(uint32_t (&w)[Unit<QT>::LW], u32x4 (&x)[GEMV_BM], uint32_t pw, uint32_t pr,
                                          uint32_t ps, uint32_t px) {
  constexpr int LW = Unit<QT>::LW;
  if constexpr (LW == 12) {
    u32x4 w4[3];
    ART_READ_M(12)
#pragma unroll
    for (int i = 0; i < 12; i++) w[i] = w4[i >> 2][i & 3];
  } else if constexpr (LW == 20 && QT == ARTLITE_Q3_K) {
    u32x4 w4[5];
    ART_READ_M(20S)
#pragma unroll
    for (int i = 0; i < 20; i++) w[i] = w4[i >> 2][i & 3];
  } else if constexpr (LW == 20) {
    u32x4 w4[5];
    ART_READ_M(20)
#pragma unroll
    for (int i = 0; i < 20; i++) w[i] = w4[i >> 2][i & 3];
  } else if constexpr (LW == 32) {
    u32x4 w4[8];
    ART_READ_M(32)
#pragma unroll
    for (int i = 0; i < 32; i++) w[i] = w4[i >> 2][i & 3];
  } else {
    u32x2 w2[LW / 2];
    uint32_t w1 = 0;
    if constexpr (LW == 9) {
      ART_READ_M(9)
    } else if constexpr (LW == 10) {
      ART_READ_M(10)
    } else {
      ART_READ_M(17)
    }
#pragma unroll
    for (int i = 0; i < LW / 2; i++) w[2 * i] = w2[i][0], w[2 * i + 1] = w2[i][1];
    if constexpr (LW % 2) w[LW - 1] = w1;
  }
}
#undef ART_READ_M
#undef ART_READ
#undef ART_OX4
#undef ART_OX3
#undef ART_OX2
#undef ART_OX1
#undef ART_OX0
#undef ART_X4
#undef ART_X3
#undef ART_X2
#undef ART_X1
#undef ART_X0
#undef ART_RX
#undef ART_OW12
#undef ART_W12
#undef ART_OW20
#undef ART_W20
#undef ART_OW32
#undef ART_W32
#undef ART_OW17
#undef ART_W17
#undef ART_OW9
#undef ART_W9
#undef ART_OW10
#undef ART_W10
#undef ART_OW1
#undef ART_OW2
#undef ART_R1
#undef ART_R2

// Codes of the lane's group H (0, 1) as 8 dwords of int8 (q[j]: values 4 j .. 4 j + 3 of the group), its scale d
// (Q4_K / Q5_K: d sc) and their dmin mn. g: the group's index in the unit (their scales, Q5_K's high bits).
template <int QT, int H>
__device__ __forceinline__ void codes(const uint32_t (&w)[Unit<QT>::LW], int g, uint32_t (&q)[8], float& d,
                                      float& mn) {
  if constexpr (QT == ARTLITE_Q4_0 || QT == ARTLITE_Q8_0 || QT == ARTLITE_IQ4_NL) {
    // Q4_0 / IQ4_NL: 18 bytes at 18 H: fp16 d, then 16 bytes whose low nibbles are values 0..15, high nibbles
    // 16..31 (IQ4_NL: the codes of IQ4[] values, looked up to int8); Q8_0: 34 bytes at 34 H: fp16 d, then 32 signed
    // bytes in value order
    constexpr int o = (QT == ARTLITE_Q8_0 ? 34 : 18) * H;
    constexpr int NQ = QT == ARTLITE_Q8_0 ? 8 : 4;
#pragma unroll
    for (int j = 0; j < NQ; j++) {
      uint32_t v;
      if constexpr (o % 4 == 0)
        v = __builtin_amdgcn_alignbit(w[o / 4 + j + 1], w[o / 4 + j], 16);
      else
        v = w[(o + 2) / 4 + j];
      if constexpr (QT == ARTLITE_Q4_0) {
        q[j] = v & 0x0F0F0F0Fu;
        q[4 + j] = (v >> 4) & 0x0F0F0F0Fu;
      } else if constexpr (QT == ARTLITE_IQ4_NL) {
        q[j] = iq4_int8(v & 0x0F0F0F0Fu);
        q[4 + j] = iq4_int8((v >> 4) & 0x0F0F0F0Fu);
      } else {
        q[j] = v;
      }
    }
    d = o % 4 == 0 ? h2f(w[o / 4] & 0xFFFFu) : h2f(w[(o - 2) / 4] >> 16);
    mn = 0.0f;
  } else if constexpr (QT == ARTLITE_Q4_1) {
    // the lane's two 20-byte blocks: block H at 20 H, fp16 d and m, then 16 bytes of nibbles as Q4_0's (w = d q + m:
    // mn = -m for the min term)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      q[j] = w[5 * H + 1 + j] & 0x0F0F0F0Fu;
      q[4 + j] = (w[5 * H + 1 + j] >> 4) & 0x0F0F0F0Fu;
    }
    d = h2f(w[5 * H] & 0xFFFFu);
    mn = -h2f(w[5 * H] >> 16);
  } else if constexpr (QT == ARTLITE_IQ4_XS) {
    // the header (fp16 d, the 16 bits of high scale crumbs, 4 bytes of low scale nibbles; w[0..1]) and the lane's
    // 32-byte run (w[4..11]: groups 2 p, 2 p + 1, 16 bytes each in Q4_0's order of IQ4[] codes); the scale
    // d (ls - 32), ls the 6-bit scale of group g
    const uint32_t sh = w[0] >> 16, sl = w[1];
    const int ls = int((sl >> (8 * (g >> 1) + 4 * (g & 1))) & 15u) | int(((sh >> (2 * g)) & 3u) << 4);
    d = h2f(w[0] & 0xFFFFu) * float(ls - 32);  // (exact: 11 x 6 significant bits)
    mn = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      q[j] = iq4_int8(w[4 + 4 * H + j] & 0x0F0F0F0Fu);
      q[4 + j] = iq4_int8((w[4 + 4 * H + j] >> 4) & 0x0F0F0F0Fu);
    }
  } else if constexpr (QT == ARTLITE_Q3_K) {
    // group g = 4 n + jj (n = p / 2, jj = 2 (p % 2) + H): value l's low bits are crumb jj of low-bit byte l of half n
    // (w[8..15]), its high bit bit 4 n + jj of high-bit byte l (w[0..7]); code - 4 as int8 (the crumb, with 0xFC
    // or'ed in where the high bit is clear); the scales of its two 16-value halves, the 6-bit sub-block scales
    // 2 g, 2 g + 1 (low nibbles in bytes 0..7 of the scales, w[16..17]: g >= 4 the high nibbles of g - 4's bytes;
    // crumbs in bytes 8..11, w[18]) less 32, times d (w[19], bytes 12..13): d in d, the second in mn
    const int n = g >> 2, jj = g & 3;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t lo = (w[8 + j] >> (2 * jj)) & 0x03030303u, hi = (w[j] >> (4 * n + jj)) & 0x01010101u;
      q[j] = lo | ((hi ^ 0x01010101u) * 0xFCu);
    }
    const uint32_t lw = (w[16 + ((g & 3) >> 1)] >> (16 * (g & 1))) >> (g < 4 ? 0 : 4);
    const uint32_t cr = w[18] >> (16 * (g & 1) + 2 * (g >> 1));
    const int sa = int((lw & 15u) | ((cr & 3u) << 4)), sb = int(((lw >> 8) & 15u) | (((cr >> 8) & 3u) << 4));
    const float dd = h2f(w[19] & 0xFFFFu);
    d = dd * float(sa - 32);  // (exact: 11 x 6 significant bits)
    mn = dd * float(sb - 32);
  } else if constexpr (QT == ARTLITE_Q6_K) {
    // group g = 4 h + jj (h = p / 2, jj = 2 (p % 2) + H): value l's low bits are a nibble of low-bit byte 32 (jj % 2)
    // + l of half h (w[0..15]: the high nibbles for jj >= 2), its high bits crumb jj of high-bit byte l (w[16..23]);
    // code - 32 as int8 (the 6-bit code with bit 5 flipped, sign-extended); the scales of its two 16-value halves,
    // int8 sub-block scales 2 g, 2 g + 1 (bytes 192.., w[24..27]) times d (bytes 208, w[28]): d in d, the second in mn
    const int p = g >> 1, jj = 2 * (p & 1) + H, sh = 4 * (p & 1);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t c = ((w[8 * H + j] >> sh) & 0x0F0F0F0Fu) | (((w[16 + j] >> (2 * jj)) & 0x03030303u) << 4);
      const uint32_t y = c ^ 0x20202020u, sgn = y & 0x20202020u;
      q[j] = y | (sgn << 1) | (sgn << 2);
    }
    const float dd = h2f(w[28] & 0xFFFFu);
    const uint32_t sw = w[24 + (g >> 1)] >> (16 * (g & 1));  // (bytes 2 g, 2 g + 1 of the scales)
    d = dd * float(int8_t(sw & 0xFFu));  // (exact: 11 x 8 significant bits)
    mn = dd * float(int8_t((sw >> 8) & 0xFFu));
  } else {
    // a super-block: fp16 d, dmin; 12 bytes of 6-bit scales / mins (w[1..3]); the lane's 32-byte run (w[4..11]),
    // its group 2 p in the low nibbles and 2 p + 1 in the high nibbles (value order)
    // (bytes g, g + 4 and g - 4 of the scales by a runtime byte select)
    const uint32_t sel = 0x0C0C0C00u | uint32_t(g);
    const uint32_t b0 = __builtin_amdgcn_perm(w[2], w[1], sel);
    const uint32_t b4 = __builtin_amdgcn_perm(w[3], w[2], sel);
    const uint32_t bm = __builtin_amdgcn_perm(w[2], w[1], 0x0C0C0C00u | uint32_t((g - 4) & 7));
    const uint32_t sc = g < 4 ? b0 & 63u : (b4 & 15u) | ((bm >> 6) << 4);
    const uint32_t m = g < 4 ? b4 & 63u : (b4 >> 4) | ((b0 >> 6) << 4);
    d = h2f(w[0] & 0xFFFFu) * float(sc);  // (exact: 11 x 6 significant bits)
    mn = h2f(w[0] >> 16) * float(m);
    if constexpr (QT == ARTLITE_Q4_K) {
#pragma unroll
      for (int j = 0; j < 8; j++) q[j] = H ? (w[4 + j] >> 4) & 0x0F0F0F0Fu : w[4 + j] & 0x0F0F0F0Fu;
    } else {  // Q5_K: the run at w[12..19]; bit g of high-bit byte l (w[4..11]) is bit 4 of value l's code
#pragma unroll
      for (int j = 0; j < 8; j++)
        q[j] = (H ? (w[12 + j] >> 4) & 0x0F0F0F0Fu : w[12 + j] & 0x0F0F0F0Fu) | (((w[4 + j] >> g) & 0x01010101u) << 4);
    }
  }
}

// The 16 dot4 of one (row of A, group) as four interleaved chains: A = a0 + a1 over plane a, B = b0 + b1 over
// plane b (a0 / b0: even dwords, a1 / b1: odd). Hazards the compiler cannot see inside the asm: a DPP instruction
// needs two wait states after a VALU write of any VGPR it reads, accumulators included (each chain's dot4 are four
// instructions apart, and start at least two after their initial values; the block opens with s_nop 1 for the inputs
// the compiler wrote just before), and a VALU other than the same dot reading a dot4 result needs three (the block
// ends with the independent scale products and an s_nop).
// x: the group's block (lane j of each 16-lane row: dword j); q0 .. q7 the codes.
#define ART_DOT(ACC, Q, L) \
  "v_dot4c_i32_i8_dpp %[" #ACC "], %[x], %[" #Q "] row_newbcast:" #L " row_mask:0xf bank_mask:0xf\n\t"
#define ART_DOTS                                                                                                \
  ART_DOT(a0, q0, 0) ART_DOT(b0, q0, 8) ART_DOT(a1, q1, 1) ART_DOT(b1, q1, 9) ART_DOT(a0, q2, 2)                \
  ART_DOT(b0, q2, 10) ART_DOT(a1, q3, 3) ART_DOT(b1, q3, 11) ART_DOT(a0, q4, 4) ART_DOT(b0, q4, 12)             \
  ART_DOT(a1, q5, 5) ART_DOT(b1, q5, 13) ART_DOT(a0, q6, 6) ART_DOT(b0, q6, 14) ART_DOT(a1, q7, 7)              \
  ART_DOT(b1, q7, 15)
// (Q6_K: the same sixteen dot4, the chains by half: a0 / b0 over dwords 0..3, a1 / b1 over 4..7, still four apart)
#define ART_DOTS_HALVES                                                                                         \
  ART_DOT(a0, q0, 0) ART_DOT(b0, q0, 8) ART_DOT(a1, q4, 4) ART_DOT(b1, q4, 12) ART_DOT(a0, q1, 1)                \
  ART_DOT(b0, q1, 9) ART_DOT(a1, q5, 5) ART_DOT(b1, q5, 13) ART_DOT(a0, q2, 2) ART_DOT(b0, q2, 10)              \
  ART_DOT(a1, q6, 6) ART_DOT(b1, q6, 14) ART_DOT(a0, q3, 3) ART_DOT(b0, q3, 11) ART_DOT(a1, q7, 7)              \
  ART_DOT(b1, q7, 15)
#define ART_QIN                                                                                   \
  [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]), [q5] "v"(q[5]), \
      [q6] "v"(q[6]), [q7] "v"(q[7])
#define ART_ACC [a0] "=&v"(a0), [a1] "=&v"(a1), [b0] "=&v"(b0), [b1] "=&v"(b1), [c] "=&v"(coef)

// acc += the term of the lane's group H for one row of A. x: the group's block dword; l: the list word (16-lane row
// lanes 2 H: s / 256, 2 H + 1: the sum of 256 a + b); xs: the sum word (lane H: the dequantised sum).
template <int QT, int H>
__device__ __forceinline__ float group_term(float acc, uint32_t x, uint32_t l, uint32_t xs, const uint32_t (&q)[8],
                                            float d, float mn) {
  int a0, a1, b0, b1;
  float coef;
  if constexpr (QT == ARTLITE_Q4_0) {
    asm("s_nop 1\n\t"
        "v_mul_i32_i24_dpp %[b0], %[l], %[m8] row_newbcast:%[l1] row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : ART_ACC
        : [x] "v"(x), [l] "v"(l), [d] "v"(d), [m8] "v"(-8), ART_QIN, [l0] "i"(2 * H), [l1] "i"(2 * H + 1));
  } else if constexpr (QT == ARTLITE_Q6_K || QT == ARTLITE_Q3_K) {
    // the halves' sums in their own chains (a0 / b0: dwords 0..3, a1 / b1: 4..7), each scaled by its sub-block's
    // scale (d: the first half's, mn: the second's); signed codes, no offset
    float c1;
    asm("s_nop 1\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[b0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS_HALVES
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[c1], %[l], %[d1] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0"
        : ART_ACC, [c1] "=&v"(c1)
        : [x] "v"(x), [l] "v"(l), [d] "v"(d), [d1] "v"(mn), ART_QIN, [l0] "i"(2 * H));
    return __builtin_fmaf(c1, float(a1 * 256 + b1), __builtin_fmaf(coef, float(a0 * 256 + b0), acc));
  } else if constexpr (QT == ARTLITE_Q8_0 || QT == ARTLITE_IQ4_NL || QT == ARTLITE_IQ4_XS) {  // (signed codes)
    asm("s_nop 1\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[b0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : ART_ACC
        : [x] "v"(x), [l] "v"(l), [d] "v"(d), ART_QIN, [l0] "i"(2 * H));
  } else {
    float mterm;
    asm("s_nop 1\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[b0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t], %[xs], %[nm] row_newbcast:%[h] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0"
        : ART_ACC, [t] "=&v"(mterm)
        : [x] "v"(x), [l] "v"(l), [xs] "v"(xs), [d] "v"(d), [nm] "v"(-mn), ART_QIN, [l0] "i"(2 * H), [h] "i"(H));
    return __builtin_fmaf(coef, float((a0 + a1) * 256 + (b0 + b1)), acc) + mterm;
  }
  return __builtin_fmaf(coef, float((a0 + a1) * 256 + (b0 + b1)), acc);
}
#undef ART_ACC
#undef ART_DOT
#undef ART_DOTS
#undef ART_DOTS_HALVES
#undef ART_QIN

template <bool SWIGLU>
struct Shape {
  static constexpr int RB = 4, S = SWIGLU ? 2 : 1, WAVES = RB * S, THREADS = 64 * WAVES;
  // (SwiGLU: whole 32-row XQ groups of h per item, 8 lanes each, at most 64 lanes for GEMV_BM rows of A)
  static_assert(!SWIGLU || (RB % 2 == 0 && 8 * RB / 2 * GEMV_BM <= 64), "SwiGLU epilogue lanes");
};

// LDS of a workgroup: each wave's D slots of 16 rows x BYTES and its record slot (GEMV_BM chunk rows of 1 KB;
// one: the next K-unit's are loaded once the current ones are read, and more slots measured no faster while they
// cost Q6_K's plain products a workgroup per CU), then (S > 1) RED_BUFS buffers of the K-ranges' partial sums and
// their counters (then the item table, sized at launch)
constexpr int RED_BUFS = 2;
// Weight slots per wave (the streams' D): two, one step in flight behind the one being read. Each wait names the
// loads issued after the one it needs (at most NMAX: LA = D - 1 steps' weights and LA + 1 K-units' records), and a
// slot is refilled right after the step that read it. Deeper queues measured no faster: with many items they cost
// workgroups per CU, and with one item per workgroup (4 slots, one token) gate / up took 17.9 µs against 15.1.
constexpr int WSLOTS = 2;
template <int QT, bool SWIGLU, int D>
constexpr size_t gemv_lds() {
  using W = Shape<SWIGLU>;
  return size_t(W::WAVES) * (D * 16 * Unit<QT>::BYTES + GEMV_BM * 1024) +
         (W::S > 1 ? size_t(RED_BUFS) * W::WAVES * (SWIGLU ? 2 : 1) * GEMV_BM * 16 * 4 + 32 : 0);
}


// A work item: one tile of rows of A times one block of 16 RB weight rows. A workgroup's items are looked up once,
// at its start, into a table in LDS (8 ints each: e, s0, m, n0 and the A rows), so that no global or scalar load
// is in flight in the stream of steps: a scalar load would hold up every LDS wait of a step.
struct Item {
  int e, s0, m, n0;
  int ar[GEMV_BM];  // the A rows (XQ rows) of the tile's rows of A
};

// The items of workgroup w of G, dealt back and forth: round j holds items j G .. j G + G - 1, forward in even rounds
// and backward in odd ones (the tiles come heaviest first, so a workgroup's items even out); item j of w, and how
// many of n_items it has.
__device__ __forceinline__ int snake_item(int w, int j, int G) { return j * G + ((j & 1) ? G - 1 - w : w); }
__device__ __forceinline__ int snake_count(int w, int G, int n_items) {
  const int full = n_items / G, r = n_items - full * G;
  return full + (r && ((full & 1) ? w >= G - r : w < r));
}

// A tile-list entry (tiles[2 t], tiles[2 t + 1]): the expert, with (lists in the GEMV's order, made by route_core)
// the tile's rows above bit 24 (0: not given, then from the expert's end in offsets), and the first sorted row.
__device__ __forceinline__ int tile_rows(int2 te, const int32_t* offsets) {
  const int m = te.x >> 24;
  return m ? m : min(GEMV_BM, offsets[(te.x & 0xFFFFFF) + 1] - te.y);
}

// (wave 0) the tile entry of item j of this workgroup (lane j), clamped into the list's bounds: loaded before the
// tile count is known, so that both are one memory round trip (an entry past the count is not used)
__device__ __forceinline__ int2 item_tile(const GemvArgs& a, const int32_t* tiles, int it0, int G, int NB, int j) {
  if (!tiles) return make_int2(0, 0);
  const int tile = min(snake_item(it0, j, G) / NB, int(a.max_tiles) - 1);
  return make_int2(tiles[2 * tile], tiles[2 * tile + 1]);
}

// wave 0: items snake_item(it0, 0, G), ... (n of them) into tab, 64 at a time, lane j one item; the tile list,
// offsets and order from tiles, offsets and order (the launch's arrays, or the workgroup's own routing in LDS, whose
// order holds the pairs' tokens: TOK); pre: the entry of item lane of the first 64, already loaded (item_tile)
template <bool TOK = false>
__device__ __forceinline__ void fill_items(const GemvArgs& a, int it0, int G, int n, int NB, int rows, int4* tab,
                                           int lane, const int32_t* tiles, const int32_t* offsets,
                                           const int32_t* order, int2 pre) {
  for (int j0 = 0; j0 < n; j0 += 64) {
    const int j = j0 + lane;
    if (j < n) {
      const int it = snake_item(it0, j, G), tile = it / NB;
      int e = 0, s0 = tile * GEMV_BM, m = min(GEMV_BM, a.dense_rows - s0);
      if (tiles) {
        const int2 te = j0 ? make_int2(tiles[2 * tile], tiles[2 * tile + 1]) : pre;
        e = te.x & 0xFFFFFF;
        s0 = te.y;
        m = tile_rows(te, offsets);
      }
      int ar[GEMV_BM];
#pragma unroll
      for (int t = 0; t < GEMV_BM; t++)
        if (a.a_gather) {
          const int o = order[min(s0 + min(t, m - 1), a.rows_total - 1)];
          ar[t] = TOK ? o : o / a.topk;
        } else {
          ar[t] = s0 + min(t, m - 1);
        }
      tab[2 * j] = make_int4(e, s0, m, (it - tile * NB) * rows);
      tab[2 * j + 1] = make_int4(ar[0], ar[1], ar[2], ar[3]);
    }
  }
}

__device__ __forceinline__ Item get_item(const int4* tab, int j) {
  const int4 u = lds_read_i4(tab + 2 * j), v = lds_read_i4(tab + 2 * j + 1);
  Item I;
  I.e = __builtin_amdgcn_readfirstlane(u.x);
  I.s0 = __builtin_amdgcn_readfirstlane(u.y);
  I.m = __builtin_amdgcn_readfirstlane(u.z);
  I.n0 = __builtin_amdgcn_readfirstlane(u.w);
  I.ar[0] = __builtin_amdgcn_readfirstlane(v.x);
  I.ar[1] = __builtin_amdgcn_readfirstlane(v.y);
  I.ar[2] = __builtin_amdgcn_readfirstlane(v.z);
  I.ar[3] = __builtin_amdgcn_readfirstlane(v.w);
  return I;
}

// the sum over the four 16-lane rows of lane (p, r), in every lane of column r (rows 0 + 1 and 2 + 3 first)
__device__ __forceinline__ float row4_sum(float s) {
  const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  s = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  const auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(y[0]) + __uint_as_float(y[1]);
}

// The state of a wave's stream of steps over its items (one step: 16 rows x one K-unit of one matrix). Every load
// of the stream is a DMA into LDS (the weights into D slots, the records of a K-unit into one slot), counted as it
// is issued (nl), so that each wait names the exact number of loads issued after the ones it needs: loads of one kind
// return in order. (Records loaded into registers instead would make the compiler wait for all loads in flight
// before each use: it cannot order them against the DMAs.)
template <int QT, bool SWIGLU, int D>
struct Stream {
  using W = Shape<SWIGLU>;
  static constexpr int RB = W::RB, S = W::S, BY = Unit<QT>::BYTES, CH = BY / 16, LW = Unit<QT>::LW;
  static constexpr int NM = SWIGLU ? 2 : 1, WCH = 16 * CH, NI = (WCH + 63) / 64, LAST = WCH - 64 * (NI - 1);
  static constexpr int LA = D - 1;                          // steps in flight ahead of the one being read
  static constexpr int XCH = GEMV_BM * 64;  // chunks of the record slot
  static constexpr int NMAX = LA * NI + (LA + 1) * GEMV_BM;  // loads issued after a step's, at most
  static_assert(NMAX < 64, "loads in flight beyond vmcnt");
  const GemvArgs& a;
  int wv, lane, p, r, rb, ks, u0, NVw;
  u32x4* my;  // the wave's weight slots, then its record slot
  uint32_t wbase, xbase, o_w, o_r, o_s;
  uint32_t lo[NI];   // the lane's byte offset in the 16 rows of each load instruction
  int nl = 0;        // loads issued so far
  int xend = 0;       // nl after the record slot's loads
  int wend[D] = {};  // nl after the weights of the last D steps issued (wend[0]: the latest)

  __device__ __forceinline__ explicit Stream(const GemvArgs& args) : a(args) {
    extern __shared__ u32x4 slab[];
    wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    lane = threadIdx.x & 63, p = lane >> 4, r = lane & 15;
    rb = wv / S, ks = wv % S;
    my = slab + wv * (D * WCH + XCH);
    const int U = a.K / 256;
    u0 = ks;  // (the wave's K-units: ks, ks + S, ...; the pair reads neighbouring units, which share lines, together)
    NVw = (U - ks + S - 1) / S * NM;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int q = min(64 * i + lane, WCH - 1), row = q / CH;
      lo[i] = uint32_t((16 * rb + row) * a.row_bytes + 16 * (q - row * CH));
    }
    wbase = lds_addr(my);
    xbase = lds_addr(my + D * WCH) + 16 * lane;
    if constexpr (QT == ARTLITE_Q6_K) {  // (low bits of half p / 2, its high bits, the scales and d)
      o_w = r * BY + 64 * (p >> 1);
      o_r = r * BY + 128 + 32 * (p >> 1);
      o_s = r * BY + 192;
    } else if constexpr (QT == ARTLITE_Q3_K) {  // (the high bits, low bits of half p / 2, the scales and d)
      o_w = r * BY;
      o_r = r * BY + 32 + 32 * (p >> 1);
      o_s = r * BY + 96;
    } else {
      constexpr bool HEAD = QT == ARTLITE_Q4_K || QT == ARTLITE_Q5_K || QT == ARTLITE_IQ4_XS;  // (header + run)
      constexpr int PB = QT == ARTLITE_Q8_0 ? 68 : QT == ARTLITE_Q4_1 ? 40 : 36;  // (the lane's two blocks)
      o_w = r * BY + (HEAD ? 0 : PB * p);
      o_r = r * BY + (QT == ARTLITE_Q5_K ? 48 : 16) + 32 * p;  // (Q4_K / Q5_K / IQ4_XS: the lane's run)
      o_s = o_w;
    }
  }
  // the weights of local step v of item (e, n0) into slot `slot`; !on: none (the end of the stream), counted alike
  template <int MX>
  __device__ __forceinline__ void issue_w(bool on, int e, int n0, int v, int slot) {
    if (on) {
      // (rows past N cannot occur: N is a multiple of the item's rows)
      const uint8_t* src = a.w[MX] + int64_t(e) * a.expert_bytes + int64_t(n0) * a.row_bytes +
                           int64_t(u0 + S * (v / NM)) * BY;
      u32x4* dst = my + slot * WCH;
#pragma unroll
      for (int i = 0; i < NI; i++)
        if (i < NI - 1 || lane < LAST)
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + lo[i]),
                                           (__attribute__((address_space(3))) void*)(dst + 64 * i), 16, 0, 0);
      nl += NI;
    }
#pragma unroll
    for (int i = D - 1; i > 0; i--) wend[i] = wend[i - 1];
    wend[0] = nl;
  }
  // the records of K-unit ku of item I's rows of A into the record slot (lane l: chunk l of each row)
  __device__ __forceinline__ void load_x(const Item& I, int ku) {
    u32x4* dst = my + D * WCH;
#pragma unroll
    for (int t = 0; t < GEMV_BM; t++)
      if (t < I.m)
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const void*>(a.xq + int64_t(I.ar[t]) * xq_row_dwords(a.K) + ku * XQ_UNIT + 4 * lane),
            (__attribute__((address_space(3))) void*)(dst + 64 * t), 16, 0, 0);
    nl += I.m;
    xend = nl;
  }
};

// the wait and read of a step: vmcnt(n), then the weights and (MX) the record chunks. n is at most NMAX (the stream's
// counts: after a step's weights come the LA steps' issued ahead (NI each) and at most LA + 1 K-units' records); a
// larger n, which the stream does not produce, would wait for every load (vmcnt(0)), never for fewer than needed
template <int QT, bool SWIGLU, int MX, int D>
__device__ __forceinline__ void wait_read(const Stream<QT, SWIGLU, D>& st, int n, uint32_t sw, uint32_t sx,
                                          uint32_t (&w)[Unit<QT>::LW], u32x4 (&x)[GEMV_BM]) {
  using SS = Stream<QT, SWIGLU, D>;
  if (n > SS::NMAX) n = 0;
  static_for<SS::NMAX + 1>([&](auto nc) {
    constexpr int N = decltype(nc)::value;
    if (n == N) wait_vm<N>();
  });
  read_unit<QT, MX>(w, x, sw + st.o_w, sw + st.o_r, sw + st.o_s, sx);
}

// The dot products of one step: the lane's two groups of the unit w against the M rows of A's records x.
template <int QT, int M>
__device__ __forceinline__ void step_terms(const uint32_t (&w)[Unit<QT>::LW], const u32x4 (&x)[GEMV_BM], int p,
                                           float (&acc)[M]) {
  static_for<2>([&](auto hc) {
    constexpr int H = decltype(hc)::value;
    uint32_t q[8];
    float d, mn;
    codes<QT, H>(w, 2 * p + H, q, d, mn);
#pragma unroll
    for (int t = 0; t < M; t++) acc[t] = group_term<QT, H>(acc[t], x[t][H], x[t][2], x[t][3], q, d, mn);
  });
}

// Item `cur` of the stream, whose first step is global step gs; `nxt` is the next item if has_next. Steps run LA
// ahead in the wave's own slots (a slot refilled right after the step that read it), across items. Each step issues
// the weights LA steps ahead, then waits for its own; at the start of each K-unit that wait also covers the
// records, which are read into registers with the weights, and the next K-unit's are loaded into the freed slot.
// Returns with the sums of the four lanes of a row in every lane.
template <int QT, bool SWIGLU, int M, int D>
__device__ __forceinline__ void run_item(Stream<QT, SWIGLU, D>& st, const Item& cur, const Item& nxt, bool has_next,
                                         int gs, float (&out)[SWIGLU ? 2 : 1][GEMV_BM]) {
  using SS = Stream<QT, SWIGLU, D>;
  constexpr int NM = SS::NM, LW = SS::LW, LA = SS::LA;
  float acc[NM][M];
#pragma unroll
  for (int mx = 0; mx < NM; mx++)
#pragma unroll
    for (int t = 0; t < M; t++) acc[mx][t] = 0.0f;
  u32x4 xc[GEMV_BM];
  for (int v0 = 0; v0 < st.NVw; v0 += NM) {
    static_for<NM>([&](auto jc) {
      constexpr int MX = decltype(jc)::value;
      const int v = v0 + MX;
      // the step LA ahead: in this item, or the next item's, or none (counted alike)
      auto issue = [&] {
        const int vi = v + LA;
        const bool here = vi < st.NVw;
        st.template issue_w<(MX + LA) % NM>(here || has_next, here ? cur.e : nxt.e, here ? cur.n0 : nxt.n0,
                                            here ? vi : vi - st.NVw, (gs + v + LA) % D);
      };
      issue();
      uint32_t w[LW];
      const uint32_t sw = st.wbase + ((gs + v) % D) * SS::WCH * 16;
      if constexpr (MX == 0) {
        // (wend[D - 1]: this step's weights), then the next K-unit's records into the slot just read
        const int nw = st.nl - st.wend[D - 1];
        wait_read<QT, SWIGLU, M, D>(st, min(nw, st.nl - st.xend), sw, st.xbase, w, xc);
        if (v0 + NM < st.NVw)
          st.load_x(cur, st.u0 + SS::S * (v0 / NM + 1));
        else if (has_next)
          st.load_x(nxt, st.u0);
      } else {
        wait_read<QT, SWIGLU, 0, D>(st, st.nl - st.wend[D - 1], sw, st.xbase, w, xc);
      }
      step_terms<QT, M>(w, xc, st.p, acc[MX]);
    });
  }
#pragma unroll
  for (int mx = 0; mx < NM; mx++)
#pragma unroll
    for (int t = 0; t < GEMV_BM; t++) {
      if (t < M) {
        out[mx][t] = row4_sum(acc[mx][t < M ? t : 0]);
      } else {
        out[mx][t] = 0.0f;
      }
    }
}

// A persistent workgroup: items snake_item(blockIdx.x, j, gridDim.x) of (tile, block of 16 RB rows), tile-major.
template <int QT, bool SWIGLU, int D>
__global__ __launch_bounds__(Shape<SWIGLU>::THREADS) __attribute__((amdgpu_waves_per_eu(QT == ARTLITE_Q4_0 ? 4 : 2))) void k_gemv(
    const GemvArgs a) {
  using W = Shape<SWIGLU>;
  using SS = Stream<QT, SWIGLU, D>;
  constexpr int RB = W::RB, S = W::S, NM = SS::NM;
  const int rows = 16 * RB, NB = (a.N + rows - 1) / rows;
  extern __shared__ u32x4 slab[];
  int n_tiles;
  bool routed = false;
  if constexpr (SWIGLU) {
    if (a.route.logits) {
      // the routing in this workgroup's LDS, over the weight and record slots (no load into them is issued before
      // the barrier after the item table); workgroup 0 also stores it for the launches after this one
      const GemvArgs::Route& r = a.route;
      auto& rl = *reinterpret_cast<RouteLds<W::THREADS>*>(slab);
      int* ro = reinterpret_cast<int*>(&rl + 1);
      RouteOut o;
      o.tiles = ro;
      o.order = ro + 2 * a.max_tiles;
      o.offsets = o.order + r.T * r.k;
      o.n_tiles = o.offsets + r.E + 1;
      o.stage = reinterpret_cast<float*>(ro + (2 * a.max_tiles + r.T * r.k + r.E + 2 + 3) / 4 * 4);
      const bool w0 = blockIdx.x == 0;
      int32_t* ids = w0 ? r.ids : nullptr;
      float* w32 = w0 ? r.w32 : nullptr;
      if (r.E <= 64)
        route_core<W::THREADS, 1, true>(r.logits, r.T, r.E, r.k, r.sigmoid, GEMV_BM, 0, ids, w32, r.d, w0, rl, o);
      else if (r.E <= 128)
        route_core<W::THREADS, 2, true>(r.logits, r.T, r.E, r.k, r.sigmoid, GEMV_BM, 0, ids, w32, r.d, w0, rl, o);
      else if (r.E <= 256)
        route_core<W::THREADS, 4, true>(r.logits, r.T, r.E, r.k, r.sigmoid, GEMV_BM, 0, ids, w32, r.d, w0, rl, o);
      else
        route_core<W::THREADS, 8, true>(r.logits, r.T, r.E, r.k, r.sigmoid, GEMV_BM, 0, ids, w32, r.d, w0, rl, o);
      __syncthreads();
      n_tiles = __builtin_amdgcn_readfirstlane(lds_read_i32(o.n_tiles));
      routed = true;
    }
  }
  const int G = gridDim.x, it0 = blockIdx.x;
  // (not routed here: the workgroup's first 64 tile entries in flight with the tile count, in every wave: lane 0's
  // gives each wave its first steps, wave 0's the table)
  const int2 pre = routed ? make_int2(0, 0) : item_tile(a, a.tiles, it0, G, NB, threadIdx.x & 63);
  if (!routed) n_tiles = a.tiles ? *a.n_tiles : (a.dense_rows + GEMV_BM - 1) / GEMV_BM;
  const int n_items = n_tiles * NB;
  if (it0 >= n_items) return;
  SS st(a);
  // [buffer][wave][matrix][row of A][row], after every wave's slots
  float* red = reinterpret_cast<float*>(slab + W::WAVES * (D * SS::WCH + SS::XCH));

  const int n_my = snake_count(it0, G, n_items);
  constexpr int RED = W::WAVES * NM * GEMV_BM * 16;  // floats of one partial-sum buffer
  int* ctr = reinterpret_cast<int*>(red + (S > 1 ? RED_BUFS * RED : 0));  // [b]: arrivals, [4 + b]: epilogues done
  int4* tab = reinterpret_cast<int4*>(ctr + (S > 1 ? 8 : 0));
  // the first item's first LA steps (its expert from a scalar load) ahead of the table; routed here: after it
  auto first_steps = [&](int e0) {
    const int n00 = (it0 % NB) * rows;
    for (int v = 0; v < SS::LA; v++) {
      if (NM == 1 || v % NM == 0)
        st.template issue_w<0>(true, e0, n00, v, v);
      else
        st.template issue_w<NM - 1>(true, e0, n00, v, v);
    }
  };
  if (!routed && st.NVw > 0) first_steps(__builtin_amdgcn_readfirstlane(pre.x) & 0xFFFFFF);
  if (st.wv == 0) {
    if (routed) {  // (the workgroup's own copies, from the LDS address itself: read as LDS)
      const int* ro = reinterpret_cast<const int*>(slab) + sizeof(RouteLds<W::THREADS>) / 4;
      const int* ord = ro + 2 * a.max_tiles;
      fill_items<true>(a, it0, G, n_my, NB, rows, tab, st.lane, ro, ord + a.rows_total, ord,
                       item_tile(a, ro, it0, G, NB, st.lane));
    } else {
      fill_items(a, it0, G, n_my, NB, rows, tab, st.lane, a.tiles, a.offsets, a.order, pre);
    }
  }
  if (S > 1 && threadIdx.x < 8) ctr[threadIdx.x] = 0;
  __syncthreads();
  Item cur = get_item(tab, 0), nxt = cur;
  if (routed && st.NVw > 0) first_steps(cur.e);
  if (st.NVw > 0) st.load_x(cur, st.u0);
  int gs = 0;
  for (int j = 0; j < n_my; j++) {
    const bool has_next = j + 1 < n_my;
    if (has_next) nxt = get_item(tab, j + 1);
    float out[NM][GEMV_BM];
    switch (cur.m) {
      case 1: run_item<QT, SWIGLU, 1, D>(st, cur, nxt, has_next, gs, out); break;
      case 2: run_item<QT, SWIGLU, 2, D>(st, cur, nxt, has_next, gs, out); break;
      case 3: run_item<QT, SWIGLU, 3, D>(st, cur, nxt, has_next, gs, out); break;
      default: run_item<QT, SWIGLU, 4, D>(st, cur, nxt, has_next, gs, out); break;
    }
    gs += st.NVw;
    if constexpr (!SWIGLU) {
      static_assert(S == 1, "plain products: one wave per row block");
      const int n = cur.n0 + 16 * st.rb + st.r;
#pragma unroll
      for (int t = 0; t < GEMV_BM; t++)
        if (t < cur.m && st.p == 0) a.y[int64_t(cur.s0 + t) * a.N + n] = out[0][t];
    } else {
      // The K-ranges' partial sums through LDS, summed in a fixed order by the last wave to deliver its own (a
      // counter per buffer, no barrier: the other waves go on with their next items); RED_BUFS buffers, a wave
      // waiting before it reuses one until the epilogue RED_BUFS items back is done. Then h = silu(gate) up of
      // the 16 RB rows, quantised into RB / 2 groups of an XQ row of N values per row of A. (The lane is recomputed
      // here rather than kept from the start: the registers are needed by the steps.)
      const int ln = __lane_id(), b = j % RED_BUFS;
      float* rd = red + b * RED;
      if (j >= RED_BUFS) {
        while (lds_read_i32(ctr + 4 + b) < j / RED_BUFS) __builtin_amdgcn_s_sleep(1);
      }
      if (ln < 16)
#pragma unroll
        for (int mx = 0; mx < NM; mx++)
#pragma unroll
          for (int t = 0; t < GEMV_BM; t++) rd[((st.wv * NM + mx) * GEMV_BM + t) * 16 + ln] = out[mx][t];
      int arrived = 0;
      if (ln == 0) arrived = lds_inc(ctr + b);
      if (__builtin_amdgcn_readfirstlane(arrived) == W::WAVES - 1) {
        if (ln < 8 * RB / 2 * cur.m) {
          // lanes 8 RB / 2 t .. + 8 RB / 2 take row of A t: 8 lanes per XQ group of 32 rows, 4 rows each
          constexpr int LPT = 8 * RB / 2;
          const int t = ln / LPT, lt = ln % LPT, l8 = lt & 7, rbb = lt >> 2, r0 = 4 * (lt & 3);
          const int UH = a.N / 256, blk = cur.n0 / 32 + (lt >> 3), g = blk & 7;
          float4 gsum = {0.0f, 0.0f, 0.0f, 0.0f}, usum = gsum;
#pragma unroll
          for (int k = 0; k < S; k++) {
            gsum += lds_read_f4(rd + (((rbb * S + k) * NM + 0) * GEMV_BM + t) * 16 + r0);
            usum += lds_read_f4(rd + (((rbb * S + k) * NM + 1) * GEMV_BM + t) * 16 + r0);
          }
          const float gv[4] = {gsum.x, gsum.y, gsum.z, gsum.w}, uv[4] = {usum.x, usum.y, usum.z, usum.w};
          float hv[4];
#pragma unroll
          for (int i = 0; i < 4; i++) hv[i] = gv[i] * __builtin_amdgcn_rcpf(1.0f + __expf(-gv[i])) * uv[i];
          int qa[4], qb[4], sum;
          float s256, xsum;
          quant_group(hv, qa, qb, s256, sum, xsum);
          uint32_t pa = 0, pb = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            pa |= uint32_t(qa[i] & 0xFF) << (8 * i);
            pb |= uint32_t(qb[i] & 0xFF) << (8 * i);
          }
          uint32_t* ub = a.hq + int64_t(cur.s0 + t) * UH * XQ_UNIT + (blk >> 3) * XQ_UNIT;
          ub[xq_block(g, l8)] = pa;
          ub[xq_block(g, 8 + l8)] = pb;
          xq_put_word(ub, g, l8, s256, sum, xsum);
          xq_put_word(ub, g, 8 + l8, s256, sum, xsum);
        }
        if (ln == 0) {
          lds_store(ctr + b, 0);
          lds_inc(ctr + 4 + b);
        }
      }
    }
    cur = nxt;
  }
}

// one wave per (row, unit) of x
template <int XT>
__global__ __launch_bounds__(256) void k_quant(const void* __restrict__ x, int64_t T, int K, uint32_t* __restrict__ xq) {
  const int64_t w = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  if (w < T * (K / 256)) xq_quant_unit<XT>(x, w, K, xq, threadIdx.x & 63);
}

// work items of a launch (the tile bound times the blocks of 16 RB rows)
template <bool SWIGLU>
int64_t gemv_items(const GemvArgs& a) {
  using W = Shape<SWIGLU>;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + GEMV_BM - 1) / GEMV_BM;
  return tiles * ((a.N + 16 * W::RB - 1) / (16 * W::RB));
}

// persistent workgroups of k_gemv<QT, SWIGLU, D>: as many as the device holds at once (queried once per kernel, with
// a table of 64 items; 0: set-up failed); their item tables take 32 bytes an item, at most lds_max in all
template <int QT, bool SWIGLU, int D>
int gemv_resident() {
  using W = Shape<SWIGLU>;
  constexpr size_t lds0 = gemv_lds<QT, SWIGLU, D>(), lds_max = lds0 + 8192;
  static const int resident = [] {
    const void* f = reinterpret_cast<const void*>(k_gemv<QT, SWIGLU, D>);
    int dev = 0, cus = 0, per_cu = 0;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_max)) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, W::THREADS, lds0 + 64 * 32) != hipSuccess)
      return 0;
    return cus * std::max(1, per_cu);
  }();
  return resident;
}

template <int QT, bool SWIGLU, int D>
int launch_t(const GemvArgs& a, hipStream_t s) {
  using W = Shape<SWIGLU>;
  const int64_t items = gemv_items<SWIGLU>(a);
  if (items <= 0) return ARTLITE_OK;
  if (items >= (int64_t(1) << 31)) return fail(ARTLITE_EINVAL, "expert GEMV: %lld work items", (long long)items);
  constexpr size_t lds0 = gemv_lds<QT, SWIGLU, D>(), lds_max = lds0 + 8192;
  const int resident = gemv_resident<QT, SWIGLU, D>();
  if (resident <= 0) return fail(ARTLITE_EHIP, "expert GEMV: kernel set-up failed");
  const unsigned grid = unsigned(std::min<int64_t>(items, resident));
  const size_t lds = lds0 + size_t((items + grid - 1) / grid) * 32;
  if (lds > lds_max) return fail(ARTLITE_EINVAL, "expert GEMV: %lld work items", (long long)items);
  if (SWIGLU && a.route.logits) {
    // the routing's LDS (scratch, then the tile list, order, offsets and tile count) within the slots
    const GemvArgs::Route& r = a.route;
    const size_t need = sizeof(RouteLds<W::THREADS>) + 4 * (size_t(2 * a.max_tiles + r.T * r.k + r.E + 2 + 3) / 4 * 4) +
                        4 * size_t(r.T) * r.E;
    const size_t slots = size_t(W::WAVES) * (D * 16 * Unit<QT>::BYTES + GEMV_BM * 1024);
    if (!gemv_route_fits(r.T, r.E, r.k) || need > slots || a.rows_total != r.T * r.k || a.topk != r.k ||
        a.max_tiles != tile_bound(int64_t(r.T) * r.k, r.E, GEMV_BM))
      return fail(ARTLITE_EINVAL, "expert GEMV: routing of %d tokens, %d experts, top %d in the launch", r.T, r.E,
                  r.k);
  }
  k_gemv<QT, SWIGLU, D><<<grid, W::THREADS, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace

// (the LDS it takes, at the most these allow: RouteLds<512>, 9.2 KB of tile list, order and offsets, 32 KB of staged
// logits; within the weight and record slots of every format, Q3_K's 61.4 KB the least)
bool gemv_route_fits(int64_t T, int E, int k) {
  return T >= 1 && k >= 1 && k <= MAX_TOPK && k <= E && E <= Shape<true>::THREADS && E % 4 == 0 &&
         T * k <= Shape<true>::THREADS && T * E <= 8192;
}

bool gemv_supported(int qtype, int K, int N) {
  return (qtype == ARTLITE_Q4_0 || qtype == ARTLITE_Q8_0 || qtype == ARTLITE_Q4_K || qtype == ARTLITE_Q5_K ||
          qtype == ARTLITE_Q6_K || qtype == ARTLITE_Q4_1 || qtype == ARTLITE_IQ4_NL || qtype == ARTLITE_IQ4_XS ||
          qtype == ARTLITE_Q3_K) &&
         K > 0 && K % 256 == 0 &&
         N > 0 && N % 64 == 0;
}

int launch_gemv(const GemvArgs& a, hipStream_t s) {
  if (!gemv_supported(a.qtype, a.K, a.N))
    return fail(ARTLITE_EINVAL,
                "expert GEMV: weight type %d with K %d, N %d (K a multiple of 256, N of 64)",
                a.qtype, a.K, a.N);
  if (a.N <= 0 || int64_t(a.N) * a.row_bytes >= (int64_t(1) << 31))
    return fail(ARTLITE_EINVAL, "expert GEMV: %d rows of %d bytes", a.N, a.row_bytes);
  const bool swiglu = a.w[1] != nullptr;
  if (swiglu && (a.N % 256 || !a.hq))
    return fail(ARTLITE_EINVAL, "expert GEMV: SwiGLU width %d is not a multiple of 256", a.N);
  if (!swiglu && !a.y) return fail(ARTLITE_EINVAL, "expert GEMV: no output");
#define ART_DISPATCH(QT) return swiglu ? launch_t<QT, true, WSLOTS>(a, s) : launch_t<QT, false, WSLOTS>(a, s)
  switch (a.qtype) {
    case ARTLITE_Q4_0: ART_DISPATCH(ARTLITE_Q4_0);
    case ARTLITE_Q8_0: ART_DISPATCH(ARTLITE_Q8_0);
    case ARTLITE_Q5_K: ART_DISPATCH(ARTLITE_Q5_K);
    case ARTLITE_Q6_K: ART_DISPATCH(ARTLITE_Q6_K);
    case ARTLITE_Q3_K: ART_DISPATCH(ARTLITE_Q3_K);
    case ARTLITE_Q4_1: ART_DISPATCH(ARTLITE_Q4_1);
    case ARTLITE_IQ4_NL: ART_DISPATCH(ARTLITE_IQ4_NL);
    case ARTLITE_IQ4_XS: ART_DISPATCH(ARTLITE_IQ4_XS);
    default: ART_DISPATCH(ARTLITE_Q4_K);
  }
#undef ART_DISPATCH
}

int launch_quant(const void* x, int x_dtype, int64_t T, int K, uint32_t* xq, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (K <= 0 || K % 256) return fail(ARTLITE_EINVAL, "quant: K %d is not a multiple of 256", K);
  const int64_t waves = T * (K / 256);
  const unsigned blocks = unsigned((waves + 3) / 4);
  if (x_dtype == ARTLITE_X_F32)
    k_quant<ARTLITE_X_F32><<<blocks, 256, 0, s>>>(x, T, K, xq);
  else
    k_quant<ARTLITE_X_BF16><<<blocks, 256, 0, s>>>(x, T, K, xq);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

void xq_dequant_row(const uint32_t* row, int K, float* out) {
  for (int u = 0; u < K / 256; u++) {
    const uint32_t* ub = row + int64_t(u) * XQ_UNIT;
    for (int g = 0; g < 8; g++) {
      float s;
      std::memcpy(&s, &ub[4 * (16 * (g >> 1) + 2 * (g & 1)) + 2], 4);
      for (int v = 0; v < 32; v++) {
        const int j = v / 4, sh = 8 * (v % 4);
        const int qa = int8_t((ub[xq_block(g, j)] >> sh) & 0xFFu);
        const int qb = int8_t((ub[xq_block(g, 8 + j)] >> sh) & 0xFFu);
        out[u * 256 + 32 * g + v] = s * float(256 * qa + qb);
      }
    }
  }
}

}  // namespace artlite
