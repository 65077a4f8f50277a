// Decode expert products on the VALU, and the XQ activations they read.
//
// A workgroup is one wave: one tile of at most GEMV_BM sorted rows of A (tokens for gate / up, pairs for down) of
// one expert, times 64 weight rows, one per lane (SwiGLU: the lane's gate row and its up row). The wave streams its
// rows in units of 8 groups of 32 values (Q4_0 / Q4_K: 144 bytes of a row, Q8_0: 272), 64 rows per unit, with
// global_load_lds_dwordx4 straight into one of D LDS slots (consecutive lanes load consecutive 16-byte chunks, so
// each load instruction reads whole runs of rows). A row occupies an odd number of 16-byte chunks of its slot, so
// the lanes' own-row ds_read_b128 fall in distinct banks. The tile's XQ records of the unit come with it (three
// dwordx4 per row of A, one record per lane of each 16-lane row), and DPP row_newbcast:j hands dword j of a group's
// block to every lane as the broadcast operand of v_dot4c_i32_i8: the activations cost no LDS traffic.
//
// Arithmetic of one (row of A, group): A = sum_j dot4(a_j, q_j) and B = C + sum_j dot4(b_j, q_j), exactly in int32,
// with q_j the group's codes as int8 (Q4_0 / Q4_K: nibbles 0..15, Q8_0: the signed bytes) and C the code offset's
// correction (Q4_0: -8 sum(256 a + b), else 0); then acc += (d s / 256) float(256 A + B), which is
// d s sum (q - 8)(a + b / 256) for Q4_0. Q4_K adds -(dmin mn) times the group's dequantised activation sum.
#include "gemv.h"

#include <cmath>
#include <cstring>
#include <utility>

namespace artlite {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }

template <int QT>
struct Unit;
template <>
struct Unit<ARTLITE_Q4_0> {
  static constexpr int BYTES = 144;
};
template <>
struct Unit<ARTLITE_Q8_0> {
  static constexpr int BYTES = 272;
};
template <>
struct Unit<ARTLITE_Q4_K> {
  static constexpr int BYTES = 144;
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

// dword i of a unit held as 16-byte chunks (i a constant after unrolling)
template <int CH>
__device__ __forceinline__ uint32_t dw(const u32x4 (&w)[CH], int i) {
  return w[i >> 2][i & 3];
}

// After vmcnt(N), the lane's row of a unit and the tile's XQ records of it from the unit's LDS slot, and their
// completion, in one asm block: the compiler would otherwise wait for every load in flight before reading LDS (it
// takes the slots' global_load_lds writes for possible producers), and it must not touch the outputs before the
// final wait. pw: the lane's row; px: record (lane % 16) of the tile's first row of A (rows 768 bytes apart).
#define ART_RW(I) "ds_read_b128 %[w" #I "], %[pw] offset:" #I "*16\n\t"
#define ART_RX(T, C) "ds_read_b128 %[x" #T #C "], %[px] offset:" #T "*768+" #C "*16\n\t"
#define ART_W9 ART_RW(0) ART_RW(1) ART_RW(2) ART_RW(3) ART_RW(4) ART_RW(5) ART_RW(6) ART_RW(7) ART_RW(8)
#define ART_W17 ART_W9 ART_RW(9) ART_RW(10) ART_RW(11) ART_RW(12) ART_RW(13) ART_RW(14) ART_RW(15) ART_RW(16)
#define ART_OW(I) [w##I] "=&v"(w[I])
#define ART_OW9 ART_OW(0), ART_OW(1), ART_OW(2), ART_OW(3), ART_OW(4), ART_OW(5), ART_OW(6), ART_OW(7), ART_OW(8)
#define ART_OW17 \
  ART_OW9, ART_OW(9), ART_OW(10), ART_OW(11), ART_OW(12), ART_OW(13), ART_OW(14), ART_OW(15), ART_OW(16)
#define ART_X1 ART_RX(0, 0) ART_RX(0, 1) ART_RX(0, 2)
#define ART_X2 ART_X1 ART_RX(1, 0) ART_RX(1, 1) ART_RX(1, 2)
#define ART_X3 ART_X2 ART_RX(2, 0) ART_RX(2, 1) ART_RX(2, 2)
#define ART_X4 ART_X3 ART_RX(3, 0) ART_RX(3, 1) ART_RX(3, 2)
#define ART_OX(T) [x##T##0] "=&v"(x[T][0]), [x##T##1] "=&v"(x[T][1]), [x##T##2] "=&v"(x[T][2])
#define ART_OX1 ART_OX(0)
#define ART_OX2 ART_OX1, ART_OX(1)
#define ART_OX3 ART_OX2, ART_OX(2)
#define ART_OX4 ART_OX3, ART_OX(3)
#define ART_READ(CHN, MN)                                                                                      \
  asm volatile("s_waitcnt vmcnt(%[n])\n\t" ART_W##CHN ART_X##MN "s_waitcnt lgkmcnt(0)"                      \
               : ART_OW##CHN, ART_OX##MN                                                                      \
               : [pw] "v"(pw), [px] "v"(px), [n] "i"(N))
template <int N, int CH, int M>
__device__ __forceinline__ void read_unit(u32x4 (&w)[CH], u32x4 (&x)[M][3], uint32_t pw, uint32_t px) {
  static_assert(N >= 0 && N < 64, "vmcnt");
  static_assert(CH == 9 || CH == 17, "unit chunks");
  if constexpr (CH == 9 && M == 1) ART_READ(9, 1);
  if constexpr (CH == 9 && M == 2) ART_READ(9, 2);
  if constexpr (CH == 9 && M == 3) ART_READ(9, 3);
  if constexpr (CH == 9 && M == 4) ART_READ(9, 4);
  if constexpr (CH == 17 && M == 1) ART_READ(17, 1);
  if constexpr (CH == 17 && M == 2) ART_READ(17, 2);
  if constexpr (CH == 17 && M == 3) ART_READ(17, 3);
  if constexpr (CH == 17 && M == 4) ART_READ(17, 4);
}
#undef ART_READ
#undef ART_OX4
#undef ART_OX3
#undef ART_OX2
#undef ART_OX1
#undef ART_OX
#undef ART_X4
#undef ART_X3
#undef ART_X2
#undef ART_X1
#undef ART_OW17
#undef ART_OW9
#undef ART_OW
#undef ART_W17
#undef ART_W9
#undef ART_RX
#undef ART_RW

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// codes of group G of a unit as 8 dwords of int8 (q[j]: values 4 j .. 4 j + 3 of the group), its scale d
// (Q4_K: d sc) and Q4_K's dmin mn
template <int QT, int G>
__device__ __forceinline__ void codes(const u32x4 (&w)[Unit<QT>::BYTES / 16], uint32_t (&q)[8], float& d, float& mn) {
  if constexpr (QT == ARTLITE_Q4_0) {
    // 18 bytes at 18 G: fp16 d, then 16 bytes whose low nibbles are values 0..15 and high nibbles 16..31
    constexpr int o = 18 * G;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t v;
      if constexpr (o % 4 == 0)
        v = __builtin_amdgcn_alignbit(dw(w, o / 4 + j + 1), dw(w, o / 4 + j), 16);
      else
        v = dw(w, (o + 2) / 4 + j);
      q[j] = v & 0x0F0F0F0Fu;
      q[4 + j] = (v >> 4) & 0x0F0F0F0Fu;
    }
    d = o % 4 == 0 ? h2f(dw(w, o / 4) & 0xFFFFu) : h2f(dw(w, (o - 2) / 4) >> 16);
    mn = 0.0f;
  } else if constexpr (QT == ARTLITE_Q8_0) {
    // 34 bytes at 34 G: fp16 d, then 32 signed bytes in value order
    constexpr int o = 34 * G;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if constexpr (o % 4 == 0)
        q[j] = __builtin_amdgcn_alignbit(dw(w, o / 4 + j + 1), dw(w, o / 4 + j), 16);
      else
        q[j] = dw(w, (o + 2) / 4 + j);
    }
    d = o % 4 == 0 ? h2f(dw(w, o / 4) & 0xFFFFu) : h2f(dw(w, (o - 2) / 4) >> 16);
    mn = 0.0f;
  } else {
    // a super-block: fp16 d, dmin; 12 bytes of 6-bit scales / mins; 4 runs of 32 bytes, run c holding group 2 c in
    // its low nibbles and group 2 c + 1 in its high nibbles (value order)
    auto sb = [&](int k) { return (dw(w, 1 + k / 4) >> (8 * (k % 4))) & 0xFFu; };
    uint32_t sc, m;
    if constexpr (G < 4) {
      sc = sb(G) & 63u;
      m = sb(G + 4) & 63u;
    } else {
      sc = (sb(G + 4) & 15u) | ((sb(G - 4) >> 6) << 4);
      m = (sb(G + 4) >> 4) | ((sb(G) >> 6) << 4);
    }
    d = h2f(dw(w, 0) & 0xFFFFu) * float(sc);  // (exact: 11 x 6 significant bits)
    mn = h2f(dw(w, 0) >> 16) * float(m);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t v = dw(w, 4 + 8 * (G / 2) + j);
      q[j] = G % 2 ? (v >> 4) & 0x0F0F0F0Fu : v & 0x0F0F0F0Fu;
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
#define ART_QIN                                                                                   \
  [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]), [q5] "v"(q[5]), \
      [q6] "v"(q[6]), [q7] "v"(q[7])
#define ART_ACC [a0] "=&v"(a0), [a1] "=&v"(a1), [b0] "=&v"(b0), [b1] "=&v"(b1), [c] "=&v"(coef)

// acc += the group's term for one row of A. x: its block dword; l: the record's list word (lane 2 G: s / 256,
// lane 2 G + 1: the sum of 256 a + b); xs: the record's sum word (lane G: the dequantised sum).
template <int QT, int G>
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
        : [x] "v"(x), [l] "v"(l), [d] "v"(d), [m8] "v"(-8), ART_QIN, [l0] "i"(2 * G), [l1] "i"(2 * G + 1));
  } else if constexpr (QT == ARTLITE_Q8_0) {
    asm("s_nop 1\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[b0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : ART_ACC
        : [x] "v"(x), [l] "v"(l), [d] "v"(d), ART_QIN, [l0] "i"(2 * G));
  } else {
    float mterm;
    asm("s_nop 1\n\t"
        "v_mov_b32 %[a0], 0\n\t"
        "v_mov_b32 %[b0], 0\n\t"
        "v_mov_b32 %[a1], 0\n\t"
        "v_mov_b32 %[b1], 0\n\t" ART_DOTS
        "v_mul_f32_dpp %[c], %[l], %[d] row_newbcast:%[l0] row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t], %[xs], %[nm] row_newbcast:%[g] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0"
        : ART_ACC, [t] "=&v"(mterm)
        : [x] "v"(x), [l] "v"(l), [xs] "v"(xs), [d] "v"(d), [nm] "v"(-mn), ART_QIN, [l0] "i"(2 * G), [g] "i"(G));
    return __builtin_fmaf(coef, float((a0 + a1) * 256 + (b0 + b1)), acc) + mterm;
  }
  return __builtin_fmaf(coef, float((a0 + a1) * 256 + (b0 + b1)), acc);
}
#undef ART_ACC
#undef ART_DOT
#undef ART_DOTS
#undef ART_QIN

// Quantise a 32-value group held by 32 / V consecutive lanes, V values each: this lane's int8 plane values, and the
// group's s / 256, sum of (256 a + b) and dequantised sum (s / 256 times that sum).
template <int V>
__device__ __forceinline__ void quant_group(const float (&x)[V], int (&qa)[V], int (&qb)[V], float& s256, int& sum,
                                            float& xsum) {
  constexpr int L = 32 / V;
  float amax = 0.0f;
  int bad = 0;
#pragma unroll
  for (int i = 0; i < V; i++) {
    amax = fmaxf(amax, fabsf(x[i]));
    bad |= !__builtin_isfinite(x[i]);
  }
#pragma unroll
  for (int o = 1; o < L; o <<= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, o));
    bad |= __shfl_xor(bad, o);
  }
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
#pragma unroll
  for (int o = 1; o < L; o <<= 1) sum += __shfl_xor(sum, o);
  s256 = bad ? __builtin_nanf("") : skip ? 0.0f : amax / 32512.0f;  // (127 x 256)
  xsum = s256 * float(sum);
}

// the group's three per-group words into unit ub (group g)
__device__ __forceinline__ void put_group_words(uint32_t* ub, int g, float s256, int sum, float xsum) {
  ub[(2 * g) * XQ_REC + 8] = __float_as_uint(s256);
  ub[(2 * g + 1) * XQ_REC + 8] = uint32_t(sum);
  ub[g * XQ_REC + 9] = __float_as_uint(xsum);
}

// LDS slot of a unit: 64 rows x CH chunks, then the tile's XQ records (up to GEMV_BM rows of 48 chunks)
template <int QT>
constexpr int slot_chunks() {
  return 64 * (Unit<QT>::BYTES / 16) + 48 * GEMV_BM;
}

template <int QT, bool SWIGLU, int D, int M>
__device__ __forceinline__ void gemv_tile(const GemvArgs& a, int e, int s0) {
  constexpr int BY = Unit<QT>::BYTES, CH = BY / 16, NM = SWIGLU ? 2 : 1;
  constexpr int XI = (48 * M + 63) / 64;  // load instructions of the records of a unit
  constexpr int LPU = CH + XI, SLOT = slot_chunks<QT>();
  static_assert((D - 1) * LPU <= 63, "loads in flight beyond vmcnt");
  static_assert(D % NM == 0, "a slot's matrix is fixed");
  static_assert(48 * GEMV_BM % 64 == 0, "record loads fill the slot's record area");
  extern __shared__ u32x4 slab[];  // D slots
  const int lane = threadIdx.x;
  const int n0 = blockIdx.y * 64;
  const int U = a.K / 256, NV = U * NM;

  // this lane's chunk of each load instruction of a unit: weight chunk 64 i + lane of the 64 x CH, record chunk
  // 64 i + lane of the M x 48 (past the last: the last again, landing in the slot's spare record area)
  int32_t off[CH];
#pragma unroll
  for (int i = 0; i < CH; i++) {
    const int q = 64 * i + lane, r = q / CH;
    off[i] = min(n0 + r, a.N - 1) * a.row_bytes + 16 * (q - r * CH);
  }
  const uint8_t* xs[XI];
#pragma unroll
  for (int i = 0; i < XI; i++) {
    const int q = min(64 * i + lane, 48 * M - 1), t = q / 48;
    const int64_t r = a.a_gather ? a.order[s0 + t] / a.topk : s0 + t;
    xs[i] = reinterpret_cast<const uint8_t*>(a.xq + r * xq_row_dwords(a.K)) + 16 * (q - 48 * t);
  }
  const uint8_t* wb[NM];
#pragma unroll
  for (int mtx = 0; mtx < NM; mtx++) wb[mtx] = a.w[mtx] + int64_t(e) * a.expert_bytes;
  float acc[NM][M];
#pragma unroll
  for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
    for (int t = 0; t < M; t++) acc[mtx][t] = 0.0f;

  // unit v (K-range v / NM of matrix v % NM) and its records into slot J = v % D
  auto issue = [&](int v, auto jc) {
    constexpr int J = decltype(jc)::value;
    const int ku = v / NM;
    const uint8_t* src = wb[J % NM] + int64_t(ku) * BY;
    u32x4* dst = slab + J * SLOT;
#pragma unroll
    for (int i = 0; i < CH; i++)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + off[i]),
                                       (__attribute__((address_space(3))) void*)(dst + 64 * i), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < XI; i++)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(xs[i] + ku * (XQ_UNIT * 4)),
                                       (__attribute__((address_space(3))) void*)(dst + 64 * CH + 64 * i), 16, 0, 0);
  };

  static_for<D - 1>([&](auto jc) {
    if (jc.value < NV) issue(jc.value, jc);
  });
  for (int v0 = 0; v0 < NV; v0 += D) {
    static_for<D>([&](auto jc) {
      constexpr int J = decltype(jc)::value;
      const int v = v0 + J;
      if (v >= NV) return;
      if (v + D - 1 < NV) issue(v + D - 1, std::integral_constant<int, (J + D - 1) % D>{});
      // unit v has landed once only the units issued after it are outstanding
      u32x4 w[CH], x[M][3];
      const uint32_t pw = lds_addr(slab + J * SLOT + lane * CH);
      const uint32_t px = lds_addr(slab + J * SLOT + 64 * CH + (lane & 15) * 3);
      const int ahead = min(D - 1, NV - 1 - v);
      if (ahead == 0)
        read_unit<0>(w, x, pw, px);
      else if (D > 1 && ahead == 1)
        read_unit<(D > 1 ? LPU : 0)>(w, x, pw, px);
      else if (D > 2 && ahead == 2)
        read_unit<(D > 2 ? 2 * LPU : 0)>(w, x, pw, px);
      else if (D > 3)
        read_unit<(D > 3 ? 3 * LPU : 0)>(w, x, pw, px);
      static_for<8>([&](auto gc) {
        constexpr int G = decltype(gc)::value;
        uint32_t q[8];
        float d, mn;
        codes<QT, G>(w, q, d, mn);
#pragma unroll
        for (int t = 0; t < M; t++)
          acc[J % NM][t] = group_term<QT, G>(acc[J % NM][t], x[t][G >> 2][G & 3], x[t][2][0], x[t][2][1], q, d, mn);
      });
    });
  }

  if constexpr (SWIGLU) {
    // h = silu(gate) up, quantised to XQ rows of N values (lanes 0..31: one group, 32..63: the next)
    const int UH = a.N / 256;
    const int g = ((n0 & 255) >> 5) + (lane >> 5), j = (lane & 31) >> 2;
#pragma unroll
    for (int t = 0; t < M; t++) {
      const float gv = acc[0][t];
      const float hv[1] = {gv / (1.0f + expf(-gv)) * acc[1][t]};
      int qa[1], qb[1], sum;
      float s256, xsum;
      quant_group<1>(hv, qa, qb, s256, sum, xsum);
      uint32_t pa = uint32_t(qa[0] & 0xFF) << (8 * (lane & 3));
      uint32_t pb = uint32_t(qb[0] & 0xFF) << (8 * (lane & 3));
      pa |= __shfl_xor(pa, 1);
      pb |= __shfl_xor(pb, 1);
      pa |= __shfl_xor(pa, 2);
      pb |= __shfl_xor(pb, 2);
      uint32_t* ub = a.hq + int64_t(s0 + t) * UH * XQ_UNIT + (n0 >> 8) * XQ_UNIT;
      if ((lane & 3) == 0) {
        ub[j * XQ_REC + g] = pa;
        ub[(8 + j) * XQ_REC + g] = pb;
      }
      if ((lane & 31) == 0) put_group_words(ub, g, s256, sum, xsum);
    }
  } else {
    const int n = n0 + lane;
    if (n < a.N)
#pragma unroll
      for (int t = 0; t < M; t++) a.y[int64_t(s0 + t) * a.N + n] = acc[0][t];
  }
}

template <int QT, bool SWIGLU, int D>
__global__ __launch_bounds__(64) void k_gemv(const GemvArgs a) {
  int e = 0, s0, m;
  if (a.tiles) {
    if (int64_t(blockIdx.x) >= *a.n_tiles) return;
    e = a.tiles[2 * blockIdx.x];
    s0 = a.tiles[2 * blockIdx.x + 1];
    m = min(GEMV_BM, a.offsets[e + 1] - s0);
  } else {
    s0 = blockIdx.x * GEMV_BM;
    m = min(GEMV_BM, a.dense_rows - s0);
  }
  static_assert(GEMV_BM == 4, "tile rows");
  switch (m) {
    case 1: gemv_tile<QT, SWIGLU, D, 1>(a, e, s0); break;
    case 2: gemv_tile<QT, SWIGLU, D, 2>(a, e, s0); break;
    case 3: gemv_tile<QT, SWIGLU, D, 3>(a, e, s0); break;
    case 4: gemv_tile<QT, SWIGLU, D, 4>(a, e, s0); break;
    default: break;
  }
}

// one wave per (row, unit): lane l holds values 4 l .. 4 l + 3 of the unit (group l / 8, plane dword l % 8)
template <int XT>
__global__ __launch_bounds__(256) void k_quant(const void* __restrict__ x, int64_t T, int K, uint32_t* __restrict__ xq) {
  const int U = K / 256;
  const int64_t w = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (w >= T * U) return;
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
  quant_group<4>(v, qa, qb, s256, sum, xsum);
  uint32_t pa = 0, pb = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    pa |= uint32_t(qa[i] & 0xFF) << (8 * i);
    pb |= uint32_t(qb[i] & 0xFF) << (8 * i);
  }
  uint32_t* ub = xq + row * (int64_t(U) * XQ_UNIT) + int64_t(u) * XQ_UNIT;
  const int g = lane >> 3, j = lane & 7;
  ub[j * XQ_REC + g] = pa;
  ub[(8 + j) * XQ_REC + g] = pb;
  if (j == 0) put_group_words(ub, g, s256, sum, xsum);
}

template <int QT, bool SWIGLU>
int launch_t(const GemvArgs& a, hipStream_t s) {
  constexpr int D = 2;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + GEMV_BM - 1) / GEMV_BM;
  if (tiles <= 0) return ARTLITE_OK;
  const dim3 grid(unsigned(tiles), unsigned((a.N + 63) / 64)), block(64);
  const size_t lds = size_t(D) * slot_chunks<QT>() * 16;
  k_gemv<QT, SWIGLU, D><<<grid, block, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace

bool gemv_supported(int qtype, int K) {
  return (qtype == ARTLITE_Q4_0 || qtype == ARTLITE_Q8_0 || qtype == ARTLITE_Q4_K) && K > 0 && K % 256 == 0;
}

int launch_gemv(const GemvArgs& a, hipStream_t s) {
  if (!gemv_supported(a.qtype, a.K))
    return fail(ARTLITE_EINVAL, "expert GEMV: weight type %d with K %d (Q4_0 / Q8_0 / Q4_K, K a multiple of 256)",
                a.qtype, a.K);
  if (a.N <= 0 || int64_t(a.N) * a.row_bytes >= (int64_t(1) << 31))
    return fail(ARTLITE_EINVAL, "expert GEMV: %d rows of %d bytes", a.N, a.row_bytes);
  const bool swiglu = a.w[1] != nullptr;
  if (swiglu && (a.N % 256 || !a.hq))
    return fail(ARTLITE_EINVAL, "expert GEMV: SwiGLU width %d is not a multiple of 256", a.N);
  if (!swiglu && !a.y) return fail(ARTLITE_EINVAL, "expert GEMV: no output");
#define ART_DISPATCH(QT) return swiglu ? launch_t<QT, true>(a, s) : launch_t<QT, false>(a, s)
  switch (a.qtype) {
    case ARTLITE_Q4_0: ART_DISPATCH(ARTLITE_Q4_0);
    case ARTLITE_Q8_0: ART_DISPATCH(ARTLITE_Q8_0);
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
      std::memcpy(&s, &ub[(2 * g) * XQ_REC + 8], 4);
      for (int v = 0; v < 32; v++) {
        const int j = v / 4, sh = 8 * (v % 4);
        const int qa = int8_t((ub[j * XQ_REC + g] >> sh) & 0xFFu);
        const int qb = int8_t((ub[(8 + j) * XQ_REC + g] >> sh) & 0xFFu);
        out[u * 256 + 32 * g + v] = s * float(256 * qa + qb);
      }
    }
  }
}

}  // namespace artlite
