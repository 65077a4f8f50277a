// Decode expert products on the VALU, and the XQ activations they read.
//
// A workgroup is one tile of at most GEMV_BM sorted rows of A (tokens for gate / up, pairs for down) of one expert,
// times 64 weight rows (SwiGLU: those rows of gate and of up), as 4 independent waves of 16 rows. A wave streams its
// rows in units of 8 groups of 32 values (Q4_0 / Q4_K: 144 bytes of a row, Q8_0: 272) with global_load_lds_dwordx4
// into one of D LDS slots of its own (consecutive lanes load consecutive 16-byte chunks), D - 1 units ahead. Lane
// (p, r) -- 16-lane row p, lane r in it -- takes row r and groups 2 p, 2 p + 1 of each unit, so four lanes share a
// row and a unit's products of 64 rows are spread over four waves (one wave per SIMD issues VALU at well under half
// rate). The activations come straight into registers, one 16-byte XQ chunk per lane per row of A: DPP
// row_newbcast:j hands every lane of 16-lane row p dword j of its groups' blocks as the broadcast operand of
// v_dot4c_i32_i8, and the per-group words the same way. The four lanes of a row are summed at the end.
//
// Arithmetic of one (row of A, group): A = sum_j dot4(a_j, q_j) and B = C + sum_j dot4(b_j, q_j), exactly in int32,
// with q_j the group's codes as int8 (Q4_0 / Q4_K: nibbles 0..15, Q8_0: the signed bytes) and C the code offset's
// correction (Q4_0: -8 sum(256 a + b), else 0); then acc += (d s / 256) float(256 A + B), which is
// d s sum (q - 8)(a + b / 256) for Q4_0. Q4_K adds -(dmin mn) times the group's dequantised activation sum.
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

// per format: bytes of a row's unit, dwords a lane reads of it (Q4_0 / Q8_0: its two groups; Q4_K: the super-block
// header and the 32-byte run holding its two groups)
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
struct Unit<ARTLITE_Q4_K> {
  static constexpr int BYTES = 144, LW = 12;
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

// After vmcnt(N), the lane's dwords of a unit (at pw; Q4_K: header at pw, its run at pr) and its XQ chunk of each
// of the M rows of A (at px, 1024 bytes apart), and their completion, in one asm block: the compiler would otherwise
// wait for every load in flight before reading LDS (it takes the slots' global_load_lds writes for possible
// producers), and it must not touch the outputs before the final wait.
#define ART_R2(I, J) "ds_read2_b32 %[w" #I "], %[pw] offset0:" #J " offset1:" #J "+1\n\t"
#define ART_R1(I, J) "ds_read_b32 %[w" #I "], %[pw] offset:" #J "*4\n\t"
#define ART_OW2(I) [w##I] "=&v"(w2[I])
#define ART_OW1(I) [w##I] "=&v"(w1)
#define ART_W9 ART_R2(0, 0) ART_R2(1, 2) ART_R2(2, 4) ART_R2(3, 6) ART_R1(4, 8)
#define ART_OW9 ART_OW2(0), ART_OW2(1), ART_OW2(2), ART_OW2(3), ART_OW1(4)
#define ART_W17 \
  ART_R2(0, 0) ART_R2(1, 2) ART_R2(2, 4) ART_R2(3, 6) ART_R2(4, 8) ART_R2(5, 10) ART_R2(6, 12) ART_R2(7, 14) ART_R1(8, 16)
#define ART_OW17 \
  ART_OW2(0), ART_OW2(1), ART_OW2(2), ART_OW2(3), ART_OW2(4), ART_OW2(5), ART_OW2(6), ART_OW2(7), ART_OW1(8)
#define ART_W12                    \
  "ds_read_b128 %[w0], %[pw]\n\t"  \
  "ds_read_b128 %[w1], %[pr]\n\t"  \
  "ds_read_b128 %[w2], %[pr] offset:16\n\t"
#define ART_OW12 [w0] "=&v"(w4[0]), [w1] "=&v"(w4[1]), [w2] "=&v"(w4[2])
#define ART_RX(T) "ds_read_b128 %[x" #T "], %[px] offset:" #T "*1024\n\t"
#define ART_X1 ART_RX(0)
#define ART_X2 ART_X1 ART_RX(1)
#define ART_X3 ART_X2 ART_RX(2)
#define ART_X4 ART_X3 ART_RX(3)
#define ART_OX1 [x0] "=&v"(x[0])
#define ART_OX2 ART_OX1, [x1] "=&v"(x[1])
#define ART_OX3 ART_OX2, [x2] "=&v"(x[2])
#define ART_OX4 ART_OX3, [x3] "=&v"(x[3])
#define ART_READ(WN, MN)                                                                             \
  asm volatile("s_waitcnt vmcnt(%[n])\n\t" ART_W##WN ART_X##MN "s_waitcnt lgkmcnt(0)"              \
               : ART_OW##WN, ART_OX##MN                                                             \
               : [pw] "v"(pw), [pr] "v"(pr), [px] "v"(px), [n] "i"(N))
#define ART_READ_M(WN)         \
  if constexpr (M == 1) ART_READ(WN, 1); \
  if constexpr (M == 2) ART_READ(WN, 2); \
  if constexpr (M == 3) ART_READ(WN, 3); \
  if constexpr (M == 4) ART_READ(WN, 4);
template <int N, int QT, int M>
__device__ __forceinline__ void read_unit(uint32_t (&w)[Unit<QT>::LW], u32x4 (&x)[M], uint32_t pw, uint32_t pr,
                                          uint32_t px) {
  static_assert(N >= 0 && N < 64, "vmcnt");
  constexpr int LW = Unit<QT>::LW;
  if constexpr (LW == 12) {
    u32x4 w4[3];
    ART_READ_M(12)
#pragma unroll
    for (int i = 0; i < 12; i++) w[i] = w4[i >> 2][i & 3];
  } else {
    u32x2 w2[LW / 2];
    uint32_t w1;
    if constexpr (LW == 9) {
      ART_READ_M(9)
    } else {
      ART_READ_M(17)
    }
#pragma unroll
    for (int i = 0; i < LW / 2; i++) w[2 * i] = w2[i][0], w[2 * i + 1] = w2[i][1];
    w[LW - 1] = w1;
  }
}
#undef ART_READ_M
#undef ART_READ
#undef ART_OX4
#undef ART_OX3
#undef ART_OX2
#undef ART_OX1
#undef ART_X4
#undef ART_X3
#undef ART_X2
#undef ART_X1
#undef ART_RX
#undef ART_OW12
#undef ART_W12
#undef ART_OW17
#undef ART_W17
#undef ART_OW9
#undef ART_W9
#undef ART_OW1
#undef ART_OW2
#undef ART_R1
#undef ART_R2

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N));
}

// Codes of the lane's group H (0, 1) as 8 dwords of int8 (q[j]: values 4 j .. 4 j + 3 of the group), its scale d
// (Q4_K: d sc) and Q4_K's dmin mn. g: the group's index in the unit (Q4_K's scales).
template <int QT, int H>
__device__ __forceinline__ void codes(const uint32_t (&w)[Unit<QT>::LW], int g, uint32_t (&q)[8], float& d,
                                      float& mn) {
  if constexpr (QT == ARTLITE_Q4_0 || QT == ARTLITE_Q8_0) {
    // Q4_0: 18 bytes at 18 H: fp16 d, then 16 bytes whose low nibbles are values 0..15, high nibbles 16..31;
    // Q8_0: 34 bytes at 34 H: fp16 d, then 32 signed bytes in value order
    constexpr int o = (QT == ARTLITE_Q4_0 ? 18 : 34) * H;
    constexpr int NQ = QT == ARTLITE_Q4_0 ? 4 : 8;
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
      } else {
        q[j] = v;
      }
    }
    d = o % 4 == 0 ? h2f(w[o / 4] & 0xFFFFu) : h2f(w[(o - 2) / 4] >> 16);
    mn = 0.0f;
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
#pragma unroll
    for (int j = 0; j < 8; j++) q[j] = H ? (w[4 + j] >> 4) & 0x0F0F0F0Fu : w[4 + j] & 0x0F0F0F0Fu;
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
  } else if constexpr (QT == ARTLITE_Q8_0) {
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
#undef ART_QIN

// LDS of a workgroup: each wave's D slots of 16 rows x BYTES, two record slots (GEMV_BM x 1 KB), then h of the
// tile (GEMV_BM x 64 fp32)
template <int QT, int D>
constexpr size_t gemv_lds() {
  return size_t(4) * D * 16 * Unit<QT>::BYTES + 2 * GEMV_BM * 1024 + GEMV_BM * 64 * 4;
}

// choose among waits vmcnt(N0), (N0 + NI), ... by a small runtime count c (< 4)
template <int N0, int NI, int CMAX>
__device__ __forceinline__ void wait_vm_c(int c) {
  if (c <= 0)
    wait_vm<N0>();
  else if (c == 1 || CMAX < 2)
    wait_vm<(CMAX >= 1 ? N0 + NI : N0)>();
  else if (c == 2 || CMAX < 3)
    wait_vm<(CMAX >= 2 ? N0 + 2 * NI : N0)>();
  else
    wait_vm<(CMAX >= 3 ? N0 + 3 * NI : N0)>();
}

template <int QT, bool SWIGLU, int D, int M>
__device__ __forceinline__ void gemv_tile(const GemvArgs& a, int e, int s0) {
  constexpr int BY = Unit<QT>::BYTES, CH = BY / 16, LW = Unit<QT>::LW, NM = SWIGLU ? 2 : 1;
  constexpr int WCH = 16 * CH;               // chunks of a wave's unit
  constexpr int NI = (WCH + 63) / 64;         // its load instructions (the last for LAST lanes)
  constexpr int LAST = WCH - 64 * (NI - 1);
  static_assert((D - 1) * NI + D * M < 64, "loads in flight beyond vmcnt");
  static_assert(D % NM == 0, "slots per matrix");
  extern __shared__ u32x4 slab[];
  // (wv through readfirstlane: wave-uniform to the compiler, so the branches on it are scalar)
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, p = lane >> 4, r = lane & 15;
  u32x4* my = slab + wv * D * WCH;
  u32x4* xslot = slab + 4 * D * WCH;  // 2 x GEMV_BM x 64 chunks
  float* hbuf = reinterpret_cast<float*>(xslot + 2 * GEMV_BM * 64);
  // plain products: a.rpw blocks of 64 rows, one after the other (SwiGLU: one)
  const int rpw = SWIGLU ? 1 : a.rpw;
  const int n0 = blockIdx.y * 64 * rpw, nw = n0 + 16 * wv;
  const int U = a.K / 256, NV = U * NM;                      // units per block of rows
  const int NVt = min(rpw, (a.N - n0 + 63) / 64) * NV, KKt = NVt / NM;  // units, K-units in all

  // the lane's chunk of each load instruction of a unit (chunk 64 i + lane of the wave's 16 x CH): its row and
  // column offset
  int rw[NI], cw[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int q = min(64 * i + lane, WCH - 1), row = q / CH;
    rw[i] = row;
    cw[i] = 16 * (q - row * CH);
  }
  const uint8_t* wb[NM];
#pragma unroll
  for (int mx = 0; mx < NM; mx++) wb[mx] = a.w[mx] + int64_t(e) * a.expert_bytes;
  // wave 0 loads the tile's record chunks of each K-unit (row t: one instruction, lane i -> chunk i)
  const uint8_t* xr[M];
  if (wv == 0)
#pragma unroll
    for (int t = 0; t < M; t++) {
      const int64_t ar = a.a_gather ? a.order[s0 + t] / a.topk : s0 + t;
      xr[t] = reinterpret_cast<const uint8_t*>(a.xq + ar * xq_row_dwords(a.K)) + 16 * lane;
    }
  auto issue_x = [&](int kk) {  // (wave 0; K-unit kk of the sequence (past the last: the last again, into the idle
                                //  slot), K-range kk % U)
    u32x4* dst = xslot + (kk & 1) * GEMV_BM * 64;
    const int ku = min(kk, KKt - 1) % U;
#pragma unroll
    for (int t = 0; t < M; t++)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(xr[t] + ku * (XQ_UNIT * 4)),
                                       (__attribute__((address_space(3))) void*)(dst + 64 * t), 16, 0, 0);
  };
  // the weights of unit v (K-range v / NM of matrix v % NM) into this wave's slot v % D
  auto issue_w = [&](int v, auto mtx_c) {
    constexpr int MX = decltype(mtx_c)::value;
    const int rb = v / NV;
    const uint8_t* src = wb[MX] + int64_t((v - rb * NV) / NM) * BY;
    u32x4* dst = my + (v % D) * WCH;
#pragma unroll
    for (int i = 0; i < NI; i++)
      if (i < NI - 1 || lane < LAST)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(
                                             src + min(nw + 64 * rb + rw[i], a.N - 1) * a.row_bytes + cw[i]),
                                         (__attribute__((address_space(3))) void*)(dst + 64 * i), 16, 0, 0);
  };

  // the lane's read addresses
  const uint32_t wbase = lds_addr(my), xbase = lds_addr(xslot) + 16 * lane;
  const uint32_t o_w = r * BY + (QT == ARTLITE_Q4_K ? 0 : (QT == ARTLITE_Q4_0 ? 36 : 68) * p);
  const uint32_t o_r = r * BY + 16 + 32 * p;  // (Q4_K)

  float acc[NM][M];
#pragma unroll
  for (int mx = 0; mx < NM; mx++)
#pragma unroll
    for (int t = 0; t < M; t++) acc[mx][t] = 0.0f;

  // Weights D - 1 units ahead in each wave's own slots (a slot refilled right after the step that read it); the
  // records of K-unit ku + 1 issued by wave 0 at ku's first step, right after the barrier that opens it: every wave is
  // then past K-unit ku - 1, whose record slot it takes, and sees K-unit ku's records, which wave 0 waited for just
  // before. The loop is unrolled by NM, which fixes each step's matrix.
  if (wv == 0) issue_x(0);
  for (int v = 0; v < D - 1 && v < NVt; v++) {
    if (NM == 1 || v % NM == 0)
      issue_w(v, std::integral_constant<int, 0>{});
    else
      issue_w(v, std::integral_constant<int, NM - 1>{});
  }
  for (int v0 = 0; v0 < NVt; v0 += NM) {
    static_for<NM>([&](auto jc) {
      constexpr int MX = decltype(jc)::value;
      const int v = v0 + MX, kk = v0 / NM;
      if (v >= NVt) return;
      if (MX == 0) {
        // wave 0: K-unit kk's records (issued before the weights of the units since its issue that were issued)
        if (wv == 0) {
          if (kk == 0)
            wait_vm_c<0, NI, 3>(min(D - 1, NVt));
          else
            wait_vm_c<0, NI, NM>(min(NM, max(0, NVt - D + 1 - (kk - 1) * NM)));
        }
        __builtin_amdgcn_s_barrier();
        if (wv == 0) issue_x(kk + 1);
      }
      if (v + D - 1 < NVt) issue_w(v + D - 1, std::integral_constant<int, (MX + D - 1) % NM>{});
      // unit v's weights have landed once only the loads issued after them are outstanding: the weights of the
      // `ahead` units after it, and (wave 0) the records issued at the K-unit starts among steps v - D + 2 .. v
      const int ahead = min(D - 1, NVt - 1 - v);
      int nx = 0;
      if (wv == 0)
        for (int j = max(0, v - D + 2); j <= v; j++) nx += j % NM == 0;
      uint32_t w[LW];
      u32x4 x[M];
      const uint32_t sw = wbase + (v % D) * WCH * 16, px = xbase + (kk & 1) * GEMV_BM * 1024;
      // (the count in one immediate: nx rows of M records plus ahead x NI)
      const int n = ahead * NI + nx * M;
      static_for<(D - 1) * NI + D * M + 1>([&](auto nc) {
        constexpr int NN = decltype(nc)::value;
        if (n == NN) read_unit<NN, QT, M>(w, x, sw + o_w, sw + o_r, px);
      });
      static_for<2>([&](auto hc) {
        constexpr int H = decltype(hc)::value;
        uint32_t q[8];
        float d, mn;
        codes<QT, H>(w, 2 * p + H, q, d, mn);
#pragma unroll
        for (int t = 0; t < M; t++) acc[MX][t] = group_term<QT, H>(acc[MX][t], x[t][H], x[t][2], x[t][3], q, d, mn);
      });
      if constexpr (!SWIGLU) {
        if (v % NV == NV - 1) {  // a block of rows done: the four lanes of a row summed, then y
          const int rb = v / NV, n = nw + 64 * rb + r;
#pragma unroll
          for (int t = 0; t < M; t++) {
            float y = acc[0][t];
            y += __shfl_xor(y, 16);
            y += __shfl_xor(y, 32);
            if (p == 0 && n < a.N) a.y[int64_t(s0 + t) * a.N + n] = y;
            acc[0][t] = 0.0f;
          }
        }
      }
    });
  }

  if constexpr (SWIGLU) {
    // the four lanes of a row: their groups' sums
#pragma unroll
    for (int mx = 0; mx < NM; mx++)
#pragma unroll
      for (int t = 0; t < M; t++) {
        acc[mx][t] += __shfl_xor(acc[mx][t], 16);
        acc[mx][t] += __shfl_xor(acc[mx][t], 32);
      }
    // h = silu(gate) up of the 64 rows, then quantised by wave 0 into XQ rows of N values (lanes 0..31: one group,
    // 32..63: the next)
    if (p == 0)
#pragma unroll
      for (int t = 0; t < M; t++) {
        const float gv = acc[0][t];
        hbuf[t * 64 + 16 * wv + r] = gv / (1.0f + expf(-gv)) * acc[1][t];
      }
    __syncthreads();
    if (wv) return;
    const int UH = a.N / 256;
    const int g = ((n0 & 255) >> 5) + (lane >> 5), v = lane & 31;
#pragma unroll
    for (int t = 0; t < M; t++) {
      const float hv[1] = {hbuf[t * 64 + lane]};
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
      if ((v & 3) == 0) {
        ub[xq_block(g, v >> 2)] = pa;
        ub[xq_block(g, 8 + (v >> 2))] = pb;
      }
      if (v < 16) xq_put_word(ub, g, v, s256, sum, xsum);
    }
  }
}

template <int QT, bool SWIGLU, int D>
__global__ __launch_bounds__(256) void k_gemv(const GemvArgs a) {
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

// one wave per (row, unit) of x
template <int XT>
__global__ __launch_bounds__(256) void k_quant(const void* __restrict__ x, int64_t T, int K, uint32_t* __restrict__ xq) {
  const int64_t w = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  if (w < T * (K / 256)) xq_quant_unit<XT>(x, w, K, xq, threadIdx.x & 63);
}

template <int QT, bool SWIGLU>
int launch_t(const GemvArgs& a, hipStream_t s) {
  constexpr int D = 2;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + GEMV_BM - 1) / GEMV_BM;
  if (tiles <= 0) return ARTLITE_OK;
  const int rpw = SWIGLU ? 1 : a.rpw;
  const dim3 grid(unsigned(tiles), unsigned((a.N + 64 * rpw - 1) / (64 * rpw))), block(256);
  k_gemv<QT, SWIGLU, D><<<grid, block, gemv_lds<QT, D>(), s>>>(a);
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
  GemvArgs b = a;
  b.rpw = std::max(1, a.rpw);
#define ART_DISPATCH(QT) return swiglu ? launch_t<QT, true>(b, s) : launch_t<QT, false>(b, s)
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
