// The experts' products over raw GGUF blocks on gfx950's MFMA, and the combine: the MFMA decode tiles (bf16, for
// batches between the GEMV's and the prefill's; every Q4_K product), the prefill tiles (fp16, below), the combine.
//
// MFMA decode tiles. Exactness of the operands: a block's integer codes are exact in bf16 -- Q4_0 as 128 + q and Q4_K as 128 + q
// (a byte 0x43 above the nibble: bf16 128 + q), Q8_0 as 128 + q through an unsigned byte conversion -- and bf16
// activations are exact; fp32 activations and the SwiGLU intermediate are split into bf16 hi + lo planes. One MFMA
// per 32-value group gives S = sum (128 + q) x exactly rounded once into fp32, its C input pre-loaded with
// -offset sum x (sum x from an MFMA against a ones operand, so the offset leaves S exactly sum (q - 8) x, or
// sum q x). The group's fp16 scale is applied in fp32: acc += d S (Q4_K: acc += (d sc) S - (dmin mn) sum x).
//
// Decode tiling (k_gemm_decode): a workgroup is one tile of DECODE_BM sorted rows of one expert (tokens for gate /
// up, pairs for down) times 4 waves x ROWS weight rows. Each wave streams its own rows' blocks, a stage of one
// ~144-byte run per row at a time: dwordx4 loads of the 16-byte-aligned cover of the run into registers (the next
// stage's loads in flight while the current stage computes), then into the wave's LDS slot, from which each lane
// decodes its row's 8 codes of a group. MFMA layout (16x16x32): lane l holds A row l % 16 and B column l % 16,
// both with K values 8 (l / 16) .. + 8; C column l % 16, rows 4 (l / 16) .. + 4. A = activations (tokens / pairs),
// B = weights (the lane's own row), so a lane's four outputs share its row's scale.
#include "experts.h"

namespace artlite {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}

__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) {
  uint16_t v;
  __builtin_memcpy(&v, p, 2);
  return v;
}

__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }

// eight nibbles (the bytes of v0, v1, each < 16) -> the B operand's four dwords of bf16 128 + q
__device__ __forceinline__ u32x4 nib8(uint32_t v0, uint32_t v1) {
  return u32x4{__builtin_amdgcn_perm(0x43434343u, v0, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v0, 0x04030402u),
               __builtin_amdgcn_perm(0x43434343u, v1, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v1, 0x04030402u)};
}

// two bf16 of the unsigned bytes 2 j, 2 j + 1 of v (exact: < 256)
__device__ __forceinline__ uint32_t byte2(uint32_t v, int j) {
  const uint32_t f0 = __float_as_uint(float((v >> (16 * j)) & 0xFFu));
  const uint32_t f1 = __float_as_uint(float((v >> (16 * j + 8)) & 0xFFu));
  return __builtin_amdgcn_perm(f1, f0, 0x07060302u);
}

// eight unsigned bytes -> the B operand's four dwords of bf16
__device__ __forceinline__ u32x4 byte8(uint32_t v0, uint32_t v1) {
  return u32x4{byte2(v0, 0), byte2(v0, 1), byte2(v1, 0), byte2(v1, 1)};
}

// Per format: a block's bytes and 32-value groups; the groups of one K-range (a stage: ~300..600 bytes of each row,
// so a 16-row stage is 16 long runs; a straddled cache line is read again by the next range of the same wave, from
// L2) and its bytes; the offset of the codes' bf16 encoding (the B operand holds 128 + c for a code byte c, or
// 128 + IQ4[c], so OFF = 128 + the format's zero point); whether the format has a min term (w = s q - m: Q4_1,
// Q4_K, Q5_K); whether its scales cover 16 values (Q3_K, Q6_K: one MFMA per half of a group, each with the other
// half's B lanes zero).
template <int BB, int GPB_, int KR_, int OFF_, bool MIN_ = false, bool SUB16_ = false>
struct FmtT {
  static constexpr int BLOCK_BYTES = BB;
  static constexpr int GPB = GPB_;  // 32-value groups per block (1 or 8)
  static constexpr int GROUP_BYTES = GPB_ == 1 ? BB : 0;  // (32-value blocks only)
  static constexpr int KR = KR_;
  static constexpr int RUN = KR_ / GPB_ * BB;  // bytes of a row's K-range
  static constexpr float OFF = float(OFF_);
  static constexpr bool MIN = MIN_;
  static constexpr bool SUB16 = SUB16_;
  static_assert(KR_ % GPB_ == 0, "K-ranges of whole blocks");
};
template <int QT>
struct Fmt;
template <>
struct Fmt<ARTLITE_Q4_0> : FmtT<18, 1, 32, 136> {};  // (128 + q) - (q - 8)
template <>
struct Fmt<ARTLITE_Q4_1> : FmtT<20, 1, 24, 128, true> {};
template <>
struct Fmt<ARTLITE_Q8_0> : FmtT<34, 1, 16, 128> {};  // (q + 128 through an unsigned byte)
template <>
struct Fmt<ARTLITE_Q3_K> : FmtT<112, 8, 32, 132, false, true> {};  // (128 + q) - (q - 4)
template <>
struct Fmt<ARTLITE_Q4_K> : FmtT<144, 8, 32, 128, true> {};
template <>
struct Fmt<ARTLITE_Q5_K> : FmtT<176, 8, 24, 128, true> {};
template <>
struct Fmt<ARTLITE_Q6_K> : FmtT<224, 8, 16, 160, false, true> {};  // (128 + q) - (q - 32); the layer's padded blocks
template <>
struct Fmt<ARTLITE_IQ4_NL> : FmtT<18, 1, 32, 128> {};
template <>
struct Fmt<ARTLITE_IQ4_XS> : FmtT<144, 8, 32, 128> {};  // (the layer's padded blocks)

// the 16-byte chunks of a 16-row stage: the aligned cover of each row's run; a row's LDS slot is an odd number of
// 16-byte units, so the 16 rows' same-offset dwords fall in 16 different banks
template <int QT>
struct Stage {
  static constexpr int BYTES = Fmt<QT>::RUN;
  static constexpr int CPR = (BYTES + 15 + 15) / 16;
  static constexpr int SLOT = 16 * (CPR | 1);
  static constexpr int LOADS = (16 * CPR + WAVE - 1) / WAVE;  // per lane
  static_assert(16 * CPR <= WEIGHT_TAIL, "a K-range's cover stays within a weight tensor's tail");
};

// four codes (bytes < 16) -> the bytes 128 + IQ4[code] (the int8 values with the top bit flipped)
__device__ __forceinline__ uint32_t iq4_bytes(uint32_t c) { return iq4_int8(c) ^ 0x80808080u; }

// Q4_K / Q5_K's 6-bit scale and min of group g from the 12 bytes at s6
__device__ __forceinline__ void k_scale_min(const uint8_t* s6, int g, int& q6, int& m6) {
  q6 = g < 4 ? s6[g] & 63 : (s6[8 + g - 4] & 15) | ((s6[g - 4] >> 6) << 4);
  m6 = g < 4 ? s6[4 + g] & 63 : (s6[8 + g - 4] >> 4) | ((s6[4 + g - 4] >> 6) << 4);
}

// Q3_K's scale of sub-block sb (of 16), minus 32, from the 12 bytes at s
__device__ __forceinline__ int q3k_scale(const uint8_t* s, int sb) {
  const int lo = sb < 8 ? s[sb] & 15 : s[sb - 8] >> 4, hi = (s[8 + (sb & 3)] >> (2 * (sb >> 2))) & 3;
  return (lo | (hi << 4)) - 32;
}

// B operand of group gl of a row's run (row: its first byte in LDS) for lane group lg (values 8 lg .. + 8 of the
// group): 8 codes as 4 dwords of bf16, and the scales: sc (the whole group's, or SUB16: its first half's, with sc2
// the second half's) and, for the formats with a min, mn with w = sc q - mn (Q4_1's w = d q + m: mn = -m)
template <int QT>
__device__ __forceinline__ u32x4 b_operand(const uint8_t* row, int gl, int lg, float& sc, float& mn, float& sc2) {
  using F = Fmt<QT>;
  const uint8_t* blk = row + F::BLOCK_BYTES * (gl / F::GPB);
  const int g = gl % F::GPB;
  if constexpr (QT == ARTLITE_Q4_0 || QT == ARTLITE_Q4_1 || QT == ARTLITE_IQ4_NL) {
    constexpr int QS = QT == ARTLITE_Q4_1 ? 4 : 2;
    sc = h2f(lds_u16(blk));
    if constexpr (QT == ARTLITE_Q4_1) mn = -h2f(lds_u16(blk + 2));
    const int sh = 4 * (lg >> 1);
    const uint32_t u0 = (lds_u32(blk + QS + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
    const uint32_t u1 = (lds_u32(blk + QS + 4 + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
    if constexpr (QT == ARTLITE_IQ4_NL) return byte8(iq4_bytes(u0), iq4_bytes(u1));
    return nib8(u0, u1);
  } else if constexpr (QT == ARTLITE_Q8_0) {
    sc = h2f(lds_u16(blk));
    return byte8(lds_u32(blk + 2 + 8 * lg) ^ 0x80808080u, lds_u32(blk + 6 + 8 * lg) ^ 0x80808080u);
  } else if constexpr (QT == ARTLITE_Q4_K || QT == ARTLITE_Q5_K) {  // group g of the super-block
    int q6, m6;
    k_scale_min(blk + 4, g, q6, m6);
    sc = __fmul_rn(h2f(lds_u16(blk)), float(q6));
    mn = __fmul_rn(h2f(lds_u16(blk + 2)), float(m6));
    const uint8_t* qs = blk + (QT == ARTLITE_Q5_K ? 48 : 16) + 32 * (g >> 1) + 8 * lg;
    const int sh = 4 * (g & 1);
    uint32_t u0 = (lds_u32(qs) >> sh) & 0x0F0F0F0Fu, u1 = (lds_u32(qs + 4) >> sh) & 0x0F0F0F0Fu;
    if constexpr (QT == ARTLITE_Q5_K) {  // bit g of qh[l] (at 16) is the code's bit 4
      u0 |= ((lds_u32(blk + 16 + 8 * lg) >> g) & 0x01010101u) << 4;
      u1 |= ((lds_u32(blk + 20 + 8 * lg) >> g) & 0x01010101u) << 4;
    }
    return nib8(u0, u1);
  } else if constexpr (QT == ARTLITE_Q6_K) {  // group g = 4 h + jj: value l at ql[64 h + 32 (jj % 2) + l], qh[32 h + l]
    const int h = g >> 2, jj = g & 3;
    const float d = h2f(lds_u16(blk + 208));
    sc = __fmul_rn(float(int8_t(blk[192 + 2 * g])), d);
    sc2 = __fmul_rn(float(int8_t(blk[193 + 2 * g])), d);
    const uint8_t *ql = blk + 64 * h + 32 * (jj & 1) + 8 * lg, *qh = blk + 128 + 32 * h + 8 * lg;
    const int sh = jj < 2 ? 0 : 4;
    const uint32_t u0 = ((lds_u32(ql) >> sh) & 0x0F0F0F0Fu) | (((lds_u32(qh) >> (2 * jj)) & 0x03030303u) << 4);
    const uint32_t u1 = ((lds_u32(ql + 4) >> sh) & 0x0F0F0F0Fu) | (((lds_u32(qh + 4) >> (2 * jj)) & 0x03030303u) << 4);
    return nib8(u0, u1);
  } else if constexpr (QT == ARTLITE_Q3_K) {  // group g = 4 n + j: value 16 h + l at qs[32 n + 16 h + l], hm[16 h + l]
    const int n = g >> 2, j = g & 3;
    const float d = h2f(lds_u16(blk + 108));
    sc = __fmul_rn(d, float(q3k_scale(blk + 96, 2 * g)));
    sc2 = __fmul_rn(d, float(q3k_scale(blk + 96, 2 * g + 1)));
    const uint8_t *qs = blk + 32 + 32 * n + 8 * lg, *hm = blk + 8 * lg;
    const int hb = 4 * n + j;
    const uint32_t u0 = ((lds_u32(qs) >> (2 * j)) & 0x03030303u) | (((lds_u32(hm) >> hb) & 0x01010101u) << 2);
    const uint32_t u1 = ((lds_u32(qs + 4) >> (2 * j)) & 0x03030303u) | (((lds_u32(hm + 4) >> hb) & 0x01010101u) << 2);
    return nib8(u0, u1);
  } else {  // IQ4_XS (a layer's 144-byte block: the 8-byte header padded to 16): group g's codes at 16 + 16 g, its
            // scale d (ls - 32)
    const int ls = ((blk[4 + g / 2] >> (4 * (g & 1))) & 15) | (((int(lds_u16(blk + 2)) >> (2 * g)) & 3) << 4);
    sc = __fmul_rn(h2f(lds_u16(blk)), float(ls - 32));
    const uint8_t* qs = blk + 16 + 16 * g + 8 * (lg & 1);
    const int sh = 4 * (lg >> 1);
    return byte8(iq4_bytes((lds_u32(qs) >> sh) & 0x0F0F0F0Fu), iq4_bytes((lds_u32(qs + 4) >> sh) & 0x0F0F0F0Fu));
  }
}

// One 16-row block's products over groups [0, gn) of its K-range (rows at rowp in LDS; this lane's A row at arow
// in LDS; gsum: -OFF times the A sums of each group, or SUB16 of each half group), ni scale FMAs per group (the
// lane's output rows that hold tokens).
template <int QT, int AP, int KR, bool FULL>
__device__ __forceinline__ f32x4 block_products(f32x4 acc, const uint8_t* rowp, const uint8_t* arow, int a_plane,
                                                const float (*gsum)[16], int g0, int gn, int lg, int ni) {
  using F = Fmt<QT>;
#pragma unroll 8
  for (int gl = 0; gl < (FULL ? KR : gn); gl++) {
    const int g = g0 + gl;
    const u32x4 ahi = *reinterpret_cast<const u32x4*>(arow + 64 * g);
    float sc, mn = 0.0f, sc2 = 0.0f;
    const u32x4 b = b_operand<QT>(rowp, gl, lg, sc, mn, sc2);
    if constexpr (!F::SUB16) {
      const f32x4 cin = *reinterpret_cast<const f32x4*>(&gsum[g][4 * lg]);
      f32x4 p = mfma(ahi, b, cin);
      if (AP == 2) p = mfma(*reinterpret_cast<const u32x4*>(arow + a_plane + 64 * g), b, p);
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (i < ni) {
          acc[i] = __builtin_fmaf(sc, p[i], acc[i]);
          if (F::MIN) acc[i] = __builtin_fmaf(mn, cin[i] * (1.0f / F::OFF), acc[i]);
        }
    } else {  // lane groups 0, 1 hold the group's first 16 values, 2, 3 its second 16
      const u32x4 zero{0, 0, 0, 0};
      const u32x4 b0 = lg < 2 ? b : zero, b1 = lg < 2 ? zero : b;
      f32x4 p0 = mfma(ahi, b0, *reinterpret_cast<const f32x4*>(&gsum[2 * g][4 * lg]));
      f32x4 p1 = mfma(ahi, b1, *reinterpret_cast<const f32x4*>(&gsum[2 * g + 1][4 * lg]));
      if (AP == 2) {
        const u32x4 alo = *reinterpret_cast<const u32x4*>(arow + a_plane + 64 * g);
        p0 = mfma(alo, b0, p0);
        p1 = mfma(alo, b1, p1);
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (i < ni) acc[i] = __builtin_fmaf(sc2, p1[i], __builtin_fmaf(sc, p0[i], acc[i]));
    }
  }
  return acc;
}

// MFMA row of tile token t (and back): token t in row 4 (t % 4) + t / 4, so a lane's output i = 0 holds tokens
// 0 .. 3 across its four lane groups and output i = 1 tokens 4 .. 7: ceil(tokens / 4) scale FMAs per group
__device__ __forceinline__ int token_of_row(int m) { return 4 * (m % 4) + m / 4; }

// Decode kernel: a workgroup is one tile of DECODE_BM sorted rows of one expert (tokens for gate / up, pairs for
// down) times RB weight rows per matrix. The tile's A rows (its valid ones, all of K; both planes when A is split)
// are staged in LDS once, with the group sums that correct the codes' offset. SwiGLU: waves 0, 1 stream gate rows,
// waves 2, 3 the same up rows (h is formed after an exchange through LDS); plain: 4 different 16-row blocks. A wave
// takes BLK 16-row blocks, each in K-ranges of Fmt::KR groups (units); two units' chunks are in flight in registers
// while the current one computes from the wave's LDS slot, and no other load is issued during the products.
template <int QT, bool SWIGLU, int AP, int BLK>
__global__ __launch_bounds__(256) void k_gemm_decode(const GemmArgs a) {
  using F = Fmt<QT>;
  using S = Stage<QT>;
  constexpr int WPM = SWIGLU ? 2 : 4;  // waves per matrix
  constexpr int RB = 16 * WPM * BLK;   // rows per matrix per workgroup
  static_assert(BLK == 1 || BLK == 2, "blocks per wave");
  static_assert(DECODE_BM <= 16, "tile rows");
  const int ng = a.K / 32;
  const int a_plane = a.K * 2;               // bytes of one plane of a staged A row
  const int arow_bytes = a_plane * AP + 16;  // (padded: the 16 lanes' rows fall in 16 bank groups)
  constexpr int NSUM = F::SUB16 ? 2 : 1;     // A sums per group (SUB16: per half)
  // LDS: the waves' slots (4 x 16 rows) | the tile's A rows | A sums [NSUM ng][16] (by MFMA row) | up accumulators
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* as = lds + 4 * 16 * S::SLOT;
  float(*gsum)[16] = reinterpret_cast<float(*)[16]>(as + DECODE_BM * arow_bytes);
  f32x4* xch = reinterpret_cast<f32x4*>(as + DECODE_BM * arow_bytes + NSUM * ng * 16 * 4);

  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE, lg = lane >> 4, lr = lane & 15;
  int e = 0, s0, m_valid;
  if (a.tiles) {
    if (int64_t(blockIdx.x) >= *a.n_tiles) return;
    e = a.tiles[2 * blockIdx.x];
    s0 = a.tiles[2 * blockIdx.x + 1];
    m_valid = min(a.bm, a.offsets[e + 1] - s0);
  } else {
    s0 = blockIdx.x * DECODE_BM;
    m_valid = min(DECODE_BM, a.dense_rows - s0);
  }
  const int mtx = SWIGLU ? wv / 2 : 0;
  const uint8_t* wbase = (mtx ? a.w[1] : a.w[0]) + e * a.expert_bytes;
  const int ns = (ng + F::KR - 1) / F::KR;  // K-ranges per block
  const int sub = SWIGLU ? wv % 2 : wv;
  const int n0 = blockIdx.y * RB;
  const int units = BLK * ns;
  uint8_t* my = lds + wv * 16 * S::SLOT;

  u32x4 wa[S::LOADS], wb[S::LOADS];  // (two units in flight)
  auto load_unit = [&](int u, u32x4(&w)[S::LOADS]) {
    const int j = u / ns, kr = u % ns;
    const int r0 = n0 + 16 * (sub + WPM * j);
    const int64_t koff = int64_t(kr) * F::RUN;
#pragma unroll
    for (int i = 0; i < S::LOADS; i++) {
      const int q = min(lane + WAVE * i, 16 * S::CPR - 1);
      const int r = min(r0 + q / S::CPR, a.N - 1);
      const int64_t o = ((int64_t(r) * a.row_bytes + koff) & ~int64_t(15)) + 16 * (q % S::CPR);
      w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wbase + o));
    }
  };
  auto store_unit = [&](const u32x4(&w)[S::LOADS]) {
#pragma unroll
    for (int i = 0; i < S::LOADS; i++) {
      const int q = min(lane + WAVE * i, 16 * S::CPR - 1);
      *reinterpret_cast<u32x4*>(my + (q / S::CPR) * S::SLOT + 16 * (q % S::CPR)) = w[i];
    }
  };
  load_unit(0, wa);
  if (units > 1) load_unit(1, wb);

  // stage the tile's valid A rows: row t = [hi plane (K bf16) | lo plane | pad]
  {
    const int per_row = a.K / 8;  // 16-byte pieces per plane
    for (int i = threadIdx.x; i < m_valid * AP * per_row; i += 256) {
      const int t = i / (AP * per_row), rest = i % (AP * per_row), pl = rest / per_row, c = rest % per_row;
      const int64_t r = a.a_gather ? int64_t(a.order[s0 + t]) / a.topk : int64_t(s0 + t);
      const uint16_t* src = (pl ? a.a_lo : a.a_hi) + r * a.K + 8 * c;
      *reinterpret_cast<u32x4*>(as + t * arow_bytes + pl * a_plane + 16 * c) = *reinterpret_cast<const u32x4*>(src);
    }
  }
  __syncthreads();
  // A sums by MFMA row m: gsum[g][m] = -OFF sum over group g (SUB16: half group g) of A[token_of_row(m)] (zero
  // past the tile)
  for (int i = threadIdx.x; i < NSUM * ng * 16; i += 256) {
    const int g = i / 16, m = i % 16, t = token_of_row(m);
    float sum = 0.0f;
    if (t < m_valid)
#pragma unroll
      for (int pl = 0; pl < AP; pl++) {
        const u32x4* p = reinterpret_cast<const u32x4*>(as + t * arow_bytes + pl * a_plane + 64 / NSUM * g);
#pragma unroll
        for (int j = 0; j < 4 / NSUM; j++) {
          const u32x4 v = p[j];
#pragma unroll
          for (int q = 0; q < 4; q++) sum += bf16_to_f32(v[q] & 0xFFFFu) + bf16_to_f32(v[q] >> 16);
        }
      }
    gsum[g][m] = -F::OFF * sum;
  }
  __syncthreads();

  // this lane's A row: the token of MFMA row lr (rows without a token repeat token 0: they only feed outputs that
  // are never stored, since MFMA output row m depends on A row m alone)
  const int tl = token_of_row(lr);
  const uint8_t* arow = as + (tl < m_valid ? tl : 0) * arow_bytes + 16 * lg;
  const int ni = (m_valid + 3) / 4;  // outputs per lane that hold tokens

  f32x4 acc[BLK];
#pragma unroll
  for (int j = 0; j < BLK; j++) acc[j] = f32x4{0, 0, 0, 0};
  for (int u = 0; u < units; u++) {
    const int j = u / ns, kr = u % ns;
    // this unit's chunks: wa (even units) or wb (odd); then the unit two ahead into the freed registers
    __builtin_amdgcn_wave_barrier();
    if (u & 1) {
      store_unit(wb);
      if (u + 2 < units) load_unit(u + 2, wb);
    } else {
      store_unit(wa);
      if (u + 2 < units) load_unit(u + 2, wa);
    }
    __builtin_amdgcn_wave_barrier();
    const int r = min(n0 + 16 * (sub + WPM * j) + lr, a.N - 1);
    const uint8_t* rowp =
        my + lr * S::SLOT + ((int64_t(r) * a.row_bytes + int64_t(kr) * F::RUN) & 15);
    const int g0 = kr * F::KR, gn = min(F::KR, ng - g0);
    f32x4 accj = (BLK > 1 && j) ? acc[BLK - 1] : acc[0];
    if (gn == F::KR)
      accj = block_products<QT, AP, F::KR, true>(accj, rowp, arow, a_plane, gsum, g0, gn, lg, ni);
    else
      accj = block_products<QT, AP, F::KR, false>(accj, rowp, arow, a_plane, gsum, g0, gn, lg, ni);
    if (BLK > 1 && j)
      acc[BLK - 1] = accj;
    else
      acc[0] = accj;
  }

  // epilogue: lane output i of block j holds token 4 i + lg of the tile, column n0 + 16 (sub + WPM j) + lr
  if (SWIGLU) {
    if (mtx == 1)
#pragma unroll
      for (int j = 0; j < BLK; j++) xch[(sub * BLK + j) * WAVE + lane] = acc[j];
    __syncthreads();
    if (mtx == 1) return;
  }
#pragma unroll
  for (int j = 0; j < BLK; j++) {
    const int n = n0 + 16 * (sub + WPM * j) + lr;
    if (n >= a.N) continue;
    f32x4 up = acc[j];
    if (SWIGLU) up = xch[(sub * BLK + j) * WAVE + lane];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = 4 * i + lg;
      if (t >= m_valid) continue;
      const int64_t o = int64_t(s0 + t) * a.N + n;
      if (SWIGLU) {
        const float g = acc[j][i];
        const float h = g / (1.0f + expf(-g)) * up[i];
        const uint32_t hi = f32_to_bf16(h);
        a.h_hi[o] = uint16_t(hi);
        a.h_lo[o] = uint16_t(f32_to_bf16(h - bf16_to_f32(hi)));
      } else {
        a.y[o] = acc[j][i];
      }
    }
  }
}

template <int QT, bool SWIGLU, int BLK>
int launch_decode(const GemmArgs& a, hipStream_t s) {
  constexpr int RB = 16 * (SWIGLU ? 2 : 4) * BLK;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + DECODE_BM - 1) / DECODE_BM;
  const dim3 grid(unsigned(tiles), unsigned((a.N + RB - 1) / RB)), block(256);
  const size_t lds = 4 * 16 * Stage<QT>::SLOT + size_t(DECODE_BM) * (size_t(a.K) * 2 * (a.a_lo ? 2 : 1) + 16) +
                     size_t(a.K / 32) * (Fmt<QT>::SUB16 ? 2 : 1) * 16 * 4 + (SWIGLU ? 2 * BLK * WAVE * 16 : 0);
  if (lds > LDS_BYTES)
    return fail(ARTLITE_EINVAL, "expert GEMM: K %d takes %zu B of LDS per workgroup (of %d)", a.K, lds, LDS_BYTES);
  if (a.a_lo)
    k_gemm_decode<QT, SWIGLU, 2, BLK><<<grid, block, lds, s>>>(a);
  else
    k_gemm_decode<QT, SWIGLU, 1, BLK><<<grid, block, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- Prefill tiling (k_prefill): fp16 products on v_mfma_f32_16x16x32_f16. A is fp16 rows, each token's row
// scaled by a power of two (2^-in_exp[token]) into [2^14, 2^15) at its largest, so bf16 activations convert
// exactly and fp32 ones round once (2^-11). The weights' blocks are decoded in registers to fp16 d (q - 8) (Q4_0)
// or d q (Q8_0): the code exactly, the product with the fp16 scale rounded once (2^-11 relative), so the MFMA's
// fp32 sums need no per-group scale FMA. The SwiGLU launch writes h in fp16 scaled by 2^-out_exp[token], where
// out_exp bounds |h| <= (sum |x|)^2 max|w_gate| max|w_up| below 2^15; the plain launch scales its fp32 outputs back
// by 2^in_exp[token].
// A workgroup is one tile of PREFILL_BM sorted rows of one expert times 256 staged weight rows (SwiGLU: 128 of gate
// and the same 128 of up; plain: 256), as 8 waves: wave w takes all 128 rows (MB = 8 MFMA row blocks) and two
// 16-row column blocks (SwiGLU: gate and up rows 16 w .. + 16, so h forms in the wave; plain: rows 32 w .. + 32), so
// each lane's decode of a block's codes feeds 8 MFMAs. K streams in stages of two 32-value groups through a ring of
// R LDS stages filled by DMA (global_load_lds, issued by asm so that the compiler, which would wait for every DMA
// in flight before any LDS read it sees, does not know of them): every wave issues the same number of loads per
// stage (past the last stage, loads of stage 0 again), so each wait is a fixed count of this wave's loads, and
// R - 1 stages are in flight while one computes. The operands of the next group are read from LDS while the
// current group computes; stage st + 1's wait and barrier sit between stage st's two groups, after which the slot
// of stage st (both groups in registers by then) takes stage st + R.
// A rows sit in LDS as 16-byte chunks of 8 values, XOR-swizzled by row, so the 16 rows of an operand read fall in
// different banks; a weight row's stage bytes (two blocks) sit packed, read as aligned dwords (a block's codes start
// 2 bytes into it: the first block's are shifted into place with alignbit). MFMA layout (16x16x32): lane l holds A
// row l % 16 and B column l % 16, both with K values 8 (l / 16) .. + 8; C column l % 16, rows 4 (l / 16) .. + 4.
template <int QT>
struct PStage {
  static constexpr int GB = Fmt<QT>::GROUP_BYTES;
  static constexpr int ROW = 2 * GB;  // weight bytes of a row per stage
  static constexpr int DW = ROW / 4;  // its dwords (9 / 17)
};
static_assert(PStage<ARTLITE_Q4_0>::ROW % 4 == 0 && PStage<ARTLITE_Q8_0>::ROW % 4 == 0, "stage rows in dwords");

template <int QT>
struct PLayout {
  static constexpr int WAVES = 8, THREADS = 64 * WAVES;
  static constexpr int WROWS = 256;                             // staged weight rows of a workgroup
  static constexpr int ACH = 8;                                 // 16-byte chunks of an A row per stage
  static constexpr int ABYTES = PREFILL_BM * ACH * 16;          // one stage of A
  static constexpr int AI = PREFILL_BM * ACH / 64 / WAVES;      // A DMA instructions per wave per stage
  static constexpr int BI = (WROWS * PStage<QT>::DW + 64 * WAVES - 1) / (64 * WAVES);  // weight dword DMAs per wave
  static constexpr int BBYTES = WAVES * BI * 256;               // one stage of weights (padded)
  static constexpr int SBYTES = ABYTES + BBYTES;
  static constexpr int R = (150 * 1024 / SBYTES) < 5 ? (150 * 1024 / SBYTES) : 5;  // stages in the ring
  static constexpr int LOADS = AI + BI;                         // DMA instructions per wave per stage
  static_assert(R >= 3, "ring");
  static_assert((R - 1) * LOADS < 64, "vmcnt");
  static_assert(AI * 64 * WAVES == PREFILL_BM * ACH, "A stage in whole instructions");
};

template <int N>
__device__ __forceinline__ void pf_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// every wave's LDS reads done, then the workgroup barrier
__device__ __forceinline__ void pf_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t pf_lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// one DMA of SIZE bytes per lane from g into LDS at lds (wave-uniform) + SIZE lane. M0 carries the LDS address; no
// compiler-generated code in these kernels uses M0 (the asm sets it before each load, with the one wait state a
// load after an M0 write needs).
template <int SIZE>
__device__ __forceinline__ void pf_dma(const void* g, uint32_t lds) {
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// the same from a uniform base (SGPRs) plus the lane's 32-bit byte offset (no 64-bit address arithmetic per load)
template <int SIZE>
__device__ __forceinline__ void pf_dma_s(const void* base, uint32_t off, uint32_t lds) {
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// the operands of one 32-value group: per row block, the lane's 8 fp16 of A; per column block, the weight row's
// fp16 scale and 8 of its code bytes (Q4_0: 16 nibbles, 8 of them the lane's)
template <int MB>
struct POps {
  u32x4 a[MB];
  uint32_t sc[2];
  uint32_t cw[2][2];
};

// Decode of a lane's 8 weights to fp16: the code bytes spread into fp16 1024 + c (c < 256 exact, one perm per two),
// the offset taken off exactly by one packed FMA (Q4_0's high nibbles, kept in place as 16 q, are scaled by 1/16 in
// it), then the product with the block's scale, rounded once.
template <int QT>
struct PDecode {
  uint32_t msk;
  f16x2 mul, add;
  __device__ __forceinline__ explicit PDecode(int lg) {
    if constexpr (QT == ARTLITE_Q4_0) {
      const bool hi = lg >= 2;  // (lane groups 2, 3 hold K values 16 .. 31: the high nibbles)
      msk = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
      mul = hi ? f16x2{_Float16(0.0625f), _Float16(0.0625f)} : f16x2{_Float16(1.0f), _Float16(1.0f)};
      add = hi ? f16x2{_Float16(-72.0f), _Float16(-72.0f)} : f16x2{_Float16(-1032.0f), _Float16(-1032.0f)};
    } else {
      msk = 0x80808080u;  // (Q8_0: the sign bits flipped, c = q + 128)
      mul = f16x2{_Float16(1.0f), _Float16(1.0f)};
      add = f16x2{_Float16(-1152.0f), _Float16(-1152.0f)};
    }
  }
  __device__ __forceinline__ u32x4 operator()(const uint32_t (&cw)[2], uint32_t sc) const {
    const uint32_t v0 = QT == ARTLITE_Q4_0 ? cw[0] & msk : cw[0] ^ msk;
    const uint32_t v1 = QT == ARTLITE_Q4_0 ? cw[1] & msk : cw[1] ^ msk;
    const uint32_t w[4] = {__builtin_amdgcn_perm(0x64646464u, v0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, v0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, v1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, v1, 0x04030402u)};
    const f16x2 d = __builtin_bit_cast(f16x2, sc | (sc << 16));
    u32x4 b;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const f16x2 c = __builtin_bit_cast(f16x2, w[j]) * mul + add;  // (exact: the code less its offset)
      b[j] = __builtin_bit_cast(uint32_t, c * d);
    }
    return b;
  }
};

__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                 0);
}

// The items (tile, column block) of a launch, in tile-major order, dealt to the 8 XCDs in contiguous runs: workgroup
// b runs on XCD b % 8 (the dispatcher's round robin), and the G = grid / 8 workgroups of an XCD take its run's items
// in turn, so the column blocks of a tile, and the tiles of an expert, run close in time on one XCD and share its L2
// (the tile's A rows, the expert's weights).
struct PItem {
  int e, s0, m_valid, n0;
};

template <bool SWIGLU>
__device__ __forceinline__ PItem prefill_item(const PrefillArgs& a, int64_t w, int nbk) {
  constexpr int WN = SWIGLU ? 128 : 256;
  const int tl = int(w / nbk);
  PItem I;
  I.n0 = int(w % nbk) * WN;
  if (a.tiles) {
    I.e = a.tiles[2 * tl];
    I.s0 = a.tiles[2 * tl + 1];
    I.m_valid = min(PREFILL_BM, a.offsets[I.e + 1] - I.s0);
  } else {
    I.e = 0;
    I.s0 = tl * PREFILL_BM;
    I.m_valid = min(PREFILL_BM, a.dense_rows - I.s0);
  }
  return I;
}

// The lane's DMA sources of an item. A: instruction i writes chunks (wv AI + i) 64 + lane of a stage's A region;
// chunk p holds row r = p / ACH, physical chunk c = p % ACH, which is logical chunk c ^ swz(r) (K values 8 c .. + 8
// of the stage); rows past the tile repeat its last (their outputs are not stored). Weights: instruction j writes
// dwords (wv BI + j) 64 + lane of the stage's weight region, staged row q / DW (SwiGLU: gate rows n0 .. + 128, then
// up's; plain: rows n0 .. + 256), dword q % DW of the row's stage bytes; dwords past the rows load the last one
// again (padding), rows past N the last row. Held as 32-bit byte offsets (A: from a.a; weights: from the
// instruction's matrix, which is uniform: 128 rows of gate are a whole number of instructions).
template <int QT, bool SWIGLU>
struct PSrc {
  using L = PLayout<QT>;
  static constexpr int GATE_INSTS = 128 * PStage<QT>::DW / 64;  // (SwiGLU: instructions of the gate rows)
  static_assert(128 * PStage<QT>::DW % 64 == 0, "matrix-uniform weight instructions");
  uint32_t a[L::AI];
  uint32_t w[L::BI];
  __device__ __forceinline__ static int swz(int r) { return (r >> 1) & 7; }
  __device__ __forceinline__ static const uint8_t* wbase(const PrefillArgs& g, int wv, int j) {
    return SWIGLU && wv * L::BI + j >= GATE_INSTS ? g.w[1] : g.w[0];
  }
  __device__ __forceinline__ void set(const PrefillArgs& g, const PItem& I, int wv, int lane) {
#pragma unroll
    for (int i = 0; i < L::AI; i++) {
      const int p = (wv * L::AI + i) * 64 + lane, r = p / L::ACH, c = (p % L::ACH) ^ swz(r);
      const int s = I.s0 + min(r, I.m_valid - 1);
      const int ar = g.a_gather ? (g.order ? g.order[s] / g.topk : s) : s;
      a[i] = (uint32_t(ar) * uint32_t(g.K) + 8 * c) * 2;  // (bytes)
    }
#pragma unroll
    for (int j = 0; j < L::BI; j++) {
      const int q = min((wv * L::BI + j) * 64 + lane, L::WROWS * PStage<QT>::DW - 1);
      const int row = q / PStage<QT>::DW, dw = q % PStage<QT>::DW;
      const int n = min(I.n0 + (SWIGLU ? row % 128 : row), g.N - 1);
      w[j] = uint32_t(I.e) * uint32_t(g.expert_bytes) + uint32_t(n) * uint32_t(g.row_bytes) + 4 * dw;
    }
  }
};

// The K loop of one item over MBN row blocks of A (the tile's rows, rounded up to 16-row blocks that hold any), in
// the workgroup's continuous stream of stages: the item's stage st is global step g0 + st in ring slot
// (g0 + st) % R; the R steps issued ahead reach into the next item's first stages (or, after the last item, load
// stage 0 again). On entry cur holds group 0 of stage 0 (read from LDS); on exit, group 0 of the next item's stage 0.
// The loads of stage st of an item (sources src) into the ring slot at byte offset so: A from a.a + 128 st, the
// weights from their matrix + ROW st (uniform bases), each lane at its own offset.
template <int QT, bool SWIGLU>
__device__ __forceinline__ void prefill_issue(const PrefillArgs& a, uint32_t lds_base, int wv,
                                              const PSrc<QT, SWIGLU>& src, int st, uint32_t so) {
  using L = PLayout<QT>;
  const uint32_t adst = lds_base + so + wv * L::AI * 1024, bdst = lds_base + so + L::ABYTES + wv * L::BI * 256;
  const uint8_t* ab = reinterpret_cast<const uint8_t*>(a.a) + 128 * st;
#pragma unroll
  for (int i = 0; i < L::AI; i++) pf_dma_s<16>(ab, src.a[i], adst + i * 1024);
#pragma unroll
  for (int i = 0; i < L::BI; i++)
    pf_dma_s<4>(PSrc<QT, SWIGLU>::wbase(a, wv, i) + st * PStage<QT>::ROW, src.w[i], bdst + i * 256);
}

// The K loop of one item over MBN row blocks of A (the tile's rows, rounded up to 16-row blocks that hold any), in
// the workgroup's continuous stream of stages through the ring: the item's stage st sits in slot (so0 + st SBYTES)
// mod R SBYTES; the step issued as stage st completes (into stage st's slot) is stage st + R, which past the item's
// last stage is the next item's stage st + R - stages (or, after the last item, stage 0 again). On entry cur holds
// group 0 of stage 0; on exit, group 0 of the next item's stage 0 (all 8 row blocks), and the slot it came from is
// returned.
template <int QT, bool SWIGLU, int MBN>
__device__ __forceinline__ uint32_t prefill_loop(const PrefillArgs& a, uint8_t* lds, uint32_t so,
                                                 const PSrc<QT, SWIGLU>& src, const PSrc<QT, SWIGLU>& nsrc,
                                                 bool has_next, POps<8>& cur, POps<8>& nxt, f32x4 (&acc)[8][2]) {
  using F = Fmt<QT>;
  using L = PLayout<QT>;
  constexpr int R = L::R, ROW = PStage<QT>::ROW, GB = F::GROUP_BYTES;
  const int lane = threadIdx.x & (WAVE - 1), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lg = lane >> 4, lr = lane & 15;
  const int stages = a.K / 64;
  const uint32_t lbase = pf_lds_addr(lds);
  // the lane's LDS read offsets in a slot: A row lr (row block mb at + 16 mb rows), group gl: the chunk of K
  // 8 lg .. + 8; B: the staged row of column block nb, its block gl
  constexpr int AMB = 16 * L::ACH * 16;
  const uint32_t aof[2] = {uint32_t(lr * L::ACH * 16 + ((0 + lg) ^ PSrc<QT, SWIGLU>::swz(lr)) * 16),
                           uint32_t(lr * L::ACH * 16 + ((4 + lg) ^ PSrc<QT, SWIGLU>::swz(lr)) * 16)};
  const uint32_t bof[2] = {uint32_t(L::ABYTES + (SWIGLU ? 16 * wv + lr : 32 * wv + lr) * ROW),
                           uint32_t(L::ABYTES + (SWIGLU ? 128 + 16 * wv + lr : 32 * wv + 16 + lr) * ROW)};
  // the code bytes of lane group lg at the block + 2 + cb: Q4_0 bytes 8 (lg & 1) .. + 8 (lane groups 0, 1 take the
  // low nibbles, 2, 3 the high ones), Q8_0 bytes 8 lg .. + 8
  const int cb = QT == ARTLITE_Q4_0 ? 8 * (lg & 1) : 8 * lg;
  auto read = [&](POps<8>& o, uint32_t sl, int gl, auto nr) {
    const uint8_t* ap = lds + sl + aof[gl];
#pragma unroll
    for (int mb = 0; mb < decltype(nr)::value; mb++) o.a[mb] = *reinterpret_cast<const u32x4*>(ap + mb * AMB);
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const uint8_t* b = lds + sl + bof[nb] + gl * GB;  // (4-byte aligned: gl GB is 0 or 2 mod 4)
      o.sc[nb] = *reinterpret_cast<const uint16_t*>(b);
      if (gl == 0) {
        const uint32_t* d = reinterpret_cast<const uint32_t*>(b + cb);
        const uint32_t d0 = d[0], d1 = d[1], d2 = d[2];
        o.cw[nb][0] = __builtin_amdgcn_alignbit(d1, d0, 16);
        o.cw[nb][1] = __builtin_amdgcn_alignbit(d2, d1, 16);
      } else {
        const uint32_t* d = reinterpret_cast<const uint32_t*>(b + 2 + cb);
        o.cw[nb][0] = d[0];
        o.cw[nb][1] = d[1];
      }
    }
  };
  const PDecode<QT> dec(lg);
  auto compute = [&](const POps<8>& o) {
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const u32x4 b = dec(o.cw[nb], o.sc[nb]);
#pragma unroll
      for (int mb = 0; mb < MBN; mb++) acc[mb][nb] = mfma16(o.a[mb], b, acc[mb][nb]);
    }
  };
  using NR = std::integral_constant<int, MBN>;
  using N8 = std::integral_constant<int, 8>;
  auto next_slot = [](uint32_t x) { return x + L::SBYTES == R * L::SBYTES ? 0u : x + L::SBYTES; };
  // one stage: group 1 read while group 0 computes; the wait for the next stage, the barrier, the step into this
  // stage's slot; the next stage's group 0 read while group 1 computes
  auto step = [&](const PSrc<QT, SWIGLU>& isrc, int ist, auto nr) {
    read(nxt, so, 1, NR{});
    compute(cur);
    pf_wait<(R - 2) * L::LOADS>();  // (the next stage: the R - 2 steps after it issued)
    pf_barrier();
    prefill_issue<QT, SWIGLU>(a, lbase, wv, isrc, ist, so);  // (into the slot every wave is past)
    so = next_slot(so);
    read(cur, so, 0, nr);
    compute(nxt);
  };
  int st = 0;
  for (; st < stages - R; st++) step(src, st + R, NR{});
  for (; st + 1 < stages; st++) step(has_next ? nsrc : src, has_next ? st + R - stages : 0, NR{});
  step(has_next ? nsrc : src, has_next ? st + R - stages : 0, N8{});
  return so;
}

template <int QT, bool SWIGLU>
__global__ __launch_bounds__(512) void k_prefill(const PrefillArgs a) {
  using L = PLayout<QT>;
  constexpr int R = L::R;
  constexpr int WN = SWIGLU ? 128 : 256;  // output columns per item
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // per row of an item: (2^in_exp, 2^-out_exp), in three buffers: item q's in buffer q % 3, filled while item q - 1
  // computes (waves 0, 1); item q - 2's epilogue, the last reader of that buffer, is behind every wave by then
  // (item q - 1's barriers), while item q - 1's may still be running in other waves (two buffers would race)
  float2* rowf = reinterpret_cast<float2*>(lds + R * L::SBYTES);
  const int lane = threadIdx.x & (WAVE - 1), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lg = lane >> 4, lr = lane & 15;
  const int nbk = (a.N + WN - 1) / WN;
  const int64_t ntl = a.tiles ? int64_t(*a.n_tiles) : (a.dense_rows + PREFILL_BM - 1) / PREFILL_BM;
  const int64_t items = ntl * nbk, per = (items + 7) / 8;
  const int G = gridDim.x / 8, x = blockIdx.x % 8, j0 = blockIdx.x / 8;
  const int64_t first = x * per + j0, end = min(items, (x + 1) * per);
  if (first >= end) return;
  const int nq = int((end - first + G - 1) / G);  // this workgroup's items: first + q G
  // the row scales of item I into buffer b
  auto row_info = [&](const PItem& I, int b) {
    if (threadIdx.x < PREFILL_BM) {
      const int m = threadIdx.x;
      float2 f = {1.0f, 1.0f};
      if (m < I.m_valid) {
        const int s = I.s0 + m, t = a.order ? a.order[s] / a.topk : s;
        f.x = __builtin_ldexpf(1.0f, a.in_exp[t]);
        if (SWIGLU) f.y = __builtin_ldexpf(1.0f, -a.out_exp[t]);
      }
      rowf[b * PREFILL_BM + m] = f;
    }
  };

  PItem I = prefill_item<SWIGLU>(a, first, nbk);
  PSrc<QT, SWIGLU> src, nsrc;
  src.set(a, I, wv, lane);
  row_info(I, 0);
  // the first item's first R stages (stages >= R: the launch checks), then its stage 0 read
#pragma unroll
  for (int j = 0; j < R; j++) prefill_issue<QT, SWIGLU>(a, pf_lds_addr(lds), wv, src, j, j * L::SBYTES);
  pf_wait<(R - 1) * L::LOADS>();  // (stage 0: R - 1 stages issued after it)
  __syncthreads();                // (and the row scales)
  POps<8> cur, nxt;
  {
    using F = Fmt<QT>;
    constexpr int AMB = 16 * L::ACH * 16, ROW = PStage<QT>::ROW;
    const uint32_t aof0 = uint32_t(lr * L::ACH * 16 + (lg ^ PSrc<QT, SWIGLU>::swz(lr)) * 16);
#pragma unroll
    for (int mb = 0; mb < 8; mb++) cur.a[mb] = *reinterpret_cast<const u32x4*>(lds + aof0 + mb * AMB);
    const int cb = QT == ARTLITE_Q4_0 ? 8 * (lg & 1) : 8 * lg;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const uint8_t* b = lds + L::ABYTES + (SWIGLU ? 128 * nb + 16 * wv + lr : 32 * wv + 16 * nb + lr) * ROW;
      cur.sc[nb] = *reinterpret_cast<const uint16_t*>(b);
      const uint32_t* d = reinterpret_cast<const uint32_t*>(b + cb);
      cur.cw[nb][0] = __builtin_amdgcn_alignbit(d[1], d[0], 16);
      cur.cw[nb][1] = __builtin_amdgcn_alignbit(d[2], d[1], 16);
      (void)F::OFF;
    }
  }

  uint32_t so = 0;  // the ring slot (byte offset) of the current item's stage 0
  for (int q = 0; q < nq; q++) {
    const bool has_next = q + 1 < nq;
    PItem J{};
    if (has_next) {
      J = prefill_item<SWIGLU>(a, first + int64_t(q + 1) * G, nbk);
      nsrc.set(a, J, wv, lane);
      row_info(J, (q + 1) % 3);  // (read after this item's barriers)
    }
    f32x4 acc[8][2];
#pragma unroll
    for (int mb = 0; mb < 8; mb++) acc[mb][0] = acc[mb][1] = f32x4{0, 0, 0, 0};
    const int mbn = (I.m_valid + 15) / 16;
    if (mbn <= 2)
      so = prefill_loop<QT, SWIGLU, 2>(a, lds, so, src, nsrc, has_next, cur, nxt, acc);
    else if (mbn <= 4)
      so = prefill_loop<QT, SWIGLU, 4>(a, lds, so, src, nsrc, has_next, cur, nxt, acc);
    else
      so = prefill_loop<QT, SWIGLU, 8>(a, lds, so, src, nsrc, has_next, cur, nxt, acc);

    // epilogue: lane output i of block (mb, nb): row 16 mb + 4 lg + i of the tile; column (SwiGLU) n0 + 16 wv + lr
    // of gate (nb 0) and up (nb 1), (plain) n0 + 32 wv + 16 nb + lr
    const float2* rf = rowf + (q % 3) * PREFILL_BM;
#pragma unroll
    for (int mb = 0; mb < 8; mb++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * mb + 4 * lg + i;
        if (m >= I.m_valid) continue;
        const int64_t o = int64_t(I.s0 + m) * a.N;
        const float2 f = rf[m];
        if constexpr (SWIGLU) {
          const int n = I.n0 + 16 * wv + lr;
          if (n >= a.N) continue;
          const float g = acc[mb][0][i] * f.x, u = acc[mb][1][i] * f.x;
          const float h = g / (1.0f + expf(-g)) * u;
          a.h[o + n] = __builtin_bit_cast(uint16_t, _Float16(h * f.y));
        } else {
#pragma unroll
          for (int nb = 0; nb < 2; nb++) {
            const int n = I.n0 + 32 * wv + 16 * nb + lr;
            if (n < a.N) a.y[o + n] = acc[mb][nb][i] * f.x;
          }
        }
      }
    }
    I = J;
    src = nsrc;
  }
  pf_wait<0>();  // (the loads past the last stage land before the workgroup's LDS is released)
}

template <int QT, bool SWIGLU>
int launch_prefill_t(const PrefillArgs& a, hipStream_t s) {
  using L = PLayout<QT>;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + PREFILL_BM - 1) / PREFILL_BM;
  const int64_t items = tiles * ((a.N + (SWIGLU ? 127 : 255)) / (SWIGLU ? 128 : 256));
  if (items <= 0) return ARTLITE_OK;
  if (items >= (int64_t(1) << 31)) return fail(ARTLITE_EINVAL, "prefill GEMM: %lld work items", (long long)items);
  if (a.K / 64 < L::R) return fail(ARTLITE_EINVAL, "prefill GEMM: K %d below %d", a.K, 64 * L::R);
  constexpr size_t lds = size_t(L::R) * L::SBYTES + 3 * PREFILL_BM * 8;
  // persistent workgroups: as many as the device holds at once (a multiple of 8, the XCDs), at most the items
  static const int resident = [] {
    const void* f = reinterpret_cast<const void*>(k_prefill<QT, SWIGLU>);
    int dev = 0, cus = 0, per_cu = 0;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, L::THREADS, lds) != hipSuccess)
      return 0;
    return cus * std::max(1, per_cu);
  }();
  if (resident < 8) return fail(ARTLITE_EHIP, "prefill GEMM: kernel set-up failed");
  const unsigned grid = unsigned(std::min<int64_t>((items + 7) / 8 * 8, resident / 8 * 8));
  k_prefill<QT, SWIGLU><<<grid, L::THREADS, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

bool prefill_supported(int qtype, int K, int N) {
  const int r = qtype == ARTLITE_Q4_0 ? PLayout<ARTLITE_Q4_0>::R : PLayout<ARTLITE_Q8_0>::R;
  return (qtype == ARTLITE_Q4_0 || qtype == ARTLITE_Q8_0) && K >= 64 * r && K % 64 == 0 && N > 0 && N % 16 == 0;
}

int launch_prefill(const PrefillArgs& a, hipStream_t s) {
  if (!prefill_supported(a.qtype, a.K, a.N))
    return fail(ARTLITE_EINVAL, "prefill GEMM: weight type %d, K %d, N %d", a.qtype, a.K, a.N);
  if (!a.a || !a.in_exp || (a.w[1] ? !a.h || !a.out_exp : !a.y) || (a.tiles && (!a.n_tiles || !a.offsets)))
    return fail(ARTLITE_EINVAL, "prefill GEMM: null argument");
  const bool swiglu = a.w[1] != nullptr;
  if (a.qtype == ARTLITE_Q4_0) return swiglu ? launch_prefill_t<ARTLITE_Q4_0, true>(a, s) : launch_prefill_t<ARTLITE_Q4_0, false>(a, s);
  return swiglu ? launch_prefill_t<ARTLITE_Q8_0, true>(a, s) : launch_prefill_t<ARTLITE_Q8_0, false>(a, s);
}

// ---- the prefill's activations: per token t, x's row in fp16 scaled by 2^-x_exp[t] (its largest |x| into
// [2^14, 2^15); exact for bf16 x unless below 2^-14 of that), and the exponents h_exp[t] of h's scale: the bound
// B = 2 (sum |x|)^2 (max |w_gate|) (max |w_up|) >= |silu(g) u| >= |h| (|g| <= sum |x| max |w_gate|, |silu(g)| <=
// |g|), h_exp = ilogb(B) - 14, so |h| 2^-h_exp < 2^15 (fp16 holds it). wmax[j]: max |w| of the bound's two matrices
// (pair j: wmax[2 j], wmax[2 j + 1]). One workgroup per token.
__global__ __launch_bounds__(256) void k_prefill_x(const void* __restrict__ x, int x_dtype, int H,
                                                   const float* __restrict__ wmax, int pairs,
                                                   uint16_t* __restrict__ x16, int32_t* __restrict__ x_exp,
                                                   int32_t* __restrict__ h_exp, int32_t* __restrict__ h_exp2) {
  __shared__ float red[2][8];
  const int64_t t = blockIdx.x;
  auto at = [&](int i) -> float {
    return x_dtype == ARTLITE_X_F32 ? static_cast<const float*>(x)[t * H + i]
                                    : bf16_to_f32(static_cast<const uint16_t*>(x)[t * H + i]);
  };
  float mx = 0.0f, l1 = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) {
    const float v = fabsf(at(i));
    mx = fmaxf(mx, v);
    l1 += v;
  }
  for (int o = 32; o; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    l1 += __shfl_xor(l1, o);
  }
  if ((threadIdx.x & 63) == 0) red[0][threadIdx.x / 64] = mx, red[1][threadIdx.x / 64] = l1;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  l1 = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  const int xe = (mx > 0.0f && mx <= 3.4e38f) ? ilogbf(mx) - 14 : 0;
  for (int i = threadIdx.x; i < H; i += 256)
    x16[t * H + i] = __builtin_bit_cast(uint16_t, _Float16(__builtin_ldexpf(at(i), -xe)));
  if (threadIdx.x < pairs) {
    // (in double: the square of a large sum stays finite)
    const double b = 2.0 * double(l1) * double(l1) * double(wmax[2 * threadIdx.x]) * double(wmax[2 * threadIdx.x + 1]);
    const int he = (b > 0.0 && b < 1e300) ? ilogb(b) - 14 : 0;
    (threadIdx.x ? h_exp2 : h_exp)[t] = max(-126, min(126, he));
  }
  if (threadIdx.x == 0) x_exp[t] = xe;
}

// The same for H a multiple of 8 up to 2048 NP: the row read once, 8 values per thread per piece (one 16-byte load for
// bf16, two for fp32), kept in registers for the fp16 pass, written as 16-byte pieces.
template <int XT, int NP>
__global__ __launch_bounds__(256) void k_prefill_x_rows(const void* __restrict__ x, int H,
                                                        const float* __restrict__ wmax, int pairs,
                                                        uint16_t* __restrict__ x16, int32_t* __restrict__ x_exp,
                                                        int32_t* __restrict__ h_exp, int32_t* __restrict__ h_exp2) {
  __shared__ float red[2][4];
  const int64_t t = blockIdx.x;
  const int n8 = H / 8;
  float v[NP][8];
  float mx = 0.0f, l1 = 0.0f;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int i = threadIdx.x + 256 * j;
    if (i < n8) {
      if (XT == ARTLITE_X_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + t * H) + 2 * i;
        const float4 a = p[0], b = p[1];
        v[j][0] = a.x, v[j][1] = a.y, v[j][2] = a.z, v[j][3] = a.w, v[j][4] = b.x, v[j][5] = b.y, v[j][6] = b.z,
        v[j][7] = b.w;
      } else {
        const uint4 q = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + t * H)[i];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int c = 0; c < 4; c++) v[j][2 * c] = bf16_to_f32(w[c] & 0xFFFFu), v[j][2 * c + 1] = bf16_to_f32(w[c] >> 16);
      }
#pragma unroll
      for (int c = 0; c < 8; c++) {
        mx = fmaxf(mx, fabsf(v[j][c]));
        l1 += fabsf(v[j][c]);
      }
    }
  }
  for (int o = 32; o; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    l1 += __shfl_xor(l1, o);
  }
  if ((threadIdx.x & 63) == 0) red[0][threadIdx.x / 64] = mx, red[1][threadIdx.x / 64] = l1;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  l1 = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  const int xe = (mx > 0.0f && mx <= 3.4e38f) ? ilogbf(mx) - 14 : 0;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int i = threadIdx.x + 256 * j;
    if (i < n8) {
      uint32_t w[4];
#pragma unroll
      for (int c = 0; c < 4; c++)
        w[c] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(__builtin_ldexpf(v[j][2 * c], -xe)))) |
               uint32_t(__builtin_bit_cast(uint16_t, _Float16(__builtin_ldexpf(v[j][2 * c + 1], -xe)))) << 16;
      reinterpret_cast<uint4*>(x16 + t * H)[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  if (threadIdx.x < pairs) {
    const double b = 2.0 * double(l1) * double(l1) * double(wmax[2 * threadIdx.x]) * double(wmax[2 * threadIdx.x + 1]);
    const int he = (b > 0.0 && b < 1e300) ? ilogb(b) - 14 : 0;
    (threadIdx.x ? h_exp2 : h_exp)[t] = max(-126, min(126, he));
  }
  if (threadIdx.x == 0) x_exp[t] = xe;
}

int launch_prefill_x(const void* x, int x_dtype, int64_t T, int H, const float* wmax, int pairs, uint16_t* x16,
                     int32_t* x_exp, int32_t* h_exp, int32_t* h_exp2, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (pairs < 1 || pairs > 2 || (pairs == 2 && !h_exp2)) return fail(ARTLITE_EINVAL, "prefill x: %d bounds", pairs);
  if (H % 8 == 0 && H <= 4 * 2048) {
    const bool f32 = x_dtype == ARTLITE_X_F32;
#define ART_PX(XT, NP) k_prefill_x_rows<XT, NP><<<unsigned(T), 256, 0, s>>>(x, H, wmax, pairs, x16, x_exp, h_exp, h_exp2)
    if (H <= 2048) {
      if (f32) ART_PX(ARTLITE_X_F32, 1); else ART_PX(ARTLITE_X_BF16, 1);
    } else if (H <= 4096) {
      if (f32) ART_PX(ARTLITE_X_F32, 2); else ART_PX(ARTLITE_X_BF16, 2);
    } else {
      if (f32) ART_PX(ARTLITE_X_F32, 4); else ART_PX(ARTLITE_X_BF16, 4);
    }
#undef ART_PX
    ART_HIP(hipGetLastError());
    return ARTLITE_OK;
  }
  k_prefill_x<<<unsigned(T), 256, 0, s>>>(x, x_dtype, H, wmax, pairs, x16, x_exp, h_exp, h_exp2);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- max |w| of a weight tensor's blocks: the fp16 scale's magnitude times the format's largest code (Q4_0: 8,
// Q8_0: 128), by an atomic max on the float's bits (non-negative floats order as their bits)
__global__ void k_weight_max(const uint8_t* __restrict__ w, int block_bytes, float code_max, int64_t nblocks,
                             uint32_t* __restrict__ out) {
  float mx = 0.0f;
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < nblocks; b += int64_t(gridDim.x) * blockDim.x) {
    uint16_t d;
    __builtin_memcpy(&d, w + b * block_bytes, 2);
    mx = fmaxf(mx, fabsf(f16_to_f32(d)));
  }
  for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(mx * code_max));
}

int launch_weight_max(const uint8_t* w, int qtype, int64_t nblocks, float* out, hipStream_t s) {
  if (qtype != ARTLITE_Q4_0 && qtype != ARTLITE_Q8_0) return fail(ARTLITE_EINVAL, "weight max: type %d", qtype);
  ART_HIP(hipMemsetAsync(out, 0, 4, s));
  if (nblocks <= 0) return ARTLITE_OK;
  const int bb = qtype == ARTLITE_Q4_0 ? 18 : 34;
  const unsigned grid = unsigned(std::min<int64_t>((nblocks + 255) / 256, 1024));
  k_weight_max<<<grid, 256, 0, s>>>(w, bb, qtype == ARTLITE_Q4_0 ? 8.0f : 128.0f, nblocks,
                                    reinterpret_cast<uint32_t*>(out));
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int launch_expert_gemm(const GemmArgs& a, hipStream_t s) {
  const QType* qt = qtype_by_id(a.qtype);
  if (!qt || qt->per < 32) return fail(ARTLITE_EINVAL, "expert GEMM: unsupported weight type %d", a.qtype);
  if (a.K <= 0 || a.K % qt->per)
    return fail(ARTLITE_EINVAL, "expert GEMM: K %d is not a multiple of the format's block", a.K);
  if (a.K / 32 > MAX_GROUPS) return fail(ARTLITE_EINVAL, "expert GEMM: K %d beyond %d", a.K, 32 * MAX_GROUPS);
  const bool swiglu = a.w[1] != nullptr;
  if (a.tiles && (a.bm < 1 || a.bm > DECODE_BM)) return fail(ARTLITE_EINVAL, "expert GEMM: tiles of %d rows", a.bm);
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + DECODE_BM - 1) / DECODE_BM;
  if (tiles <= 0) return ARTLITE_OK;
#define ART_DISPATCH(QT) return swiglu ? launch_decode<QT, true, 2>(a, s) : launch_decode<QT, false, 2>(a, s)
  switch (a.qtype) {
    case ARTLITE_Q4_0: ART_DISPATCH(ARTLITE_Q4_0);
    case ARTLITE_Q4_1: ART_DISPATCH(ARTLITE_Q4_1);
    case ARTLITE_Q8_0: ART_DISPATCH(ARTLITE_Q8_0);
    case ARTLITE_Q3_K: ART_DISPATCH(ARTLITE_Q3_K);
    case ARTLITE_Q4_K: ART_DISPATCH(ARTLITE_Q4_K);
    case ARTLITE_Q5_K: ART_DISPATCH(ARTLITE_Q5_K);
    case ARTLITE_Q6_K: ART_DISPATCH(ARTLITE_Q6_K);
    case ARTLITE_IQ4_NL: ART_DISPATCH(ARTLITE_IQ4_NL);
    case ARTLITE_IQ4_XS: ART_DISPATCH(ARTLITE_IQ4_XS);
    default: return fail(ARTLITE_EINVAL, "expert GEMM: unsupported weight type %d", a.qtype);
  }
#undef ART_DISPATCH
}

// ---- combine: y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] (the reference CombineOperator's sum,
// src/artlite/moe/gather.py:12-18: the shared term first, then the slots in order, fp32)
__global__ void k_combine(const float* __restrict__ Y, const int32_t* __restrict__ slot, const float* __restrict__ w,
                          int k, const float* __restrict__ ys, const float* __restrict__ ws_logit, int ws_sigmoid,
                          int64_t T, int H, const void* __restrict__ res, int res_dtype, float* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  if (h4 * 4 >= H) return;
  float4 acc = make_float4(0, 0, 0, 0);
  if (ys) {
    float ws = 1.0f;
    if (ws_logit) ws = ws_sigmoid ? 1.0f / (1.0f + expf(-ws_logit[t])) : ws_logit[t];
    const float4 v = reinterpret_cast<const float4*>(ys + t * H)[h4];
    acc.x = ws * v.x, acc.y = ws * v.y, acc.z = ws * v.z, acc.w = ws * v.w;
  }
  for (int i = 0; i < k; i++) {
    const float wi = w[t * k + i];
    const float4 v = reinterpret_cast<const float4*>(Y + int64_t(slot[t * k + i]) * H)[h4];
    acc.x = __builtin_fmaf(wi, v.x, acc.x);
    acc.y = __builtin_fmaf(wi, v.y, acc.y);
    acc.z = __builtin_fmaf(wi, v.z, acc.z);
    acc.w = __builtin_fmaf(wi, v.w, acc.w);
  }
  if (res) {  // (the residual add after the block: y = moe + x)
    float4 r;
    if (res_dtype == ARTLITE_X_F32) {
      r = reinterpret_cast<const float4*>(static_cast<const float*>(res) + t * H)[h4];
    } else {
      const uint2 v = reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(res) + t * H)[h4];
      r = make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16), bf16_to_f32(v.y & 0xFFFFu),
                      bf16_to_f32(v.y >> 16));
    }
    acc.x = acc.x + r.x, acc.y = acc.y + r.y, acc.z = acc.z + r.z, acc.w = acc.w + r.w;
  }
  reinterpret_cast<float4*>(y + t * H)[h4] = acc;
}

int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, const void* res, int res_dtype, float* y, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (H % 4) return fail(ARTLITE_EINVAL, "combine: H %d not a multiple of 4", H);
  const dim3 grid(unsigned((H / 4 + 255) / 256), unsigned(T)), block(256);
  k_combine<<<grid, block, 0, s>>>(Y, slot, w, k, ys, ws_logit, ws_sigmoid, T, H, res, res_dtype, y);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

__global__ void k_split(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const uint32_t h = f32_to_bf16(v);
  hi[i] = uint16_t(h);
  lo[i] = uint16_t(f32_to_bf16(v - bf16_to_f32(h)));
}

int launch_split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n <= 0) return ARTLITE_OK;
  k_split<<<unsigned((n + 255) / 256), 256, 0, s>>>(x, n, hi, lo);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace artlite
