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

// ---- the prefill's activations: per token t, x's row in fp16 scaled by 2^-xe (its largest |x| into [2^14, 2^15);
// exact for bf16 x unless below 2^-14 of that), and the factors of the expert products' rows: gu[t] = (2^xe, 2^-he),
// he the exponent of h's scale from a bound B >= 2 |g| |u| >= |silu(g) u| = |h| (|silu(g)| <= |g|), where each of
// |g|, |u| is at most the smaller of (sum |x|) (max |w|) and (max |x|) (the matrix's largest row L1 norm):
// he = ilogb(B) - 14, so |h| 2^-he < 2^15 (fp16 holds it). wmax[2 j], wmax[2 j + 1]: max |w| of pair j's matrices,
// wmax[5 + 2 j], wmax[6 + 2 j] their largest row L1 norms (a block with an outlier scale raises its row's L1 norm by
// its 32 values' share, not every row's bound by the outlier's factor). The down launch's sums over F fp16 values of
// h 2^-he (below 2^15) times a row of weights (of L1 norm at most L1d = wmax[9], up to fp16 rounding) stay below
// 2^15 L1d (1 + 2^-11): with ye = ilogb(L1d) + 1 they stay below 2^15 (1 + 2^-11) < 65504 after the factor 2^-ye,
// so the expert launch writes fp16 sums times 2^-ye and the true output is that times 2^(he + ye):
// dn[t] = (2^(he + ye), 2^-ye). The shared expert's down writes fp32: dn2[t] = (2^he, 1). One workgroup per token.
// the bounds prefill_x_factors reads for pair min(tid, pairs - 1), loaded at a kernel's start: wmax[2 q], wmax[2 q + 1],
// wmax[5 + 2 q], wmax[6 + 2 q], wmax[4], wmax[9] (an empty asm statement takes them, so that the compiler does not
// move the loads to their use after the row's own round trips)
struct PXBounds {
  float g, u, gl, ul, d, dl;
};
__device__ __forceinline__ PXBounds px_bounds(const float* wmax, int tid, int pairs) {
  const int q = min(tid, pairs - 1);
  PXBounds b{wmax[2 * q], wmax[2 * q + 1], wmax[5 + 2 * q], wmax[6 + 2 * q], wmax[4], wmax[9]};
  asm volatile("" : : "v"(b.g), "v"(b.u), "v"(b.gl), "v"(b.ul), "v"(b.d), "v"(b.dl));
  return b;
}
__device__ __forceinline__ void prefill_x_factors(int64_t t, int tid, int xe, float mx, float l1, const PXBounds& w,
                                                  int pairs, int F, float2* gu, float2* dn, float2* gu2, float2* dn2) {
  if (tid < pairs) {
    // (in double: the product of two large bounds stays finite)
    const double bg = fmin(double(l1) * double(w.g), double(mx) * double(w.gl));
    const double bu = fmin(double(l1) * double(w.u), double(mx) * double(w.ul));
    const double b = 2.0 * bg * bu;
    const int he = max(-126, min(126, (b > 0.0 && b < 1e300) ? ilogb(b) - 14 : 0));
    (tid ? gu2 : gu)[t] = make_float2(__builtin_ldexpf(1.0f, xe), __builtin_ldexpf(1.0f, -he));
    if (tid) {
      dn2[t] = make_float2(__builtin_ldexpf(1.0f, he), 1.0f);
    } else {
      const double bd = fmin(double(F) * double(w.d), double(w.dl));
      const int ye = (bd > 0.0 && bd < 1e300) ? min(min(126, 126 - he), max(max(-126, -126 - he), ilogb(bd) + 1)) : 0;
      dn[t] = make_float2(__builtin_ldexpf(1.0f, he + ye), __builtin_ldexpf(1.0f, -ye));
    }
  }
}

__global__ __launch_bounds__(256) void k_prefill_x(const void* __restrict__ x, int x_dtype, int H,
                                                   const float* __restrict__ wmax, int pairs, int F,
                                                   uint16_t* __restrict__ x16, float2* gu, float2* dn, float2* gu2,
                                                   float2* dn2) {
  __shared__ float red[2][8];
  const int64_t t = blockIdx.x;
  const PXBounds wb = px_bounds(wmax, threadIdx.x, pairs);
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
  prefill_x_factors(t, threadIdx.x, xe, mx, l1, wb, pairs, F, gu, dn, gu2, dn2);
}

// The same for H a multiple of 8 up to 2048 NP: the row read once, 8 values per thread per piece (one 16-byte load for
// bf16, two for fp32), kept in registers for the fp16 pass, written as 16-byte pieces.
template <int XT, int NP>
__global__ __launch_bounds__(256) void k_prefill_x_rows(const void* __restrict__ x, int H,
                                                        const float* __restrict__ wmax, int pairs, int F,
                                                        uint16_t* __restrict__ x16, float2* gu, float2* dn, float2* gu2,
                                                        float2* dn2) {
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
  const PXBounds wb = px_bounds(wmax, threadIdx.x, pairs);
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
  prefill_x_factors(t, threadIdx.x, xe, mx, l1, wb, pairs, F, gu, dn, gu2, dn2);
}

// The same, a wave per token (four tokens a workgroup): lane l holds pieces l + 64 j of the row (8 values each, H =
// 512 NP), every load in flight at once; the row's largest magnitude and L1 norm by reductions within the wave alone
// (no LDS, no barrier), so that a workgroup costs one round trip to memory.
template <int XT, int NP>
__global__ __launch_bounds__(256) void k_prefill_x_wave(const void* __restrict__ x, int64_t T, int H,
                                                        const float* __restrict__ wmax, int pairs, int F,
                                                        uint16_t* __restrict__ x16, float2* gu, float2* dn,
                                                        float2* gu2, float2* dn2) {
  const int lane = threadIdx.x & 63;
  const int64_t t = int64_t(blockIdx.x) * 4 + threadIdx.x / 64;
  if (t >= T) return;
  float v[NP][8];
  if (XT == ARTLITE_X_F32) {
    float4 q[NP][2];
#pragma unroll
    for (int j = 0; j < NP; j++) {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + t * H) + 2 * (lane + 64 * j);
      q[j][0] = p[0], q[j][1] = p[1];
    }
#pragma unroll
    for (int j = 0; j < NP; j++) {
      v[j][0] = q[j][0].x, v[j][1] = q[j][0].y, v[j][2] = q[j][0].z, v[j][3] = q[j][0].w;
      v[j][4] = q[j][1].x, v[j][5] = q[j][1].y, v[j][6] = q[j][1].z, v[j][7] = q[j][1].w;
    }
  } else {
    uint4 q[NP];
#pragma unroll
    for (int j = 0; j < NP; j++) q[j] = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + t * H)[lane + 64 * j];
#pragma unroll
    for (int j = 0; j < NP; j++) {
      const uint32_t w[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
      for (int c = 0; c < 4; c++) v[j][2 * c] = bf16_to_f32(w[c] & 0xFFFFu), v[j][2 * c + 1] = bf16_to_f32(w[c] >> 16);
    }
  }
  const PXBounds wb = px_bounds(wmax, lane, pairs);
  float mx = 0.0f, l1 = 0.0f;
#pragma unroll
  for (int j = 0; j < NP; j++)
#pragma unroll
    for (int c = 0; c < 8; c++) {
      mx = fmaxf(mx, fabsf(v[j][c]));
      l1 += fabsf(v[j][c]);
    }
  for (int o = 32; o; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    l1 += __shfl_xor(l1, o);
  }
  const int xe = (mx > 0.0f && mx <= 3.4e38f) ? ilogbf(mx) - 14 : 0;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    uint32_t w[4];
#pragma unroll
    for (int c = 0; c < 4; c++)
      w[c] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(__builtin_ldexpf(v[j][2 * c], -xe)))) |
             uint32_t(__builtin_bit_cast(uint16_t, _Float16(__builtin_ldexpf(v[j][2 * c + 1], -xe)))) << 16;
    reinterpret_cast<uint4*>(x16 + t * H)[lane + 64 * j] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  prefill_x_factors(t, lane, xe, mx, l1, wb, pairs, F, gu, dn, gu2, dn2);
}

int launch_prefill_x(const void* x, int x_dtype, int64_t T, int H, const float* wmax, int pairs, int F, uint16_t* x16,
                     float2* gu, float2* dn, float2* gu2, float2* dn2, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (pairs < 1 || pairs > 2 || (pairs == 2 && (!gu2 || !dn2))) return fail(ARTLITE_EINVAL, "prefill x: %d bounds", pairs);
  if (H % 512 == 0 && (H / 512 == 1 || H / 512 == 2 || H / 512 == 4 || H / 512 == 8)) {
    const bool f32 = x_dtype == ARTLITE_X_F32;
    const unsigned g = unsigned((T + 3) / 4);
#define ART_PXW(XT, NP) k_prefill_x_wave<XT, NP><<<g, 256, 0, s>>>(x, T, H, wmax, pairs, F, x16, gu, dn, gu2, dn2)
#define ART_PXW2(NP) \
  if (f32)           \
    ART_PXW(ARTLITE_X_F32, NP); \
  else               \
    ART_PXW(ARTLITE_X_BF16, NP);
    switch (H / 512) {
      case 1: ART_PXW2(1) break;
      case 2: ART_PXW2(2) break;
      case 4: ART_PXW2(4) break;
      default: ART_PXW2(8) break;
    }
#undef ART_PXW2
#undef ART_PXW
    ART_HIP(hipGetLastError());
    return ARTLITE_OK;
  }
  if (H % 8 == 0 && H <= 4 * 2048) {
    const bool f32 = x_dtype == ARTLITE_X_F32;
#define ART_PX(XT, NP) k_prefill_x_rows<XT, NP><<<unsigned(T), 256, 0, s>>>(x, H, wmax, pairs, F, x16, gu, dn, gu2, dn2)
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
  k_prefill_x<<<unsigned(T), 256, 0, s>>>(x, x_dtype, H, wmax, pairs, F, x16, gu, dn, gu2, dn2);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- a bound on max |w| of a weight tensor's blocks: the fp16 scale's magnitude times the format's largest code
// (Q4_0: 8, Q8_0: 128; Q4_K: |d| 63 15 + |dmin| 63, its 6-bit scale and min at their largest), by an atomic max on the
// float's bits (non-negative floats order as their bits)
__global__ void k_weight_max(const uint8_t* __restrict__ w, int block_bytes, float code_max, float min_max,
                             int64_t nblocks, uint32_t* __restrict__ out) {
  float mx = 0.0f;
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < nblocks; b += int64_t(gridDim.x) * blockDim.x) {
    uint16_t d, dm;
    __builtin_memcpy(&d, w + b * block_bytes, 2);
    __builtin_memcpy(&dm, w + b * block_bytes + 2, 2);
    mx = fmaxf(mx, fabsf(f16_to_f32(d)) + (min_max > 0.0f ? fabsf(f16_to_f32(dm)) * min_max : 0.0f));
  }
  for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(mx * code_max));  // (min_max: already over code_max)
}

int launch_weight_max(const uint8_t* w, int qtype, int64_t nblocks, float* out, hipStream_t s) {
  if (qtype != ARTLITE_Q4_0 && qtype != ARTLITE_Q8_0 && qtype != ARTLITE_Q4_K) {
    // (no bound of this form: the largest fp32 value, so that the rows' L1 norms bound the products alone)
    ART_HIP(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(out), 0x7F7FFFFF, 1, s));
    return ARTLITE_OK;
  }
  ART_HIP(hipMemsetAsync(out, 0, 4, s));
  if (nblocks <= 0) return ARTLITE_OK;
  const int bb = qtype == ARTLITE_Q4_0 ? 18 : qtype == ARTLITE_Q8_0 ? 34 : 144;
  const float code = qtype == ARTLITE_Q4_0 ? 8.0f : qtype == ARTLITE_Q8_0 ? 128.0f : 945.0f;
  const float mins = qtype == ARTLITE_Q4_K ? 63.0f / 945.0f * 1.0001f : 0.0f;  // (a bound: rounded up)
  const unsigned grid = unsigned(std::min<int64_t>((nblocks + 255) / 256, 1024));
  k_weight_max<<<grid, 256, 0, s>>>(w, bb, code, mins, nblocks, reinterpret_cast<uint32_t*>(out));
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
  // (KC pairs at a time: their slots and weights, then their rows, all in flight before the sums, which go in pair
  // order; pairs past k load pair k - 1 again, unused, so that no branch separates the loads)
  constexpr int KC = 8;
  for (int i0 = 0; i0 < k; i0 += KC) {
    int r[KC];
    float wi[KC];
    f32x4 v[KC];
#pragma unroll
    for (int i = 0; i < KC; i++) {
      const int64_t pi = t * k + min(i0 + i, k - 1);
      r[i] = slot[pi], wi[i] = w[pi];
    }
    // (the slots as outputs of an empty asm: every slot load issued before any row's address is formed from one)
    asm volatile("" : "+s"(r[0]), "+s"(r[1]), "+s"(r[2]), "+s"(r[3]), "+s"(r[4]), "+s"(r[5]), "+s"(r[6]), "+s"(r[7]));
#pragma unroll
    for (int i = 0; i < KC; i++) v[i] = reinterpret_cast<const f32x4*>(Y + int64_t(r[i]) * H)[h4];
    // (every row in registers before the first sum: else the compiler moves each load into the branch that uses it)
    asm volatile("" : : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]));
    asm volatile("" : : "s"(wi[0]), "s"(wi[1]), "s"(wi[2]), "s"(wi[3]), "s"(wi[4]), "s"(wi[5]), "s"(wi[6]), "s"(wi[7]));
#pragma unroll
    for (int i = 0; i < KC; i++) {
      if (i0 + i >= k) break;
      acc.x = __builtin_fmaf(wi[i], v[i].x, acc.x);
      acc.y = __builtin_fmaf(wi[i], v[i].y, acc.y);
      acc.z = __builtin_fmaf(wi[i], v[i].z, acc.z);
      acc.w = __builtin_fmaf(wi[i], v[i].w, acc.w);
    }
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

// The same over fp16 pair outputs, 8 columns per thread (16-byte loads): Y[s] = Y16[s] yf[s].x, the factor folded
// into the weight (a power of two: (w f) v = w (f v) exactly), so the sum is the fp32 one over those values. The
// shared expert's output may come in ys_parts parts of a split K (T x H each, one after another), added in part
// order before its gate.
__global__ void k_combine16(const uint16_t* __restrict__ Y16, const float2* __restrict__ yf,
                            const int32_t* __restrict__ slot, const float* __restrict__ w, int k,
                            const float* __restrict__ ys, int ys_parts, const float* __restrict__ ws_logit,
                            int ws_sigmoid, int64_t T, int H, const void* __restrict__ res, int res_dtype,
                            float* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int h8 = blockIdx.x * blockDim.x + threadIdx.x;
  if (h8 * 8 >= H) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (ys) {
    float ws = 1.0f;
    if (ws_logit) ws = ws_sigmoid ? 1.0f / (1.0f + expf(-ws_logit[t])) : ws_logit[t];
    float v[8];
    for (int j = 0; j < ys_parts; j++) {
      const float4* p = reinterpret_cast<const float4*>(ys + (j * T + t) * H) + 2 * h8;
      const float4 a = p[0], b = p[1];
      const float u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = j ? v[i] + u[i] : u[i];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = ws * v[i];
  }
  // (KC pairs at a time: their slots and weights, then their factors and rows, all in flight before the sums, which
  // go in pair order; pairs past k load pair k - 1 again, unused, so that no branch separates the loads)
  constexpr int KC = 8;
  for (int i0 = 0; i0 < k; i0 += KC) {
    int r[KC];
    float wi[KC];
    u32x4 v[KC];
#pragma unroll
    for (int i = 0; i < KC; i++) {
      const int64_t pi = t * k + min(i0 + i, k - 1);
      r[i] = slot[pi], wi[i] = w[pi];
    }
    // (the slots as outputs of an empty asm: every slot load issued before any row's address is formed from one)
    asm volatile("" : "+s"(r[0]), "+s"(r[1]), "+s"(r[2]), "+s"(r[3]), "+s"(r[4]), "+s"(r[5]), "+s"(r[6]), "+s"(r[7]));
#pragma unroll
    for (int i = 0; i < KC; i++) wi[i] *= yf[r[i]].x, v[i] = reinterpret_cast<const u32x4*>(Y16 + int64_t(r[i]) * H)[h8];
    // (every row in registers before the first sum: else the compiler moves each load into the branch that uses it)
    asm volatile("" : : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]));
    asm volatile("" : : "s"(wi[0]), "s"(wi[1]), "s"(wi[2]), "s"(wi[3]), "s"(wi[4]), "s"(wi[5]), "s"(wi[6]), "s"(wi[7]));
#pragma unroll
    for (int i = 0; i < KC; i++) {
      if (i0 + i >= k) break;
      const uint32_t q[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[2 * j] = __builtin_fmaf(wi[i], h2f(q[j] & 0xFFFFu), acc[2 * j]);
        acc[2 * j + 1] = __builtin_fmaf(wi[i], h2f(q[j] >> 16), acc[2 * j + 1]);
      }
    }
  }
  if (res) {
    float r[8];
    if (res_dtype == ARTLITE_X_F32) {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(res) + t * H) + 2 * h8;
      const float4 a = p[0], b = p[1];
      r[0] = a.x, r[1] = a.y, r[2] = a.z, r[3] = a.w, r[4] = b.x, r[5] = b.y, r[6] = b.z, r[7] = b.w;
    } else {
      const uint4 v = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(res) + t * H)[h8];
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) r[2 * j] = bf16_to_f32(q[j] & 0xFFFFu), r[2 * j + 1] = bf16_to_f32(q[j] >> 16);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = acc[j] + r[j];
  }
  float4* o = reinterpret_cast<float4*>(y + t * H) + 2 * h8;
  o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

int launch_combine16(const uint16_t* Y16, const float2* yf, const int32_t* slot, const float* w, int k,
                     const float* ys, int ys_parts, const float* ws_logit, int ws_sigmoid, int64_t T, int H,
                     const void* res, int res_dtype, float* y, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (H % 8) return fail(ARTLITE_EINVAL, "combine: H %d not a multiple of 8", H);
  if (ys && ys_parts < 1) return fail(ARTLITE_EINVAL, "combine: %d shared parts", ys_parts);
  const dim3 grid(unsigned((H / 8 + 255) / 256), unsigned(T)), block(256);
  k_combine16<<<grid, block, 0, s>>>(Y16, yf, slot, w, k, ys, ys_parts, ws_logit, ws_sigmoid, T, H, res, res_dtype,
                                     y);
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
