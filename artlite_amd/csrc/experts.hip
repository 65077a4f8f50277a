// The experts' products over raw GGUF blocks on gfx950's bf16 MFMA (v_mfma_f32_16x16x32_bf16), and the combine.
//
// Exactness of the operands: a block's integer codes are exact in bf16 -- Q4_0 as 128 + q and Q4_K as 128 + q
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

// Per format: bytes per 32-value group (in a run of whole blocks), the 32-value groups of one K-range (a stage:
// ~560 bytes of each row, so a 16-row stage is 16 long runs; a straddled cache line is read again by the next range
// of the same wave, from L2), the offset of the codes' bf16 encoding.
template <int QT>
struct Fmt;
template <>
struct Fmt<ARTLITE_Q4_0> {
  static constexpr int GROUP_BYTES = 18;
  static constexpr int KR = 32;
  static constexpr float OFF = 136.0f;  // (128 + q) - (q - 8)
};
template <>
struct Fmt<ARTLITE_Q8_0> {
  static constexpr int GROUP_BYTES = 34;
  static constexpr int KR = 16;
  static constexpr float OFF = 128.0f;
};
template <>
struct Fmt<ARTLITE_Q4_K> {
  static constexpr int GROUP_BYTES = 18;  // (144 bytes per super-block of 8 groups)
  static constexpr int KR = 32;
  static constexpr float OFF = 128.0f;
};

// the 16-byte chunks of a 16-row stage: the aligned cover of each row's run; a row's LDS slot is an odd number of
// 16-byte units, so the 16 rows' same-offset dwords fall in 16 different banks
template <int QT>
struct Stage {
  static constexpr int BYTES = Fmt<QT>::KR * Fmt<QT>::GROUP_BYTES;
  static constexpr int CPR = (BYTES + 15 + 15) / 16;
  static constexpr int SLOT = 16 * (CPR | 1);
  static constexpr int LOADS = (16 * CPR + WAVE - 1) / WAVE;  // per lane
};

// B operand of group gl of a row's run (row: its first byte in LDS) for lane group lg: 8 codes as 4 dwords of bf16,
// and the scale (Q4_K: d sc, with dmin mn in mn)
template <int QT>
__device__ __forceinline__ u32x4 b_operand(const uint8_t* row, int gl, int lg, float& sc, float& mn) {
  if (QT == ARTLITE_Q4_0) {
    const uint8_t* blk = row + 18 * gl;
    sc = h2f(lds_u16(blk));
    const int sh = 4 * (lg >> 1);
    const uint32_t u0 = (lds_u32(blk + 2 + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
    const uint32_t u1 = (lds_u32(blk + 6 + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
    return nib8(u0, u1);
  } else if (QT == ARTLITE_Q8_0) {
    const uint8_t* blk = row + 34 * gl;
    sc = h2f(lds_u16(blk));
    return byte8(lds_u32(blk + 2 + 8 * lg) ^ 0x80808080u, lds_u32(blk + 6 + 8 * lg) ^ 0x80808080u);
  } else {  // Q4_K: group gl % 8 of the super-block at gl / 8
    const uint8_t* sb = row + 144 * (gl >> 3);
    const int g = gl & 7;
    const float d = h2f(lds_u16(sb)), dmin = h2f(lds_u16(sb + 2));
    const uint8_t* s6 = sb + 4;
    const int q6 = g < 4 ? s6[g] & 63 : (s6[8 + g - 4] & 15) | ((s6[g - 4] >> 6) << 4);
    const int m6 = g < 4 ? s6[4 + g] & 63 : (s6[8 + g - 4] >> 4) | ((s6[4 + g - 4] >> 6) << 4);
    sc = __fmul_rn(d, float(q6));
    mn = __fmul_rn(dmin, float(m6));
    const uint8_t* qs = sb + 16 + 32 * (g >> 1) + 8 * lg;
    const int sh = 4 * (g & 1);
    return nib8((lds_u32(qs) >> sh) & 0x0F0F0F0Fu, (lds_u32(qs + 4) >> sh) & 0x0F0F0F0Fu);
  }
}

// One 16-row block's products over groups [0, gn) of its K-range (rows at rowp in LDS; this lane's A row at arow
// in LDS; cin: -OFF group sums), ni scale FMAs per group (the lane's output rows that hold tokens).
template <int QT, int AP, int KR, bool FULL>
__device__ __forceinline__ f32x4 block_products(f32x4 acc, const uint8_t* rowp, const uint8_t* arow, int a_plane,
                                                const float (*gsum)[16], int g0, int gn, int lg, int ni) {
#pragma unroll 8
  for (int gl = 0; gl < (FULL ? KR : gn); gl++) {
    const int g = g0 + gl;
    const u32x4 ahi = *reinterpret_cast<const u32x4*>(arow + 64 * g);
    const f32x4 cin = *reinterpret_cast<const f32x4*>(&gsum[g][4 * lg]);
    float sc, mn = 0.0f;
    const u32x4 b = b_operand<QT>(rowp, gl, lg, sc, mn);
    f32x4 p = mfma(ahi, b, cin);
    if (AP == 2) p = mfma(*reinterpret_cast<const u32x4*>(arow + a_plane + 64 * g), b, p);
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (i < ni) {
        acc[i] = __builtin_fmaf(sc, p[i], acc[i]);
        if (QT == ARTLITE_Q4_K) acc[i] = __builtin_fmaf(mn, cin[i] * (1.0f / Fmt<QT>::OFF), acc[i]);
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
  // LDS: the waves' slots (4 x 16 rows) | the tile's A rows | group sums [ng][16] (by MFMA row) | up accumulators
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* as = lds + 4 * 16 * S::SLOT;
  float(*gsum)[16] = reinterpret_cast<float(*)[16]>(as + DECODE_BM * arow_bytes);
  f32x4* xch = reinterpret_cast<f32x4*>(as + DECODE_BM * arow_bytes + ng * 16 * 4);

  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE, lg = lane >> 4, lr = lane & 15;
  int e = 0, s0, m_valid;
  if (a.tiles) {
    if (int64_t(blockIdx.x) >= *a.n_tiles) return;
    e = a.tiles[2 * blockIdx.x];
    s0 = a.tiles[2 * blockIdx.x + 1];
    m_valid = min(DECODE_BM, a.offsets[e + 1] - s0);
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
    const int64_t koff = int64_t(kr) * F::KR * F::GROUP_BYTES;
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
  // group sums by MFMA row m: gsum[g][m] = -OFF sum over group g of A[token_of_row(m)] (zero past the tile)
  for (int i = threadIdx.x; i < ng * 16; i += 256) {
    const int g = i / 16, m = i % 16, t = token_of_row(m);
    float sum = 0.0f;
    if (t < m_valid)
#pragma unroll
      for (int pl = 0; pl < AP; pl++) {
        const u32x4* p = reinterpret_cast<const u32x4*>(as + t * arow_bytes + pl * a_plane + 64 * g);
#pragma unroll
        for (int j = 0; j < 4; j++) {
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
        my + lr * S::SLOT + ((int64_t(r) * a.row_bytes + int64_t(kr) * F::KR * F::GROUP_BYTES) & 15);
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
                     size_t(a.K / 32) * 16 * 4 + (SWIGLU ? 2 * BLK * WAVE * 16 : 0);
  if (a.a_lo)
    k_gemm_decode<QT, SWIGLU, 2, BLK><<<grid, block, lds, s>>>(a);
  else
    k_gemm_decode<QT, SWIGLU, 1, BLK><<<grid, block, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- Prefill tiling (k_gemm_prefill): a workgroup is one tile of PREFILL_BM sorted rows of one expert times 128
// weight rows (of each matrix), as 2 x 4 waves: wave (wm, wn) takes rows of A 64 wm .. + 64 (4 MFMA row blocks) and
// weight rows 32 wn .. + 32 (2 column blocks per matrix; SwiGLU: those rows of gate and of up, so h is formed in
// the wave). K streams in stages of two 32-value groups through a ring of R LDS stages filled by DMA
// (global_load_lds, issued by asm so that the compiler, which would wait for every DMA in flight before any LDS read
// it sees, does not know of them): every wave issues the same number of loads per stage (past the last stage, loads
// of stage 0 again), so each wait is a fixed count of this wave's loads, and R - 1 stages are in flight while one
// computes. The operands of the next group are read from LDS while the current group computes; stage st + 1's wait
// and barrier sit between stage st's two groups, after which the slot of stage st (both groups in registers by
// then) takes stage st + R.
// A rows sit in LDS as 16-byte chunks of 8 values, XOR-swizzled by row, so the 16 rows of an operand read fall in
// different banks; a weight row's stage bytes (two blocks) sit packed, read as aligned dwords (a block's codes start
// 2 bytes into it: the first block's are shifted into place with alignbit).
template <int QT>
struct PStage {
  static constexpr int GB = Fmt<QT>::GROUP_BYTES;
  static constexpr int ROW = 2 * GB;  // weight bytes of a row per stage
  static constexpr int DW = ROW / 4;  // its dwords (9 / 17)
};
static_assert(PStage<ARTLITE_Q4_0>::ROW % 4 == 0 && PStage<ARTLITE_Q8_0>::ROW % 4 == 0, "stage rows in dwords");

template <int QT, bool SWIGLU, int AP>
struct PLayout {
  static constexpr int NM = SWIGLU ? 2 : 1;
  static constexpr int WAVES = 8, THREADS = 64 * WAVES;
  static constexpr int WROWS = 128 * NM;                        // weight rows of a workgroup
  static constexpr int ACH = 8 * AP;                            // 16-byte chunks of an A row per stage
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

// the operands of one 32-value group: per row block and A plane, the lane's 8 bf16 of A; per column block, the
// weight row's fp16 scale and 8 of its code bytes (Q4_0: 16 nibbles, 8 of them the lane's)
template <int QT, int NB, int AP>
struct POps {
  u32x4 a[4][AP];
  uint32_t sc[NB];
  uint32_t cw[NB][2];
};

template <int QT, bool SWIGLU, int AP>
__global__ __launch_bounds__(512) void k_gemm_prefill(const GemmArgs a) {
  using F = Fmt<QT>;
  using L = PLayout<QT, SWIGLU, AP>;
  constexpr int NM = L::NM, NB = 2 * NM;  // column blocks per wave (matrix-major)
  constexpr int MB = 4;                   // row blocks per wave
  constexpr int R = L::R;
  constexpr int ROW = PStage<QT>::ROW, GB = F::GROUP_BYTES;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & (WAVE - 1), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lg = lane >> 4, lr = lane & 15, wm = wv & 1, wn = wv >> 1;
  int e = 0, s0, m_valid;
  if (a.tiles) {
    if (int64_t(blockIdx.x) >= *a.n_tiles) return;
    e = a.tiles[2 * blockIdx.x];
    s0 = a.tiles[2 * blockIdx.x + 1];
    m_valid = min(PREFILL_BM, a.offsets[e + 1] - s0);
  } else {
    s0 = blockIdx.x * PREFILL_BM;
    m_valid = min(PREFILL_BM, a.dense_rows - s0);
  }
  const int n0 = blockIdx.y * 128;
  const int stages = a.K / 64;

  // chunk swizzle of row r: the 16 rows an operand read touches hit 16 different 16-byte bank slots
  auto swz = [](int r) { return AP == 2 ? (r & 15) : ((r >> 1) & 7); };
  // The lane's DMA sources. A: instruction i writes chunks (wv AI + i) 64 + lane of the stage's A region; chunk p
  // holds row r = p / ACH, physical chunk c = p % ACH, which is logical chunk c ^ swz(r) (logical: plane c / 8, K
  // values 8 (c % 8) .. + 8 of the stage).
  const uint16_t* asrc[L::AI];
#pragma unroll
  for (int i = 0; i < L::AI; i++) {
    const int p = (wv * L::AI + i) * 64 + lane, r = p / L::ACH, c = (p % L::ACH) ^ swz(r);
    const int rr = min(r, m_valid - 1);  // (rows past the tile repeat its last: their outputs are not stored)
    const int ar = a.a_gather ? a.order[s0 + rr] / a.topk : s0 + rr;
    asrc[i] = (AP == 2 && c >= 8 ? a.a_lo : a.a_hi) + int64_t(ar) * a.K + 8 * (c % 8);
  }
  // weights: instruction j writes dwords (wv BI + j) 64 + lane of the stage's weight region, row q / DW (matrix-major,
  // 128 rows each), dword q % DW of the row's stage bytes; dwords past the rows load the last one again (padding)
  const uint8_t* wsrc[L::BI];
#pragma unroll
  for (int j = 0; j < L::BI; j++) {
    const int q = min((wv * L::BI + j) * 64 + lane, L::WROWS * PStage<QT>::DW - 1);
    const int row = q / PStage<QT>::DW, dw = q % PStage<QT>::DW;
    const int mtx = NM == 2 ? row / 128 : 0, n = min(n0 + row % 128, a.N - 1);
    wsrc[j] = a.w[mtx] + int64_t(e) * a.expert_bytes + int64_t(n) * a.row_bytes + 4 * dw;
  }
  const uint32_t lbase = pf_lds_addr(lds);
  const uint32_t adst = lbase + wv * L::AI * 1024, bdst = lbase + L::ABYTES + wv * L::BI * 256;
  // the loads of stage j (past the last stage: stage 0 again) into ring slot j % R
  auto issue = [&](int j) {
    const int st = j < stages ? j : 0;
    const uint32_t so = (j % R) * L::SBYTES;
#pragma unroll
    for (int i = 0; i < L::AI; i++) pf_dma<16>(asrc[i] + 64 * st, adst + so + i * 1024);
#pragma unroll
    for (int i = 0; i < L::BI; i++) pf_dma<4>(wsrc[i] + st * ROW, bdst + so + i * 256);
  };

  // the lane's LDS read offsets in ring slot 0. A, row 64 wm + lr (row block mb at + 16 mb rows), group gl, plane pl:
  // the chunk of K 8 lg .. + 8. B, row 32 wn + lr (+ the column block's rows): its block gl.
  constexpr int AMB = 16 * L::ACH * 16;
  uint32_t aof[2][AP];
  {
    const int r = 64 * wm + lr, s = swz(r);
#pragma unroll
    for (int gl = 0; gl < 2; gl++)
#pragma unroll
      for (int pl = 0; pl < AP; pl++) aof[gl][pl] = r * L::ACH * 16 + ((8 * pl + 4 * gl + lg) ^ s) * 16;
  }
  const uint32_t bof = L::ABYTES + (32 * wn + lr) * ROW;
  const int sh = 4 * (lg >> 1);  // (Q4_0: the nibble half of lane group lg)
  auto brow = [](int nb) { return (nb / 2) * 128 + 16 * (nb % 2); };

  auto read = [&](POps<QT, NB, AP>& o, uint32_t so, int gl) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int pl = 0; pl < AP; pl++) {
        o.a[mb][pl] = *reinterpret_cast<const u32x4*>(lds + so + aof[gl][pl] + mb * AMB);
      }
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      const uint8_t* b = lds + so + bof + brow(nb) * ROW + gl * GB;  // (4-byte aligned: gl GB is 0 or 2 mod 4)
      o.sc[nb] = *reinterpret_cast<const uint16_t*>(b);
      // the 8 code bytes at b + 2 + CB: Q4_0 bytes 8 (lg & 1) .. + 8 (of which lane group lg takes the low nibbles
      // for lg < 2, else the high ones), Q8_0 bytes 8 lg .. + 8
      const int cb = QT == ARTLITE_Q4_0 ? 8 * (lg & 1) : 8 * lg;
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

  // the -OFF operand of the group sums (bf16, exact)
  const uint32_t noff = f32_to_bf16(-F::OFF) * 0x10001u;
  const u32x4 bneg = {noff, noff, noff, noff};
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[mb][nb] = f32x4{0, 0, 0, 0};
  // One group's products: the -OFF group sums (MFMAs against bneg) with the B operands decoded between them, then
  // the MB x NB products, each followed by the scale FMAs of the product two before it (the MFMA result's latency),
  // as sched_group_barrier orders them.
  auto compute = [&](const POps<QT, NB, AP>& o) {
    f32x4 cin[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      cin[mb] = mfma(o.a[mb][0], bneg, f32x4{0, 0, 0, 0});
      if (AP == 2) cin[mb] = mfma(o.a[mb][AP - 1], bneg, cin[mb]);
    }
    u32x4 b[NB];
    float d[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      if constexpr (QT == ARTLITE_Q4_0)
        b[nb] = nib8((o.cw[nb][0] >> sh) & 0x0F0F0F0Fu, (o.cw[nb][1] >> sh) & 0x0F0F0F0Fu);
      else
        b[nb] = byte8(o.cw[nb][0] ^ 0x80808080u, o.cw[nb][1] ^ 0x80808080u);
      d[nb] = h2f(o.sc[nb]);
    }
    f32x4 p[NB][MB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int mb = 0; mb < MB; mb++) {
        p[nb][mb] = mfma(o.a[mb][0], b[nb], cin[mb]);
        if (AP == 2) p[nb][mb] = mfma(o.a[mb][AP - 1], b[nb], p[nb][mb]);
      }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[mb][nb][i] = __builtin_fmaf(d[nb], p[nb][mb][i], acc[mb][nb][i]);
    constexpr int DEC = QT == ARTLITE_Q4_0 ? 7 : 18;  // decode VALU per column block (about)
#pragma unroll
    for (int mb = 0; mb < MB * AP; mb++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, (DEC * NB + MB * AP - 1) / (MB * AP), 0);
    }
#pragma unroll
    for (int t = 0; t < MB * NB; t++) {
      __builtin_amdgcn_sched_group_barrier(0x008, AP, 0);
      if (t >= 2) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
  };
  // waves whose 64 rows of A are all past the tile skip the products (rows past it otherwise repeat its last row)
  const bool active = 64 * wm < m_valid;

  POps<QT, NB, AP> cur, nxt;
#pragma unroll
  for (int j = 0; j < R; j++) issue(j);
  pf_wait<(R - 1) * L::LOADS>();  // (stage 0: R - 1 stages issued after it)
  pf_barrier();
  if (active) read(cur, 0, 0);
  for (int st = 0; st < stages; st++) {
    const uint32_t so = (st % R) * L::SBYTES;
    if (active) {
      read(nxt, so, 1);
      compute(cur);
    }
    if (st + 1 < stages) {
      pf_wait<(R - 2) * L::LOADS>();  // (stage st + 1: stages up to st + R - 1 issued)
      pf_barrier();
      issue(st + R);  // (into the slot of stage st, whose operands every wave holds in registers)
      if (active) read(cur, ((st + 1) % R) * L::SBYTES, 0);
    }
    if (active) compute(nxt);
  }
  pf_wait<0>();  // (the loads past the last stage land before the workgroup's LDS is released)

  // epilogue: lane output i of block (mb, nb): row of A 64 wm + 16 mb + 4 lg + i, weight row n0 + 32 wn + 16 (nb % 2)
  // + lr of matrix nb / 2
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = n0 + 32 * wn + 16 * j + lr;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 64 * wm + 16 * mb + 4 * lg + i;
        if (m >= m_valid) continue;
        const int64_t o = int64_t(s0 + m) * a.N + n;
        if constexpr (SWIGLU) {
          const float g = acc[mb][j][i], u = acc[mb][2 + j][i];
          const float h = g / (1.0f + expf(-g)) * u;
          const uint32_t hi = f32_to_bf16(h);
          a.h_hi[o] = uint16_t(hi);
          a.h_lo[o] = uint16_t(f32_to_bf16(h - bf16_to_f32(hi)));
        } else {
          a.y[o] = acc[mb][j][i];
        }
      }
    }
  }
}

template <int QT, bool SWIGLU, int AP>
int launch_prefill_ap(const GemmArgs& a, hipStream_t s) {
  using L = PLayout<QT, SWIGLU, AP>;
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + PREFILL_BM - 1) / PREFILL_BM;
  const dim3 grid(unsigned(tiles), unsigned((a.N + 127) / 128)), block(L::THREADS);
  constexpr size_t lds = size_t(L::R) * L::SBYTES;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_prefill<QT, SWIGLU, AP>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
  ART_HIP(attr);
  k_gemm_prefill<QT, SWIGLU, AP><<<grid, block, lds, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

template <int QT, bool SWIGLU>
int launch_prefill(const GemmArgs& a, hipStream_t s) {
  return a.a_lo ? launch_prefill_ap<QT, SWIGLU, 2>(a, s) : launch_prefill_ap<QT, SWIGLU, 1>(a, s);
}

bool prefill_supported(int qtype, int K, int N) {
  return (qtype == ARTLITE_Q4_0 || qtype == ARTLITE_Q8_0) && K > 0 && K % 64 == 0 && N > 0 && N % 128 == 0;
}

int launch_expert_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.K % 32 || (a.qtype == ARTLITE_Q4_K && a.K % 256))
    return fail(ARTLITE_EINVAL, "expert GEMM: K %d is not a multiple of the format's block", a.K);
  if (a.K / 32 > MAX_GROUPS) return fail(ARTLITE_EINVAL, "expert GEMM: K %d beyond %d", a.K, 32 * MAX_GROUPS);
  const bool swiglu = a.w[1] != nullptr;
  // tiles of PREFILL_BM rows (a tile list made for them, or dense rows enough to fill them): the prefill tiling
  const bool pre = a.tiles ? a.bm == PREFILL_BM
                            : a.dense_rows >= PREFILL_BM / 2 && prefill_supported(a.qtype, a.K, a.N);
  if (pre) {
    if (!prefill_supported(a.qtype, a.K, a.N))
      return fail(ARTLITE_EINVAL, "expert GEMM: prefill tiles of weight type %d, K %d, N %d", a.qtype, a.K, a.N);
    const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + PREFILL_BM - 1) / PREFILL_BM;
    if (tiles <= 0) return ARTLITE_OK;
    if (a.qtype == ARTLITE_Q4_0) return swiglu ? launch_prefill<ARTLITE_Q4_0, true>(a, s) : launch_prefill<ARTLITE_Q4_0, false>(a, s);
    return swiglu ? launch_prefill<ARTLITE_Q8_0, true>(a, s) : launch_prefill<ARTLITE_Q8_0, false>(a, s);
  }
  if (a.tiles && a.bm != DECODE_BM) return fail(ARTLITE_EINVAL, "expert GEMM: tiles of %d rows", a.bm);
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + DECODE_BM - 1) / DECODE_BM;
  if (tiles <= 0) return ARTLITE_OK;
#define ART_DISPATCH(QT) return swiglu ? launch_decode<QT, true, 2>(a, s) : launch_decode<QT, false, 2>(a, s)
  switch (a.qtype) {
    case ARTLITE_Q4_0: ART_DISPATCH(ARTLITE_Q4_0);
    case ARTLITE_Q8_0: ART_DISPATCH(ARTLITE_Q8_0);
    case ARTLITE_Q4_K: ART_DISPATCH(ARTLITE_Q4_K);
    default: return fail(ARTLITE_EINVAL, "expert GEMM: unsupported weight type %d", a.qtype);
  }
#undef ART_DISPATCH
}

// ---- combine: y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] (the reference CombineOperator's sum,
// src/artlite/moe/gather.py:12-18: the shared term first, then the slots in order, fp32)
__global__ void k_combine(const float* __restrict__ Y, const int32_t* __restrict__ slot, const float* __restrict__ w,
                          int k, const float* __restrict__ ys, const float* __restrict__ ws_logit, int ws_sigmoid,
                          int64_t T, int H, float* __restrict__ y) {
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
  reinterpret_cast<float4*>(y + t * H)[h4] = acc;
}

int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, float* y, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (H % 4) return fail(ARTLITE_EINVAL, "combine: H %d not a multiple of 4", H);
  const dim3 grid(unsigned((H / 4 + 255) / 256), unsigned(T)), block(256);
  k_combine<<<grid, block, 0, s>>>(Y, slot, w, k, ys, ws_logit, ws_sigmoid, T, H, y);
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
