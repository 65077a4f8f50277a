// The prefill tiles: the experts' grouped GEMMs at prefill sizes (tens to hundreds of rows per expert) over raw GGUF
// Q4_0 / Q8_0 / Q4_K blocks, on gfx950's fp16 MFMA (v_mfma_f32_16x16x32_f16).
//
// Numerics. A is fp16 rows, each token's row scaled by a power of two (2^-in_exp[token]) so that its largest |x| sits
// in [2^14, 2^15): bf16 activations convert exactly, fp32 ones round once (2^-11). Each lane decodes its 8 codes of a
// block to fp16 d (q - 8) (Q4_0) or d q (Q8_0): the code exactly, the product with the block's fp16 scale rounded
// once (2^-11 relative); Q4_K: q (d sc) - dmin m in fp32 (the products exact), rounded once to fp16. The MFMA
// accumulates all of K in fp32, so no per-group scale work is left. Each row's factors (x, y) undo the scales: the
// SwiGLU launch writes h = silu(x g) (x u) y in fp16 (y bounds |h| below 2^15); the plain launch writes fp16 y sum
// (y bounds it below 2^15; the row's true values are x times these) or fp32 x y sum.
//
// Shape of the work. An expert's sorted rows are cut into tiles of at most 256 rows of nearly equal size
// (balanced_rows: 270 rows are two tiles of 144 and 126, not 256 and 14). An item is one tile times 256 staged
// weight rows (SwiGLU: 128 rows of gate and the same 128 of up; plain: 256 rows). A workgroup is 8 waves, two per
// SIMD: wave w takes all of the tile's rows (up to 16 MFMA row blocks) times 32 weight rows (2 column blocks: SwiGLU
// gate rows 16 w .. + 16 and the same up rows, so h forms in the wave; plain rows 32 w .. + 32), 128 fp32
// accumulators per lane; the K loop is instantiated per even row-block count so that they stay in registers.
// Per 32-value group a wave reads an A operand from LDS per row block and decodes 2 B operands (Q4_0: about 13
// VALU each; Q4_K: about 25, in fp32).
//
// Data movement. K streams in stages of 64 values (two groups) through a ring of R = 3 LDS slots filled by DMA
// (global_load_lds, issued by asm from uniform bases with 32-bit lane offsets, so that the compiler, which would wait
// for every DMA in flight before any LDS read it sees, does not know of them), the stage's loads spread over the
// step's MFMA iterations. Every wave issues the same loads per stage, so each wait is a fixed count of this wave's
// loads: at step st, stage st must have landed and stage st + 1 may still be in flight; after the barrier (every
// wave past its reads of the previous slot) stage st + 2 is issued into that slot, two steps ahead. Each item's row
// metadata (tokens, scale factors) arrives by DMA too, and the workgroup's item table is read once at its start, so
// no global load is waited for in the K loop. The issue side runs on across items (the next item's first stages load
// while the current one finishes and writes its epilogue) and, past the last item, reloads a stage of it (dummies
// keep the counts fixed).
// A rows sit in LDS as 16-byte chunks of 8 values, XOR-swizzled by row (16 rows of an operand read in different
// banks); a weight row's stage bytes (two blocks, 36 / 68 B; Q4_K: the super-block header and the quarter's 32
// code bytes, in two regions) sit packed, read as aligned dwords (Q4_0 / Q8_0: the first block's codes start 2 bytes
// into it, shifted into place with alignbit).
// MFMA layout (16x16x32): lane l holds A row l % 16 and B column l % 16, both with K values 8 (l / 16) .. + 8;
// C column l % 16, rows 4 (l / 16) .. + 4. The decoded weights are the A operand and the activations B, so C is the
// output transposed: a lane holds one tile row's 4 consecutive output columns, stored as one 8 / 16 B write.
#include "experts.h"
#include "route.h"

#include <utility>

namespace artlite {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int TILE_ROWS = 256;  // A rows of a tile, at most

template <int QT>
struct PG {
  // Q4_K: a stage is a quarter of a 256-value super-block (144 B: d, dmin, 12 bytes of 6-bit scales and mins, 128
  // code bytes); a row's stage bytes are its super-block's 16-byte header and the quarter's 32 code bytes, staged in
  // two regions (the headers of the item's 256 rows, then their codes), each DMA instruction reading one of them.
  // PQ6 (the prefill layout of the other block formats, PREFILL_PQ6): a stage is 64 bytes of a row, four 16-byte
  // chunks (the scales, two of nibbles, one of crumbs), staged whole, each row's chunks swizzled by pq6_swz.
  static constexpr bool K4 = QT == ARTLITE_Q4_K;
  static constexpr bool P6 = QT == PREFILL_PQ6;
  static constexpr bool F32D = K4 || P6;                  // (weights decoded in fp32: pg_k4_word)
  static constexpr int GB = QT == ARTLITE_Q4_0 ? 18 : 34;  // bytes of a 32-value block (Q4_0, Q8_0)
  static constexpr int WN = 256;                          // weight rows staged per item
  static constexpr int WROW = K4 ? 48 : P6 ? 64 : 2 * GB;  // stage bytes of a staged weight row (two blocks)
  static constexpr int WDW = WROW / 4;                    // its dwords (9 / 17 / 12 / 16)
  static constexpr int THREADS = 512;                     // 8 waves, two per SIMD
  static constexpr int ABYTES = TILE_ROWS * 128;          // a stage of A: 64 fp16 per row
  static constexpr int AI = ABYTES / 16 / THREADS;        // A DMAs (16 B) per lane per stage
  // Q4_0: a row's 36 stage bytes in three 12-byte DMA pieces, 12 instructions a stage: waves 0-3 issue two, waves 4-7
  // (the younger wave of each SIMD, whose step is the longer) one. A 12-byte DMA writes each lane's piece into 16 bytes
  // of LDS (its last dword untouched), so a row takes 48 LDS bytes, piece k at 16 k: stage byte x at x + 4 (x / 12).
  // Else 4-byte pieces, the same count for every wave, a row's stage bytes packed.
  static constexpr bool X3 = QT == ARTLITE_Q4_0;
  // weight DMAs per lane per stage (at most; PQ6: 16-byte pieces, 4 a row, 2 per lane)
  static constexpr int BI = X3 ? 2 : P6 ? WN * 4 / THREADS : (WN * WDW + THREADS - 1) / THREADS;
  static constexpr int WLDS = X3 ? 48 : WROW;             // LDS bytes of a staged weight row
  static constexpr int KHDR = WN * 16;                    // Q4_K: the header region's bytes (the codes follow)
  static constexpr int WBYTES = X3 || P6 ? WN * WLDS : BI * THREADS * 4;  // (4-byte pieces: the last dwords padding)
  static constexpr int SBYTES = ABYTES + WBYTES;
  static constexpr int MI = 2;           // item metadata DMAs (4 B) per lane per stage
  static constexpr int META = MI * THREADS * 4;  // an item's metadata: 256 row tokens (int), 256 row factors (float2),
                                                 // padding
  static constexpr int LOADS = AI + BI + MI;  // (X3: waves 4-7 issue one fewer)
  static constexpr int R = 3;
  static constexpr int MAXQ = 128;  // items of a workgroup the item table holds
  static constexpr int LDS = R * SBYTES + 2 * META + MAXQ * 16;
  static_assert(AI * 16 * THREADS == ABYTES, "whole A DMAs");
  static_assert(META >= 3 * 1024, "metadata");
  static_assert(K4 || 128 * WDW % 64 == 0, "a wave's weight DMA reads one matrix (gate or up)");
  static_assert(!X3 || (WROW == 36 && GB == 18 && WN * 3 == 12 * 64 && 128 * 3 % 64 == 0),
                "Q4_0: 12 DMAs of 12-byte pieces");
  static_assert(!K4 || (BI == 6 && WN * WDW == BI * THREADS), "Q4_K: two header and four code DMAs, no padding");
  static_assert(!P6 || (BI == 2 && WBYTES == WN * 64 && 128 * 4 == THREADS), "PQ6: a DMA of gate rows, one of up's");
  static_assert(LDS <= LDS_BYTES, "LDS");
  static_assert((R - 1) * LOADS < 64, "vmcnt");
};

// the LDS row of weight row r with 48-byte rows (and back: an involution): bit 2 flipped where bit 4 is set, so that
// the 16 rows a lane group reads at once sit in distinct banks (12-dword rows repeat their bank every 16 rows, and the
// plain products' lanes read rows r and r + 16 together)
__device__ __forceinline__ int pg_x3_row(int r) { return r ^ (((r >> 4) & 1) << 2); }

// PQ6: the LDS chunk of a staged row r's chunk c is c ^ pq6_swz(r) (rows 64 bytes apart repeat their banks every 4 rows:
// the 16 rows a lane group reads, SwiGLU's consecutive ones or the plain products' runs of 4 rows 8 apart, take 4
// different chunk orders within each set of rows that share banks)
__device__ __forceinline__ int pq6_swz(int r) { return ((r >> 2) ^ (r >> 3)) & 3; }

template <int N>
__device__ __forceinline__ void pg_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// until only the window just issued is in flight (wv: the wave; with 12-byte weight pieces waves 4-7 issue one load
// fewer a window)
template <int QT>
__device__ __forceinline__ void pg_wait_window(int wv) {
  if (PG<QT>::X3 && wv >= 4)
    pg_wait<PG<QT>::LOADS - 1>();
  else
    pg_wait<PG<QT>::LOADS>();
}

// every wave's LDS reads done, then the workgroup barrier
__device__ __forceinline__ void pg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t pg_lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// One DMA of SIZE bytes per lane from base (uniform) + off (the lane's 32-bit byte offset) into LDS at lds (uniform) +
// SIZE lane. M0 carries the LDS address; no compiler-generated code in this kernel uses M0 (the asm sets it before
// each load, with the one wait state a load after an M0 write needs).
template <int SIZE>
__device__ __forceinline__ void pg_dma(const void* base, uint32_t off, uint32_t lds) {
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
  else if constexpr (SIZE == 12)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx3 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                 0);
}

// v as a value the compiler cannot hoist: what the rare paths (item switches, epilogues) compute from a lane's index
// is computed there, not kept in registers (or spilled) throughout the K loop
__device__ __forceinline__ int pg_fresh(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// f(std::integral_constant<int, i>{}) for i = 0 .. N - 1, expanded at compile time (loops this long and this large
// are not always unrolled, and their registers, accumulators included, must be indexed by constants)
template <typename F, int... I>
__device__ __forceinline__ void pg_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void pg_for(F&& f) {
  pg_for_impl(f, std::make_integer_sequence<int, N>{});
}

// A column block's operand (a lane's 8 weights of a group, as 4 words of fp16 pairs) is decoded in 5 tasks that a step
// spreads over its iterations (the matrix cores take only a few other instructions per MFMA for free): the
// preparation, then the 4 words. PGPrep holds what the words take: the code dwords (Q4_0: masked to its nibbles;
// Q8_0: sign bits flipped; Q4_K: each byte < 16), and the scale (Q4_0 / Q8_0: as an fp16 pair; Q4_K: the sub-block's
// scale s and min o in fp32).
struct PGPrep {
  uint32_t v0, v1, d;
  float s, o;
};

// Q4_0 / Q8_0 decode of a lane's 8 weights to fp16: the code bytes spread into fp16 1024 + c (c < 256 exact, one perm
// per two), the offset taken off exactly by one packed FMA (Q4_0's high nibbles, kept in place as 16 q, are scaled by
// 1/16 in it), then the product with the block's scale, rounded once.
template <int QT>
struct PGDecode {
  uint32_t msk;
  f16x2 mul, add;
  __device__ __forceinline__ explicit PGDecode(int lg) {
    if constexpr (QT == ARTLITE_Q4_0) {
      const bool hi = lg >= 2;  // (lane groups 2, 3 hold K values 16 .. 31 of a block: the high nibbles)
      msk = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
      mul = hi ? f16x2{_Float16(0.0625f), _Float16(0.0625f)} : f16x2{_Float16(1.0f), _Float16(1.0f)};
      add = hi ? f16x2{_Float16(-72.0f), _Float16(-72.0f)} : f16x2{_Float16(-1032.0f), _Float16(-1032.0f)};
    } else {
      msk = 0x80808080u;  // (Q8_0: the sign bits flipped, c = q + 128)
      mul = f16x2{_Float16(1.0f), _Float16(1.0f)};
      add = f16x2{_Float16(-1152.0f), _Float16(-1152.0f)};
    }
  }
  __device__ __forceinline__ PGPrep prep(uint32_t c0, uint32_t c1, uint32_t sc) const {
    PGPrep p;
    p.v0 = QT == ARTLITE_Q4_0 ? c0 & msk : c0 ^ msk;
    p.v1 = QT == ARTLITE_Q4_0 ? c1 & msk : c1 ^ msk;
    p.d = sc | (sc << 16);
    return p;
  }
  __device__ __forceinline__ uint32_t word(const PGPrep& p, int j) const {
    const uint32_t w = __builtin_amdgcn_perm(0x64646464u, j < 2 ? p.v0 : p.v1, j & 1 ? 0x04030402u : 0x04010400u);
    const f16x2 c = __builtin_bit_cast(f16x2, w) * mul + add;  // (exact: the code less its offset)
    return __builtin_bit_cast(uint32_t, c * __builtin_bit_cast(f16x2, p.d));
  }
};

// Q4_K: the scale and min of the lane's two sub-blocks of stage quarter qi (sub-blocks 2 qi, 2 qi + 1) from its row's
// super-block header h (d, dmin; 12 bytes of 6-bit scales and mins, packed as the format packs them: sub-blocks 0-3
// in the low 6 bits of bytes 0-3 (scales) and 4-7 (mins), sub-blocks 4-7 in the nibbles of bytes 8-11 with their top
// 2 bits in the top bits of bytes 0-7), as fp32: s = d sc and o = dmin m, both exact.
__device__ __forceinline__ void pg_k4_scales(const u32x4& h, int qi, float (&s)[2], float (&o)[2]) {
  const float d = float(__builtin_bit_cast(_Float16, uint16_t(h[0] & 0xFFFFu)));
  const float dm = float(__builtin_bit_cast(_Float16, uint16_t(h[0] >> 16)));
#pragma unroll
  for (int g = 0; g < 2; g++) {
    const int sh = 8 * (2 * (qi & 1) + g);  // (the sub-block's byte within each 4-byte run)
    uint32_t sc, m;
    if (qi < 2) {
      sc = (h[1] >> sh) & 63;
      m = (h[2] >> sh) & 63;
    } else {
      sc = ((h[3] >> sh) & 0xF) | (((h[1] >> (sh + 6)) & 3) << 4);
      m = ((h[3] >> (sh + 4)) & 0xF) | (((h[2] >> (sh + 6)) & 3) << 4);
    }
    s[g] = d * float(sc);
    o[g] = dm * float(m);
  }
}

// Q4_K: word j of the lane's 8 weights of one sub-block from its 8 codes (the bytes of v0, v1, each < 16): q s - o in
// fp32 (the product exact, one rounding), then rounded to fp16.
__device__ __forceinline__ uint32_t pg_k4_word(const PGPrep& p, int j) {
  const uint32_t v = j < 2 ? p.v0 : p.v1;
  const int sh = 16 * (j & 1);
  const f16x2 h = {_Float16(__builtin_fmaf(float((v >> sh) & 0xFF), p.s, -p.o)),
                   _Float16(__builtin_fmaf(float((v >> (sh + 8)) & 0xFF), p.s, -p.o))};
  return __builtin_bit_cast(uint32_t, h);
}

// An item: product p of the launch, expert e, its sorted rows s0 .. s0 + m_valid, output columns n0 .. (SwiGLU: + 128
// of gate and up; plain: + 256), the product's K stages
struct PGItem {
  int e, s0, m_valid, n0, p, stages;
};

// the column blocks of a product, its tiles (the tile list's count, or the dense rows' tiles)
template <bool SWIGLU>
__device__ __forceinline__ int pg_nbk(const PrefillProblem& P) {
  constexpr int WN = SWIGLU ? 128 : 256;
  return (P.N + WN - 1) / WN;
}
// dense rows: the rows of a tile
__host__ __device__ __forceinline__ int pg_dense_rows(const PrefillProblem& P) {
  return P.dense_tile > 0 ? P.dense_tile : balanced_rows(P.dense_rows, TILE_ROWS);
}
__device__ __forceinline__ int64_t pg_tiles(const PrefillProblem& P) {
  if (P.tiles) return *P.n_tiles;
  const int rows = pg_dense_rows(P);
  return (P.dense_rows + rows - 1) / rows;
}

// item w of product p (tile w / nbk, column block w % nbk); global loads: read once per workgroup, at its start
template <bool SWIGLU>
__device__ __forceinline__ PGItem pg_item(const PrefillProblem& P, int p, int64_t w) {
  constexpr int WN = SWIGLU ? 128 : 256;
  const int nbk = pg_nbk<SWIGLU>(P);
  const int tl = int(w / nbk);
  PGItem I;
  I.n0 = int(w % nbk) * WN;
  I.p = p;
  I.stages = P.K / 64;
  if (P.tiles) {
    I.e = P.tiles[2 * tl];
    I.s0 = P.tiles[2 * tl + 1];
    const int lo = P.offsets[I.e], hi = P.offsets[I.e + 1];
    I.m_valid = min(balanced_rows(hi - lo, TILE_ROWS), hi - I.s0);
  } else {
    const int rows = pg_dense_rows(P);
    I.e = 0;
    I.s0 = tl * rows;
    I.m_valid = min(rows, P.dense_rows - I.s0);
  }
  return I;
}

// The lane's DMA sources of an item at stage 0. A: instruction i of wave w writes chunks (4 i + w) 64 + lane of a
// stage's A region; chunk p holds row r = p / 8, physical chunk c = p % 8, which is logical chunk c ^ swz(r) (K values
// 8 c .. + 8 of the stage); rows past the tile's valid ones repeat its last (their outputs are not stored); a row's A
// row comes from the item's metadata in LDS (tok). Weights: instruction j of wave w writes dwords (8 j + w) 64 + lane
// of the stage's weight region: staged row q / WDW (SwiGLU: gate rows n0 .. + 128, then the same rows of up; plain:
// rows n0 .. + 256), dword q % WDW of the row's stage bytes (q = 512 j + tid: consecutive lanes read consecutive
// dwords of a row); rows past N load the last row. Offsets in bytes (A: from a.a; weights: from the instruction's
// matrix).
template <int QT, bool SWIGLU>
struct PGSrc {
  using L = PG<QT>;
  uint32_t a[L::AI];
  uint32_t w[L::BI];
  __device__ __forceinline__ static int swz(int r) { return (r >> 1) & 7; }
  // the A sources (a's row tokens from its metadata in LDS)
  __device__ __forceinline__ void set_a(const PrefillProblem& g, const PGItem& I, const int32_t* tok, int tid) {
    tid = pg_fresh(tid);
#pragma unroll
    for (int i = 0; i < L::AI; i++) {
      const int p = i * L::THREADS + tid, r = p >> 3, c = (p & 7) ^ swz(r);
      const int row = min(r, I.m_valid - 1);
      const int ar = g.row_a ? tok[row] : I.s0 + row;
      a[i] = (uint32_t(ar) * uint32_t(g.lda) + 8 * c) * 2;
    }
  }
  // the weight sources
  __device__ __forceinline__ void set_w(const PrefillProblem& g, const PGItem& I, int tid) {
    tid = pg_fresh(tid);
#pragma unroll
    for (int j = 0; j < L::BI; j++) {  // (dwords past the staged rows: padding, loading the last dword again)
      int row, dw;
      if constexpr (L::K4) {  // (instructions 0, 1: the headers, 4 dwords a row; 2 .. 5: the codes, 8 a row)
        const int q = (j < 2 ? j : j - 2) * L::THREADS + tid;
        row = j < 2 ? q >> 2 : q >> 3;
        dw = j < 2 ? q & 3 : q & 7;
      } else if constexpr (L::P6) {  // (piece q: LDS row q / 4, LDS chunk q % 4, which holds the row's chunk q % 4 ^ swz)
        const int q = j * L::THREADS + tid;
        row = q >> 2;
        dw = 4 * ((q & 3) ^ pq6_swz(row));
      } else if constexpr (L::X3) {  // (piece q: LDS row q / 3, its dwords 3 (q % 3) .. + 3; waves 4-7 have no second)
        const int q = min(j * L::THREADS + tid, L::WN * 3 - 1);
        row = pg_x3_row(q / 3);
        dw = 3 * (q % 3);
      } else {
        const int q = min(j * L::THREADS + tid, L::WN * L::WDW - 1);
        row = q / L::WDW;
        dw = q % L::WDW;
      }
      const int n = min(I.n0 + (SWIGLU ? row % 128 : row), g.N - 1);
      w[j] = uint32_t(I.e) * uint32_t(g.expert_bytes) + uint32_t(n) * uint32_t(g.row_bytes) + 4 * dw;
    }
  }
};

// The lane's metadata DMA sources of an item: dword u = j 512 + tid of the item's metadata (u < 256: the A row of
// tile row u, from row_a (without it, from row_scale: unread); u < 768: the row factors, float2 per row, as dwords,
// from row_scale; past that, padding: a reload of row 0's first dword), tile rows past the valid ones repeating the
// last. Offsets in bytes.
struct PGMeta {
  uint32_t m[2];
  __device__ __forceinline__ void set(const PGItem& I, int tid) {
    tid = pg_fresh(tid);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int u = j * 512 + tid;
      if (u < 256) {
        m[j] = uint32_t(I.s0 + min(u, I.m_valid - 1)) * 4;
      } else if (u < 768) {
        const int row = (u - 256) >> 1;
        m[j] = (uint32_t(I.s0 + min(row, I.m_valid - 1)) * 2 + (u & 1)) * 4;
      } else {
        m[j] = uint32_t(I.s0) * 4;
      }
    }
  }
};

// The DMA sources of the open window (an A stage, the weight stage after it, the metadata of item mq): uniform base
// pointers (at those stages) and destinations (dst: the A stage's slot; dstw: the weight region of the next slot);
// the lanes' offsets are in PGSrc and PGMeta.
struct PGBases {
  const uint8_t *ab, *wb0, *wb1, *mt, *ms;
  const uint8_t *wq0, *wq1;  // (Q4_K: the stage's code bytes; wb0, wb1 its super-block headers)
  uint32_t dst, dstw, mdst;
};

// The issue side: the A stream (item qa of na stages, stage sta of the window last opened, its ring slot) and the
// weight stream one stage ahead of it (item qw of nw stages, stage stw: its stage index runs one ahead, and so does
// its slot), the item whose metadata the windows carry (mq), their products' base pointers (A: ab0; weights: w0, w1;
// metadata: mt0, ms0), and the open window's bases. Past the last item a stream reloads stage 0 of it (dummies keep
// the counts fixed).
template <int QT, bool SWIGLU, bool MP>
struct PGIssue {
  PGSrc<QT, SWIGLU> src;
  PGMeta meta;
  PGBases b;
  int sta, qa, na, stw, qw, nw;
  int slot;
  int mq;
  const uint8_t *ab0, *w0, *w1, *mt0, *ms0;
  // the base pointers of product P for the A stream, the weight stream, the metadata
  __device__ __forceinline__ void use_a(const PrefillProblem& P) {
    ab0 = reinterpret_cast<const uint8_t*>(P.a);
  }
  __device__ __forceinline__ void use_w(const PrefillProblem& P) {
    w0 = P.w[0];
    w1 = SWIGLU ? P.w[1] : P.w[0];
  }
  __device__ __forceinline__ void use_m(const PrefillProblem& P) {
    ms0 = reinterpret_cast<const uint8_t*>(P.row_scale);
    mt0 = P.row_a ? reinterpret_cast<const uint8_t*>(P.row_a) : ms0;
  }
};

// One DMA of the open window: n < BI the weights' dwords (first: they come from HBM), then the A chunks, then the
// metadata's dwords (instruction i of wave w writes the region's bytes (8 i + w) 64 + lane times the DMA's size).
template <int QT, bool SWIGLU, bool MP>
__device__ __forceinline__ void pg_dma_n(int n, const PGIssue<QT, SWIGLU, MP>& is, int wv) {
  using L = PG<QT>;
  const PGBases& b = is.b;
  if (n < L::BI) {
    const int j = n;
    const uint8_t* base;
    if constexpr (L::K4)  // (headers: instruction 1 reads up's; codes: instructions 4, 5)
      base = j < 2 ? (SWIGLU && j == 1 ? b.wb1 : b.wb0) : (SWIGLU && j >= 4 ? b.wq1 : b.wq0);
    else if constexpr (L::X3 || L::P6)  // (X3: instructions 6 .. 11: up's rows, the wave's bases; P6: instruction 1)
      base = j == 0 ? b.wb0 : b.wb1;
    else
      base = SWIGLU && (j * L::THREADS + 64 * wv) >= 128 * L::WDW ? b.wb1 : b.wb0;
    if constexpr (L::X3) {
      if (j == 1 && wv >= 4) return;
      pg_dma<12>(base, is.src.w[j], b.dstw + (8 * j + wv) * 1024);
    } else if constexpr (L::P6) {
      pg_dma<16>(base, is.src.w[j], b.dstw + (8 * j + wv) * 1024);
    } else {
      pg_dma<4>(base, is.src.w[j], b.dstw + (8 * j + wv) * 256);
    }
  } else if (n < L::BI + L::AI) {
    const int i = n - L::BI;
    pg_dma<16>(b.ab, is.src.a[i], b.dst + (8 * i + wv) * 1024);
  } else {
    const int j = n - L::BI - L::AI;
    pg_dma<4>(j == 0 ? b.mt : b.ms, is.meta.m[j], b.mdst + (8 * j + wv) * 256);
  }
}

// The lane's fixed places: its A chunk in a slot for row block 0 of group 0 (aof0) and of group 1 (aof1); its staged
// weight row per column block (bof: the row's stage bytes in a slot; Q4_K: the row itself, its header and codes in
// their regions): SwiGLU gate rows 16 wv .. + 16 (column block 0) and the same rows of up (staged
// at + 128); plain: of rows 32 wv .. + 32, MFMA row i of block nb is row 32 wv + 8 (i / 4) + 4 nb + i % 4, so that a
// lane's outputs of the two blocks are 8 consecutive columns; cb its code bytes' offset in a block (Q4_K: in the
// quarter's 32 bytes, 8 lg). PQ6: bof is the row's scale chunk (its chunk c at bof ^ 16 c: rows are 64-byte aligned),
// and the launch's decode mode (pmode, poff: PrefillArgs) with the lane's half of a 32-value group (hi16).
template <int QT>
struct PGLane {
  uint32_t aof0, aof1, bof[2];
  int cb;
  int pmode;
  float poff;
  bool hi16;
  PGDecode<QT> dec;
  __device__ __forceinline__ PGLane(int lr, int lg, int wv, bool swiglu, int mode = 0, float off = 0.0f) : dec(lg) {
    const int sz = (lr >> 1) & 7;  // (the A rows' chunk swizzle, PGSrc::swz)
    aof0 = uint32_t(lr * 128 + ((0 + lg) ^ sz) * 16);
    aof1 = uint32_t(lr * 128 + ((4 + lg) ^ sz) * 16);
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const int row = swiglu ? 128 * nb + 16 * wv + lr : 32 * wv + 8 * (lr >> 2) + 4 * nb + (lr & 3);
      if constexpr (PG<QT>::K4)
        bof[nb] = uint32_t(row);
      else if constexpr (PG<QT>::P6)
        bof[nb] = uint32_t(PG<QT>::ABYTES + row * PG<QT>::WLDS + 16 * pq6_swz(row));
      else
        bof[nb] = uint32_t(PG<QT>::ABYTES + (PG<QT>::X3 ? pg_x3_row(row) : row) * PG<QT>::WLDS);
    }
    cb = QT == ARTLITE_Q4_0 ? 8 * (lg & 1) : 8 * lg;
    pmode = mode;
    poff = off;
    hi16 = (lg & 2) != 0;
  }
};

// The weight operands a step starts with: group 0's weights decoded, group 1's codes and scale (Q4_K: the code bytes'
// high nibbles, the second sub-block's scale and min). The previous step reads and decodes them in its last
// iterations, past the barrier that certifies their stage, so that a step's MFMAs start as soon as the last ones of
// the previous step. (Its first 4 A operands come the same way, through the ring of A operands.)
template <int QT>
struct PGOps {
  u32x4 b0[2];
  uint32_t c10[2], c11[2], sc1[2];  // (Q4_0 / Q8_0: the scale in sc1's high half)
  float ks1[2], ko1[2];
};

// What the decode of group 0 takes, as read from LDS: its code dwords and scale (Q4_0 / Q8_0: the codes start two bytes
// into d[0], and the scale is sc0's low half; shifted and masked at the decode, not at the read, so that the read's
// iteration does not wait for the data; Q4_K: d[0], d[1] the code bytes, h the super-block headers).
template <int QT>
struct PGRaw {
  uint32_t d[3][2], sc0[2];
  u32x4 h[2];
};

// The LDS reads of a step's weight codes from its slot s, all aligned dwords: per column block, group 0's from the lane
// group's code byte offset cb (Q4_0: 8 (lg & 1), both nibbles of those 8 bytes; Q8_0: 8 lg) two bytes past the
// block's scale (the row's first dword: the scale in its low half); group 1's from GB + 2 + cb (20 or 36), its scale
// the high half of the dword at GB - 2. Q4_K: the header, the code dwords 2 lg, 2 lg + 1. PQ6: the scale chunk, each
// group's nibble and crumb dwords.
template <int QT>
__device__ __forceinline__ void pg_read_codes(const uint8_t* s, const PGLane<QT>& ln, PGOps<QT>& o, PGRaw<QT>& r) {
  using L = PG<QT>;
  auto dw = [](const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); };
#pragma unroll
  for (int nb = 0; nb < 2; nb++) {
    if constexpr (L::P6) {  // (the scales; group g's nibble dword: chunk 1 + g, dword lg; its crumbs: chunk 3, dword
                            // 2 g + lg / 2)
      const uint32_t hd = ln.bof[nb], nbx = hd + 4 * uint32_t(ln.cb >> 3), cr = hd + 4 * uint32_t(ln.cb >> 4);
      r.h[nb] = *reinterpret_cast<const u32x4*>(s + hd);
      r.d[0][nb] = dw(s + (nbx ^ 16u));
      r.d[1][nb] = dw(s + (cr ^ 48u));
      r.d[2][nb] = dw(s + (nbx ^ 32u));
      r.sc0[nb] = dw(s + (cr ^ 48u) + 8);
    } else if constexpr (L::K4) {
      r.h[nb] = *reinterpret_cast<const u32x4*>(s + L::ABYTES + ln.bof[nb] * 16);
      const uint8_t* c = s + L::ABYTES + L::KHDR + ln.bof[nb] * 32 + ln.cb;
      r.d[0][nb] = dw(c);
      r.d[1][nb] = dw(c + 4);
    } else if constexpr (L::X3) {  // (the same dwords from the 48-byte LDS rows: cb 0 or 8, cx its image 0 or 12)
      const uint8_t* row = s + ln.bof[nb];
      const int cx = ln.cb + (ln.cb >> 1);
      r.d[0][nb] = dw(row + ln.cb);
      r.d[1][nb] = dw(row + cx + 4);
      r.d[2][nb] = dw(row + cx + 8);
      r.sc0[nb] = dw(row);
      o.c10[nb] = dw(row + cx + 24);
      o.c11[nb] = dw(row + ln.cb + 32);
      o.sc1[nb] = dw(row + 20);
    } else {
      const uint8_t* row = s + ln.bof[nb];
      r.d[0][nb] = dw(row + ln.cb);
      r.d[1][nb] = dw(row + ln.cb + 4);
      r.d[2][nb] = dw(row + ln.cb + 8);
      r.sc0[nb] = dw(row);
      o.c10[nb] = dw(row + L::GB + 2 + ln.cb);
      o.c11[nb] = dw(row + L::GB + 6 + ln.cb);
      o.sc1[nb] = dw(row + L::GB - 2);
    }
  }
}

// A operand j < 4 of a step from its slot s: iteration j's (group j < MBN ? 0 : 1, row block j % MBN; small: the
// step's tile has 2 row blocks, so operands 2, 3 are group 1's row blocks 0, 1)
template <int QT>
__device__ __forceinline__ u32x4 pg_read_a0(const uint8_t* s, const PGLane<QT>& ln, bool small, int j) {
  const uint32_t o = j < 2 ? ln.aof0 + j * 2048 : small ? ln.aof1 + (j - 2) * 2048 : ln.aof0 + j * 2048;
  return *reinterpret_cast<const u32x4*>(s + o);
}

// PQ6: the lane's 8 codes of a group (values 8 lg .. + 8 of its 32) as two dwords of bytes, from its nibble dword n
// (byte k: value k's low 4 bits, value k + 4's in the high nibble) and its crumb dword x (byte k: the high 2 bits of
// lane group 2 m + 1's values k and k + 4 in bits 0-3, lane group 2 m's in bits 4-7); mode 2 (IQ4): the nibble is an
// index of IQ4's table, whose value + 128 is the code (the offset 128 comes off in the decode)
__device__ __forceinline__ void pq6_codes(uint32_t n, uint32_t x, bool odd, int mode, uint32_t& v0, uint32_t& v1) {
  const uint32_t lo0 = n & 0x0F0F0F0Fu, lo1 = (n >> 4) & 0x0F0F0F0Fu;
  if (mode == 2) {
    v0 = iq4_int8(lo0) ^ 0x80808080u;
    v1 = iq4_int8(lo1) ^ 0x80808080u;
  } else {
    const uint32_t y = odd ? x << 4 : x;
    v0 = lo0 | (y & 0x30303030u);
    v1 = lo1 | ((y >> 2) & 0x30303030u);
  }
}

// PQ6: the scale s and the offset o of the lane's 8 values of group g (w = s c - o) from the row's scale chunk h: modes
// 0, 2: per 16 values s = h[2 g + hi16], o = off s (exact: off a power of two); mode 1: per 32, (s, o) = (h[2 g],
// h[2 g + 1])
template <int QT>
__device__ __forceinline__ void pq6_scale(const u32x4& h, int g, const PGLane<QT>& ln, float& s, float& o) {
  const float a = __uint_as_float(h[2 * g]), b = __uint_as_float(h[2 * g + 1]);
  if (ln.pmode == 1) {
    s = a;
    o = b;
  } else {
    s = ln.hi16 ? b : a;
    o = s * ln.poff;
  }
}

// The preparation of group 0's operand of column block nb from what was read (Q4_K: also group 1's codes, scale and
// min into o; qi the stage's quarter of its super-block), and a word of an operand.
template <int QT>
__device__ __forceinline__ PGPrep pg_prep0(PGOps<QT>& o, const PGRaw<QT>& r, const PGLane<QT>& ln, int qi, int nb) {
  if constexpr (PG<QT>::P6) {  // (group 1's codes, scale and offset into o)
    const bool odd = (ln.cb >> 3) & 1;
    pq6_codes(r.d[2][nb], r.sc0[nb], odd, ln.pmode, o.c10[nb], o.c11[nb]);
    pq6_scale<QT>(r.h[nb], 1, ln, o.ks1[nb], o.ko1[nb]);
    PGPrep p;
    pq6_codes(r.d[0][nb], r.d[1][nb], odd, ln.pmode, p.v0, p.v1);
    pq6_scale<QT>(r.h[nb], 0, ln, p.s, p.o);
    return p;
  } else if constexpr (PG<QT>::K4) {
    float ks[2], ko[2];
    pg_k4_scales(r.h[nb], qi, ks, ko);
    o.ks1[nb] = ks[1];
    o.ko1[nb] = ko[1];
    o.c10[nb] = (r.d[0][nb] >> 4) & 0x0F0F0F0Fu;
    o.c11[nb] = (r.d[1][nb] >> 4) & 0x0F0F0F0Fu;
    PGPrep p;
    p.v0 = r.d[0][nb] & 0x0F0F0F0Fu;
    p.v1 = r.d[1][nb] & 0x0F0F0F0Fu;
    p.s = ks[0];
    p.o = ko[0];
    return p;
  } else {
    return ln.dec.prep(__builtin_amdgcn_alignbit(r.d[1][nb], r.d[0][nb], 16),
                       __builtin_amdgcn_alignbit(r.d[2][nb], r.d[1][nb], 16), r.sc0[nb] & 0xFFFFu);
  }
}

// the preparation of group 1's operand of column block nb (its codes read a step before)
template <int QT>
__device__ __forceinline__ PGPrep pg_prep1(const PGOps<QT>& o, const PGLane<QT>& ln, int nb) {
  if constexpr (PG<QT>::F32D) {
    PGPrep p;
    p.v0 = o.c10[nb];
    p.v1 = o.c11[nb];
    p.s = o.ks1[nb];
    p.o = o.ko1[nb];
    return p;
  } else {
    return ln.dec.prep(o.c10[nb], o.c11[nb], o.sc1[nb] >> 16);
  }
}

template <int QT>
__device__ __forceinline__ uint32_t pg_word(const PGPrep& p, const PGLane<QT>& ln, int j) {
  if constexpr (PG<QT>::F32D)
    return pg_k4_word(p, j);
  else
    return ln.dec.word(p, j);
}

// group 0's whole operand of column block nb (the set-up's, for the first step)
template <int QT>
__device__ __forceinline__ void pg_decode0(PGOps<QT>& o, const PGRaw<QT>& r, const PGLane<QT>& ln, int qi, int nb) {
  const PGPrep p = pg_prep0<QT>(o, r, ln, qi, nb);
#pragma unroll
  for (int j = 0; j < 4; j++) o.b0[nb][j] = pg_word<QT>(p, ln, j);
}

// silu(g) u with the hardware's exp2 and reciprocal (each within an ulp or two of fp32; the fp16 rounding of h,
// 2^-11, dominates)
__device__ __forceinline__ float pg_swiglu(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-1.4426950408889634f * g);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The workgroup's state shared by its items.
struct PGCtx {
  uint8_t* lds;
  uint32_t lbase;
  int tid, wv, lane, lg, lr;
  int nq;
  int stages;  // (a launch of one product: its stages, those of every item)
  const int4* table;  // (in LDS) the items: (e + 2^24 p, s0, m_valid, n0 + 2^24 stages)
};

template <int QT>
__device__ __forceinline__ const int32_t* pg_tok(const PGCtx& c, int q) {
  return reinterpret_cast<const int32_t*>(c.lds + PG<QT>::R * PG<QT>::SBYTES + (q & 1) * PG<QT>::META);
}

template <int QT>
__device__ __forceinline__ const float2* pg_rowf(const PGCtx& c, int q) {  // (after the 256 row tokens)
  return reinterpret_cast<const float2*>(c.lds + PG<QT>::R * PG<QT>::SBYTES + (q & 1) * PG<QT>::META + 1024);
}

__device__ __forceinline__ int4 pg_pack(const PGItem& I) {
  return make_int4(I.e | (I.p << 24), I.s0, I.m_valid, I.n0 | (I.stages << 24));
}

// (MP: the launch holds several products; else every item is product 0's, known at compile time)
template <bool MP>
__device__ __forceinline__ PGItem pg_table(const PGCtx& c, int q) {
  const int4 v = c.table[q];
  const int x = __builtin_amdgcn_readfirstlane(v.x), w = __builtin_amdgcn_readfirstlane(v.w);
  return PGItem{x & 0xFFFFFF, __builtin_amdgcn_readfirstlane(v.y), __builtin_amdgcn_readfirstlane(v.z),
                w & 0xFFFFFF, MP ? x >> 24 : 0, w >> 24};
}

// the weight bases of stage sw (Q4_K: super-block sw / 4, its quarter sw % 4) from the weight stream's matrices w0, w1
template <int QT, bool SWIGLU>
__device__ __forceinline__ void pg_wbases(const uint8_t* w0, const uint8_t* w1, int sw, PGBases& b, int wv) {
  using L = PG<QT>;
  if constexpr (L::X3) {  // (the wave's own: instruction 0's matrix, instruction 1's)
    b.wb0 = (SWIGLU && wv >= 6 ? w1 : w0) + sw * L::WROW;
    b.wb1 = w1 + sw * L::WROW;
    b.wq0 = b.wq1 = nullptr;
  } else if constexpr (L::P6) {  // (instruction 0: rows 0 .. 127, gate's; 1: up's)
    b.wb0 = w0 + sw * L::WROW;
    b.wb1 = w1 + sw * L::WROW;
    b.wq0 = b.wq1 = nullptr;
  } else if constexpr (L::K4) {
    b.wb0 = w0 + (sw >> 2) * 144;
    b.wb1 = w1 + (sw >> 2) * 144;
    b.wq0 = b.wb0 + 16 + 32 * (sw & 3);
    b.wq1 = b.wb1 + 16 + 32 * (sw & 3);
  } else {
    b.wb0 = w0 + sw * L::WROW;
    b.wb1 = w1 + sw * L::WROW;
    b.wq0 = b.wq1 = nullptr;
  }
}

// Opens the next window: the A stream's next stage and the weight stream's (past an item's last stage, the next item:
// the A sources from its metadata, which landed two windows after the first that carried it; the weight sources from
// its table entry), into the next ring slot (weights: the slot after it), with the metadata of item mq (>= 0: a new one)
// into its buffer.
template <int QT, bool SWIGLU, bool MP>
__device__ __forceinline__ void pg_open(const PrefillArgs& a, const PGCtx& c, PGIssue<QT, SWIGLU, MP>& is, int mq) {
  using L = PG<QT>;
  if (mq >= 0 && mq != is.mq) {
    is.mq = mq;
    const PGItem M = pg_table<MP>(c, mq);
    is.meta.set(M, c.tid);
    is.use_m(a.p[M.p]);
  }
  is.slot = is.slot + 1 == L::R ? 0 : is.slot + 1;
  if (is.qa < c.nq && ++is.sta == (MP ? is.na : c.stages)) {
    is.sta = 0;
    if (++is.qa < c.nq) {
      const PGItem A = pg_table<MP>(c, is.qa);
      is.src.set_a(a.p[A.p], A, pg_tok<QT>(c, is.qa), c.tid);
      is.use_a(a.p[A.p]);
      is.na = A.stages;
    }
  }
  if (is.qw < c.nq && ++is.stw == (MP ? is.nw : c.stages)) {
    is.stw = 0;
    if (++is.qw < c.nq) {
      const PGItem W = pg_table<MP>(c, is.qw);
      is.src.set_w(a.p[W.p], W, c.tid);
      is.use_w(a.p[W.p]);
      is.nw = W.stages;
    }
  }
  const int sa = __builtin_amdgcn_readfirstlane(is.qa < c.nq ? is.sta : 0);
  PGBases& b = is.b;
  // (one product: its pointers read from the kernel's arguments, which the compiler may reload rather than hold)
  PGIssue<QT, SWIGLU, MP> one;
  if constexpr (!MP) {
    one.use_a(a.p[0]);
    one.use_w(a.p[0]);
    one.use_m(a.p[0]);
  }
  const PGIssue<QT, SWIGLU, MP>& ptr = MP ? is : one;
  b.ab = ptr.ab0 + 128 * sa;
  pg_wbases<QT, SWIGLU>(ptr.w0, ptr.w1, __builtin_amdgcn_readfirstlane(is.qw < c.nq ? is.stw : 0), b, c.wv);
  b.ms = ptr.ms0;
  b.mt = c.wv < 4 ? ptr.mt0 : ptr.ms0;  // (the wave's metadata DMA 0)
  const int ws = is.slot + 1 == L::R ? 0 : is.slot + 1;
  b.dst = __builtin_amdgcn_readfirstlane(c.lbase + is.slot * L::SBYTES);
  b.dstw = __builtin_amdgcn_readfirstlane(c.lbase + ws * L::SBYTES + L::ABYTES);
  b.mdst = __builtin_amdgcn_readfirstlane(c.lbase + L::R * L::SBYTES + (is.mq & 1) * L::META);
}

// One step g: the products of the stage in slot s (two groups) -- MBN row blocks of the tile times the wave's 2 column
// blocks -- laid out as IT = 2 MBN iterations (group 0's row blocks, then group 1's) pinned in order by scheduling
// barriers. Iteration it issues its row block's 2 MFMAs on A operand av[it % 4] and then reads into that register the
// operand of iteration it + 4 (IT is a multiple of 4, so the ring runs on from step to step: the last 4 iterations
// read the next step's first 4 operands). The step opens a window at its start and issues its DMAs over the
// iterations before its barrier: A stage g + 2 into the slot the previous barrier freed, weight stage g + 3 into the
// slot whose codes the previous step read. The weights run a stage ahead: the first two iterations decode a column
// block each of this stage's group 1 (from codes read a step ago); iteration RD, 8 before the end (or the third; 2 row
// blocks: the first, ahead of its barrier), reads the next stage's codes from the next slot ns (certified by the
// previous step's barrier), so that the last two decode the next stage's group 0 (nqi: that stage's quarter) from
// data long landed. Four iterations before the end comes the workgroup's barrier: this wave's reads of the A stage in
// slot s are all issued by then (the next step's window may overwrite it), and the A stage in ns has landed (vmcnt:
// only this step's window may be in flight); past it the wave reads the next step's first A operands from ns
// (nsmall: its tile has 2 row blocks). 2 row blocks: the window, its DMAs and the codes' read come before the barrier
// at the step's start. nmq >= 0: the item whose metadata the windows carry from now on.
template <int QT, bool SWIGLU, bool MP, int MBN>
__device__ __forceinline__ void pg_step(const PrefillArgs& a, const PGCtx& c, PGIssue<QT, SWIGLU, MP>& is,
                                        const PGLane<QT>& ln, PGOps<QT>& ops, u32x4 (&av)[4], const uint8_t* s,
                                        const uint8_t* ns, int nqi, bool nsmall, int nmq, f32x4 (&acc)[MBN][2]) {
  using L = PG<QT>;
  constexpr int IT = 2 * MBN, HEAD = IT - 4, RD = MBN > 4 ? MBN - 4 : 0;
  auto a_addr = [&](int it) { return s + (it < MBN ? ln.aof0 : ln.aof1) + (it % MBN) * 2048; };
  u32x4 b1[2];
  PGOps<QT> nx;
  PGRaw<QT> raw;
  PGPrep p1[2], p0[2];
  if constexpr (HEAD == 0) {  // (2 row blocks: the window and the codes' read before the step's barrier)
    pg_open<QT, SWIGLU, MP>(a, c, is, nmq);
#pragma unroll
    for (int n = 0; n < L::LOADS; n++) pg_dma_n<QT, SWIGLU, MP>(n, is, c.wv);
    pg_read_codes<QT>(ns, ln, nx, raw);
  }
  static_assert(HEAD == 0 || RD < HEAD, "the next stage's codes are read before the barrier that frees their slot");
  pg_for<IT>([&](auto itc) __attribute__((always_inline)) {
    constexpr int it = decltype(itc)::value;
    if constexpr (it == 0 && HEAD > 0) pg_open<QT, SWIGLU, MP>(a, c, is, nmq);
    if constexpr (it == HEAD) {
      pg_wait_window<QT>(c.wv);
      pg_barrier();
    }
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      if constexpr (it < MBN)
        acc[it][nb] = mfma16(ops.b0[nb], av[it % 4], acc[it][nb]);
      else
        acc[it - MBN][nb] = mfma16(b1[nb], av[it % 4], acc[it - MBN][nb]);
    }
    if constexpr (it == RD && HEAD > 0) pg_read_codes<QT>(ns, ln, nx, raw);
    if constexpr (it < HEAD)
      av[it % 4] = *reinterpret_cast<const u32x4*>(a_addr(it + 4));
    else
      av[it % 4] = pg_read_a0<QT>(ns, ln, nsmall, it - HEAD);
    // the decodes, each a column block's preparation and 4 words (10 tasks), dealt over group 0's iterations (this
    // stage's group 1) and group 1's (the next stage's group 0)
    pg_for<10>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value, nb = t / 5, k = t % 5;
      // (Q4_K and PQ6, whose decoded operands and group-1 state take more registers than what is read: a column
      // block's 5 tasks together, at the last iterations before the operand is used)
      constexpr int ti1 = L::F32D ? MBN - 2 + nb : t * MBN / 10, ti0 = L::F32D ? IT - 2 + nb : MBN + t * MBN / 10;
      if constexpr (ti1 == it) {
        if constexpr (k == 0)
          p1[nb] = pg_prep1<QT>(ops, ln, nb);
        else
          b1[nb][k - 1] = pg_word<QT>(p1[nb], ln, k - 1);
      }
      if constexpr (ti0 == it) {
        if constexpr (k == 0)
          p0[nb] = pg_prep0<QT>(nx, raw, ln, nqi, nb);
        else
          nx.b0[nb][k - 1] = pg_word<QT>(p0[nb], ln, k - 1);
      }
    });
    if constexpr (it < HEAD) {  // (the window's DMAs: weights first)
#pragma unroll
      for (int n = it * L::LOADS / HEAD; n < (it + 1) * L::LOADS / HEAD; n++) pg_dma_n<QT, SWIGLU, MP>(n, is, c.wv);
    }
    __builtin_amdgcn_sched_barrier(0);  // (nothing moves from one iteration to another)
  });
  ops = nx;
}

// One item: its K loop (stage by stage through the ring; cslot: the slot of its stage 0) and its epilogue. Its first
// step's operands are read already (ops, av), and its last step reads those of the next item's first.
template <int QT, bool SWIGLU, bool MP, int MBN>
__device__ __forceinline__ int pg_run(const PrefillArgs& a, const PGCtx& c, PGIssue<QT, SWIGLU, MP>& is,
                                      const PGLane<QT>& ln, PGOps<QT>& ops, u32x4 (&av)[4], const PGItem& I, int q,
                                      int cslot) {
  using L = PG<QT>;
  const int wv = c.wv;
  f32x4 acc[MBN][2];
#pragma unroll
  for (int mb = 0; mb < MBN; mb++) acc[mb][0] = acc[mb][1] = f32x4{0, 0, 0, 0};
  // From the item's second step on (past its first barrier) the windows carry the metadata of item q + 1 (into the
  // buffer of item q - 1, whose epilogue every wave is past by then), else item q's again. The last step's reads are
  // for the next item.
  const int nmq = q + 1 < c.nq ? q + 1 : q;
  bool nsmall = false;
  if (q + 1 < c.nq) nsmall = pg_table<MP>(c, q + 1).m_valid <= 32;
  const int stages = MP ? I.stages : c.stages;
#pragma clang loop unroll(disable)  // (one copy of the step: none peeled for the first)
  for (int st = 0; st < stages; st++) {
    const int ns = cslot + 1 == L::R ? 0 : cslot + 1;
    pg_step<QT, SWIGLU, MP, MBN>(a, c, is, ln, ops, av, c.lds + cslot * L::SBYTES, c.lds + ns * L::SBYTES, (st + 1) & 3,
                                 st + 1 < stages ? MBN == 2 : nsmall, st == 1 ? nmq : -1, acc);
    cslot = __builtin_amdgcn_readfirstlane(ns);
  }
  // epilogue: lane output i of block (mb, nb): row 16 mb + lr of the tile; column (SwiGLU) n0 + 16 wv + 4 lg + i, gate
  // in nb 0 and up in nb 1; (plain) n0 + 32 wv + 8 lg + 4 nb + i. A lane stores its row's 4 (8) columns at once.
  const float2* rf = pg_rowf<QT>(c, q);
  const int lr = pg_fresh(c.lr), lg = pg_fresh(c.lg);
  const PrefillProblem& P = a.p[I.p];
  float2 fr[3];  // (the row factors, read two row blocks ahead; rows past the valid ones hold the last one's)
  fr[0] = rf[lr];
  fr[1] = rf[16 + lr];
  pg_for<MBN>([&](auto mbc) __attribute__((always_inline)) {
    constexpr int mb = decltype(mbc)::value;
    if constexpr (mb + 2 < MBN) fr[(mb + 2) % 3] = rf[16 * (mb + 2) + lr];
    const int m = 16 * mb + lr;
    const float2 f = fr[mb % 3];
    const int64_t o = int64_t(I.s0 + m) * P.N;
    if constexpr (SWIGLU) {
      const int n = I.n0 + 16 * wv + 4 * lg;
      if (m < I.m_valid && n < P.N) {
        uint32_t v[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const f16x2 h = {_Float16(pg_swiglu(acc[mb][0][2 * i] * f.x, acc[mb][1][2 * i] * f.x) * f.y),
                           _Float16(pg_swiglu(acc[mb][0][2 * i + 1] * f.x, acc[mb][1][2 * i + 1] * f.x) * f.y)};
          v[i] = __builtin_bit_cast(uint32_t, h);
        }
        *reinterpret_cast<uint2*>(P.h + o + n) = make_uint2(v[0], v[1]);
      }
    } else {
      const int n = I.n0 + 32 * wv + 8 * lg;  // (the lane's 8 columns: 4 of each column block)
      if (m < I.m_valid && n < P.N) {
        if (P.y16) {  // (fp16: the sums times f.y)
          uint32_t v[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const f16x2 h = {_Float16(acc[mb][i / 2][2 * (i % 2)] * f.y), _Float16(acc[mb][i / 2][2 * (i % 2) + 1] * f.y)};
            v[i] = __builtin_bit_cast(uint32_t, h);
          }
          *reinterpret_cast<uint4*>(P.y16 + o + n) = make_uint4(v[0], v[1], v[2], v[3]);
        } else {  // (fp32: the sums times f.x f.y, a power of two)
          const float fs = f.x * f.y;
#pragma unroll
          for (int nb = 0; nb < 2; nb++)
            *reinterpret_cast<float4*>(P.y + o + n + 4 * nb) =
                make_float4(acc[mb][nb][0] * fs, acc[mb][nb][1] * fs, acc[mb][nb][2] * fs, acc[mb][nb][3] * fs);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // (a row block at a time: its factors read two ahead)
  });
  return cslot;
}

template <int QT, bool SWIGLU, bool MP>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pgemm(const PrefillArgs a) {
  using L = PG<QT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  PGCtx c;
  c.lds = lds;
  c.lbase = pg_lds_addr(lds);
  c.tid = threadIdx.x;
  c.lane = c.tid & (WAVE - 1);
  c.wv = __builtin_amdgcn_readfirstlane(c.tid / WAVE);
  c.lg = c.lane >> 4;
  c.lr = c.lane & 15;
  c.stages = a.p[0].K / 64;
  int4* table = reinterpret_cast<int4*>(lds + L::R * L::SBYTES + 2 * L::META);
  c.table = table;
  // Each product's items are dealt to the 8 XCDs in contiguous runs (workgroup b runs on XCD b % 8): the column blocks
  // of a tile, and an expert's tiles, run close in time on one XCD and share its L2 (the tile's A rows, the expert's
  // weights); an XCD's run holds its share of every product. Within a run, an item costs about its stages times its
  // tile's row blocks (plus a step's fixed part), so the XCD's G workgroups take the run's items ranked by that cost
  // (most first, then by place in the run), dealt back and forth: position q G + j0 in even rounds, q G + G - 1 - j0
  // in odd ones. Every workgroup of the XCD ranks the same way, so each item is taken once (any assignment gives the
  // same results: each item writes its own outputs).
  const int G = gridDim.x / 8, x = blockIdx.x % 8, j0 = blockIdx.x / 8;
  int64_t lo[PREFILL_MAXP];
  int cnt[PREFILL_MAXP + 1];
  cnt[0] = 0;
  int most = 1;  // (the largest item cost of the launch: the cost unit)
  for (int p = 0; p < PREFILL_MAXP; p++) {
    int n = 0;
    lo[p] = 0;
    if (p < (MP ? a.np : 1)) {
      const int64_t items = pg_tiles(a.p[p]) * pg_nbk<SWIGLU>(a.p[p]), per = (items + 7) / 8;
      lo[p] = x * per;
      const int64_t hi = min(items, (x + 1) * per);
      n = hi > lo[p] ? int(hi - lo[p]) : 0;
      most = max(most, a.p[p].K / 64 * (TILE_ROWS / 32 + 1));
    }
    cnt[p + 1] = cnt[p] + n;
  }
  const int n_run = cnt[PREFILL_MAXP], full = n_run / G, rem = n_run - full * G;
  c.nq = full + (rem && ((full & 1) ? j0 >= G - rem : j0 < rem));  // (at most MAXQ: the launch checks)
  if (c.nq == 0) return;
  // the ranking and the item table: every global load of the tiles and offsets, once, before any DMA is in flight
  // (the ranking's keys, order and the run's items in the ring's memory, not yet in use: n_run <= MAXQ G <= 4096)
  constexpr int KM = 16;  // (cost keys 1 .. KM)
  const int unit = (most + KM - 1) / KM;
  uint8_t* key = lds;
  uint16_t* order = reinterpret_cast<uint16_t*>(lds + 4096);
  int4* run = reinterpret_cast<int4*>(lds + 12288);
  static_assert(12288 + 4096 * 16 <= L::R * L::SBYTES, "the ranking's LDS");
  for (int i = c.tid; i < n_run; i += L::THREADS) {
    int p = 0;
#pragma unroll
    for (int q = 1; q < PREFILL_MAXP; q++) p += i >= cnt[q] ? 1 : 0;
    const PGItem J = pg_item<SWIGLU>(a.p[p], p, lo[p] + (i - cnt[p]));
    const int cost = J.stages * ((J.m_valid + 31) / 32 + 1);
    key[i] = uint8_t(min(KM, max(1, (cost + unit - 1) / unit)));
    run[i] = pg_pack(J);
  }
  __syncthreads();
  if (c.wv == 0) {  // (one wave: per key, ballots over runs of 64 items)
    int tot[KM + 1] = {}, start[KM + 1];
    for (int i0 = 0; i0 < n_run; i0 += WAVE) {
      const int k = i0 + c.lane < n_run ? key[i0 + c.lane] : 0;
#pragma unroll
      for (int kk = 1; kk <= KM; kk++) tot[kk] += __popcll(__ballot(k == kk));
    }
    start[KM] = 0;  // (key KM first)
#pragma unroll
    for (int kk = KM - 1; kk >= 1; kk--) start[kk] = start[kk + 1] + tot[kk + 1];
    const uint64_t below = (uint64_t(1) << c.lane) - 1;
    for (int i0 = 0; i0 < n_run; i0 += WAVE) {
      const int i = i0 + c.lane, k = i < n_run ? key[i] : 0;
#pragma unroll
      for (int kk = 1; kk <= KM; kk++) {
        const uint64_t m = __ballot(k == kk);
        if (k == kk) order[start[kk] + __popcll(m & below)] = uint16_t(i);
        start[kk] += __popcll(m);
      }
    }
  }
  __syncthreads();
  if (c.tid < c.nq) {
    const int q = c.tid, pos = q * G + ((q & 1) ? G - 1 - j0 : j0);
    table[q] = run[order[pos]];
  }
  __syncthreads();
  // item 0's metadata, landed before its sources are made (buffer 0)
  PGIssue<QT, SWIGLU, MP> is;
  PGItem I = pg_table<MP>(c, 0);
  is.meta.set(I, c.tid);
  is.use_m(a.p[I.p]);
  {
    const uint32_t mdst = __builtin_amdgcn_readfirstlane(c.lbase + L::R * L::SBYTES);
#pragma unroll
    for (int j = 0; j < L::MI; j++)
      pg_dma<4>(j == 0 && c.wv < 4 ? is.mt0 : is.ms0, is.meta.m[j], mdst + (8 * j + c.wv) * 256);
    pg_wait<0>();
    __syncthreads();
  }
  // The weight stream runs a stage ahead of the A stream: weight stage 0 into slot 0; the windows of A stages 0, 1
  // (weights 1, 2; stages >= R + 2: prefill_supported), carrying item 1's metadata (item 0's again when there is
  // none); the barrier that certifies A stage 0 and weight stages 0, 1; the first step's operands (group 0's weights
  // decoded, group 1's codes, the first A operands); a barrier (every wave past its reads of weight stage 0, into whose
  // slot the first step's window loads weight stage 3).
  is.src.set_a(a.p[I.p], I, pg_tok<QT>(c, 0), c.tid);
  is.src.set_w(a.p[I.p], I, c.tid);
  is.use_a(a.p[I.p]);
  is.use_w(a.p[I.p]);
  is.qa = is.qw = 0;
  is.na = is.nw = I.stages;
  is.sta = -1;
  is.stw = 0;
  is.slot = -1;
  is.mq = 0;
  pg_wbases<QT, SWIGLU>(is.w0, is.w1, 0, is.b, c.wv);
  is.b.dstw = __builtin_amdgcn_readfirstlane(c.lbase + L::ABYTES);
#pragma unroll
  for (int n = 0; n < L::BI; n++) pg_dma_n<QT, SWIGLU, MP>(n, is, c.wv);
  const int mq = c.nq > 1 ? 1 : 0;
#pragma unroll
  for (int w = 0; w < 2; w++) {
    pg_open<QT, SWIGLU, MP>(a, c, is, mq);
#pragma unroll
    for (int n = 0; n < L::LOADS; n++) pg_dma_n<QT, SWIGLU, MP>(n, is, c.wv);
  }
  pg_wait_window<QT>(c.wv);
  pg_barrier();
  const PGLane<QT> ln(c.lr, c.lg, c.wv, SWIGLU, a.pq_mode, a.pq_off);
  PGOps<QT> ops;
  u32x4 av[4];
  {
    PGRaw<QT> raw;
    pg_read_codes<QT>(c.lds, ln, ops, raw);
#pragma unroll
    for (int j = 0; j < 4; j++) av[j] = pg_read_a0<QT>(c.lds, ln, I.m_valid <= 32, j);
#pragma unroll
    for (int nb = 0; nb < 2; nb++) pg_decode0<QT>(ops, raw, ln, 0, nb);
  }
  pg_barrier();

  int cslot = 0;
  for (int q = 0; q < c.nq; q++) {
    I = pg_table<MP>(c, q);
    // the tile's row blocks, rounded up to an even count (an instance of the K loop per count)
    switch ((I.m_valid + 31) / 32) {
      case 1: cslot = pg_run<QT, SWIGLU, MP, 2>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 2: cslot = pg_run<QT, SWIGLU, MP, 4>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 3: cslot = pg_run<QT, SWIGLU, MP, 6>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 4: cslot = pg_run<QT, SWIGLU, MP, 8>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 5: cslot = pg_run<QT, SWIGLU, MP, 10>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 6: cslot = pg_run<QT, SWIGLU, MP, 12>(a, c, is, ln, ops, av, I, q, cslot); break;
      case 7: cslot = pg_run<QT, SWIGLU, MP, 14>(a, c, is, ln, ops, av, I, q, cslot); break;
      default: cslot = pg_run<QT, SWIGLU, MP, 16>(a, c, is, ln, ops, av, I, q, cslot); break;
    }
  }
  pg_wait<0>();  // (the dummy loads past the last stage land before the workgroup's LDS is released)
}

// a product's work items at most (its tile bound times its column blocks)
int64_t pg_items_bound(const PrefillProblem& P, bool swiglu) {
  const int64_t tiles = P.tiles ? P.max_tiles : (P.dense_rows + pg_dense_rows(P) - 1) / pg_dense_rows(P);
  return tiles * ((P.N + (swiglu ? 127 : 255)) / (swiglu ? 128 : 256));
}

template <int QT, bool SWIGLU, bool MP>
int launch_pgemm(const PrefillArgs& a, hipStream_t s) {
  using L = PG<QT>;
  int64_t items = 0, run = 0;
  for (int p = 0; p < a.np; p++) {
    const int64_t n = pg_items_bound(a.p[p], SWIGLU);
    items += n;
    run += (n + 7) / 8;  // (an XCD's run: its share of each product)
  }
  if (items <= 0) return ARTLITE_OK;
  // persistent workgroups: as many as the device holds at once (a multiple of 8, the XCDs), at most the items
  static const int resident = [] {
    const void* f = reinterpret_cast<const void*>(k_pgemm<QT, SWIGLU, MP>);
    int dev = 0, cus = 0, per_cu = 0;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, L::LDS) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, L::THREADS, L::LDS) != hipSuccess)
      return 0;
    return cus * std::max(1, per_cu);
  }();
  if (resident < 8) return fail(ARTLITE_EHIP, "prefill GEMM: kernel set-up failed");
  const int64_t grid = std::min<int64_t>(run * 8, resident / 8 * 8);
  // a workgroup's items (an XCD's run, dealt over its grid / 8 workgroups) fit its item table (and an XCD's run fits
  // the ranking's 4096 entries)
  if ((run + grid / 8 - 1) / (grid / 8) > L::MAXQ || run > 4096)
    return fail(ARTLITE_EINVAL, "prefill GEMM: %lld work items, more than %d per workgroup", (long long)items, L::MAXQ);
  k_pgemm<QT, SWIGLU, MP><<<unsigned(grid), L::THREADS, L::LDS, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace

bool prefill_supported(int qtype, int K, int N) {
  // (K: whole stages of 64, at least R + 2 of them: the window of an item's stage 0 opens at the previous item's step
  // stages - R, which must come at least two windows after that item's first step opened the first window carrying
  // the next item's metadata: stages - R >= 2)
  // (Q4_K: whole super-blocks)
  return (qtype == ARTLITE_Q4_0 || qtype == ARTLITE_Q8_0 || qtype == ARTLITE_Q4_K || qtype == PREFILL_PQ6) &&
         K >= 64 * (PG<ARTLITE_Q4_0>::R + 2) && K % (qtype == ARTLITE_Q4_K ? 256 : 64) == 0 && K / 64 < 256 && N > 0 &&
         N % 16 == 0;
}

bool prefill_fits(int64_t experts, int64_t expert_bytes, int64_t a_rows, int64_t K) {
  // (the lane offsets of the weight DMAs reach e expert_bytes + the row's bytes, those of A rows row K 2 bytes)
  return experts > 0 && experts * expert_bytes + WEIGHT_TAIL < (int64_t(1) << 32) && a_rows * K * 2 < (int64_t(1) << 32);
}

int launch_prefill(const PrefillArgs& a, hipStream_t s) {
  if (a.np < 1 || a.np > PREFILL_MAXP) return fail(ARTLITE_EINVAL, "prefill GEMM: %d products", a.np);
  const bool swiglu = a.p[0].w[1] != nullptr;
  for (int p = 0; p < a.np; p++) {
    const PrefillProblem& P = a.p[p];
    if (!prefill_supported(a.qtype, P.K, P.N))
      return fail(ARTLITE_EINVAL, "prefill GEMM: weight type %d, K %d, N %d", a.qtype, P.K, P.N);
    if (!P.a || !P.row_scale || !P.w[0] || (P.w[1] != nullptr) != swiglu || (swiglu ? !P.h : !P.y && !P.y16) ||
        (P.tiles && (!P.n_tiles || !P.offsets)) || P.lda < P.K ||
        P.dense_tile < 0 || P.dense_tile > TILE_ROWS)
      return fail(ARTLITE_EINVAL, "prefill GEMM: product %d: null or mismatched argument", p);
    if (P.expert_bytes >= (int64_t(1) << 32) || int64_t(P.N) * P.row_bytes >= (int64_t(1) << 32) ||
        (!P.tiles && P.dense_rows > (1 << 24)))
      return fail(ARTLITE_EINVAL, "prefill GEMM: product %d beyond the tiles' 32-bit offsets", p);
  }
  // (one product: the kernel with product 0 known at compile time)
#define ART_PG(QT) \
  return swiglu ? (a.np > 1 ? launch_pgemm<QT, true, true>(a, s) : launch_pgemm<QT, true, false>(a, s)) \
                : (a.np > 1 ? launch_pgemm<QT, false, true>(a, s) : launch_pgemm<QT, false, false>(a, s))
  if (a.qtype == ARTLITE_Q4_0) ART_PG(ARTLITE_Q4_0);
  if (a.qtype == ARTLITE_Q4_K) ART_PG(ARTLITE_Q4_K);
  if (a.qtype == PREFILL_PQ6) {
    if (a.pq_mode < 0 || a.pq_mode > 2) return fail(ARTLITE_EINVAL, "prefill GEMM: PQ6 mode %d", a.pq_mode);
    ART_PG(PREFILL_PQ6);
  }
  ART_PG(ARTLITE_Q8_0);
#undef ART_PG
}

}  // namespace artlite
