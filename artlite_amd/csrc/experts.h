// The experts' grouped GEMMs over raw GGUF blocks (experts.hip) and the combine.
#pragma once

#include "common.h"

namespace artlite {

// One grouped GEMM launch: for each tile (expert e, sorted rows s0 .. s0 + BM) and each N-tile of output rows,
// out[s][n] = sum_k A[row(s)][k] W_e[n][k] with W_e's rows raw GGUF blocks. SwiGLU launches (w[1] set) write
// h = silu(A W_gate^T) * (A W_up^T) as bf16 hi + lo planes; plain launches write fp32.
struct GemmArgs {
  const uint8_t* w[2];     // weight tensors: (gate, up) or (down, null); expert e at w + e expert_bytes
  int64_t expert_bytes;
  int row_bytes;
  int N, K;                // output rows per expert, values per row
  int qtype;               // ARTLITE_Q4_0 / Q8_0 / Q4_K
  const uint16_t* a_hi;    // A: rows of K bf16 (hi plane)
  const uint16_t* a_lo;    // lo plane (null: A is exactly bf16)
  int a_gather;            // 1: A row of sorted row s = order[s] / topk (tokens); 0: A row = s
  const int32_t* order;
  int topk;
  const int32_t* tiles;    // (expert, first sorted row) per tile; null: dense rows 0 .. dense_rows of expert 0
  const int32_t* n_tiles;  // the tile count (device)
  const int32_t* offsets;  // E + 1 expert offsets in the sorted order
  int dense_rows;
  int64_t max_tiles;       // grid bound
  int bm;                  // rows of A per tile of the tile list (at most DECODE_BM)
  uint16_t* h_hi;          // SwiGLU output planes (row stride N)
  uint16_t* h_lo;
  float* y;                // plain output (row stride N)
};

// rows of A (tokens / pairs) per tile of the MFMA decode tiles, and the most of a prefill tile (an expert's rows in
// tiles of balanced_rows(count, PREFILL_BM) rows)
constexpr int DECODE_BM = 8;
constexpr int PREFILL_BM = 256;

// One product of a prefill launch (prefill.hip: fp16 MFMA tiles of at most PREFILL_BM rows): for each tile and each
// block of output rows, out[s][n] = sum_k A[row_a(s)][k] W_e[n][k] over the product's K values, with A in fp16 (its
// rows scaled by powers of two) and W_e's rows raw GGUF blocks; row_scale[s] = (x, y) undoes the scales: plain
// products write fp32 x y sum (y set) or fp16 y sum (y16 set: the row's true values are x times these), SwiGLU
// products (w[1] set) write h = silu(x g) (x u) y in fp16. A product may cover a range of K (a part of a split K):
// w and a then point at its first value, lda is A's row stride and the weights' rows keep their own stride.
struct PrefillProblem {
  const uint8_t* w[2];     // weight tensors: (gate, up) or (down, null); expert e at w + e expert_bytes
  int64_t expert_bytes;
  int row_bytes;
  int N, K;                // output rows per expert; the product's values of K (whole 64-value stages)
  int lda;                 // A's row stride (values)
  const uint16_t* a;       // A: fp16 rows
  const int32_t* row_a;    // per output row s: its A row (a token); null: A row s
  const float2* row_scale; // per output row s: (x, y) as above
  const int32_t* tiles;    // (expert, first sorted row) per tile; null: dense rows 0 .. dense_rows of expert 0
  const int32_t* n_tiles;  // the tile count (device)
  const int32_t* offsets;  // E + 1 expert offsets in the sorted order
  int dense_rows;
  int dense_tile;          // dense rows: a tile's rows, at most 256 (0: balanced_rows(dense_rows, 256))
  int64_t max_tiles;       // grid bound
  uint16_t* h;             // SwiGLU output: fp16 (row stride N)
  float* y;                // plain output: fp32 (row stride N)
  uint16_t* y16;           // or fp16 (row stride N)
};

// The prefill layout of the block formats the prefill tiles do not read from the file's bytes (Q3_K, Q5_K, Q6_K, Q4_1,
// IQ4_NL, IQ4_XS): made at upload (launch_pq6_pack), 64 bytes per 64 values of a row (a stage of the tiles), four
// 16-byte chunks: the scales (4 fp32), two of nibbles, one of crumbs. Value 32 g + 8 l + i (g < 2, l < 4, i < 8) has
// code c (6 bits): its low 4 bits are nibble (i / 4) of byte i % 4 of dword 4 g + l (bytes 16 ..), its high 2 bits
// bits 2 (i / 4) + 4 (1 - l % 2) of byte i % 4 of dword 2 g + l / 2 of the crumbs (bytes 48 ..). Its weight is
// w = s c - o, in one of three modes: 0 (Q3_K, Q6_K) s the fp32 scale of its 16 values (scale 4 g + 2 l / 2 ... of
// the stage: s[2 g + l / 2]), o = off s (off: 4, 32); 1 (Q4_1, Q5_K) (s, o) = the fp32 scale and min of its 32 values
// (scales 2 g, 2 g + 1); 2 (IQ4_NL, IQ4_XS) as mode 0 with off 128, c = IQ4[nibble] + 128. Every s and o is the block's
// own product of fp16 and integer fields, exact in fp32, so w is the file's value.
constexpr int PREFILL_PQ6 = 0x106;  // (a prefill launch's qtype: weights in the prefill layout)
// the mode and offset of a block format's prefill layout; false: the format has none
bool pq6_mode(int qtype, int& mode, float& off);
// rows of K values (K a multiple of 64 and of the format's block) of a tensor as the layer stores it (row_bytes apart)
// -> the prefill layout (K bytes a row)
int launch_pq6_pack(const uint8_t* src, int qtype, int64_t rows, int K, size_t row_bytes, uint8_t* dst, hipStream_t s);

// A prefill launch: up to PREFILL_MAXP products of one weight format and kind (all SwiGLU or all plain), their work
// items dealt over the device together (a routed product and the shared expert's; the parts of a split K).
constexpr int PREFILL_MAXP = 4;
struct PrefillArgs {
  PrefillProblem p[PREFILL_MAXP];
  int np;
  int qtype;               // ARTLITE_Q4_0 / Q8_0 / Q4_K, or PREFILL_PQ6 (every product's weights in the prefill layout)
  int pq_mode;             // PREFILL_PQ6: the products' mode and offset (pq6_mode)
  float pq_off;
};

// whether the prefill tiling takes N rows of K values of weights of this type
bool prefill_supported(int qtype, int K, int N);
// whether the 32-bit offsets of the prefill tiles reach every byte: E experts of expert_bytes (their weights and the
// zeroed tail), rows of A of K fp16 values
bool prefill_fits(int64_t experts, int64_t expert_bytes, int64_t a_rows, int64_t K);

int launch_prefill(const PrefillArgs& a, hipStream_t s);

// x (T rows of H fp32 / bf16 values) -> the prefill's fp16 rows x16 = x 2^-xe[t] (each token's largest |x| into
// [2^14, 2^15)), and per token the row factors of the expert products: gu[t] = (2^xe, 2^-he) for the gate / up
// launch (he: the exponent of h's scale, from the bound on |h| that the gate and up matrices' max |w| (wmax[0],
// wmax[1]) and largest row L1 norms (wmax[5], wmax[6]) give) and dn[t] = (2^(he + ye), 2^-ye) for the down launch's
// fp16 output (ye from the bound on its sums that the down matrix's largest row L1 norm wmax[9] gives:
// |sum| 2^-ye < 2^15); pairs 2: the same for a second (shared) expert's matrices (wmax[2], wmax[3]; wmax[7], wmax[8])
// into gu2, and dn2 = (2^he, 1) for its fp32 down output
int launch_prefill_x(const void* x, int x_dtype, int64_t T, int H, const float* wmax, int pairs, int F, uint16_t* x16,
                     float2* gu, float2* dn, float2* gu2, float2* dn2, hipStream_t s);

// *out = a bound on max |w| over a tensor's nblocks GGUF blocks (Q4_0, Q8_0: exact; Q4_K: from d, dmin and the
// largest 6-bit scale and min; other formats: the largest fp32 value, no bound, so that the L1 norms govern)
int launch_weight_max(const uint8_t* w, int qtype, int64_t nblocks, float* out, hipStream_t s);
// *out = a bound on the largest L1 norm (sum |w|) of a tensor's rows of cols values as the layer stores them
// (dequant.hip)
int launch_weight_l1(const uint8_t* w, int qtype, int64_t rows, size_t row_bytes, int cols, float* out, hipStream_t s);
// the most 32-value groups of a row (K <= 32 MAX_GROUPS)
constexpr int MAX_GROUPS = 128;

int launch_expert_gemm(const GemmArgs& a, hipStream_t s);

// y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] in fp32 (ys / ws optional)
// res (optional; x_dtype res_dtype): added last, y[t] += res[t] (the block's residual)
int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, const void* res, int res_dtype, float* y, hipStream_t s);
// the same over fp16 pair outputs: Y[s] = Y16[s] yf[s].x (the down launch's row factors; H a multiple of 8); ys in
// ys_parts parts of T x H (a split K), added in order
int launch_combine16(const uint16_t* Y16, const float2* yf, const int32_t* slot, const float* w, int k,
                     const float* ys, int ys_parts, const float* ws_logit, int ws_sigmoid, int64_t T, int H,
                     const void* res, int res_dtype, float* y, hipStream_t s);

// fp32 activations -> bf16 hi + lo planes (x = hi + lo to 2^-16 relative)
int launch_split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s);

}  // namespace artlite
