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

// rows of A (tokens / pairs) per tile of the decode (GEMV-like) kernel, and of the prefill tiling
constexpr int DECODE_BM = 8;
constexpr int PREFILL_BM = 128;

// One prefill launch (fp16 MFMA tiles of PREFILL_BM rows): for each tile and each block of output rows,
// out[s][n] = sum_k A[row(s)][k] W_e[n][k] with A in fp16, its rows scaled by 2^-in_exp[token], and W_e's rows raw
// GGUF blocks. SwiGLU launches (w[1] set) write h = silu(A W_gate^T) * (A W_up^T) in fp16 scaled by
// 2^-out_exp[token]; plain launches write fp32 (the A scale undone).
struct PrefillArgs {
  const uint8_t* w[2];     // weight tensors: (gate, up) or (down, null); expert e at w + e expert_bytes
  int64_t expert_bytes;
  int row_bytes;
  int N, K;                // output rows per expert, values per row
  int qtype;               // ARTLITE_Q4_0 / Q8_0
  const uint16_t* a;       // A: fp16 rows of K values
  int a_gather;            // 1: A row of sorted row s = token(s); 0: A row = s
  const int32_t* order;    // token(s) = order[s] / topk (null: token(s) = s)
  int topk;
  const int32_t* tiles;    // (expert, first sorted row) per tile; null: dense rows 0 .. dense_rows of expert 0
  const int32_t* n_tiles;  // the tile count (device)
  const int32_t* offsets;  // E + 1 expert offsets in the sorted order
  int dense_rows;
  int64_t max_tiles;       // grid bound
  const int32_t* in_exp;   // per token: the exponent of A's row scale
  const int32_t* out_exp;  // SwiGLU: per token, the exponent of h's scale
  uint16_t* h;             // SwiGLU output: fp16 h 2^-out_exp[token(s)] (row stride N)
  float* y;                // plain output: fp32 (row stride N)
};

// whether the prefill tiling takes N rows of K values of weights of this type
bool prefill_supported(int qtype, int K, int N);

int launch_prefill(const PrefillArgs& a, hipStream_t s);

// x (T rows of H fp32 / bf16 values) -> the prefill's fp16 rows x16 scaled by 2^-x_exp[t], and per token the
// exponents h_exp (h_exp2) of the h scale from the bound on |h| that wmax[0], wmax[1] (wmax[2], wmax[3]) give: max
// |w| of the gate and up matrices (pairs: 1 or 2)
int launch_prefill_x(const void* x, int x_dtype, int64_t T, int H, const float* wmax, int pairs, uint16_t* x16,
                     int32_t* x_exp, int32_t* h_exp, int32_t* h_exp2, hipStream_t s);

// *out = max |w| over a tensor's nblocks GGUF blocks (Q4_0, Q8_0)
int launch_weight_max(const uint8_t* w, int qtype, int64_t nblocks, float* out, hipStream_t s);
// the most 32-value groups of a row (K <= 32 MAX_GROUPS)
constexpr int MAX_GROUPS = 128;

int launch_expert_gemm(const GemmArgs& a, hipStream_t s);

// y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] in fp32 (ys / ws optional)
// res (optional; x_dtype res_dtype): added last, y[t] += res[t] (the block's residual)
int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, const void* res, int res_dtype, float* y, hipStream_t s);

// fp32 activations -> bf16 hi + lo planes (x = hi + lo to 2^-16 relative)
int launch_split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s);

}  // namespace artlite
