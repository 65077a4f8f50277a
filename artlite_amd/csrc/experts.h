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
  int bm;                  // rows of A per tile of the tile list: DECODE_BM or PREFILL_BM
  uint16_t* h_hi;          // SwiGLU output planes (row stride N)
  uint16_t* h_lo;
  float* y;                // plain output (row stride N)
};

// rows of A (tokens / pairs) per tile of the decode (GEMV-like) kernel, and of the prefill tiling
constexpr int DECODE_BM = 8;
constexpr int PREFILL_BM = 128;

// whether the prefill tiling takes N rows of K values of weights of this type
bool prefill_supported(int qtype, int K, int N);
// the most 32-value groups of a row (K <= 32 MAX_GROUPS)
constexpr int MAX_GROUPS = 128;

int launch_expert_gemm(const GemmArgs& a, hipStream_t s);

// y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] in fp32 (ys / ws optional)
int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, float* y, hipStream_t s);

// fp32 activations -> bf16 hi + lo planes (x = hi + lo to 2^-16 relative)
int launch_split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s);

}  // namespace artlite
