// The decode path's expert products (gemv.hip): a VALU GEMV over raw GGUF blocks for tiles of a few tokens, and
// the quantisation of its activations.
#pragma once

#include "common.h"
#include "route.h"

namespace artlite {

// rows of A (tokens for gate / up, pairs for down) per decode tile
constexpr int GEMV_BM = 4;

// XQ, the decode activations: each row of K values (K a multiple of 256) as units of 256 values, a unit as 8
// groups of 32 and each group as two int8 planes, x ~ s (a + b / 256) with s = max |x| / 127 over the group. A
// group's block is 16 dwords: plane a (8 dwords of 4 int8 in value order), then plane b. Per group three words:
// s / 256 (fp32), the sum over the group of 256 a + b (int32), and s / 256 times that sum (fp32: the group's
// dequantised sum). A group with a non-finite value has s = NaN; a group of zeros has s = 0.
// A unit is 64 chunks of 4 dwords, chunk 16 p + r (p < 4, r < 16) = [dword r of group 2 p's block, dword r of group
// 2 p + 1's block, L, S], with L = (s / 256 of group 2 p, its sum, s / 256 of group 2 p + 1, its sum)[r % 4] and
// S = (dequantised sum of group 2 p, of group 2 p + 1)[r % 2]: chunk i is exactly what lane i of the GEMV needs.
constexpr int XQ_UNIT = 256;  // dwords per unit

__host__ __device__ inline int64_t xq_row_dwords(int K) { return int64_t(K / 256) * XQ_UNIT; }

struct GemvArgs {
  const uint8_t* w[2];     // weight tensors: (gate, up) or (down, null); expert e at w + e expert_bytes
  int64_t expert_bytes;
  int row_bytes;
  int N, K;                // output rows per expert, values per row
  int qtype;               // ARTLITE_Q4_0 / Q8_0 / Q4_K
  const uint32_t* xq;      // A rows in XQ
  int a_gather;            // 1: A row of sorted row s = order[s] / topk (tokens); 0: A row = s
  const int32_t* order;
  int topk;
  int rows_total;          // a_gather: the entries of order
  const int32_t* tiles;    // (expert, first sorted row) per tile of GEMV_BM rows; null: dense rows of expert 0
  const int32_t* n_tiles;  // the tile count (device)
  const int32_t* offsets;  // E + 1 expert offsets in the sorted order
  int dense_rows;
  int64_t max_tiles;       // grid bound
  uint32_t* hq;            // SwiGLU: h = silu(gate) up as XQ rows (by sorted row)
  float* y;                // plain: fp32 rows (by sorted row), stride N
  // (SwiGLU, optional) the routing done by the launch itself: when logits is given, every workgroup routes the T
  // tokens' (T, E) logits in its LDS (gemv_route_fits) and takes its items from that; workgroup 0 also stores ids,
  // weights and the dispatch (d: counts, offsets, order, slot, tiles, ctrl[CTRL_TILES]) for the launches after it.
  // tiles, n_tiles, offsets and order above are then not read.
  struct Route {
    const float* logits = nullptr;
    int T = 0, E = 0, k = 0, sigmoid = 0;
    int32_t* ids = nullptr;
    float* w32 = nullptr;
    DispatchBufs d{};
  } route;
};

// whether a SwiGLU GEMV launch can route T tokens of E experts, top k, itself (GemvArgs::route)
bool gemv_route_fits(int64_t T, int E, int k);

// whether the GEMV takes N rows of K values of weights of this type
bool gemv_supported(int qtype, int K, int N);

int launch_gemv(const GemvArgs& a, hipStream_t s);

// x (T rows of K fp32 or bf16 values) -> XQ rows
int launch_quant(const void* x, int x_dtype, int64_t T, int K, uint32_t* xq, hipStream_t s);

// one XQ row back to fp32 (host side, for inspection)
void xq_dequant_row(const uint32_t* row, int K, float* out);

}  // namespace artlite
