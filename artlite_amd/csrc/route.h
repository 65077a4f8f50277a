// Routing kernels' launchers (route.hip) and the dispatch's (dispatch.hip).
#pragma once

#include "common.h"

namespace artlite {

constexpr int MAX_EXPERTS = 1024;  // (keys per lane: 16)
constexpr int MAX_TOPK = 64;       // (one lane per chosen expert)
constexpr int ROUTER_TG = 16;      // tokens per router block (at most)
constexpr int ROUTER_EW = 8;       // experts (waves) per router block
constexpr int ROUTER_LDS = 64 * 1024;  // bytes of staged token rows per router block

int check_route_args(int64_t n, int per_col, int E, int k);

int launch_topk(const float* logits, int64_t n, int64_t row, int per_col, int64_t pitch, int E, int k, int sigmoid,
                int32_t* ids, float* w32, double* w64, hipStream_t s);

int launch_router(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* out, int64_t out_row,
                  hipStream_t s);

// ---- dispatch: the stable counting sort of the (token, slot) pairs by expert
constexpr int DISPATCH_BLOCK = 1024;  // pairs per block

// ctrl words (int32) of a dispatch
enum DispatchCtrl {
  CTRL_DONE = 0,      // blocks finished counting (reset by the last)
  CTRL_BAD = 1,       // an id outside [0, E) was seen
  CTRL_BAD_ID = 2,    // one such id
  CTRL_TILES = 3,     // expert GEMM tiles of the tile list
  CTRL_CHUNKS = 4,    // plan chunks
  CTRL_OVER_CAP = 5,  // a column needs more than cap chunks
  CTRL_BAD_FIRST = 6, // P - (the first pair with a bad id): the reference reports the first in pair order
  CTRL_WORDS = 8,
};

struct DispatchBufs {
  const int32_t* ids;  // P pair ids (t k + i order)
  int64_t P;
  int E, k;
  int32_t* table;    // NB x E: per-block counts, then per-block bases
  int32_t* ctrl;     // CTRL_WORDS, zero before the first launch (kept zero-ready by the kernels)
  int32_t* counts;   // E
  int32_t* offsets;  // E + 1
  int32_t* order;    // P
  int32_t* slot;     // P
  int32_t* tiles;    // 2 x tile bound: (expert, first sorted row) per M-tile of BM rows, experts ascending
  int BM;            // rows per tile (0: no tile list)
  int32_t* cstart;   // E + 1 chunk prefix (plan only; may be null)
  int chunk;         // plan chunk size (0: no plan)
};

// blocks of a dispatch of P pairs
inline int64_t dispatch_blocks(int64_t P) { return P > 0 ? (P + DISPATCH_BLOCK - 1) / DISPATCH_BLOCK : 1; }
// an upper bound on the tiles of P pairs over E experts with BM rows per tile
inline int64_t tile_bound(int64_t P, int E, int BM) { return (P + BM - 1) / BM + (P < E ? P : E); }

int launch_dispatch(const DispatchBufs& d, hipStream_t s);
int launch_dispatch_count(const DispatchBufs& d, int64_t nb, hipStream_t s);
int launch_dispatch_scatter(const DispatchBufs& d, int64_t nb, hipStream_t s);

struct PlanBufs {
  int cols, cap;
  int32_t* experts;  // cols x cap
  int32_t* ccounts;  // cols
  int32_t* sizes;    // cols x cap
  int32_t* rows;     // cols x cap x chunk
  int64_t* pos;      // P
};
int launch_plan(const DispatchBufs& d, const PlanBufs& p, hipStream_t s);

}  // namespace artlite
