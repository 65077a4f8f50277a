// Routing kernels' launchers (route.hip) and the dispatch's (dispatch.hip).
#pragma once

#include "common.h"

namespace artlite {

constexpr int MAX_EXPERTS = 1024;  // (keys per lane: 16)
constexpr int MAX_TOPK = 64;       // (one lane per chosen expert)
constexpr int ROUTER_TG = 16;      // tokens per router block (at most)
constexpr int ROUTER_GROUPS = 4;   // token groups of the one-launch router + routing (k_router_route), at most
constexpr int GTICK_STRIDE = 64;   // ints between its group tickets (each in lines of its own)
constexpr int ROUTER_EW = 8;       // experts (waves) per router block
constexpr int ROUTER_LDS = 64 * 1024;  // bytes of staged token rows per router block

// ---- the top k of one token's logits, one wave (shared by k_topk and the small-batch routing)
//
// Ranking follows the reference's host step (csrc/artlite/moe_host.cpp:45-73): a logit's 64-bit key is its ordered
// fp32 bits (after l + 0, so -0 ranks as +0) above ~id, so larger logits win and equal logits go to the lower id.
// The weights follow moe_host.cpp:62-72: e^(l - l_max) (or sigmoid(l)) in double, their sum in numpy's pairwise
// order (moe_host.cpp:25-39), e / sum rounded to fp32.
__device__ __forceinline__ uint64_t logit_key(float l, int e) {
  uint32_t u = __float_as_uint(l);
  if (u == 0x80000000u) u = 0;  // (-0 ranks as +0)
  const uint32_t ord = (u >> 31) ? ~u : (u | 0x80000000u);
  return (uint64_t(ord) << 32) | uint32_t(~uint32_t(e));
}

// the logit of ordered bits (the high half of logit_key; -0 comes back as +0, which every use of it treats alike)
__device__ __forceinline__ float key_logit(uint32_t ord) {
  return __uint_as_float((ord >> 31) ? (ord & 0x7FFFFFFFu) : ~ord);
}

// numpy's pairwise sum of n <= 128 doubles (moe_host.cpp:25-39)
__device__ __forceinline__ double row_sum(const double* a, int n) {
  if (n < 8) {
    double s = 0;
    for (int i = 0; i < n; i++) s += a[i];
    return s;
  }
  double r[8];
  for (int j = 0; j < 8; j++) r[j] = a[j];
  int i = 8;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; j++) r[j] += a[i + j];
  double s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; i++) s += a[i];
  return s;
}

// a wave's 32-bit maximum, in every lane: DPP within 16-lane rows, then the permlane swaps across rows
template <int C>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), C, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  const auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(uint32_t(s16[0]), uint32_t(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(uint32_t(s32[0]), uint32_t(s32[1]));
}

// One token's top k by one wave: R logits per lane (expert e = lane + 64 r of the logits p, expert e at
// (e / per_col) pitch + e % per_col) as their ordered bits (the high half of logit_key), k rounds of: the largest
// ordered bits among the experts not yet taken (a 32-bit wave maximum), then the lowest id holding them (ballots: the
// low half of logit_key decides ties), lane j keeping the j-th; then the weights. ev (64 doubles) and sum (1): the
// wave's LDS scratch. Lane j < k writes ids[j] and the weights (w32 / w64 when given) and returns its id; other lanes
// return -1. COHERENT: the logits are read at device scope (written by other workgroups of the same launch);
// DEV_IDS: the ids are stored at device scope (read by other workgroups of the same launch).
template <int R, bool COHERENT = false, bool DEV_IDS = false>
__device__ __forceinline__ int topk_wave(const float* __restrict__ p, int per_col, int64_t pitch, int E, int k,
                                         int sigmoid, double* ev, double* sum, int lane, int32_t* __restrict__ ids,
                                         float* __restrict__ w32, double* __restrict__ w64) {
  static_assert(R <= 32, "keys per lane");
  uint32_t ord[R], live = 0;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int e = lane + WAVE * r;
    float l = 0.0f;
    if (e < E) {
      const float* q = per_col == E ? p + e : p + int64_t(e / per_col) * pitch + e % per_col;
      l = COHERENT ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *q;
    }
    ord[r] = e < E ? uint32_t(logit_key(l, e) >> 32) : 0;
    if (e < E) live |= 1u << r;
  }
  int mine = 0;
  uint32_t mkey = 0;  // (lane j: the ordered bits of its logit, which give the logit back)
  for (int j = 0; j < k; j++) {
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < R; r++) m = ((live >> r) & 1) && ord[r] > m ? ord[r] : m;
    m = wave_max_u32(m);
    // the lowest id among the live keys equal to m: the first r with a hit, its lowest lane
    int wr = 0, wl = 0;
#pragma unroll
    for (int r = R - 1; r >= 0; r--) {
      const uint64_t b = __ballot(((live >> r) & 1) && ord[r] == m);
      if (b) wr = r, wl = __builtin_ctzll(b);
    }
    if (lane == wl) live &= ~(1u << wr);
    if (lane == j) mine = wl + WAVE * wr, mkey = m;
  }
  const int id = mine;
  const bool on = lane < k;
  const float l = on ? key_logit(mkey) : 0.0f;
  const double l0 = __shfl(double(l), 0, WAVE);
  double e = 0;
  if (on) e = sigmoid ? 1.0 / (1.0 + exp(-double(l))) : exp(double(l) - l0);
  ev[lane] = e;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane == 0) {
    double s = row_sum(ev, k);
    if (sigmoid) s = s < 6.103515625e-5 ? 6.103515625e-5 : s;  // (std::max(s, 2^-14): a NaN sum stays NaN)
    *sum = s;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const double s = *sum;
  __builtin_amdgcn_wave_barrier();  // (the scratch is free again once every lane has read the sum)
  if (!on) return -1;
  if constexpr (DEV_IDS)
    __hip_atomic_store(ids + lane, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    ids[lane] = id;
  const double w = e / s;
  if (w32) w32[lane] = float(w);
  if (w64) w64[lane] = w;
  return id;
}

int check_route_args(int64_t n, int per_col, int E, int k);

int launch_topk(const float* logits, int64_t n, int64_t row, int per_col, int64_t pitch, int E, int k, int sigmoid,
                int32_t* ids, float* w32, double* w64, hipStream_t s);

// Router logits out[t out_row + e] = x[t] . W[e] (float64 accumulation, rounded once). xq: when given, x is also
// quantised into XQ rows (gemv.h) by extra workgroups of the same launch (H a multiple of 256). part (part_elems
// doubles, router_part_elems for the most tokens of a layer; may be null): the fp64 partial sums of prefill-sized
// batches whose tiles are too few for the device, K split over workgroups and the parts added in a fixed order.
int launch_router(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* out, int64_t out_row,
                  uint32_t* xq, double* part, size_t part_elems, hipStream_t s);
size_t router_part_elems(int64_t max_T, int E, int H);

// out (T x H fp32) = x / sqrt(mean(x^2) + eps) * w per row (float64 mean and quotient, rounded once, then fp32 w)
int launch_rmsnorm(const void* x, int x_dtype, const float* w, float eps, int64_t T, int H, float* out,
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
  CTRL_ROUTED = 7,    // router workgroups finished (k_router_route; reset by the last)
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
  int balanced = 0;  // 1: an expert's c rows in tiles of balanced_rows(c, BM) rows (the last one shorter)
  // (optional, the one-launch routing of more than one token group) a ticket per group, GTICK_STRIDE ints apart,
  // zero before the first launch (kept zero by the launches)
  int32_t* gtick = nullptr;
  // (optional, the prefill path) per sorted row s, filled by the scatter: its token t = order[s] / k into row_a, and
  // that token's row factors row_f[0][t], row_f[1][t] into row_out[0][s], row_out[1][s]
  int32_t* row_a = nullptr;
  const float2* row_f[2] = {nullptr, nullptr};
  float2* row_out[2] = {nullptr, nullptr};
};

// rows per tile when an expert's c rows are split into tiles of at most bm rows of nearly equal size: the fewest
// tiles, their size rounded up to a multiple of 16 (whole MFMA row blocks); the tiles are ceil(c / that)
__host__ __device__ inline int balanced_rows(int c, int bm) {
  if (c <= 0) return bm;
  const int nt = (c + bm - 1) / bm, r = ((c + nt - 1) / nt + 15) / 16 * 16;
  return r < bm ? r : bm;
}

// blocks of a dispatch of P pairs
inline int64_t dispatch_blocks(int64_t P) { return P > 0 ? (P + DISPATCH_BLOCK - 1) / DISPATCH_BLOCK : 1; }
// an upper bound on the tiles of P pairs over E experts with BM rows per tile
inline int64_t tile_bound(int64_t P, int E, int BM) { return (P + BM - 1) / BM + (P < E ? P : E); }

// exclusive prefix of one value per thread of a DISPATCH_BLOCK block; *total the sum (all threads)
__device__ __forceinline__ int block_scan(int v, int* total) {
  __shared__ int wsum[DISPATCH_BLOCK / WAVE];
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  int x = v;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int y = __shfl_up(x, o, WAVE);
    if (lane >= o) x += y;
  }
  if (lane == WAVE - 1) wsum[wv] = x;
  __syncthreads();
  if (wv == 0) {
    int s = lane < DISPATCH_BLOCK / WAVE ? wsum[lane] : 0;
#pragma unroll
    for (int o = 1; o < DISPATCH_BLOCK / WAVE; o <<= 1) {
      const int y = __shfl_up(s, o, WAVE);
      if (lane >= o) s += y;
    }
    if (lane < DISPATCH_BLOCK / WAVE) wsum[lane] = s;  // (inclusive over waves)
  }
  __syncthreads();
  const int before = (wv ? wsum[wv - 1] : 0) + x - v;
  *total = wsum[DISPATCH_BLOCK / WAVE - 1];
  __syncthreads();
  return before;
}

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

// Small batches (n k <= DISPATCH_BLOCK pairs, E <= MAX_EXPERTS): the top k of n tokens' plain (n, E) logits and the
// dispatch of their pairs (d.ids receives the ids; counts, offsets, order, slot, tiles, ctrl[CTRL_TILES]) in one
// workgroup: the results of launch_topk followed by launch_dispatch.
int launch_route_small(const float* logits, int64_t n, int E, int k, int sigmoid, int32_t* ids, float* w32,
                       const DispatchBufs& d, hipStream_t s);

// Router logits (as launch_router, into logits (T, E)) and the routing of launch_route_small in one launch, for T <=
// ROUTER_GROUPS ROUTER_TG tokens, H a multiple of 256 (at least 2 values per wave), T k <= DISPATCH_BLOCK pairs, E <= MAX_EXPERTS
// (router_route_fits). xq: when given, x is also quantised into XQ rows.
bool router_route_fits(int64_t T, int H, int E, int k);
int launch_router_route(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* logits,
                        uint32_t* xq, int k, int sigmoid, int32_t* ids, float* w32, const DispatchBufs& d,
                        hipStream_t s);

}  // namespace artlite
