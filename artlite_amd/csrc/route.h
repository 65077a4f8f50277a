// Routing kernels' launchers (route.hip) and the dispatch's (dispatch.hip).
#pragma once

#include "common.h"

#include <type_traits>

namespace artlite {

constexpr int MAX_EXPERTS = 1024;  // (keys per lane: 16)
constexpr int MAX_TOPK = 64;       // (one lane per chosen expert)
constexpr int ROUTER_TG = 16;      // tokens per router block (at most)
constexpr int ROUTER_GROUPS = 4;   // token groups of the few-token router (k_router_few), at most
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
// return -1 (ids null: none written; w32 and w64 null: no weights computed).
// (topk_wave_by: the logit of expert e < E from load(e), called by the lane that ranks it)
template <int R, typename LOAD>
__device__ __forceinline__ int topk_wave_by(LOAD load, int E, int k, int sigmoid, double* ev, double* sum, int lane,
                                            int32_t* __restrict__ ids, float* __restrict__ w32,
                                            double* __restrict__ w64) {
  static_assert(R <= 32, "keys per lane");
  uint32_t ord[R], live = 0;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int e = lane + WAVE * r;
    float l = 0.0f;
    if (e < E) l = load(e);
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
  if (!w32 && !w64) {  // (the ids alone)
    if (ids && on) ids[lane] = id;
    return on ? id : -1;
  }
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
  if (ids) ids[lane] = id;
  const double w = e / s;
  if (w32) w32[lane] = float(w);
  if (w64) w64[lane] = w;
  return id;
}
template <int R>
__device__ __forceinline__ int topk_wave(const float* __restrict__ p, int per_col, int64_t pitch, int E, int k,
                                         int sigmoid, double* ev, double* sum, int lane, int32_t* __restrict__ ids,
                                         float* __restrict__ w32, double* __restrict__ w64) {
  return topk_wave_by<R>(
      [&](int e) { return per_col == E ? p[e] : p[int64_t(e / per_col) * pitch + e % per_col]; }, E, k, sigmoid, ev,
      sum, lane, ids, w32, w64);
}

// the 32-bit maximum / minimum over each group of W lanes (16: a DPP row; 32: two rows, then the permlane16 swap
// that pairs rows 0 / 1 and 2 / 3, as in wave_max_u32), in every lane of the group
template <int W>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(W == 16 || W == 32, "group width");
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  if constexpr (W == 32) {
    const auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(uint32_t(s16[0]), uint32_t(s16[1]));
  }
  return v;
}
template <int W>
__device__ __forceinline__ uint32_t group_min_u32(uint32_t v) {
  static_assert(W == 16 || W == 32, "group width");
  v = min(v, dpp_u32<0xB1>(v));
  v = min(v, dpp_u32<0x4E>(v));
  v = min(v, dpp_u32<0x141>(v));
  v = min(v, dpp_u32<0x140>(v));
  if constexpr (W == 32) {
    const auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = min(uint32_t(s16[0]), uint32_t(s16[1]));
  }
  return v;
}

// A lane's RR keys sorted in descending order in place, by a sorting network (RR = 1, 2, 4, 8; 8: Batcher's odd-even
// merge sort, 19 compare-exchanges)
template <int RR>
__device__ __forceinline__ void sort_desc(uint64_t (&k)[RR]) {
  auto cx = [&](int i, int j) {
    const uint64_t a = k[i], b = k[j];
    k[i] = b > a ? b : a;
    k[j] = b > a ? a : b;
  };
  if constexpr (RR == 2) {
    cx(0, 1);
  } else if constexpr (RR == 4) {
    cx(0, 1), cx(2, 3), cx(0, 2), cx(1, 3), cx(1, 2);
  } else if constexpr (RR == 8) {
    cx(0, 1), cx(2, 3), cx(4, 5), cx(6, 7), cx(0, 2), cx(1, 3), cx(4, 6), cx(5, 7), cx(1, 2), cx(5, 6);
    cx(0, 4), cx(1, 5), cx(2, 6), cx(3, 7), cx(2, 4), cx(3, 5), cx(1, 2), cx(3, 4), cx(5, 6);
  } else {
    static_assert(RR == 1, "keys per lane: 1, 2, 4 or 8");
  }
}

// The top k of 64 / W tokens' logits at once, one group of W lanes each (E <= W RR experts, k <= W): lane c of a
// group holds experts W r + c (r < RR) of its token's logits p as logit_key's keys (ordered bits above ~id; 0 for
// none), sorted in descending order within the lane, then k rounds of: the group's largest ordered bits among the
// lanes' first keys (a group maximum), the largest ~id among the first keys holding them (a second group maximum:
// the lowest id), the lane holding that key dropping it from its list, lane j of the group keeping the j-th. A lane's
// first key is its best one left, so the round takes the best key left in the group: the same choice, in the same
// order, as topk_wave (larger logits first, equal logits to the lower id), with the groups' rounds side by side. on:
// the group has a token. Lane j < k of a group gets its id (the return value) and the logit's ordered bits (key);
// other lanes get -1.
template <int W, int RR>
__device__ __forceinline__ int topk_rows(const float* __restrict__ p, int E, int k, bool on, int c, uint32_t& key) {
  float l[RR];
#pragma unroll
  for (int r = 0; r < RR; r++) l[r] = p[min(W * r + c, E - 1)];  // (every load issued before any is used)
  uint64_t kk[RR];
#pragma unroll
  for (int r = 0; r < RR; r++) {
    const int e = W * r + c;
    kk[r] = on && e < E ? logit_key(l[r], e) : 0;  // (a real key's low half, ~id, is never 0)
  }
  sort_desc<RR>(kk);
  int mine = -1;
  uint32_t mkey = 0;
  for (int j = 0; j < k; j++) {
    const uint32_t hi = uint32_t(kk[0] >> 32), lo = uint32_t(kk[0]);
    const uint32_t m = group_max_u32<W>(hi);
    const uint32_t cl = group_max_u32<W>(hi == m ? lo : 0u);
    if (hi == m && lo == cl) {  // (the one lane holding the round's key: the ids, hence ~ids, are distinct)
#pragma unroll
      for (int r = 0; r + 1 < RR; r++) kk[r] = kk[r + 1];
      kk[RR - 1] = 0;
    }
    if (c == j) mine = int(~cl), mkey = m;
  }
  key = mkey;
  return on && c < k ? mine : -1;
}

// The weights of the tokens of topk_rows (lane j < k of a group of W lanes: its id's logit as ordered bits, key), as
// topk_wave computes them: e^(l - l_0) (l_0 the group's first, its largest) or sigmoid(l) in double, their sum in
// numpy's pairwise order by the group's lane 0, e / sum rounded to fp32 into w32[j] of the group's token. ev (64
// doubles) and sum (64 / W): the wave's LDS scratch.
template <int W>
__device__ __forceinline__ void rows_weights(uint32_t key, int k, int sigmoid, bool on, int c, double* ev, double* sum,
                                             float* __restrict__ w32) {
  const int lane = threadIdx.x & (WAVE - 1), grp = lane / W;
  const bool mine = on && c < k;
  const float l = mine ? key_logit(key) : 0.0f;
  const double l0 = __shfl(double(l), grp * W, WAVE);
  double e = 0;
  if (mine) e = sigmoid ? 1.0 / (1.0 + exp(-double(l))) : exp(double(l) - l0);
  ev[lane] = e;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (c == 0) {
    double s = row_sum(ev + W * grp, k);
    if (sigmoid) s = s < 6.103515625e-5 ? 6.103515625e-5 : s;  // (std::max(s, 2^-14): a NaN sum stays NaN)
    sum[grp] = s;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const double s = sum[grp];
  __builtin_amdgcn_wave_barrier();  // (the scratch is free again once every lane has read the sum)
  if (mine) w32[c] = float(e / s);
}

int check_route_args(int64_t n, int per_col, int E, int k);

int launch_topk(const float* logits, int64_t n, int64_t row, int per_col, int64_t pitch, int E, int k, int sigmoid,
                int32_t* ids, float* w32, double* w64, hipStream_t s);
// the same over a split router's fp64 parts (launch_router with parts_left): each logit is the sum of its parts in
// part order, rounded once, and is also stored to out[t out_row + e]
int launch_topk_parts(const double* part, int parts, int64_t n, int E, float* out, int64_t out_row, int k, int sigmoid,
                      int32_t* ids, float* w32, hipStream_t s);

// Router logits out[t out_row + e] = x[t] . W[e] (float64 accumulation, rounded once). xq: when given, x is also
// quantised into XQ rows (gemv.h) by extra workgroups of the same launch (H a multiple of 256). part (part_elems
// doubles, router_part_elems for the most tokens of a layer; may be null): the fp64 partial sums of prefill-sized
// batches whose tiles are too few for the device, K split over workgroups and the parts added in a fixed order.
// parts_left (optional): the parts are then not added here: *parts_left = their count (for launch_topk_parts), or 0
// when the logits are in out.
int launch_router(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* out, int64_t out_row,
                  uint32_t* xq, double* part, size_t part_elems, hipStream_t s, int* parts_left = nullptr);
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

// ---- the routing of a few tokens by one workgroup (route_core): top k, then the stable counting sort of the pairs

// a workgroup barrier over LDS alone: global stores issued before it are not waited for (nothing in the workgroup
// reads them back)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// a wave's inclusive prefix sum by DPP (row shifts within 16-lane rows, then the row broadcasts of lanes 15 and 31):
// x + the values of 1, 2, 3 lanes back, then 4 back in lanes 4..15 of a row, 8 back in lanes 8..15, lane 15's in
// rows 1 and 3, lane 31's in rows 2 and 3 (a disabled or out-of-row source adds 0)
__device__ __forceinline__ int wave_scan_dpp(int a) {
  int x = a + __builtin_amdgcn_update_dpp(0, a, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, a, 0x112, 0xF, 0xF, false);         // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, a, 0x113, 0xF, 0xF, false);         // row_shr:3
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xE, false);         // row_shr:4, banks 1-3
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xC, false);         // row_shr:8, banks 2-3
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);         // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);         // row_bcast:31, rows 2 and 3
  return x;
}

// exclusive prefixes of S values per thread of an NT-thread workgroup (ex), and their sums (tot, every thread):
// wave scans, the waves' sums scanned by wave 0; two LDS barriers (ws: S x NW ints of LDS, free again only after a
// further barrier)
template <int NT, int S>
__device__ __forceinline__ void block_scan_n(const int (&v)[S], int (&ex)[S], int (&tot)[S], int (*ws)[NT / WAVE]) {
  constexpr int NW = NT / WAVE;
  static_assert(NW <= WAVE, "one wave scans the waves' sums");
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  int x[S];
#pragma unroll
  for (int j = 0; j < S; j++) x[j] = wave_scan_dpp(v[j]);
  if (lane == WAVE - 1)
#pragma unroll
    for (int j = 0; j < S; j++) ws[j][wv] = x[j];
  lds_barrier();
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < S; j++) {
      const int y = wave_scan_dpp(lane < NW ? ws[j][lane] : 0);
      if (lane < NW) ws[j][lane] = y;  // (inclusive over waves)
    }
  }
  lds_barrier();
#pragma unroll
  for (int j = 0; j < S; j++) {
    ex[j] = (wv ? ws[j][wv - 1] : 0) + x[j] - v[j];
    tot[j] = ws[j][NW - 1];
  }
}

// LDS scratch of route_core in an NT-thread workgroup (at most NT pairs and NT experts)
template <int NT>
struct RouteLds {
  static constexpr int NW = NT / WAVE;
  static_assert(NT % 8 == 0, "wcnt rows in 16-byte pieces");
  double ev[NW][WAVE];
  double sum[NW][4];
  int sid[NT];
  int base[NT];
  __align__(16) uint16_t wcnt[NW][NT];
  int ws[3][NW];
};

// route_core's outputs into memory of the workgroup's own (LDS), each optional: the tile list (2 ints a tile), the
// sorted pairs' tokens (P: order / k, the rows of A a gate / up tile reads), the expert offsets (E + 1) and the tile
// count (1); and (route_core's STAGE) room for the n E
// logits, which are then copied there first, all loads in flight at once, rather than read a token at a time by its
// wave
struct RouteOut {
  int* tiles = nullptr;
  int* order = nullptr;
  int* offsets = nullptr;
  int* n_tiles = nullptr;
  float* stage = nullptr;
};

// the logits of n tokens (n E floats) into LDS at stage by an NT-thread workgroup: 16-byte loads (E a multiple of
// 4; at most 8 a thread), every one issued before the first is stored; complete for every thread after a barrier
template <int NT>
__device__ __forceinline__ void stage_logits(const float* __restrict__ logits, int nE, float* stage) {
  const int nv = nE / 4, tid = threadIdx.x, nj = (nv + NT - 1) / NT;
  const float4* src = reinterpret_cast<const float4*>(logits);
  float4* dst = reinterpret_cast<float4*>(stage);
  float4 v0, v1, v2, v3, v4, v5, v6, v7;
  // (past the end: the last vector again, not stored)
  auto ld = [&](int j) { return src[min(tid + j * NT, nv - 1)]; };
  v0 = ld(0);
  if (nj > 1) v1 = ld(1);
  if (nj > 2) v2 = ld(2), v3 = ld(3);
  if (nj > 4) v4 = ld(4), v5 = ld(5), v6 = ld(6), v7 = ld(7);
  auto st = [&](int j, const float4& v) {
    if (tid + j * NT < nv) dst[tid + j * NT] = v;
  };
  st(0, v0);
  if (nj > 1) st(1, v1);
  if (nj > 2) st(2, v2), st(3, v3);
  if (nj > 4) st(4, v4), st(5, v5), st(6, v6), st(7, v7);
}

// The routing of n tokens' (n, E) logits by one NT-thread workgroup (n k <= NT pairs, E <= NT experts, R >= E / 64
// keys per lane): the top k of each token (a wave per token; ids and w32, when given, receive the ids and the
// weights), then the counts, offsets, the tile list of BM rows a tile (BM 0: none; balanced: balanced_rows; the
// GEMV's order, BM <= 4: each tile's rows above bit 24 of its expert) and each pair's sorted position, into g's
// arrays (when gw: counts, offsets, order, slot, tiles, ctrl[CTRL_TILES]) and into o's (when given). Every exchange is through LDS (no barrier waits for the global stores); o's arrays are
// complete for every thread after one more barrier.
template <int NT, int R, bool STAGE = false>
__device__ __forceinline__ void route_core(const float* __restrict__ logits, int n, int E, int k, int sigmoid,
                                           int BM, int balanced, int32_t* __restrict__ ids, float* __restrict__ w32,
                                           const DispatchBufs& g, bool gw, RouteLds<NT>& s, const RouteOut& o) {
  constexpr int NW = NT / WAVE;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid / WAVE;
  if (tid < E) s.base[tid] = 0;
  for (int i = tid; i < NW * NT / 8; i += NT) reinterpret_cast<uint4*>(&s.wcnt[0][0])[i] = uint4{0, 0, 0, 0};
  const float* lg = logits;
  if constexpr (STAGE) {
    stage_logits<NT>(logits, n * E, o.stage);
    __syncthreads();
    lg = o.stage;
  }
  if constexpr (R <= 2) {
    // (a token per group of 32 lanes, two a wave, while the waves have enough of those groups for every token;
    // else of 16 lanes, four a wave)
    auto rows = [&](auto wc) {
      constexpr int W = decltype(wc)::value, G = WAVE / W;
      const int c = lane % W;
      for (int t0 = G * wv; t0 < n; t0 += G * NW) {
        const int t = t0 + lane / W;
        const bool on = t < n;
        uint32_t key;
        const int id = topk_rows<W, R * WAVE / W>(lg + int64_t(on ? t : 0) * E, E, k, on, c, key);
        if (id >= 0) {
          s.sid[t * k + c] = id;
          if (ids) ids[t * k + c] = id;
        }
        if (w32) rows_weights<W>(key, k, sigmoid, on, c, s.ev[wv], s.sum[wv], w32 + int64_t(on ? t : 0) * k);
      }
    };
    if (k <= 16) {
      if (n <= 2 * NW)
        rows(std::integral_constant<int, 32>{});
      else
        rows(std::integral_constant<int, 16>{});
    }
  }
  if (R > 2 || k > 16) {
    for (int t = wv; t < n; t += NW) {  // (one wave per token)
      const int id = topk_wave<R>(lg + int64_t(t) * E, E, 0, E, k, sigmoid, s.ev[wv], &s.sum[wv][0], lane,
                                  ids ? ids + t * k : nullptr, w32 ? w32 + t * k : nullptr, nullptr);
      if (lane < k) s.sid[t * k + lane] = id;
    }
  }
  lds_barrier();
  const int P = n * k, p = tid;
  const bool valid = p < P;
  const int id = valid ? s.sid[p] : -1;
  if (valid) atomicAdd(&s.base[id], 1);  // (counts: order-free)
  // each pair's rank among the earlier pairs of its expert: the lanes of its wave with the same expert (ballots over
  // the id bits), then the earlier waves' counts (read once every wave has written its own)
  uint64_t peers = __ballot(valid);
  for (int bit = 0; (1 << bit) < E; bit++) {
    const bool set = (id >> bit) & 1;
    const uint64_t b = __ballot(set);
    peers &= set ? b : ~b;
  }
  const uint64_t below = (uint64_t(1) << lane) - 1;
  int rank = __popcll(peers & below);
  if (valid && !(peers & below)) s.wcnt[wv][id] = uint16_t(__popcll(peers));
  lds_barrier();
  // the prefixes: the expert's count (low 16 bits) and its tiles of the expert GEMMs (high 16 bits; both sums stay
  // below 2^16: at most NT pairs); for the GEMV's tile order, its full tiles and its last tile's class
  const int e = tid;
  const int c = e < E ? s.base[e] : 0;
  const int rows = balanced ? balanced_rows(c, BM) : BM;
  const int nt = e < E && BM > 0 ? (c + rows - 1) / rows : 0;
  const bool gemv_order = BM > 0 && !balanced && BM <= 4;
  const int full = gemv_order && e < E ? c / rows : 0, rem = gemv_order && e < E ? c % rows : 0;
  // (11-bit class fields: a class holds at most MAX_EXPERTS tiles; the last field's prefix stays below 2^10 and its
  // total, which may reach 2^10 and carry out of the word, is not read)
  const int v[3] = {c | (nt << 16), full, (rem == 3) | (rem == 2) << 11 | (rem == 1) << 22};
  int ex[3], tot[3];
  block_scan_n<NT, 3>(v, ex, tot, s.ws);
  const int packed = ex[0], packed_total = tot[0];
  const int start = packed & 0xFFFF, total = packed_total & 0xFFFF;
  if (e < E) {
    if (gw) {
      g.counts[e] = c;
      g.offsets[e] = start;
    }
    if (o.offsets) o.offsets[e] = start;
    s.base[e] = start;
  }
  if (e == 0) {
    if (gw) g.offsets[E] = total;
    if (o.offsets) o.offsets[E] = total;
  }
  // (the GEMV's order: the tile's rows above bit 24 of its expert)
  auto put_tile = [&](int t, int s0, int m = 0) {
    const int em = e | (m << 24);
    if (gw) {
      g.tiles[2 * t] = em;
      g.tiles[2 * t + 1] = s0;
    }
    if (o.tiles) {
      o.tiles[2 * t] = em;
      o.tiles[2 * t + 1] = s0;
    }
  };
  if (BM > 0 && !gemv_order) {  // the expert GEMMs' tiles: experts ascending, BM sorted rows each
    const int t0 = packed >> 16;
    for (int m = 0; m < nt; m++) put_tile(t0 + m, start + m * rows);
  } else if (gemv_order) {
    // the GEMV's tiles by rows, most first: every expert's full tiles of BM rows, then the last tiles of BM - 1
    // rows, ..., of 1 row (experts ascending within each class), so that a persistent launch dealing its items back
    // and forth hands each workgroup items of about equal total rows
    const int pf = ex[1], nfull = tot[1];
    for (int m = 0; m < full; m++) put_tile(pf + m, start + m * rows, rows);
    if (rem) {  // (class base: the full tiles, then the classes of more rows)
      const uint32_t up = uint32_t(ex[2]), ut = uint32_t(tot[2]);
      const int n3 = int(ut & 0x7FF), n2 = int((ut >> 11) & 0x7FF);
      const int t = nfull + (rem == 3 ? int(up & 0x7FF) : rem == 2 ? n3 + int((up >> 11) & 0x7FF) : n3 + n2 + int(up >> 22));
      put_tile(t, start + full * rows, rem);
    }
  }
  if (BM > 0 && e == 0) {
    if (gw) g.ctrl[CTRL_TILES] = packed_total >> 16;
    if (o.n_tiles) *o.n_tiles = packed_total >> 16;
  }
  lds_barrier();  // (base now holds each expert's start)
  if (valid) {
#pragma unroll
    for (int w = 0; w < NW; w++)  // (all the reads in flight at once)
      if (w < wv) rank += s.wcnt[w][id];
    const int dest = s.base[id] + rank;
    if (gw) {
      g.order[dest] = p;
      g.slot[p] = dest;
    }
    if (o.order) o.order[dest] = p / k;
  }
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

// Router logits (as launch_router, into logits (T, E)) of small batches: T <= ROUTER_GROUPS ROUTER_TG tokens, H a
// multiple of 256 (at least 2 values per wave), E <= MAX_EXPERTS (router_few_fits). xq: when given, x is also
// quantised into XQ rows.
bool router_few_fits(int64_t T, int H, int E);
int launch_router_few(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* logits,
                        uint32_t* xq, hipStream_t s);

}  // namespace artlite
