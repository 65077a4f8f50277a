// Routing: the router's logits (x W^T with float64 accumulation) and the top k of each token's logits with their
// weights, one wave64 per token; the C entry points artlite_moe_route / artlite_moe_top_k.
//
// Ranking follows the reference's host step (csrc/artlite/moe_host.cpp:45-73): a logit's 64-bit key is its ordered
// fp32 bits (after l + 0, so -0 ranks as +0) above ~id, so larger logits win and equal logits go to the lower id.
// The weights follow moe_host.cpp:62-72: e^(l - l_max) (or sigmoid(l)) in double, their sum in numpy's pairwise
// order (moe_host.cpp:25-39), e / sum rounded to fp32.
#include "route.h"
#include "xq.h"

#include <algorithm>

namespace artlite {

constexpr int TOPK_WAVES = 4;

// one wave per token (topk_wave, route.h)
template <int R>
__global__ __launch_bounds__(TOPK_WAVES * WAVE) void k_topk(const float* __restrict__ logits, int64_t n, int64_t row,
                                                            int per_col, int64_t pitch, int E, int k, int sigmoid,
                                                            int32_t* __restrict__ ids, float* __restrict__ w32,
                                                            double* __restrict__ w64) {
  __shared__ double ev[TOPK_WAVES][WAVE];
  __shared__ double sum[TOPK_WAVES];
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  const int64_t t = int64_t(blockIdx.x) * TOPK_WAVES + wv;
  if (t >= n) return;  // (uniform per wave)
  const int id = topk_wave<R>(logits + t * row, per_col, pitch, E, k, sigmoid, ev[wv], &sum[wv], lane, ids + t * k,
                              w32 ? w32 + t * k : nullptr, w64 ? w64 + t * k : nullptr);
  (void)id;
}

constexpr int TOPK_MAXPARTS = 16;  // (router_split's parts at most)

// one wave per token over a split router's parts: lane e's logit the sum of its parts in part order (as
// k_router_parts adds them), rounded once and stored
template <int R>
__global__ __launch_bounds__(TOPK_WAVES * WAVE) void k_topk_parts(const double* __restrict__ part, int parts,
                                                                  int64_t n, int E, float* __restrict__ out,
                                                                  int64_t out_row, int k, int sigmoid,
                                                                  int32_t* __restrict__ ids, float* __restrict__ w32) {
  __shared__ double ev[TOPK_WAVES][WAVE];
  __shared__ double sum[TOPK_WAVES];
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  const int64_t t = int64_t(blockIdx.x) * TOPK_WAVES + wv, pn = n * E;
  if (t >= n) return;  // (uniform per wave)
  auto load = [&](int e) {
    const double* q = part + t * E + e;
    double v[TOPK_MAXPARTS];  // (every part's load in flight together)
#pragma unroll
    for (int z = 0; z < TOPK_MAXPARTS; z++) v[z] = z < parts ? q[int64_t(z) * pn] : 0.0;
    double c = v[0];
#pragma unroll
    for (int z = 1; z < TOPK_MAXPARTS; z++)
      if (z < parts) c += v[z];
    const float l = float(c);
    out[t * out_row + e] = l;
    return l;
  };
  topk_wave_by<R>(load, E, k, sigmoid, ev[wv], &sum[wv], lane, ids + t * k, w32 ? w32 + t * k : nullptr, nullptr);
}

int launch_topk_parts(const double* part, int parts, int64_t n, int E, float* out, int64_t out_row, int k, int sigmoid,
                      int32_t* ids, float* w32, hipStream_t s) {
  if (n <= 0) return ARTLITE_OK;
  if (parts < 1 || parts > TOPK_MAXPARTS || E < 1 || E > MAX_EXPERTS || k < 1 || k > E || k > MAX_TOPK)
    return fail(ARTLITE_EINVAL, "top-k over router parts: %d parts, E %d, k %d", parts, E, k);
  const dim3 grid(unsigned((n + TOPK_WAVES - 1) / TOPK_WAVES)), block(TOPK_WAVES * WAVE);
#define ART_TOPK(RR) \
  k_topk_parts<RR><<<grid, block, 0, s>>>(part, parts, n, E, out, out_row, k, sigmoid, ids, w32)
  if (E <= 64)
    ART_TOPK(1);
  else if (E <= 128)
    ART_TOPK(2);
  else if (E <= 256)
    ART_TOPK(4);
  else if (E <= 512)
    ART_TOPK(8);
  else
    ART_TOPK(16);
#undef ART_TOPK
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int launch_topk(const float* logits, int64_t n, int64_t row, int per_col, int64_t pitch, int E, int k, int sigmoid,
                int32_t* ids, float* w32, double* w64, hipStream_t s) {
  if (n <= 0) return ARTLITE_OK;
  const dim3 grid(unsigned((n + TOPK_WAVES - 1) / TOPK_WAVES)), block(TOPK_WAVES * WAVE);
#define ART_TOPK(RR) k_topk<RR><<<grid, block, 0, s>>>(logits, n, row, per_col, pitch, E, k, sigmoid, ids, w32, w64)
  if (E <= 64)
    ART_TOPK(1);
  else if (E <= 128)
    ART_TOPK(2);
  else if (E <= 256)
    ART_TOPK(4);
  else if (E <= 512)
    ART_TOPK(8);
  else
    ART_TOPK(16);
#undef ART_TOPK
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// Router logits: a block of EW waves (one expert each) over a tile of up to ROUTER_TG tokens whose rows are staged
// in LDS; each lane accumulates float64 partial dot products (exact products of fp32 / bf16 values) over
// h = 4 lane + 256 j, its weights for 8 j at a time loaded up front, then a fixed shuffle tree; the sum is rounded
// once to fp32. With xq, workgroups past the router's (blockIdx.x >= nbx, first token tile) quantise x into XQ,
// one wave per (row, unit).
template <int XT, int EW>
__global__ __launch_bounds__(EW * WAVE) void k_router(const void* __restrict__ xv, const float* __restrict__ W, int H,
                                                     int E, int64_t T, int tt, float* __restrict__ out,
                                                     int64_t out_row, uint32_t* __restrict__ xq, int nbx) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // tt rows of H values (x's own dtype)
  constexpr int XB = XT == ARTLITE_X_F32 ? 4 : 2;
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  if (int(blockIdx.x) >= nbx) {  // XQ of x
    if (blockIdx.y) return;
    const int64_t w = int64_t(blockIdx.x - nbx) * EW + wv;
    if (w < T * (H / 256)) xq_quant_unit<XT>(xv, w, H, xq, lane);
    return;
  }
  const int64_t t0 = int64_t(blockIdx.y) * tt;
  const int nt = int(min(int64_t(tt), T - t0));
  {  // stage the tile's rows (16-byte pieces)
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(xv) + t0 * H * XB);
    uint4* dst = reinterpret_cast<uint4*>(xs);
    const int n16 = nt * H * XB / 16;
    int i = threadIdx.x;
    for (; i + 7 * EW * WAVE < n16; i += 8 * EW * WAVE) {  // (eight loads in flight per lane)
      uint4 v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = src[i + j * EW * WAVE];
#pragma unroll
      for (int j = 0; j < 8; j++) dst[i + j * EW * WAVE] = v[j];
    }
    for (; i < n16; i += EW * WAVE) dst[i] = src[i];
  }
  __syncthreads();
  const int e = blockIdx.x * EW + wv;
  if (e >= E) return;
  const float* w = W + int64_t(e) * H;
  double acc[ROUTER_TG];
#pragma unroll
  for (int t = 0; t < ROUTER_TG; t++) acc[t] = 0.0;
  for (int h0 = 0; h0 < H; h0 += 8 * 4 * WAVE) {
    float4 wq[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int h = h0 + 4 * lane + 4 * WAVE * j;
      wq[j] = h < H ? *reinterpret_cast<const float4*>(w + h) : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int h = h0 + 4 * lane + 4 * WAVE * j;
      if (h >= H) break;
#pragma unroll
      for (int t = 0; t < ROUTER_TG; t++) {
        if (t < nt) {
          float x0, x1, x2, x3;
          if (XT == ARTLITE_X_F32) {
            const float4 v = *reinterpret_cast<const float4*>(xs + (int64_t(t) * H + h) * 4);
            x0 = v.x, x1 = v.y, x2 = v.z, x3 = v.w;
          } else {
            const uint2 v = *reinterpret_cast<const uint2*>(xs + (int64_t(t) * H + h) * 2);
            x0 = bf16_to_f32(v.x & 0xFFFFu), x1 = bf16_to_f32(v.x >> 16);
            x2 = bf16_to_f32(v.y & 0xFFFFu), x3 = bf16_to_f32(v.y >> 16);
          }
          acc[t] += double(x0) * double(wq[j].x);
          acc[t] += double(x1) * double(wq[j].y);
          acc[t] += double(x2) * double(wq[j].z);
          acc[t] += double(x3) * double(wq[j].w);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < ROUTER_TG; t++) {
    double v = acc[t];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    if (lane == 0 && t < nt) out[(t0 + t) * out_row + e] = float(v);
  }
}

// The 16 tokens' sums across a wave by halving exchanges: at lane bit o (32, 16, 8, 4) a lane keeps the half of its
// remaining tokens that its bit selects and adds the partner's sums of those (n: the tokens left, a compile-time
// count, so that every index is a constant), then bits 2 and 1 add up the four lanes left per token. Lane l ends with
// the sum of token sum_token(l) (each token's in four lanes).
template <int N>
__device__ __forceinline__ void halve_tokens(double (&v)[ROUTER_TG], int lane, int o) {
  const bool hi = lane & o;
#pragma unroll
  for (int i = 0; i < N; i++) {
    const double keep = hi ? v[N + i] : v[i], give = hi ? v[i] : v[N + i];
    v[i] = keep + __shfl_xor(give, o, WAVE);
  }
}
__device__ __forceinline__ double token_sums(double (&v)[ROUTER_TG], int lane) {
  static_assert(ROUTER_TG == 16, "halving exchanges of 16 tokens");
  halve_tokens<8>(v, lane, 32);
  halve_tokens<4>(v, lane, 16);
  halve_tokens<2>(v, lane, 8);
  halve_tokens<1>(v, lane, 4);
  double s = v[0] + __shfl_xor(v[0], 2, WAVE);
  return s + __shfl_xor(s, 1, WAVE);
}
__device__ __forceinline__ int sum_token(int lane) {
  return ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
}

// Router logits for small batches (T <= ROUTER_TG tokens per tile, H a multiple of 1024): a workgroup per expert,
// its 4 waves each a quarter of H (lane: h = quarter + 4 lane + 256 j), x read straight from memory (L2), float64
// products and per-wave shuffle trees, then the quarters summed in order; rounded once to fp32. With xq, workgroups
// past the experts' quantise x into XQ as k_router's do.
template <int XT>
__global__ __launch_bounds__(4 * WAVE) void k_router_small(const void* __restrict__ xv, const float* __restrict__ W,
                                                          int H, int E, int64_t T, float* __restrict__ out,
                                                          int64_t out_row, uint32_t* __restrict__ xq) {
  __shared__ double part[4][ROUTER_TG];
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  if (int(blockIdx.x) >= E) {  // XQ of x
    if (blockIdx.y) return;
    const int64_t w = int64_t(blockIdx.x - E) * 4 + wv;
    if (w < T * (H / 256)) xq_quant_unit<XT>(xv, w, H, xq, lane);
    return;
  }
  const int e = blockIdx.x;
  const int64_t t0 = int64_t(blockIdx.y) * ROUTER_TG;
  const int nt = int(min(int64_t(ROUTER_TG), T - t0));
  const int q = H / 4, nj = q / (4 * WAVE);
  const float* w = W + int64_t(e) * H + wv * q;
  double acc[ROUTER_TG];
#pragma unroll
  for (int t = 0; t < ROUTER_TG; t++) acc[t] = 0.0;
  for (int j0 = 0; j0 < nj; j0 += 2) {
    float4 wq[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
      wq[j] = j0 + j < nj ? *reinterpret_cast<const float4*>(w + 4 * lane + 4 * WAVE * (j0 + j)) : make_float4(0, 0, 0, 0);
    float xf[ROUTER_TG][2][4];
#pragma unroll
    for (int t = 0; t < ROUTER_TG; t++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int64_t i = (t0 + min(t, nt - 1)) * H + wv * q + 4 * lane + 4 * WAVE * (j0 + j);
        if (XT == ARTLITE_X_F32) {
          const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(xv) + i);
          xf[t][j][0] = v.x, xf[t][j][1] = v.y, xf[t][j][2] = v.z, xf[t][j][3] = v.w;
        } else {
          const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(xv) + i);
          xf[t][j][0] = bf16_to_f32(v.x & 0xFFFFu), xf[t][j][1] = bf16_to_f32(v.x >> 16);
          xf[t][j][2] = bf16_to_f32(v.y & 0xFFFFu), xf[t][j][3] = bf16_to_f32(v.y >> 16);
        }
      }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      if (j0 + j >= nj) break;
      const double w0 = wq[j].x, w1 = wq[j].y, w2 = wq[j].z, w3 = wq[j].w;
#pragma unroll
      for (int t = 0; t < ROUTER_TG; t++) {
        acc[t] += double(xf[t][j][0]) * w0;
        acc[t] += double(xf[t][j][1]) * w1;
        acc[t] += double(xf[t][j][2]) * w2;
        acc[t] += double(xf[t][j][3]) * w3;
      }
    }
  }
  const double v = token_sums(acc, lane);
  if ((lane & 3) == 0) part[wv][sum_token(lane)] = v;
  __syncthreads();
  if (threadIdx.x < nt) {
    const int t = threadIdx.x;
    out[(t0 + t) * out_row + e] = float(((part[0][t] + part[1][t]) + part[2][t]) + part[3][t]);
  }
}

// Router logits for prefill-sized batches on the fp64 MFMA (v_mfma_f64_16x16x4_f64; fp32 x fp32 products are exact
// in fp64, the sums in fp64, rounded once to fp32 like the other router kernels). A workgroup is a tile of 32 tokens
// times TE experts, waves of 16 x 16 (wave w: token block w & 1, expert block w / 2). K streams in stages of 64
// values through two LDS buffers (x and W rows as fp32, rows padded to 68 values so that a wave's 16 rows read
// different banks), each thread loading 16-byte pieces of x and W, two stages ahead in registers. MFMA layout: lane l holds A row l % 16 (token) and B column l % 16 (expert), both at K position l / 16 of
// the step; result element i of lane l is row 4 i + l / 16, column l % 16. The K values of a 16-value block are dealt
// as step s, lane group g -> k0 + 4 g + s, so each lane's four steps are one 16-byte LDS read of its x row and one of
// its W row; step s accumulates into acc[s] (consecutive MFMAs independent), the four summed at the end. Rows past T,
// experts past E load the last one (not stored); K past H loads zeros. KP parts of K: the workgroup's waves are KP
// sets of the above, set p taking K values [p Kp, (p + 1) Kp) of the workgroup's range through LDS buffers of its
// own (more waves a SIMD to issue MFMAs while others wait); the sets' sums are added in set order at the end.
// Split K (part set): workgroup z of the grid takes K values [z kchunk, (z + 1) kchunk) and stores its fp64 sums as
// part[(z T + t) E + e]; launch_router adds the parts in z order and rounds once. Else (kchunk >= H) the fp32 logits.
template <int XT, int TE, int KP>
__global__ __launch_bounds__(KP * 2 * TE / 16 * WAVE) void k_router_mfma(const void* __restrict__ xv,
                                                                         const float* __restrict__ W, int H, int E,
                                                                         int64_t T, float* __restrict__ out,
                                                                         int64_t out_row, int kchunk,
                                                                         double* __restrict__ part_out) {
  typedef double d4 __attribute__((ext_vector_type(4)));
  constexpr int TM = 32, KS = 64, PAD = 68, THREADS = 2 * TE / 16 * WAVE;  // (threads of one set)
  constexpr int NX = TM * 16 / THREADS, NW = TE * 16 / THREADS;  // 16-byte pieces per thread per stage
  __shared__ __attribute__((aligned(16))) float xs_all[KP][2][TM][PAD];
  __shared__ __attribute__((aligned(16))) float ws_all[KP][2][TE][PAD];
  const int part = int(threadIdx.x) / THREADS;
  float(&xs)[2][TM][PAD] = xs_all[part];
  float(&ws)[2][TE][PAD] = ws_all[part];
  const int kz = int(blockIdx.z) * kchunk, kze = min(H, kz + kchunk);
  const int Kp = (kchunk / KP + KS - 1) / KS * KS, kb = kz + part * Kp, ke = min(kze, kb + Kp);
  const int tid = threadIdx.x % THREADS, lane = tid & (WAVE - 1), wv = tid / WAVE;
  const int tb = wv & 1, eb = wv >> 1, g = lane >> 4, r = lane & 15;
  const int64_t t0 = int64_t(blockIdx.x) * TM;
  const int e0 = int(blockIdx.y) * TE;
  // the thread's loads: piece i is row (tid + i THREADS) / 16 of x (or W), values 4 lq .. + 4 of each stage
  const int lq = tid & 15;
  const void* xp[NX];
  const float* wp[NW];
#pragma unroll
  for (int i = 0; i < NX; i++) {
    const int64_t xt = min(t0 + (tid + i * THREADS) / 16, T - 1);
    xp[i] = XT == ARTLITE_X_F32 ? static_cast<const void*>(static_cast<const float*>(xv) + xt * H)
                                : static_cast<const void*>(static_cast<const uint16_t*>(xv) + xt * H);
  }
#pragma unroll
  for (int i = 0; i < NW; i++) wp[i] = W + int64_t(min(e0 + (tid + i * THREADS) / 16, E - 1)) * H;
  struct Piece {
    float4 x[NX], w[NW];
  };
  // (loads past H read the last piece again, unconditionally, so that no branch makes the compiler wait for loads in
  // flight; the store into LDS puts zeros in their place)
  auto gload = [&](int k0) -> Piece {
    const int k = min(kb + k0 + 4 * lq, H - 4);
    Piece p;
#pragma unroll
    for (int i = 0; i < NX; i++) {
      if (XT == ARTLITE_X_F32) {
        p.x[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(xp[i]) + k);
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(xp[i]) + k);
        p.x[i] = make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16), bf16_to_f32(v.y & 0xFFFFu),
                             bf16_to_f32(v.y >> 16));
      }
    }
#pragma unroll
    for (int i = 0; i < NW; i++) p.w[i] = *reinterpret_cast<const float4*>(wp[i] + k);
    return p;
  };
  // (values, not references or lvalue selects, which the compiler turns into pointer selects over scratch copies)
  auto sstore = [&](int st, Piece p) {
    const float m = kb + st * KS + 4 * lq < ke ? 1.0f : 0.0f;  // (x 1 exact; x 0 gives +-0, adding nothing)
#pragma unroll
    for (int i = 0; i < NX; i++)
      *reinterpret_cast<float4*>(&xs[st & 1][(tid + i * THREADS) / 16][4 * lq]) =
          make_float4(p.x[i].x * m, p.x[i].y * m, p.x[i].z * m, p.x[i].w * m);
#pragma unroll
    for (int i = 0; i < NW; i++)
      *reinterpret_cast<float4*>(&ws[st & 1][(tid + i * THREADS) / 16][4 * lq]) =
          make_float4(p.w[i].x * m, p.w[i].y * m, p.w[i].z * m, p.w[i].w * m);
  };
  d4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = d4{0, 0, 0, 0};
  const int S = (Kp + KS - 1) / KS;  // (the same in every set: the barriers are the workgroup's)
  // stage st: its products from buffer st & 1, then the next stage's piece (loaded two stages before) into the other
  // buffer (whose reads ended before the last barrier), then a barrier; the loop is unrolled by two so that the two
  // pieces in flight keep their registers (a copy would wait for the loads)
  auto products = [&](int st) {
    const float* xrow = &xs[st & 1][16 * tb + r][4 * g];
    const float* wrow = &ws[st & 1][16 * eb + r][4 * g];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 a = *reinterpret_cast<const float4*>(xrow + 16 * j);
      const float4 b = *reinterpret_cast<const float4*>(wrow + 16 * j);
      acc[0] = __builtin_amdgcn_mfma_f64_16x16x4f64(double(a.x), double(b.x), acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f64_16x16x4f64(double(a.y), double(b.y), acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f64_16x16x4f64(double(a.z), double(b.z), acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f64_16x16x4f64(double(a.w), double(b.w), acc[3], 0, 0, 0);
    }
  };
  Piece pa = gload(0);
  sstore(0, pa);
  Piece pb = gload(KS);
  __syncthreads();
  for (int st = 0; st < S; st += 2) {
    pa = gload((st + 2) * KS);  // (past the last stage: never stored)
    products(st);
    if (st + 1 < S) sstore(st + 1, pb);
    __syncthreads();
    if (st + 1 >= S) break;
    pb = gload((st + 3) * KS);
    products(st + 1);
    if (st + 2 < S) sstore(st + 2, pa);
    __syncthreads();
  }
  d4 c = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  if constexpr (KP > 1) {  // (the staging buffers are free: every read ended before the loop's last barrier)
    double* red = reinterpret_cast<double*>(&xs_all[0][0][0][0]);
    static_assert(sizeof(xs_all) >= size_t(KP - 1) * THREADS * 4 * sizeof(double), "the sets' sums in LDS");
    if (part > 0)
#pragma unroll
      for (int i = 0; i < 4; i++) red[((part - 1) * THREADS + tid) * 4 + i] = c[i];
    __syncthreads();
    if (part > 0) return;
#pragma unroll
    for (int q = 1; q < KP; q++)
#pragma unroll
      for (int i = 0; i < 4; i++) c[i] += red[((q - 1) * THREADS + tid) * 4 + i];
  }
  const int e = e0 + 16 * eb + r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int64_t tt = t0 + 16 * tb + 4 * i + g;
    if (tt < T && e < E) {
      if (part_out)
        part_out[(int64_t(blockIdx.z) * T + tt) * E + e] = c[i];
      else
        out[tt * out_row + e] = float(c[i]);
    }
  }
}

// the split router's parts added in part order, rounded once: a thread per logit
__global__ __launch_bounds__(256) void k_router_parts(const double* __restrict__ part, int parts, int64_t T, int E,
                                                     float* __restrict__ out, int64_t out_row) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x, n = T * E;
  if (i >= n) return;
  double c = part[i];
  for (int z = 1; z < parts; z++) c += part[int64_t(z) * n + i];
  out[(i / E) * out_row + i % E] = float(c);
}

// ---- RMSNorm of the block's input (the reference's rms_norm, tests/np_ops.py:27-32): the mean of x^2 in float64
// (the squares of fp32 values exact), x / sqrt(mean + eps) in float64 rounded once to fp32, then times w in fp32
// (this file is built without FMA contraction, so the product rounds on its own). One workgroup per token.
template <int XT>
__global__ __launch_bounds__(256) void k_rmsnorm(const void* __restrict__ xv, const float* __restrict__ w, float eps,
                                                 int H, float* __restrict__ out) {
  __shared__ double part[4];
  const int64_t t = blockIdx.x;
  auto at = [&](int i) -> float {
    return XT == ARTLITE_X_F32 ? static_cast<const float*>(xv)[t * H + i]
                               : bf16_to_f32(static_cast<const uint16_t*>(xv)[t * H + i]);
  };
  double ss = 0.0;
  for (int i = threadIdx.x; i < H; i += 256) {
    const double v = at(i);
    ss += v * v;
  }
  for (int o = 32; o; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = ss;
  __syncthreads();
  const double d = sqrt((((part[0] + part[1]) + part[2]) + part[3]) / double(H) + double(eps));
  for (int i = threadIdx.x; i < H; i += 256) out[t * H + i] = float(double(at(i)) / d) * w[i];
}

int launch_rmsnorm(const void* x, int x_dtype, const float* w, float eps, int64_t T, int H, float* out,
                   hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (x_dtype == ARTLITE_X_F32)
    k_rmsnorm<ARTLITE_X_F32><<<unsigned(T), 256, 0, s>>>(x, w, eps, H, out);
  else
    k_rmsnorm<ARTLITE_X_BF16><<<unsigned(T), 256, 0, s>>>(x, w, eps, H, out);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

namespace {

// the fp64 MFMA router's tile (TE experts) and its K parts across workgroups for T tokens: enough workgroups for the
// device (about 256; one a CU, the kernel's LDS), each part at least 128 values of K (whole stages of each wave set)
struct RouterSplit {
  int te, parts, kchunk;
};
RouterSplit router_split(int64_t T, int E, int H) {
  RouterSplit r;
  r.te = E <= 32 ? 32 : 64;
  const int64_t tiles = (T + 31) / 32 * ((E + r.te - 1) / r.te);
  int parts = int(std::min<int64_t>(TOPK_MAXPARTS, std::max<int64_t>(1, 256 / std::max<int64_t>(1, tiles))));
  parts = std::min(parts, std::max(1, H / 128));
  r.kchunk = (H + parts - 1) / parts;
  r.kchunk = (r.kchunk + 127) / 128 * 128;
  r.parts = (H + r.kchunk - 1) / r.kchunk;
  return r;
}

bool router_mfma_path(int64_t T, int E, int H, bool xq) { return !xq && T >= 64 && E >= 16 && H % 16 == 0; }

}  // namespace

size_t router_part_elems(int64_t max_T, int E, int H) {
  size_t most = 0;
  for (int64_t T = 64; T <= max_T; T++) {
    const RouterSplit r = router_split(T, E, H);
    if (r.parts > 1) most = std::max(most, size_t(r.parts) * size_t(T) * size_t(E));
    if (r.parts == 1) break;  // (fewer parts for more tokens)
  }
  return most;
}

int launch_router(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* out, int64_t out_row,
                  uint32_t* xq, double* part, size_t part_elems, hipStream_t s, int* parts_left) {
  if (parts_left) *parts_left = 0;
  if (T <= 0) return ARTLITE_OK;
  if (H % 8) return fail(ARTLITE_EINVAL, "router: H %d not a multiple of 8", H);
  if (xq && H % 256) return fail(ARTLITE_EINVAL, "router: XQ of H %d (not a multiple of 256)", H);
  const int xb = x_dtype == ARTLITE_X_F32 ? 4 : 2;
  const int tt = int(std::min<int64_t>(ROUTER_TG, std::max<int64_t>(1, ROUTER_LDS / (int64_t(H) * xb))));
  if (int64_t(H) * xb > ROUTER_LDS) return fail(ARTLITE_EINVAL, "router: H %d too wide", H);
  const size_t lds = size_t(tt) * H * xb;
  if (router_mfma_path(T, E, H, xq)) {  // (prefill-sized: the fp64 MFMA)
    // (tiles of 32 x 64, 8 waves a K part: measured faster than 32 x 32 with two workgroups per CU; 32 x 32 for at
    // most 32 experts; K split over workgroups when the tiles are fewer than the device's CUs)
    constexpr int KP = 2;
    RouterSplit r = router_split(T, E, H);
    if (r.parts > 1 && (!part || size_t(r.parts) * size_t(T) * size_t(E) > part_elems)) r = RouterSplit{r.te, 1, H};
    double* po = r.parts > 1 ? part : nullptr;
    const dim3 g(unsigned((T + 31) / 32), unsigned((E + r.te - 1) / r.te), unsigned(r.parts));
    if (r.te == 32) {
      const dim3 b(KP * 2 * 32 / 16 * WAVE);
      if (x_dtype == ARTLITE_X_F32)
        k_router_mfma<ARTLITE_X_F32, 32, KP><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, r.kchunk, po);
      else
        k_router_mfma<ARTLITE_X_BF16, 32, KP><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, r.kchunk, po);
    } else {
      const dim3 b(KP * 2 * 64 / 16 * WAVE);
      if (x_dtype == ARTLITE_X_F32)
        k_router_mfma<ARTLITE_X_F32, 64, KP><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, r.kchunk, po);
      else
        k_router_mfma<ARTLITE_X_BF16, 64, KP><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, r.kchunk, po);
    }
    ART_HIP(hipGetLastError());
    if (po && parts_left) {
      *parts_left = r.parts;
    } else if (po) {
      const int64_t n = T * E;
      k_router_parts<<<unsigned((n + 255) / 256), 256, 0, s>>>(po, r.parts, T, E, out, out_row);
      ART_HIP(hipGetLastError());
    }
    return ARTLITE_OK;
  }
  if (T <= ROUTER_TG && H % 1024 == 0) {  // (a workgroup per expert)
    const int nq = xq ? int((T * (H / 256) + 3) / 4) : 0;
    const dim3 g(unsigned(E + nq), 1), b(4 * WAVE);
    if (x_dtype == ARTLITE_X_F32)
      k_router_small<ARTLITE_X_F32><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, xq);
    else
      k_router_small<ARTLITE_X_BF16><<<g, b, 0, s>>>(x, W, H, E, T, out, out_row, xq);
    ART_HIP(hipGetLastError());
    return ARTLITE_OK;
  }
  // (small batches: 4 experts per workgroup, for more workgroups)
  const bool small = T <= 4 * ROUTER_TG;
  const int ew = small ? 4 : ROUTER_EW;
  const int nbx = (E + ew - 1) / ew;
  const int nq = xq ? int((T * (H / 256) + ew - 1) / ew) : 0;
  const dim3 grid(unsigned(nbx + nq), unsigned((T + tt - 1) / tt)), block(ew * WAVE);
#define ART_ROUTER(XT, EWN) k_router<XT, EWN><<<grid, block, lds, s>>>(x, W, H, E, T, tt, out, out_row, xq, nbx)
  if (x_dtype == ARTLITE_X_F32) {
    if (small)
      ART_ROUTER(ARTLITE_X_F32, 4);
    else
      ART_ROUTER(ARTLITE_X_F32, ROUTER_EW);
  } else {
    if (small)
      ART_ROUTER(ARTLITE_X_BF16, 4);
    else
      ART_ROUTER(ARTLITE_X_BF16, ROUTER_EW);
  }
#undef ART_ROUTER
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

// ---- small batches: the top k of every token, then the stable counting sort of the pairs, in one workgroup
// (the results of k_topk, k_count and k_scatter for a single block of pairs)

template <int R>
__global__ __launch_bounds__(DISPATCH_BLOCK) void k_route_small(const float* __restrict__ logits, int64_t n, int E,
                                                                int k, int sigmoid, int32_t* __restrict__ ids,
                                                                float* __restrict__ w32, DispatchBufs d) {
  __shared__ RouteLds<DISPATCH_BLOCK> lds;
  route_core<DISPATCH_BLOCK, R>(logits, int(n), E, k, sigmoid, d.BM, d.balanced, ids, w32, d, true, lds, RouteOut{});
}

// Router logits of small batches (T <= ROUTER_GROUPS ROUTER_TG tokens, H a multiple of 256, at least 2 values a
// wave). A workgroup per EPW experts and group of ROUTER_TG tokens (workgroup b: experts EPW (b % (E / EPW)) .., tokens
// ROUTER_TG (b / (E / EPW)) ..): each expert's NW / EPW waves each take a slice of H / (NW / EPW) values of K (lane:
// values 2 lane + 128 j of the wave's slice), x read straight from memory (L2), float64 products; a wave's 16 token
// sums by halving exchanges, then the expert's slices' sums added in slice order, rounded once to fp32. Workgroups past them quantise x into XQ, a wave per unit. (Whatever reads the logits
// runs in a later launch: the launch boundary publishes them.)
template <int XT, int EPW>
__global__ __launch_bounds__(DISPATCH_BLOCK) void k_router_few(const void* __restrict__ xv,
                                                                 const float* __restrict__ W, int H, int E, int64_t T,
                                                                 float* __restrict__ logits,
                                                                 uint32_t* __restrict__ xq) {
  constexpr int NW = DISPATCH_BLOCK / WAVE, WE = NW / EPW;  // (waves a workgroup, waves an expert)
  __shared__ double part[NW][ROUTER_TG];
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  const int G = int((T + ROUTER_TG - 1) / ROUTER_TG), EB = E / EPW;  // (token groups, expert blocks)
  if (int(blockIdx.x) >= EB * G) {  // XQ of x
    const int64_t w = int64_t(blockIdx.x - EB * G) * NW + wv;
    if (w < T * (H / 256)) xq_quant_unit<XT>(xv, w, H, xq, lane);
    return;
  }
  const int eb = int(blockIdx.x) % EB, gi = int(blockIdx.x) / EB, t0 = gi * ROUTER_TG, nt = min(ROUTER_TG, int(T) - t0);
  const int e = eb * EPW + wv / WE, ew = wv % WE;  // (this wave's expert, its slice of H)
  const int q = H / WE;
  const float* wr = W + int64_t(e) * H + ew * q;
  double acc[ROUTER_TG];
#pragma unroll
  for (int t = 0; t < ROUTER_TG; t++) acc[t] = 0.0;
  // (EPW steps of 128 values at a time: every load of them issued before any is used, one memory round trip, not
  // one per token or per step)
  const int J = (q + 2 * WAVE - 1) / (2 * WAVE);
  for (int j0 = 0; j0 < J; j0 += EPW) {
    float2 wl[EPW], xl[EPW][ROUTER_TG];
#pragma unroll
    for (int u = 0; u < EPW; u++) {
      const int i = min(2 * (lane + WAVE * (j0 + u)), q - 2);  // (lanes past the slice load its last pair, unused)
      wl[u] = *reinterpret_cast<const float2*>(wr + i);
#pragma unroll
      for (int t = 0; t < ROUTER_TG; t++) {
        const int64_t o = int64_t(t0 + min(t, nt - 1)) * H + ew * q + i;
        if (XT == ARTLITE_X_F32) {
          xl[u][t] = *reinterpret_cast<const float2*>(static_cast<const float*>(xv) + o);
        } else {
          const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(xv) + o);
          xl[u][t] = make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xFFFF0000u));
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < EPW; u++) {
      float xf[ROUTER_TG][2];
#pragma unroll
      for (int t = 0; t < ROUTER_TG; t++) xf[t][0] = xl[u][t].x, xf[t][1] = xl[u][t].y;
      const double w0 = wl[u].x, w1 = wl[u].y;
      if (j0 + u < J && 2 * (lane + WAVE * (j0 + u)) < q) {
#pragma unroll
        for (int t = 0; t < ROUTER_TG; t++) {
          acc[t] += double(xf[t][0]) * w0;
          acc[t] += double(xf[t][1]) * w1;
        }
      }
    }
  }
  const double v = token_sums(acc, lane);
  if ((lane & 3) == 0) part[wv][sum_token(lane)] = v;
  lds_barrier();
  if (ew == 0 && lane < nt) {  // (the expert's first wave: its slices' sums in slice order)
    double sum = part[wv][lane];
#pragma unroll
    for (int w = 1; w < WE; w++) sum += part[wv + w][lane];
    logits[int64_t(t0 + lane) * E + e] = float(sum);
  }
}

int launch_route_small(const float* logits, int64_t n, int E, int k, int sigmoid, int32_t* ids, float* w32,
                       const DispatchBufs& d, hipStream_t s) {
  if (n <= 0) return ARTLITE_OK;
  if (n * k > DISPATCH_BLOCK || E > MAX_EXPERTS)
    return fail(ARTLITE_EINVAL, "route_small: %lld pairs of %d experts", (long long)(n * k), E);
#define ART_RS(RR) k_route_small<RR><<<1, DISPATCH_BLOCK, 0, s>>>(logits, n, E, k, sigmoid, ids, w32, d)
  if (E <= 64)
    ART_RS(1);
  else if (E <= 128)
    ART_RS(2);
  else if (E <= 256)
    ART_RS(4);
  else if (E <= 512)
    ART_RS(8);
  else
    ART_RS(16);
#undef ART_RS
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

bool router_few_fits(int64_t T, int H, int E) {
  return T >= 1 && T <= ROUTER_GROUPS * ROUTER_TG && H % 256 == 0 && H / (DISPATCH_BLOCK / WAVE) >= 2 &&
         E <= MAX_EXPERTS;
}

int launch_router_few(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* logits,
                        uint32_t* xq, hipStream_t s) {
  if (!router_few_fits(T, H, E))
    return fail(ARTLITE_EINVAL, "router_few: %lld tokens, H %d, %d experts", (long long)T, H, E);
  constexpr int NW = DISPATCH_BLOCK / WAVE;
  const int nq = xq ? int((T * (H / 256) + NW - 1) / NW) : 0;
  // (past two token groups, two experts a workgroup: fewer, longer workgroups, which the device holds in one round)
  const int epw = T > 2 * ROUTER_TG && E % 2 == 0 ? 2 : 1;
  const dim3 g(unsigned(E / epw * ((T + ROUTER_TG - 1) / ROUTER_TG) + nq)), b(DISPATCH_BLOCK);
  if (epw == 2) {
    if (x_dtype == ARTLITE_X_F32)
      k_router_few<ARTLITE_X_F32, 2><<<g, b, 0, s>>>(x, W, H, E, T, logits, xq);
    else
      k_router_few<ARTLITE_X_BF16, 2><<<g, b, 0, s>>>(x, W, H, E, T, logits, xq);
  } else {
    if (x_dtype == ARTLITE_X_F32)
      k_router_few<ARTLITE_X_F32, 1><<<g, b, 0, s>>>(x, W, H, E, T, logits, xq);
    else
      k_router_few<ARTLITE_X_BF16, 1><<<g, b, 0, s>>>(x, W, H, E, T, logits, xq);
  }
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int check_route_args(int64_t n, int per_col, int E, int k) {
  if (k < 1 || k > E || per_col < 1 || E % per_col)
    return fail(ARTLITE_EINVAL, "moe_route: k %d of E %d (%d per column)", k, E, per_col);
  if (n < 0) return fail(ARTLITE_EINVAL, "moe_route: %lld tokens", (long long)n);
  if (E > MAX_EXPERTS || k > MAX_TOPK)
    return fail(ARTLITE_EINVAL, "moe_route: E %d / k %d beyond this build's %d / %d", E, k, MAX_EXPERTS, MAX_TOPK);
  return ARTLITE_OK;
}

}  // namespace artlite

using namespace artlite;

extern "C" int artlite_moe_route(const float* logits, size_t logits_len, int64_t n, int64_t row, int per_col,
                                 int64_t pitch, int E, int k, int sigmoid, int32_t* ids, float* weights) {
  ART_TRY(check_route_args(n, per_col, E, k));
  if (n == 0) return ARTLITE_OK;
  if (!logits || !ids || !weights) return fail(ARTLITE_EINVAL, "moe_route: null array");
  if (row < 0 || pitch < 0) return fail(ARTLITE_EINVAL, "moe_route: negative row / pitch");
  const int64_t need = (n - 1) * row + int64_t(E / per_col - 1) * pitch + per_col;
  if (int64_t(logits_len) < need) return fail(ARTLITE_EINVAL, "moe_route: arrays too small");
  HostCtx* c;
  ART_TRY(host_ctx(&c));
  ART_TRY(c->in.reserve(size_t(need) * 4));
  ART_TRY(c->out.reserve(size_t(n) * k * 4));
  ART_TRY(c->out2.reserve(size_t(n) * k * 4));
  ART_HIP(hipMemcpyAsync(c->in.p, logits, size_t(need) * 4, hipMemcpyHostToDevice, c->stream));
  ART_TRY(launch_topk(c->in.as<float>(), n, row, per_col, pitch, E, k, sigmoid, c->out.as<int32_t>(),
                      c->out2.as<float>(), nullptr, c->stream));
  ART_HIP(hipMemcpyAsync(ids, c->out.p, size_t(n) * k * 4, hipMemcpyDeviceToHost, c->stream));
  ART_HIP(hipMemcpyAsync(weights, c->out2.p, size_t(n) * k * 4, hipMemcpyDeviceToHost, c->stream));
  ART_HIP(hipStreamSynchronize(c->stream));
  return ARTLITE_OK;
}

extern "C" int artlite_moe_top_k(const float* logits, int64_t n, int E, int k, int sigmoid, int32_t* ids,
                                 double* weights) {
  ART_TRY(check_route_args(n, E, E, k));
  if (n == 0) return ARTLITE_OK;
  if (!logits || !ids || !weights) return fail(ARTLITE_EINVAL, "top_k: null array");
  HostCtx* c;
  ART_TRY(host_ctx(&c));
  ART_TRY(c->in.reserve(size_t(n) * E * 4));
  ART_TRY(c->out.reserve(size_t(n) * k * 4));
  ART_TRY(c->out2.reserve(size_t(n) * k * 8));
  ART_HIP(hipMemcpyAsync(c->in.p, logits, size_t(n) * E * 4, hipMemcpyHostToDevice, c->stream));
  ART_TRY(launch_topk(c->in.as<float>(), n, E, E, 0, E, k, sigmoid, c->out.as<int32_t>(), nullptr,
                      c->out2.as<double>(), c->stream));
  ART_HIP(hipMemcpyAsync(ids, c->out.p, size_t(n) * k * 4, hipMemcpyDeviceToHost, c->stream));
  ART_HIP(hipMemcpyAsync(weights, c->out2.p, size_t(n) * k * 8, hipMemcpyDeviceToHost, c->stream));
  ART_HIP(hipStreamSynchronize(c->stream));
  return ARTLITE_OK;
}
