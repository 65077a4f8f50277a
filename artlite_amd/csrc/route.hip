// Routing: the router's logits (x W^T with float64 accumulation) and the top k of each token's logits with their
// weights, one wave64 per token; the C entry points artlite_moe_route / artlite_moe_top_k.
//
// Ranking follows the reference's host step (csrc/artlite/moe_host.cpp:45-73): a logit's 64-bit key is its ordered
// fp32 bits (after l + 0, so -0 ranks as +0) above ~id, so larger logits win and equal logits go to the lower id.
// The weights follow moe_host.cpp:62-72: e^(l - l_max) (or sigmoid(l)) in double, their sum in numpy's pairwise
// order (moe_host.cpp:25-39), e / sum rounded to fp32.
#include "route.h"

#include <algorithm>

namespace artlite {

__device__ __forceinline__ uint64_t logit_key(float l, int e) {
  uint32_t u = __float_as_uint(l);
  if (u == 0x80000000u) u = 0;  // (-0 ranks as +0)
  const uint32_t ord = (u >> 31) ? ~u : (u | 0x80000000u);
  return (uint64_t(ord) << 32) | uint32_t(~uint32_t(e));
}

// numpy's pairwise sum of n <= 128 doubles (moe_host.cpp:25-39)
__device__ double row_sum(const double* a, int n) {
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

constexpr int TOPK_WAVES = 4;

// One wave per token: R keys per lane (expert e = lane + 64 r), k rounds of a wave maximum (the winner's key
// cleared), lane j keeping the j-th; then the weights.
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
  const float* p = logits + t * row;
  uint64_t key[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int e = lane + WAVE * r;
    key[r] = e < E ? logit_key(p[int64_t(e / per_col) * pitch + e % per_col], e) : 0;
  }
  uint64_t mine = 0;
  for (int j = 0; j < k; j++) {
    uint64_t m = 0;
#pragma unroll
    for (int r = 0; r < R; r++) m = key[r] > m ? key[r] : m;
    m = wave_max_u64(m);
#pragma unroll
    for (int r = 0; r < R; r++)
      if (key[r] == m) key[r] = 0;
    if (lane == j) mine = m;
  }
  const int id = int(~uint32_t(mine));
  const bool on = lane < k;
  const float l = on ? p[int64_t(id / per_col) * pitch + id % per_col] : 0.0f;
  const double l0 = __shfl(double(l), 0, WAVE);
  double e = 0;
  if (on) e = sigmoid ? 1.0 / (1.0 + exp(-double(l))) : exp(double(l) - l0);
  ev[wv][lane] = e;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane == 0) {
    double s = row_sum(ev[wv], k);
    if (sigmoid) s = s < 6.103515625e-5 ? 6.103515625e-5 : s;  // (std::max(s, 2^-14): a NaN sum stays NaN)
    sum[wv] = s;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const double s = sum[wv];
  if (on) {
    ids[t * k + lane] = id;
    const double w = e / s;
    if (w32) w32[t * k + lane] = float(w);
    if (w64) w64[t * k + lane] = w;
  }
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

// Router logits: a block of ROUTER_EW waves (one expert each) over a tile of up to ROUTER_TG tokens whose rows are
// staged in LDS; each lane accumulates float64 partial dot products (exact products of fp32 / bf16 values) over
// h = 4 lane + 256 j, then a fixed shuffle tree; the sum is rounded once to fp32.
template <int XT>
__global__ __launch_bounds__(ROUTER_EW * WAVE) void k_router(const void* __restrict__ xv, const float* __restrict__ W,
                                                            int H, int E, int64_t T, int tt, float* __restrict__ out,
                                                            int64_t out_row) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // tt rows of H values (x's own dtype)
  constexpr int XB = XT == ARTLITE_X_F32 ? 4 : 2;
  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE;
  const int64_t t0 = int64_t(blockIdx.y) * tt;
  const int nt = int(min(int64_t(tt), T - t0));
  {  // stage the tile's rows (16-byte pieces)
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(xv) + t0 * H * XB);
    uint4* dst = reinterpret_cast<uint4*>(xs);
    const int n16 = nt * H * XB / 16;
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
  }
  __syncthreads();
  const int e = blockIdx.x * ROUTER_EW + wv;
  if (e >= E) return;
  const float* w = W + int64_t(e) * H;
  double acc[ROUTER_TG];
#pragma unroll
  for (int t = 0; t < ROUTER_TG; t++) acc[t] = 0.0;
  for (int h = 4 * lane; h < H; h += 4 * WAVE) {
    const float4 wq = *reinterpret_cast<const float4*>(w + h);
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
        acc[t] += double(x0) * double(wq.x);
        acc[t] += double(x1) * double(wq.y);
        acc[t] += double(x2) * double(wq.z);
        acc[t] += double(x3) * double(wq.w);
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

int launch_router(const void* x, int x_dtype, const float* W, int H, int E, int64_t T, float* out, int64_t out_row,
                  hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (H % 8) return fail(ARTLITE_EINVAL, "router: H %d not a multiple of 8", H);
  const int xb = x_dtype == ARTLITE_X_F32 ? 4 : 2;
  const int tt = int(std::min<int64_t>(ROUTER_TG, std::max<int64_t>(1, ROUTER_LDS / (int64_t(H) * xb))));
  if (int64_t(H) * xb > ROUTER_LDS) return fail(ARTLITE_EINVAL, "router: H %d too wide", H);
  const dim3 grid(unsigned((E + ROUTER_EW - 1) / ROUTER_EW), unsigned((T + tt - 1) / tt)), block(ROUTER_EW * WAVE);
  const size_t lds = size_t(tt) * H * xb;
  if (x_dtype == ARTLITE_X_F32)
    k_router<ARTLITE_X_F32><<<grid, block, lds, s>>>(x, W, H, E, T, tt, out, out_row);
  else
    k_router<ARTLITE_X_BF16><<<grid, block, lds, s>>>(x, W, H, E, T, tt, out, out_row);
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
