// The experts' products over raw GGUF blocks on gfx950's bf16 MFMA (v_mfma_f32_16x16x32_bf16), and the combine.
//
// Exactness of the operands: a block's integer codes are exact in bf16 -- Q4_0 as 128 + q and Q4_K as 128 + q
// (a byte 0x43 above the nibble: bf16 128 + q), Q8_0 as 128 + q through an unsigned byte conversion -- and bf16
// activations are exact; fp32 activations and the SwiGLU intermediate are split into bf16 hi + lo planes. One MFMA
// per 32-value group gives S = sum (128 + q) x exactly rounded once into fp32, its C input pre-loaded with
// -offset sum x (sum x from an MFMA against a ones operand, so the offset leaves S exactly sum (q - 8) x, or
// sum q x). The group's fp16 scale is applied in fp32: acc += d S (Q4_K: acc += (d sc) S - (dmin mn) sum x).
//
// Decode tiling (k_gemm_decode): a workgroup is one tile of DECODE_BM sorted rows of one expert (tokens for gate /
// up, pairs for down) times 4 waves x ROWS weight rows. Each wave streams its own rows' blocks, a stage of one
// ~144-byte run per row at a time: dwordx4 loads of the 16-byte-aligned cover of the run into registers (the next
// stage's loads in flight while the current stage computes), then into the wave's LDS slot, from which each lane
// decodes its row's 8 codes of a group. MFMA layout (16x16x32): lane l holds A row l % 16 and B column l % 16,
// both with K values 8 (l / 16) .. + 8; C column l % 16, rows 4 (l / 16) .. + 4. A = activations (tokens / pairs),
// B = weights (the lane's own row), so a lane's four outputs share its row's scale.
#include "experts.h"

namespace artlite {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}

__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) {
  uint16_t v;
  __builtin_memcpy(&v, p, 2);
  return v;
}

__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }

// eight nibbles (the bytes of v0, v1, each < 16) -> the B operand's four dwords of bf16 128 + q
__device__ __forceinline__ u32x4 nib8(uint32_t v0, uint32_t v1) {
  return u32x4{__builtin_amdgcn_perm(0x43434343u, v0, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v0, 0x04030402u),
               __builtin_amdgcn_perm(0x43434343u, v1, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v1, 0x04030402u)};
}

// two bf16 of the unsigned bytes 2 j, 2 j + 1 of v (exact: < 256)
__device__ __forceinline__ uint32_t byte2(uint32_t v, int j) {
  const uint32_t f0 = __float_as_uint(float((v >> (16 * j)) & 0xFFu));
  const uint32_t f1 = __float_as_uint(float((v >> (16 * j + 8)) & 0xFFu));
  return __builtin_amdgcn_perm(f1, f0, 0x07060302u);
}

// eight unsigned bytes -> the B operand's four dwords of bf16
__device__ __forceinline__ u32x4 byte8(uint32_t v0, uint32_t v1) {
  return u32x4{byte2(v0, 0), byte2(v0, 1), byte2(v1, 0), byte2(v1, 1)};
}

template <int QT>
struct Fmt;
template <>
struct Fmt<ARTLITE_Q4_0> {
  static constexpr int GROUPS = 8;         // 32-value groups per stage
  static constexpr int STAGE_BYTES = 144;  // a stage's bytes of a row
  static constexpr float OFF = 136.0f;     // (128 + q) - (q - 8)
};
template <>
struct Fmt<ARTLITE_Q8_0> {
  static constexpr int GROUPS = 4;
  static constexpr int STAGE_BYTES = 136;
  static constexpr float OFF = 128.0f;
};
template <>
struct Fmt<ARTLITE_Q4_K> {
  static constexpr int GROUPS = 8;  // (one super-block)
  static constexpr int STAGE_BYTES = 144;
  static constexpr float OFF = 128.0f;
};

constexpr int CPR = 10;                 // 16-byte chunks per row and stage (the cover of <= 144 bytes at any offset)
constexpr int SLOT = CPR * 16 + 16;     // a row's LDS bytes (padded: rows' groups fall in different banks)
constexpr uint32_t ONES = 0x3F803F80u;  // bf16 1.0 pair

// a stage's weight chunks (the 16-byte-aligned cover of each row's run) and A groups into registers
template <class F, int LOADS, int AP>
__device__ __forceinline__ void load_stage(int s, u32x4 (&wreg)[LOADS], u32x4 (&areg)[F::GROUPS][AP],
                                           const int64_t (&roff)[LOADS], uint32_t second, const uint8_t* w0,
                                           const uint8_t* w1, int lane, int lg, const uint16_t* ah,
                                           const uint16_t* al, bool arow_ok, int ng) {
  const int64_t off = int64_t(s) * F::STAGE_BYTES;
#pragma unroll
  for (int i = 0; i < LOADS; i++) {
    const int64_t o = ((roff[i] + off) & ~int64_t(15)) + 16 * ((lane + WAVE * i) % CPR);
    wreg[i] = *reinterpret_cast<const u32x4*>(((second >> i) & 1 ? w1 : w0) + o);
  }
  const int g0 = s * F::GROUPS;
#pragma unroll
  for (int g = 0; g < F::GROUPS; g++) {
    const int k = min(g0 + g, ng - 1) * 32 + 8 * lg;
    const bool ok = arow_ok && g0 + g < ng;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ah + k);
    areg[g][0] = ok ? v : u32x4{0, 0, 0, 0};
    if (AP == 2) {
      const u32x4 u = *reinterpret_cast<const u32x4*>(al + k);
      areg[g][AP - 1] = ok ? u : u32x4{0, 0, 0, 0};
    }
  }
}

template <int LOADS>
__device__ __forceinline__ void store_stage(const u32x4 (&wreg)[LOADS], uint8_t* my, int lane) {
#pragma unroll
  for (int i = 0; i < LOADS; i++) {
    const int q = lane + WAVE * i;
    *reinterpret_cast<u32x4*>(my + (q / CPR) * SLOT + 16 * (q % CPR)) = wreg[i];
  }
}

template <int QT, int NMAT, int CB, int AP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_gemm_decode(const GemmArgs a) {
  using F = Fmt<QT>;
  constexpr int RW = 16 * CB;      // rows per matrix per wave
  constexpr int ROWS = NMAT * RW;  // rows per wave
  constexpr int LOADS = ROWS * CPR / WAVE;
  static_assert(ROWS * CPR % WAVE == 0, "loads per lane");
  __shared__ __attribute__((aligned(16))) uint8_t lds[4][ROWS * SLOT];

  const int lane = threadIdx.x & (WAVE - 1), wv = threadIdx.x / WAVE, lg = lane >> 4, lr = lane & 15;
  // the tile
  int e = 0, s0, m_valid;
  if (a.tiles) {
    if (int64_t(blockIdx.x) >= *a.n_tiles) return;
    e = a.tiles[2 * blockIdx.x];
    s0 = a.tiles[2 * blockIdx.x + 1];
    m_valid = min(DECODE_BM, a.offsets[e + 1] - s0);
  } else {
    s0 = blockIdx.x * DECODE_BM;
    m_valid = min(DECODE_BM, a.dense_rows - s0);
  }
  const int n0 = (blockIdx.y * 4 + wv) * RW;  // the wave's first row of each matrix
  uint8_t* my = lds[wv];

  // A row of this lane (row lr of the tile; lanes past the tile read row s0 and are zeroed)
  const bool arow_ok = lr < m_valid;
  const int64_t arow = a.a_gather ? a.order[s0 + (arow_ok ? lr : 0)] / a.topk : s0 + (arow_ok ? lr : 0);
  const uint16_t* ah = a.a_hi + arow * a.K;
  const uint16_t* al = a.a_lo + (AP == 2 ? arow * a.K : 0);

  // the loader's chunks: chunk q = lane + 64 i -> (row q / CPR, chunk q % CPR); rows past N read row N - 1
  int64_t roff[LOADS];
  uint32_t second = 0;  // bit i: chunk i is of the second matrix
#pragma unroll
  for (int i = 0; i < LOADS; i++) {
    const int q = lane + WAVE * i, r = q / CPR;
    const int m = r / RW, rr = min(n0 + r % RW, a.N - 1);
    second |= uint32_t(m) << i;
    roff[i] = e * a.expert_bytes + int64_t(rr) * a.row_bytes;
  }
  const uint8_t* w0 = a.w[0];
  const uint8_t* w1 = a.w[NMAT - 1];
  // the lane's rows' address low bits (matrix m, column block c)
  int mis0[CB];
#pragma unroll
  for (int c = 0; c < CB; c++) mis0[c] = int((e * a.expert_bytes + int64_t(n0 + 16 * c + lr) * a.row_bytes) & 15);

  const int ng = a.K / 32;  // groups per row
  const int ns = (ng + F::GROUPS - 1) / F::GROUPS;

  u32x4 wreg[LOADS];
  u32x4 acur[F::GROUPS][AP], anext[F::GROUPS][AP];
  load_stage<F, LOADS, AP>(0, wreg, acur, roff, second, w0, w1, lane, lg, ah, al, arow_ok, ng);
  store_stage<LOADS>(wreg, my, lane);

  f32x4 acc[NMAT][CB];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
#pragma unroll
    for (int c = 0; c < CB; c++) acc[m][c] = f32x4{0, 0, 0, 0};

  for (int s = 0; s < ns; s++) {
    if (s + 1 < ns) load_stage<F, LOADS, AP>(s + 1, wreg, anext, roff, second, w0, w1, lane, lg, ah, al, arow_ok, ng);
    __builtin_amdgcn_wave_barrier();
    const int gn = min(F::GROUPS, ng - s * F::GROUPS);
    const int64_t off = int64_t(s) * F::STAGE_BYTES;
#pragma unroll
    for (int g = 0; g < F::GROUPS; g++) {
      if (g < gn) {
        // sum x of the lane's four outputs' tokens: the C input of the group's products
        f32x4 sx = mfma(acur[g][0], u32x4{ONES, ONES, ONES, ONES}, f32x4{0, 0, 0, 0});
        if (AP == 2) sx = mfma(acur[g][AP - 1], u32x4{ONES, ONES, ONES, ONES}, sx);
        const f32x4 cin = sx * (-F::OFF);
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
          for (int c = 0; c < CB; c++) {
            const uint8_t* row = my + (m * RW + 16 * c + lr) * SLOT + ((mis0[c] + off) & 15);
            u32x4 b;
            float sc;
            float mn = 0.0f;
            if (QT == ARTLITE_Q4_0) {
              const uint8_t* blk = row + 18 * g;
              sc = h2f(lds_u16(blk));
              const int sh = 4 * (lg >> 1);
              const uint32_t u0 = (lds_u32(blk + 2 + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
              const uint32_t u1 = (lds_u32(blk + 6 + 8 * (lg & 1)) >> sh) & 0x0F0F0F0Fu;
              b = nib8(u0, u1);
            } else if (QT == ARTLITE_Q8_0) {
              const uint8_t* blk = row + 34 * g;
              sc = h2f(lds_u16(blk));
              const uint32_t u0 = lds_u32(blk + 2 + 8 * lg) ^ 0x80808080u;
              const uint32_t u1 = lds_u32(blk + 6 + 8 * lg) ^ 0x80808080u;
              b = byte8(u0, u1);
            } else {  // Q4_K: group g of the stage's super-block
              const float d = h2f(lds_u16(row)), dmin = h2f(lds_u16(row + 2));
              const uint8_t* s6 = row + 4;
              const int q6 = g < 4 ? s6[g] & 63 : (s6[8 + g - 4] & 15) | ((s6[g - 4] >> 6) << 4);
              const int m6 = g < 4 ? s6[4 + g] & 63 : (s6[8 + g - 4] >> 4) | ((s6[4 + g - 4] >> 6) << 4);
              sc = __fmul_rn(d, float(q6));
              mn = __fmul_rn(dmin, float(m6));
              const uint8_t* qs = row + 16 + 32 * (g >> 1) + 8 * lg;
              const int sh = 4 * (g & 1);
              b = nib8((lds_u32(qs) >> sh) & 0x0F0F0F0Fu, (lds_u32(qs + 4) >> sh) & 0x0F0F0F0Fu);
            }
            f32x4 p = mfma(acur[g][0], b, cin);
            if (AP == 2) p = mfma(acur[g][AP - 1], b, p);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              acc[m][c][i] = __builtin_fmaf(sc, p[i], acc[m][c][i]);
              if (QT == ARTLITE_Q4_K) acc[m][c][i] = __builtin_fmaf(-mn, sx[i], acc[m][c][i]);
            }
          }
      }
    }
    if (s + 1 < ns) {
      __builtin_amdgcn_wave_barrier();
      store_stage<LOADS>(wreg, my, lane);
#pragma unroll
      for (int g = 0; g < F::GROUPS; g++)
#pragma unroll
        for (int p = 0; p < AP; p++) acur[g][p] = anext[g][p];
    }
  }

  // epilogue: lane holds rows (tokens / pairs) 4 lg + i of output column n0 + 16 c + lr
#pragma unroll
  for (int c = 0; c < CB; c++) {
    const int n = n0 + 16 * c + lr;
    if (n >= a.N) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 4 * lg + i;
      if (m >= m_valid) continue;
      const int64_t o = int64_t(s0 + m) * a.N + n;
      if (NMAT == 2) {
        const float g = acc[0][c][i], u = acc[1][c][i];
        const float h = g / (1.0f + expf(-g)) * u;
        const uint32_t hi = f32_to_bf16(h);
        a.h_hi[o] = uint16_t(hi);
        a.h_lo[o] = uint16_t(f32_to_bf16(h - bf16_to_f32(hi)));
      } else {
        a.y[o] = acc[0][c][i];
      }
    }
  }
}

template <int QT, int NMAT, int CB>
int launch_decode(const GemmArgs& a, hipStream_t s) {
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + DECODE_BM - 1) / DECODE_BM;
  const dim3 grid(unsigned(tiles), unsigned((a.N + 4 * 16 * CB - 1) / (4 * 16 * CB))), block(256);
  if (a.a_lo)
    k_gemm_decode<QT, NMAT, CB, 2><<<grid, block, 0, s>>>(a);
  else
    k_gemm_decode<QT, NMAT, CB, 1><<<grid, block, 0, s>>>(a);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int launch_expert_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.K % 32 || (a.qtype == ARTLITE_Q4_K && a.K % 256))
    return fail(ARTLITE_EINVAL, "expert GEMM: K %d is not a multiple of the format's block", a.K);
  const int64_t tiles = a.tiles ? a.max_tiles : (a.dense_rows + DECODE_BM - 1) / DECODE_BM;
  if (tiles <= 0) return ARTLITE_OK;
  const bool swiglu = a.w[1] != nullptr;
#define ART_DISPATCH(QT) \
  return swiglu ? launch_decode<QT, 2, 2>(a, s) : launch_decode<QT, 1, 4>(a, s)
  switch (a.qtype) {
    case ARTLITE_Q4_0: ART_DISPATCH(ARTLITE_Q4_0);
    case ARTLITE_Q8_0: ART_DISPATCH(ARTLITE_Q8_0);
    case ARTLITE_Q4_K: ART_DISPATCH(ARTLITE_Q4_K);
    default: return fail(ARTLITE_EINVAL, "expert GEMM: unsupported weight type %d", a.qtype);
  }
#undef ART_DISPATCH
}

// ---- combine: y[t] = ws[t] ys[t] + sum_i w[t, i] Y[slot[t k + i]] (the reference CombineOperator's sum,
// src/artlite/moe/gather.py:12-18: the shared term first, then the slots in order, fp32)
__global__ void k_combine(const float* __restrict__ Y, const int32_t* __restrict__ slot, const float* __restrict__ w,
                          int k, const float* __restrict__ ys, const float* __restrict__ ws_logit, int ws_sigmoid,
                          int64_t T, int H, float* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  if (h4 * 4 >= H) return;
  float4 acc = make_float4(0, 0, 0, 0);
  if (ys) {
    float ws = 1.0f;
    if (ws_logit) ws = ws_sigmoid ? 1.0f / (1.0f + expf(-ws_logit[t])) : ws_logit[t];
    const float4 v = reinterpret_cast<const float4*>(ys + t * H)[h4];
    acc.x = ws * v.x, acc.y = ws * v.y, acc.z = ws * v.z, acc.w = ws * v.w;
  }
  for (int i = 0; i < k; i++) {
    const float wi = w[t * k + i];
    const float4 v = reinterpret_cast<const float4*>(Y + int64_t(slot[t * k + i]) * H)[h4];
    acc.x = __builtin_fmaf(wi, v.x, acc.x);
    acc.y = __builtin_fmaf(wi, v.y, acc.y);
    acc.z = __builtin_fmaf(wi, v.z, acc.z);
    acc.w = __builtin_fmaf(wi, v.w, acc.w);
  }
  reinterpret_cast<float4*>(y + t * H)[h4] = acc;
}

int launch_combine(const float* Y, const int32_t* slot, const float* w, int k, const float* ys, const float* ws_logit,
                   int ws_sigmoid, int64_t T, int H, float* y, hipStream_t s) {
  if (T <= 0) return ARTLITE_OK;
  if (H % 4) return fail(ARTLITE_EINVAL, "combine: H %d not a multiple of 4", H);
  const dim3 grid(unsigned((H / 4 + 255) / 256), unsigned(T)), block(256);
  k_combine<<<grid, block, 0, s>>>(Y, slot, w, k, ys, ws_logit, ws_sigmoid, T, H, y);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

__global__ void k_split(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const uint32_t h = f32_to_bf16(v);
  hi[i] = uint16_t(h);
  lo[i] = uint16_t(f32_to_bf16(v - bf16_to_f32(h)));
}

int launch_split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n <= 0) return ARTLITE_OK;
  k_split<<<unsigned((n + 255) / 256), 256, 0, s>>>(x, n, hi, lo);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

}  // namespace artlite
