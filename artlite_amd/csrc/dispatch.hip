// Dispatch: the stable counting sort of the (token, slot) pairs p = t k + i by expert, deterministic on the GPU
// (reference csrc/artlite/moe_host.cpp:201-215: histogram, exclusive prefix, scatter in p order), and the chunk plan
// dealt to the columns (moe_host.cpp:216-234); the C entry point artlite_moe_plan.
//
// Two launches over blocks of DISPATCH_BLOCK consecutive pairs:
//  1. k_count: per-block histograms (LDS atomics: counts are order-free) into table[b][e]; the last block to finish
//     (a device-scope ticket) sums them into counts, scans them into offsets and per-(block, expert) bases (the
//     table staged through LDS in tiles of whole rows), and writes the tile list of the expert GEMMs and the plan's
//     chunk prefix. When the whole table fits in LDS (e.g. 32 blocks of 128 experts), k_count_one does the same in
//     one workgroup, without the ticket and its device-scope fences.
//  2. k_scatter: each pair's rank among the earlier pairs of its block with the same expert (wave ballots over the
//     id bits give the peers and the in-wave rank; a per-wave count table orders the waves) plus its block's base:
//     its position in the sorted order. Stable by construction: no atomics decide any position.
#include <mutex>

#include "route.h"

// The device memory of artlite_moe_plan_static (the entry point that allocates nothing): one array per GPU, held until
// the process ends. Kernels never name it: host code looks its per-device address up with hipGetSymbolAddress and
// passes that address, as it passes the buffers of artlite_moe_plan.
constexpr size_t PLAN_SCRATCH_BYTES = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[PLAN_SCRATCH_BYTES];

namespace artlite {

constexpr int COUNT_TILE = 8192;  // table cells staged in LDS at a time

// one pair's id into a histogram (LDS); a bad id is flagged instead (the first in pair order kept)
__device__ __forceinline__ void count_pair(const DispatchBufs& d, int64_t p, int id, int* hist) {
  if (id < 0 || id >= d.E) {
    atomicOr(&d.ctrl[CTRL_BAD], 1);
    atomicMax(&d.ctrl[CTRL_BAD_FIRST], int(d.P - p));
  } else {
    atomicAdd(&hist[id], 1);
  }
}

// The end of a count, in one block of DISPATCH_BLOCK threads, for expert e = thread: c its count, `start` and
// `total` the scan's; writes counts, offsets, the expert GEMMs' tile list and the plan's chunk prefix.
__device__ void count_tail(const DispatchBufs& d, int c, int start, int total) {
  const int e = threadIdx.x;
  if (e < d.E) {
    d.counts[e] = c;
    d.offsets[e] = start;
  }
  if (e == 0) d.offsets[d.E] = total;
  if (d.BM > 0) {  // the expert GEMMs' tiles: experts ascending, BM sorted rows each (balanced: balanced_rows)
    const int rows = d.balanced ? balanced_rows(c, d.BM) : d.BM;
    const int nt = e < d.E ? (c + rows - 1) / rows : 0;
    int nt_total;
    const int t0 = block_scan(nt, &nt_total);
    for (int m = 0; m < nt; m++) {
      d.tiles[2 * (t0 + m)] = e;
      d.tiles[2 * (t0 + m) + 1] = start + m * rows;
    }
    if (e == 0) d.ctrl[CTRL_TILES] = nt_total;
  }
  if (d.chunk > 0) {  // the plan's chunks per expert
    const int nc = e < d.E ? (c + d.chunk - 1) / d.chunk : 0;
    int nc_total;
    const int c0 = block_scan(nc, &nc_total);
    if (e < d.E) d.cstart[e] = c0;
    if (e == 0) {
      d.cstart[d.E] = nc_total;
      d.ctrl[CTRL_CHUNKS] = nc_total;
    }
  }
}

// Dispatches whose table (blocks x experts) fits in LDS: one workgroup counts every block's pairs into its row of
// the table in LDS (no ticket, no device-scope fences), then scans it as k_count's last block does.
__global__ __launch_bounds__(DISPATCH_BLOCK) void k_count_one(DispatchBufs d, int nb) {
  __shared__ int hist[COUNT_TILE];
  const int tid = threadIdx.x;
  for (int i = tid; i < nb * d.E; i += DISPATCH_BLOCK) hist[i] = 0;
  __syncthreads();
  constexpr int U = 8;  // (blocks' ids loaded together)
  for (int b0 = 0; b0 < nb; b0 += U) {
    int id[U];
#pragma unroll
    for (int j = 0; j < U; j++) {
      const int64_t p = int64_t(b0 + j) * DISPATCH_BLOCK + tid;
      id[j] = b0 + j < nb && p < d.P ? d.ids[p] : 0;
    }
#pragma unroll
    for (int j = 0; j < U; j++) {
      const int64_t p = int64_t(b0 + j) * DISPATCH_BLOCK + tid;
      if (b0 + j < nb && p < d.P) count_pair(d, p, id[j], hist + (b0 + j) * d.E);
    }
  }
  __syncthreads();
  const int e = tid;
  int c = 0;
  if (e < d.E)
    for (int b = 0; b < nb; b++) c += hist[b * d.E + e];
  int total;
  const int start = block_scan(c, &total);
  if (e < d.E) {
    int run = start;
    for (int b = 0; b < nb; b++) {
      const int v = hist[b * d.E + e];
      hist[b * d.E + e] = run;
      run += v;
    }
  }
  __syncthreads();
  for (int i = tid; i < nb * d.E; i += DISPATCH_BLOCK) d.table[i] = hist[i];
  count_tail(d, c, start, total);
}

__global__ __launch_bounds__(DISPATCH_BLOCK) void k_count(DispatchBufs d) {
  __shared__ int hist[MAX_EXPERTS];
  __shared__ int tile[COUNT_TILE];
  __shared__ int last;
  const int tid = threadIdx.x;
  const int64_t nb = gridDim.x;
  for (int e = tid; e < d.E; e += DISPATCH_BLOCK) hist[e] = 0;
  __syncthreads();
  const int64_t p = int64_t(blockIdx.x) * DISPATCH_BLOCK + tid;
  if (p < d.P) count_pair(d, p, d.ids[p], hist);
  __syncthreads();
  for (int e = tid; e < d.E; e += DISPATCH_BLOCK) d.table[int64_t(blockIdx.x) * d.E + e] = hist[e];
  __threadfence();
  __syncthreads();
  if (tid == 0) last = atomicAdd(&d.ctrl[CTRL_DONE], 1) == int(nb - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();  // (acquire: the other blocks' tables)
  // counts, offsets, per-block bases (one expert per thread: E <= MAX_EXPERTS == DISPATCH_BLOCK), the table read
  // (and rewritten) in tiles of whole blocks' rows staged in LDS by all threads, coalesced
  const int e = tid;
  const int64_t rows = COUNT_TILE / d.E;
  auto stage = [&](int64_t b0, int64_t nr) {
    for (int64_t i = tid; i < nr * d.E; i += DISPATCH_BLOCK) tile[i] = __builtin_nontemporal_load(&d.table[b0 * d.E + i]);
    __syncthreads();
  };
  int c = 0;
  for (int64_t b0 = 0; b0 < nb; b0 += rows) {
    const int64_t nr = nb - b0 < rows ? nb - b0 : rows;
    stage(b0, nr);
    if (e < d.E)
      for (int64_t r = 0; r < nr; r++) c += tile[r * d.E + e];
    __syncthreads();
  }
  int total;
  const int start = block_scan(c, &total);
  int run = start;
  for (int64_t b0 = 0; b0 < nb; b0 += rows) {
    const int64_t nr = nb - b0 < rows ? nb - b0 : rows;
    stage(b0, nr);
    if (e < d.E)
      for (int64_t r = 0; r < nr; r++) {
        const int v = tile[r * d.E + e];
        tile[r * d.E + e] = run;
        run += v;
      }
    __syncthreads();
    for (int64_t i = tid; i < nr * d.E; i += DISPATCH_BLOCK) d.table[b0 * d.E + i] = tile[i];
    __syncthreads();
  }
  count_tail(d, c, start, total);
  if (e == 0) d.ctrl[CTRL_DONE] = 0;  // (ready for the next dispatch)
}

__global__ __launch_bounds__(DISPATCH_BLOCK) void k_scatter(DispatchBufs d, PlanBufs pl) {
  __shared__ uint16_t wcnt[DISPATCH_BLOCK / WAVE][MAX_EXPERTS];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid / WAVE;
  const int64_t p = int64_t(blockIdx.x) * DISPATCH_BLOCK + tid;
  const int id = p < d.P ? d.ids[p] : -1;
  for (int i = tid; i < (DISPATCH_BLOCK / WAVE) * d.E; i += DISPATCH_BLOCK) wcnt[i / d.E][i % d.E] = 0;
  __syncthreads();
  const bool valid = id >= 0 && id < d.E;
  // (the block's base of this expert and the pair's token factors, which need the id alone, loaded together now;
  // the empty asm statement keeps the compiler from moving each load to its use, one round trip after another)
  const int t = int((p < d.P ? p : d.P - 1) / d.k);  // (pairs past P: the last pair's token, unused)
  const int base = d.table[int64_t(blockIdx.x) * d.E + (valid ? id : 0)];
  float2 f0 = {0.0f, 0.0f}, f1 = f0;
  if (d.row_a) f0 = d.row_f[0][t], f1 = d.row_f[1][t];
  asm volatile("" : : "v"(base), "v"(f0.x), "v"(f0.y), "v"(f1.x), "v"(f1.y));
  // the lanes of this wave with the same expert (ballots over the id bits)
  uint64_t peers = __ballot(valid);
  for (int bit = 0; (1 << bit) < d.E; bit++) {
    const bool set = (id >> bit) & 1;
    const uint64_t b = __ballot(set);
    peers &= set ? b : ~b;
  }
  const uint64_t below = (uint64_t(1) << lane) - 1;
  int rank = __popcll(peers & below);
  if (valid && !(peers & below)) wcnt[wv][id] = uint16_t(__popcll(peers));
  __syncthreads();
  if (!valid) return;
  for (int w = 0; w < wv; w++) rank += wcnt[w][id];
  const int dest = base + rank;
  d.order[dest] = int32_t(p);
  d.slot[p] = dest;
  if (d.row_a) {  // (the prefill's per-row token and factors, gathered here rather than by a launch of their own)
    d.row_a[dest] = t;
    d.row_out[0][dest] = f0;
    d.row_out[1][dest] = f1;
  }
  if (pl.pos) {  // the plan's row of this pair
    const int o = dest - d.offsets[id];
    const int j = d.cstart[id] + o / d.chunk, i = o % d.chunk;
    const int c = j % pl.cols, kk = j / pl.cols;
    if (kk < pl.cap) {
      const int64_t g = (int64_t(c) * pl.cap + kk) * d.chunk + i;
      pl.pos[p] = g;
      pl.rows[g] = int32_t(p / d.k);
    }
  }
}

// per chunk j: its column's expert and size, the padding rows (the chunk's first token); the columns' counts
__global__ void k_plan_fill(DispatchBufs d, PlanBufs pl) {
  const int total = d.ctrl[CTRL_CHUNKS];
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j == 0 && total > int64_t(pl.cols) * pl.cap) d.ctrl[CTRL_OVER_CAP] = 1;
  if (j < pl.cols) pl.ccounts[j] = total > j ? int32_t((total - 1 - j) / pl.cols + 1) : 0;
  if (j >= total) return;
  const int c = int(j % pl.cols), kk = int(j / pl.cols);
  if (kk >= pl.cap) return;
  int lo = 0, hi = d.E;  // the expert e with cstart[e] <= j < cstart[e + 1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (d.cstart[mid] <= j)
      lo = mid;
    else
      hi = mid;
  }
  const int e = lo, q = int(j) - d.cstart[e];
  const int size = min(d.chunk, d.counts[e] - q * d.chunk);
  pl.experts[int64_t(c) * pl.cap + kk] = e;
  pl.sizes[int64_t(c) * pl.cap + kk] = size;
  const int32_t first = d.order[d.offsets[e] + q * d.chunk] / d.k;
  int32_t* r = pl.rows + (int64_t(c) * pl.cap + kk) * d.chunk;
  for (int i = size; i < d.chunk; i++) r[i] = first;
}

int launch_dispatch_count(const DispatchBufs& d, int64_t nb, hipStream_t s) {
  if (d.E < 1 || d.E > MAX_EXPERTS) return fail(ARTLITE_EINVAL, "dispatch: E %d outside [1, %d]", d.E, MAX_EXPERTS);
  if (nb * d.E <= COUNT_TILE)
    k_count_one<<<1, DISPATCH_BLOCK, 0, s>>>(d, int(nb));
  else
    k_count<<<unsigned(nb), DISPATCH_BLOCK, 0, s>>>(d);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int launch_dispatch_scatter(const DispatchBufs& d, int64_t nb, hipStream_t s) {
  k_scatter<<<unsigned(nb), DISPATCH_BLOCK, 0, s>>>(d, PlanBufs{0, 0, nullptr, nullptr, nullptr, nullptr, nullptr});
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

int launch_dispatch(const DispatchBufs& d, hipStream_t s) {
  const int64_t nb = dispatch_blocks(d.P);
  ART_TRY(launch_dispatch_count(d, nb, s));
  return launch_dispatch_scatter(d, nb, s);
}

int launch_plan(const DispatchBufs& d, const PlanBufs& pl, hipStream_t s) {
  if (d.E < 1 || d.E > MAX_EXPERTS) return fail(ARTLITE_EINVAL, "dispatch: E %d outside [1, %d]", d.E, MAX_EXPERTS);
  const int64_t nb = dispatch_blocks(d.P);
  ART_TRY(launch_dispatch_count(d, nb, s));
  k_scatter<<<unsigned(nb), DISPATCH_BLOCK, 0, s>>>(d, pl);
  ART_HIP(hipGetLastError());
  const int64_t bound = d.E + (d.P + d.chunk - 1) / d.chunk;
  const int64_t threads = bound > pl.cols ? bound : pl.cols;
  k_plan_fill<<<unsigned((threads + 255) / 256), 256, 0, s>>>(d, pl);
  ART_HIP(hipGetLastError());
  return ARTLITE_OK;
}

namespace {

// The device memory of one host-pointer plan call: the staged ids, the per-block histogram table, counts / offsets /
// chunk prefix, order / slot, pos, the plan's rows / experts / sizes / column counts, the control words.
struct PlanMem {
  int32_t *ids, *table, *o2, *o3, *o5, *ctrl;
  int64_t* pos;
};

// bytes of each PlanMem region, in order (each followed by a 256-byte tail the vector loads may touch)
void plan_sizes(int64_t P, int E, int cols, int cap, int chunk, size_t (&b)[7]) {
  const size_t slots = size_t(cols) * cap;
  b[0] = size_t(P) * 4;
  b[1] = size_t(dispatch_blocks(P)) * E * 4;
  b[2] = size_t(3 * E + 3) * 4;
  b[3] = size_t(2 * P) * 4;
  b[4] = size_t(P) * 8;
  b[5] = (slots * chunk + 2 * slots + cols) * 4;
  b[6] = CTRL_WORDS * 4;
}

__global__ void k_zero_words(int32_t* p, int n) {
  if (int(threadIdx.x) < n) p[threadIdx.x] = 0;
}
static_assert(CTRL_WORDS <= 64, "k_zero_words: one 64-thread block");

int check_plan_args(const char* who, const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk,
                    const int32_t* experts, const int32_t* counts, const int32_t* sizes, const int32_t* rows,
                    const int64_t* pos) {
  if (n < 0 || k < 1 || E < 1 || cols < 1 || cap < 0 || chunk < 1)
    return fail(ARTLITE_EINVAL, "%s: n %lld, k %d, E %d, cols %d, cap %d, chunk %d", who, (long long)n, k, E, cols,
                cap, chunk);
  if (E > MAX_EXPERTS) return fail(ARTLITE_EINVAL, "%s: E %d beyond this build's %d", who, E, MAX_EXPERTS);
  if (!counts || (n && (!ids || !pos)) || (cap && (!experts || !sizes || !rows)))
    return fail(ARTLITE_EINVAL, "%s: null array", who);
  return ARTLITE_OK;
}

// The plan of n x k ids on stream s in the device memory m, the results copied to the caller's host arrays.
int plan_run(const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk, int32_t* experts,
             int32_t* counts, int32_t* sizes, int32_t* rows, int64_t* pos, const PlanMem& m, hipStream_t s) {
  const int64_t P = n * k;
  const size_t slots = size_t(cols) * cap;
  if (P) ART_HIP(hipMemcpyAsync(m.ids, ids, size_t(P) * 4, hipMemcpyHostToDevice, s));
  k_zero_words<<<1, 64, 0, s>>>(m.ctrl, CTRL_WORDS);  // (a fill kernel: no memset node if a caller captures)
  ART_HIP(hipGetLastError());
  DispatchBufs d{m.ids, P, E, k, m.table, m.ctrl, m.o2, m.o2 + E, m.o3, m.o3 + P, nullptr, 0, m.o2 + 2 * E + 1, chunk};
  PlanBufs pl{cols, cap, m.o5 + slots * chunk, m.o5 + slots * chunk + 2 * slots, m.o5 + slots * chunk + slots, m.o5,
              m.pos};
  ART_TRY(launch_plan(d, pl, s));
  int32_t ctrl[CTRL_WORDS];
  ART_HIP(hipMemcpyAsync(ctrl, m.ctrl, sizeof ctrl, hipMemcpyDeviceToHost, s));
  ART_HIP(hipStreamSynchronize(s));
  if (ctrl[CTRL_BAD]) return fail(ARTLITE_EINVAL, "moe_plan: expert id %d of %d", ids[P - ctrl[CTRL_BAD_FIRST]], E);
  if (ctrl[CTRL_OVER_CAP]) return fail(ARTLITE_EINVAL, "moe_plan: more than %d chunks in a column", cap);
  const int total = ctrl[CTRL_CHUNKS];
  ART_HIP(hipMemcpyAsync(counts, pl.ccounts, size_t(cols) * 4, hipMemcpyDeviceToHost, s));
  // (only the dealt slots are written: the reference's arrays keep their other entries)
  for (int col = 0; col < cols; col++) {
    const int mc = total > col ? (total - 1 - col) / cols + 1 : 0;
    if (!mc) continue;
    ART_HIP(hipMemcpyAsync(experts + size_t(col) * cap, pl.experts + size_t(col) * cap, size_t(mc) * 4,
                           hipMemcpyDeviceToHost, s));
    ART_HIP(hipMemcpyAsync(sizes + size_t(col) * cap, pl.sizes + size_t(col) * cap, size_t(mc) * 4,
                           hipMemcpyDeviceToHost, s));
    ART_HIP(hipMemcpyAsync(rows + size_t(col) * cap * chunk, pl.rows + size_t(col) * cap * chunk,
                           size_t(mc) * chunk * 4, hipMemcpyDeviceToHost, s));
  }
  if (P) ART_HIP(hipMemcpyAsync(pos, pl.pos, size_t(P) * 8, hipMemcpyDeviceToHost, s));
  ART_HIP(hipStreamSynchronize(s));
  return ARTLITE_OK;
}

// ---- the no-allocation variant's device memory: one static array per GPU, its address looked up once per device
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES] = {};

// the current device's copy of scratch (hipGetSymbolAddress on its first use on each device, that device current);
// host code uses this address, never the array's name
int scratch_of_device(uint8_t** out) {
  int dev = 0;
  ART_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(ARTLITE_EINVAL, "moe_plan_static: device %d beyond %d", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(ARTLITE_EHIP, "moe_plan_static: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = static_cast<uint8_t*>(g_scratch[dev]);
  return ARTLITE_OK;
}

}  // namespace

}  // namespace artlite

using namespace artlite;

extern "C" int artlite_moe_plan(const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk,
                                int32_t* experts, int32_t* counts, int32_t* sizes, int32_t* rows, int64_t* pos) {
  ART_TRY(check_plan_args("moe_plan", ids, n, k, E, cols, cap, chunk, experts, counts, sizes, rows, pos));
  HostCtx* c;
  ART_TRY(host_ctx(&c));
  size_t b[7];
  plan_sizes(n * k, E, cols, cap, chunk, b);
  // in: ids | out: table | out2: counts, offsets, cstart | out3: order, slot | out4: pos | out5: rows, experts, sizes,
  // column counts | flag: ctrl
  ART_TRY(c->in.reserve(b[0]));
  ART_TRY(c->out.reserve(b[1]));
  ART_TRY(c->out2.reserve(b[2]));
  ART_TRY(c->out3.reserve(b[3]));
  ART_TRY(c->out4.reserve(b[4]));
  ART_TRY(c->out5.reserve(b[5]));
  ART_TRY(c->flag.reserve(b[6]));
  const PlanMem m{c->in.as<int32_t>(), c->out.as<int32_t>(), c->out2.as<int32_t>(), c->out3.as<int32_t>(),
                  c->out5.as<int32_t>(), c->flag.as<int32_t>(), c->out4.as<int64_t>()};
  return plan_run(ids, n, k, E, cols, cap, chunk, experts, counts, sizes, rows, pos, m, c->stream);
}

extern "C" int artlite_moe_plan_static(const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk,
                                       int32_t* experts, int32_t* counts, int32_t* sizes, int32_t* rows,
                                       int64_t* pos) {
  ART_TRY(check_plan_args("moe_plan_static", ids, n, k, E, cols, cap, chunk, experts, counts, sizes, rows, pos));
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return fail(ARTLITE_EHIP, "moe_plan_static: no HIP device");
  size_t b[7], at[7], total = 0;
  plan_sizes(n * k, E, cols, cap, chunk, b);
  for (int i = 0; i < 7; i++) {
    at[i] = total;
    total += (b[i] + 255) / 256 * 256 + 256;
  }
  if (total > PLAN_SCRATCH_BYTES)
    return fail(ARTLITE_EINVAL,
                "moe_plan_static: n %lld x k %d, E %d, %d x %d chunks of %d need %zu bytes of device scratch, beyond "
                "its %zu (use artlite_moe_plan)",
                (long long)n, k, E, cols, cap, chunk, total, PLAN_SCRATCH_BYTES);
  uint8_t* base = nullptr;
  ART_TRY(scratch_of_device(&base));
  const PlanMem m{reinterpret_cast<int32_t*>(base + at[0]), reinterpret_cast<int32_t*>(base + at[1]),
                  reinterpret_cast<int32_t*>(base + at[2]), reinterpret_cast<int32_t*>(base + at[3]),
                  reinterpret_cast<int32_t*>(base + at[5]), reinterpret_cast<int32_t*>(base + at[6]),
                  reinterpret_cast<int64_t*>(base + at[4])};
  // the null stream: nothing is created (a stream's creation may allocate)
  return plan_run(ids, n, k, E, cols, cap, chunk, experts, counts, sizes, rows, pos, m, nullptr);
}
