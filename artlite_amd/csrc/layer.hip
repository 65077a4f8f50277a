// The MoE layer object: its weights in HBM as the GGUF file lays them out (no repacking), its activations, and the
// forward pass on one HIP stream: router -> top k -> dispatch -> gate / up (SwiGLU) -> down -> combine, plus the
// shared expert. The semantics are the reference's oracle (tests/moe/ref.py:43-60) with its routing
// (csrc/artlite/moe_host.cpp:45-73) and combine (src/artlite/moe/gather.py:12-18).
#include <cmath>
#include <string>
#include <vector>

#include "experts.h"
#include "gemv.h"
#include "route.h"

using namespace artlite;

struct artlite_moe_layer {
  artlite_moe_desc d{};
  int device = 0, cus = 0;  // (the device's compute units)
  hipStream_t stream = nullptr;
  const QType *gq = nullptr, *dq = nullptr, *sq = nullptr, *sdq = nullptr;  // (sdq: the shared down's)
  size_t gate_row = 0, down_row = 0, sgate_row = 0, sdown_row = 0;  // row bytes in the layer (QType::dev blocks)
  DevBuf router, gate, up, down, sgate, sup, sdown, sinp, norm;
  bool have[9] = {};
  // activations of the staged input
  int x_dtype = ARTLITE_X_BF16;
  int64_t staged = -1;  // tokens staged, -1: none
  DevBuf x, xhi, xlo;
  DevBuf xn;  // the RMS-normalised x (norm_eps > 0)
  DevBuf x16;                     // the prefill's fp16 activations (each token's row scaled by a power of two)
  DevBuf gu_tok, dn_tok, sgu_tok, sdn_tok;  // per token, the row factors of the prefill's products (float2)
  DevBuf row_a, gu_row, dn_row;   // per sorted pair row: its token and its factors
  DevBuf wmax;  // max |w| of gate, up, shared gate, shared up (the bounds on |h|), down; then the largest row L1 norm
                // of each
  DevBuf logits, ids, w, sg;
  DevBuf rpart;  // the router's fp64 partial sums (K split over workgroups), router_part_elems doubles
  size_t rpart_elems = 0;
  DevBuf table, ctrl, counts, offsets, order, slot, tiles;
  DevBuf hhi, hlo, ypairs, shhi, shlo, ys, y;
  DevBuf h16, sh16;  // the prefill's h (fp16, scaled per token)
  // the prefill tiles' weights of the formats they do not read from the file's bytes: the prefill layout (experts.h,
  // PREFILL_PQ6) of gate, up, down, shared gate, shared up, shared down, made at upload
  DevBuf pq_gate, pq_up, pq_down, pq_sgate, pq_sup, pq_sdown;
  int pre_g = 0, pre_d = 0, pre_sg = 0, pre_sd = 0;  // the prefill launches' weight format of each product (0: none)
  DevBuf xq, hq, shq;  // the decode path's XQ activations
  bool gemv_ok = false, shared_gemv_ok = false, prefill_ok = false, shared_prefill_ok = false;
  int64_t last_T = -1;
  bool last_gemv = false, last_prefill = false;
  int last_ys_parts = 1;  // (the shared expert's output of the last run: parts of its K, summed by the combine)
};

namespace {

// bytes of a row of cols values of type q as a GGUF file stores it
size_t file_row(const QType* q, int cols) { return q ? size_t(cols) / q->per * q->bytes : 0; }

// the block type of a weight tensor (null: the fp32 ones)
const QType* tensor_type(const artlite_moe_layer* L, int t) {
  switch (t) {
    case ARTLITE_GATE_EXPS:
    case ARTLITE_UP_EXPS: return L->gq;
    case ARTLITE_DOWN_EXPS: return L->dq;
    case ARTLITE_GATE_SHEXP:
    case ARTLITE_UP_SHEXP: return L->sq;
    case ARTLITE_DOWN_SHEXP: return L->sdq;
    default: return nullptr;
  }
}

// the bytes a tensor takes as uploaded (tensor_bytes, its file size)
size_t tensor_bytes(const artlite_moe_layer* L, int t) {
  const artlite_moe_desc& d = L->d;
  switch (t) {
    case ARTLITE_ROUTER: return size_t(d.n_experts) * d.hidden * 4;
    case ARTLITE_GATE_EXPS:
    case ARTLITE_UP_EXPS: return size_t(d.n_experts) * d.expert_ffn * file_row(L->gq, d.hidden);
    case ARTLITE_DOWN_EXPS: return size_t(d.n_experts) * d.hidden * file_row(L->dq, d.expert_ffn);
    case ARTLITE_GATE_SHEXP:
    case ARTLITE_UP_SHEXP: return size_t(d.shared_ffn) * file_row(L->sq, d.hidden);
    case ARTLITE_DOWN_SHEXP: return size_t(d.hidden) * file_row(L->sdq, d.shared_ffn);
    case ARTLITE_GATE_INP_SHEXP: return size_t(d.hidden) * 4;
    case ARTLITE_FFN_NORM: return d.norm_eps > 0 ? size_t(d.hidden) * 4 : 0;
    default: return 0;
  }
}

DevBuf* tensor_buf(artlite_moe_layer* L, int t) {
  switch (t) {
    case ARTLITE_ROUTER: return &L->router;
    case ARTLITE_GATE_EXPS: return &L->gate;
    case ARTLITE_UP_EXPS: return &L->up;
    case ARTLITE_DOWN_EXPS: return &L->down;
    case ARTLITE_GATE_SHEXP: return &L->sgate;
    case ARTLITE_UP_SHEXP: return &L->sup;
    case ARTLITE_DOWN_SHEXP: return &L->sdown;
    case ARTLITE_GATE_INP_SHEXP: return &L->sinp;
    case ARTLITE_FFN_NORM: return &L->norm;
    default: return nullptr;
  }
}

// the block formats of the experts' kernels (every quantized type the dequantizer reads)
bool is_expert_type(const QType* q) { return q && q->per >= 32; }

// the prefill tiles' weight format of a block format: its own (Q4_0, Q8_0, Q4_K: read from the file's bytes) or the
// prefill layout (the others)
int prefill_type(const QType* q) {
  int mode;
  float off;
  if (!q) return 0;
  if (q->id == ARTLITE_Q4_0 || q->id == ARTLITE_Q8_0 || q->id == ARTLITE_Q4_K) return q->id;
  return pq6_mode(q->id, mode, off) ? PREFILL_PQ6 : 0;
}

// a prefill launch's weight format (and the prefill layout's mode) for products of block format q
void prefill_format(const QType* q, PrefillArgs& a) {
  a.qtype = prefill_type(q);
  a.pq_mode = 0;
  a.pq_off = 0.0f;
  if (a.qtype == PREFILL_PQ6) pq6_mode(q->id, a.pq_mode, a.pq_off);
}

// a product's weights and row bytes as the prefill tiles read them (the prefill layout: one byte a value)
const uint8_t* prefill_w(const DevBuf& raw, const DevBuf& pq, int pre) {
  return pre == PREFILL_PQ6 ? pq.as<uint8_t>() : raw.as<uint8_t>();
}
size_t prefill_row(size_t raw_row, int K, int pre) { return pre == PREFILL_PQ6 ? size_t(K) : raw_row; }

int check_ready(const artlite_moe_layer* L) {
  for (int t = ARTLITE_ROUTER; t <= ARTLITE_DOWN_EXPS; t++)
    if (!L->have[t]) return fail(ARTLITE_EINVAL, "moe layer: tensor %d not uploaded", t);
  if (L->d.shared_ffn) {
    for (int t = ARTLITE_GATE_SHEXP; t <= ARTLITE_DOWN_SHEXP; t++)
      if (!L->have[t]) return fail(ARTLITE_EINVAL, "moe layer: shared tensor %d not uploaded", t);
    if (L->d.shared_gated && !L->have[ARTLITE_GATE_INP_SHEXP])
      return fail(ARTLITE_EINVAL, "moe layer: shared gate not uploaded");
  }
  if (L->d.norm_eps > 0 && !L->have[ARTLITE_FFN_NORM]) return fail(ARTLITE_EINVAL, "moe layer: ffn_norm not uploaded");
  return ARTLITE_OK;
}

// The kernels a forward pass of T tokens takes. Decode-sized passes (at most GEMV_BM pairs per expert on
// average) run the experts on the VALU GEMV over XQ activations (it takes every block format); larger ones on the
// fp16 MFMA prefill tiles (every block format: Q4_0, Q8_0, Q4_K from the file's bytes, the others through the prefill
// layout), and where those do not take a product's shape (K below 320 or not a multiple of 64) on the MFMA decode
// tiles over bf16 planes. (At 128 tokens of config 2, 8 pairs per expert, the prefill tiles' tiles of 32 rows took
// 208 us against 323 on the MFMA decode tiles: the decode tiles do twice the MFMA work on bf16 hi / lo planes.)
struct Path {
  bool gemv;            // routed experts (gate / up and down) on the GEMV (XQ of x; tiles of GEMV_BM rows)
  bool shared_gemv;     // the shared expert on the GEMV
  bool prefill;         // routed experts on the prefill tiles
  bool shared_prefill;  // the shared expert on the prefill tiles
  bool split;           // bf16 hi / lo planes of fp32 x needed (the MFMA decode tiles)
  bool quant;           // XQ of x needed (made by the router's launch)
  bool few_router;      // the router's launch of few tokens: a workgroup per expert and 16 tokens (and XQ of x)
  bool gemv_route;      // top k and dispatch in the gate / up GEMV's launch (each workgroup in its LDS)
  bool small;           // ... else in one workgroup of a launch of their own
};

Path path_of(const artlite_moe_layer* L, int64_t T) {
  Path p{};
  p.gemv = L->gemv_ok && T * L->d.top_k <= int64_t(GEMV_BM) * L->d.n_experts;
  p.shared_gemv = L->d.shared_ffn && p.gemv && L->shared_gemv_ok;
  p.prefill = !p.gemv && L->prefill_ok;
  p.shared_prefill = L->d.shared_ffn && p.prefill && L->shared_prefill_ok && T >= 64;
  const bool planes = (!p.gemv && !p.prefill) || (L->d.shared_ffn && !p.shared_gemv && !p.shared_prefill);
  p.split = planes && (L->x_dtype == ARTLITE_X_F32 || L->d.norm_eps > 0);  // (the normalised x is fp32)
  p.quant = p.gemv;
  p.few_router = p.gemv && router_few_fits(T, L->d.hidden, L->d.n_experts);
  p.gemv_route = p.few_router && gemv_route_fits(T, L->d.n_experts, L->d.top_k);
  p.small = p.gemv && !p.gemv_route && T * L->d.top_k <= DISPATCH_BLOCK && L->d.n_experts <= MAX_EXPERTS;
  return p;
}

// whether the shared expert's gate / up (down) products join the routed launch on the prefill tiles: the same block
// format (the launch's kernel is instantiated per format)
bool shared_gu_merged(const artlite_moe_layer* L) { return L->sq && L->sq->id == L->gq->id; }
bool shared_dn_merged(const artlite_moe_layer* L) { return L->sdq && L->sdq->id == L->dq->id; }

// the named kernels of a forward pass, in launch order
std::vector<std::string> kernel_list(const artlite_moe_layer* L, int64_t T) {
  const Path p = path_of(L, T);
  std::vector<std::string> k;
  if (L->d.norm_eps > 0) k.push_back("rmsnorm");
  if (p.prefill) k.push_back("prefill_x");
  if (p.split) k.push_back("split");
  k.push_back(p.quant ? "router_quant" : "router");
  if (L->d.shared_ffn && L->d.shared_gated) k.push_back("shared_gate");
  if (p.gemv_route) {
  } else if (p.small) {
    k.push_back("route");
  } else {
    k.push_back("topk");
    k.push_back("dispatch_count");
    k.push_back("dispatch_scatter");
  }
  const bool sp = p.prefill && p.shared_prefill;  // (the shared expert's items in the routed launches, or beside them)
  k.push_back("gate_up");
  if (sp && !shared_gu_merged(L)) k.push_back("shared_gate_up");
  k.push_back("down");
  if (sp && !shared_dn_merged(L)) k.push_back("shared_down");
  if (L->d.shared_ffn && !sp) {
    k.push_back("shared_gate_up");
    k.push_back("shared_down");
  }
  k.push_back("combine");
  return k;
}

// The shared expert's down on the prefill tiles splits its K (the shared width) into parts, each a product of the
// launch with a partial output of its own (T x H fp32; the combine adds them in order): whole blocks (K-quants: 256
// values) a part, at least 5 stages (320 values) each, the first ones a block longer where they do not divide evenly.
int shared_parts(const artlite_moe_layer* L, bool merged) {
  const int Ks = L->d.shared_ffn, unit = L->sdq->per >= 256 ? 256 : 64, units = Ks / unit;
  // (beside the routed down: parts about as long as its items' K; alone: as many as the launch takes)
  int parts = merged ? std::max(1, std::min(PREFILL_MAXP - 1, (Ks + L->d.expert_ffn / 2) / L->d.expert_ffn))
                     : PREFILL_MAXP;
  while (parts > 1 && units / parts * unit < 320) parts--;
  return parts;
}

// the shared down's part j of n: the product over its range of K, into ys part j
PrefillProblem shared_down_part(const artlite_moe_layer* L, int64_t T, int j, int n) {
  const int Ks = L->d.shared_ffn, unit = L->sdq->per >= 256 ? 256 : 64, units = Ks / unit;
  const int u0 = j * (units / n) + std::min(j, units % n), nu = units / n + (j < units % n ? 1 : 0);
  const int k0 = u0 * unit;
  PrefillProblem p{};
  const bool pq = L->pre_sd == PREFILL_PQ6;  // (the prefill layout: a byte a value)
  p.w[0] = pq ? L->pq_sdown.as<uint8_t>() + k0 : L->sdown.as<uint8_t>() + size_t(k0 / L->sdq->per) * L->sdq->dev;
  p.row_bytes = int(prefill_row(L->sdown_row, Ks, L->pre_sd));
  p.N = L->d.hidden;
  p.K = nu * unit;
  p.lda = Ks;
  p.a = L->sh16.as<uint16_t>() + k0;
  p.dense_rows = int(T);
  p.row_scale = L->sdn_tok.as<float2>();
  p.y = L->ys.as<float>() + size_t(j) * size_t(T) * L->d.hidden;
  return p;
}

// The forward pass of the staged T tokens. ev (optional): an event recorded before each kernel and one after the
// last (kernel_list order).
int run(artlite_moe_layer* L, int64_t T, hipEvent_t* ev) {
  const artlite_moe_desc& d = L->d;
  hipStream_t s = L->stream;
  const int H = d.hidden, E = d.n_experts, k = d.top_k, F = d.expert_ffn;
  const int64_t P = T * k;
  int ei = 0;
  auto mark = [&]() -> int {
    if (ev) ART_HIP(hipEventRecord(ev[ei++], s));
    return ARTLITE_OK;
  };
  const Path path = path_of(L, T);
  int ys_parts = 1;  // (the shared expert's output: its parts on the prefill tiles)
  // the block's input: x as staged, or (norm_eps > 0) its RMS normalisation in fp32
  const void* xin = L->x.p;
  int xdt = L->x_dtype;
  if (d.norm_eps > 0) {
    ART_TRY(mark());
    ART_TRY(launch_rmsnorm(L->x.p, L->x_dtype, L->norm.as<float>(), d.norm_eps, T, H, L->xn.as<float>(), s));
    xin = L->xn.p;
    xdt = ARTLITE_X_F32;
  }
  const uint16_t *ahi = static_cast<const uint16_t*>(xin), *alo = nullptr;
  if (path.prefill) {
    ART_TRY(mark());
    ART_TRY(launch_prefill_x(xin, xdt, T, H, L->wmax.as<float>(), path.shared_prefill ? 2 : 1, F,
                             L->x16.as<uint16_t>(), L->gu_tok.as<float2>(), L->dn_tok.as<float2>(),
                             L->sgu_tok.as<float2>(), L->sdn_tok.as<float2>(), s));
  }
  if (path.split) {
    ART_TRY(mark());
    ART_TRY(launch_split(static_cast<const float*>(xin), T * H, L->xhi.as<uint16_t>(), L->xlo.as<uint16_t>(), s));
    ahi = L->xhi.as<uint16_t>();
    alo = L->xlo.as<uint16_t>();
  }
  const int BM = path.gemv ? GEMV_BM : path.prefill ? PREFILL_BM : DECODE_BM;
  DispatchBufs db{L->ids.as<int32_t>(), P, E, k, L->table.as<int32_t>(), L->ctrl.as<int32_t>(),
                  L->counts.as<int32_t>(), L->offsets.as<int32_t>(), L->order.as<int32_t>(), L->slot.as<int32_t>(),
                  L->tiles.as<int32_t>(), BM, nullptr, 0, path.prefill ? 1 : 0};
  if (path.prefill) {  // (the scatter also writes each sorted row's token and factors)
    db.row_a = L->row_a.as<int32_t>();
    db.row_f[0] = L->gu_tok.as<float2>();
    db.row_f[1] = L->dn_tok.as<float2>();
    db.row_out[0] = L->gu_row.as<float2>();
    db.row_out[1] = L->dn_row.as<float2>();
  }
  ART_TRY(mark());
  // (a split router's parts, when the top k follows as a launch of its own: added by the top k)
  int parts = 0;
  const bool topk_launch = !path.gemv_route && !path.small;
  if (path.few_router)
    ART_TRY(launch_router_few(xin, xdt, L->router.as<float>(), H, E, T, L->logits.as<float>(),
                                path.quant ? L->xq.as<uint32_t>() : nullptr, s));
  else
    ART_TRY(launch_router(xin, xdt, L->router.as<float>(), H, E, T, L->logits.as<float>(), E,
                          path.quant ? L->xq.as<uint32_t>() : nullptr, L->rpart.as<double>(), L->rpart_elems, s,
                          topk_launch ? &parts : nullptr));
  if (d.shared_ffn && d.shared_gated) {
    ART_TRY(mark());
    ART_TRY(launch_router(xin, xdt, L->sinp.as<float>(), H, 1, T, L->sg.as<float>(), 1, nullptr, nullptr, 0, s));
  }
  if (path.gemv_route) {
  } else if (path.small) {
    ART_TRY(mark());
    ART_TRY(launch_route_small(L->logits.as<float>(), T, E, k, d.gating, L->ids.as<int32_t>(), L->w.as<float>(), db,
                               s));
  } else {
    ART_TRY(mark());
    if (parts)
      ART_TRY(launch_topk_parts(L->rpart.as<double>(), parts, T, E, L->logits.as<float>(), E, k, d.gating,
                                L->ids.as<int32_t>(), L->w.as<float>(), s));
    else
      ART_TRY(launch_topk(L->logits.as<float>(), T, E, E, 0, E, k, d.gating, L->ids.as<int32_t>(), L->w.as<float>(),
                          nullptr, s));
    const int64_t nb = dispatch_blocks(P);
    ART_TRY(mark());
    ART_TRY(launch_dispatch_count(db, nb, s));
    ART_TRY(mark());
    ART_TRY(launch_dispatch_scatter(db, nb, s));
  }
  if (path.gemv) {
    GemvArgs g{};
    g.w[0] = L->gate.as<uint8_t>();
    g.w[1] = L->up.as<uint8_t>();
    g.expert_bytes = int64_t(F) * L->gate_row;
    g.row_bytes = int(L->gate_row);
    g.N = F;
    g.K = H;
    g.qtype = d.gate_type;
    g.xq = L->xq.as<uint32_t>();
    g.a_gather = 1;
    g.order = L->order.as<int32_t>();
    g.topk = k;
    g.rows_total = int(P);
    g.tiles = L->tiles.as<int32_t>();
    g.n_tiles = L->ctrl.as<int32_t>() + CTRL_TILES;
    g.offsets = L->offsets.as<int32_t>();
    g.max_tiles = tile_bound(P, E, BM);
    g.hq = L->hq.as<uint32_t>();
    if (path.gemv_route) {
      g.route.logits = L->logits.as<float>();
      g.route.T = int(T);
      g.route.E = E;
      g.route.k = k;
      g.route.sigmoid = d.gating;
      g.route.ids = L->ids.as<int32_t>();
      g.route.w32 = L->w.as<float>();
      g.route.d = db;
    }
    ART_TRY(mark());
    ART_TRY(launch_gemv(g, s));
    GemvArgs dn = g;
    dn.route = GemvArgs::Route{};
    dn.w[0] = L->down.as<uint8_t>();
    dn.w[1] = nullptr;
    dn.expert_bytes = int64_t(H) * L->down_row;
    dn.row_bytes = int(L->down_row);
    dn.N = H;
    dn.K = F;
    dn.qtype = d.down_type;
    dn.xq = L->hq.as<uint32_t>();
    dn.a_gather = 0;
    dn.hq = nullptr;
    dn.y = L->ypairs.as<float>();
    ART_TRY(mark());
    ART_TRY(launch_gemv(dn, s));
  } else if (path.prefill) {
    // gate / up (SwiGLU), then down; the shared expert's products join them (its down in parts of its K) when their
    // formats match, else run as launches of their own right after
    const bool sp = d.shared_ffn && path.shared_prefill;
    PrefillArgs gu{};
    prefill_format(L->gq, gu);
    gu.np = 1;
    PrefillProblem& g = gu.p[0];
    g.w[0] = prefill_w(L->gate, L->pq_gate, L->pre_g);
    g.w[1] = prefill_w(L->up, L->pq_up, L->pre_g);
    g.row_bytes = int(prefill_row(L->gate_row, H, L->pre_g));
    g.expert_bytes = int64_t(F) * g.row_bytes;
    g.N = F;
    g.K = H;
    g.lda = H;
    g.a = L->x16.as<uint16_t>();
    g.row_a = L->row_a.as<int32_t>();
    g.row_scale = L->gu_row.as<float2>();
    g.tiles = L->tiles.as<int32_t>();
    g.n_tiles = L->ctrl.as<int32_t>() + CTRL_TILES;
    g.offsets = L->offsets.as<int32_t>();
    g.max_tiles = tile_bound(P, E, BM);
    g.h = L->h16.as<uint16_t>();
    PrefillArgs sgu{};  // (the shared gate / up: in gu, or a launch of its own)
    if (sp) {
      PrefillArgs& into = shared_gu_merged(L) ? gu : sgu;
      prefill_format(L->sq, into);
      PrefillProblem& q = into.p[into.np++];
      q.w[0] = prefill_w(L->sgate, L->pq_sgate, L->pre_sg);
      q.w[1] = prefill_w(L->sup, L->pq_sup, L->pre_sg);
      q.row_bytes = int(prefill_row(L->sgate_row, H, L->pre_sg));
      q.N = d.shared_ffn;
      q.K = H;
      q.lda = H;
      q.a = L->x16.as<uint16_t>();
      q.dense_rows = int(T);
      q.row_scale = L->sgu_tok.as<float2>();
      q.h = L->sh16.as<uint16_t>();
    }
    ART_TRY(mark());
    ART_TRY(launch_prefill(gu, s));
    if (sgu.np) {
      ART_TRY(mark());
      ART_TRY(launch_prefill(sgu, s));
    }
    PrefillArgs dn{};
    prefill_format(L->dq, dn);
    dn.np = 1;
    PrefillProblem& q = dn.p[0];
    q = g;
    q.w[0] = prefill_w(L->down, L->pq_down, L->pre_d);
    q.w[1] = nullptr;
    q.row_bytes = int(prefill_row(L->down_row, F, L->pre_d));
    q.expert_bytes = int64_t(H) * q.row_bytes;
    q.N = H;
    q.K = F;
    q.lda = F;
    q.a = L->h16.as<uint16_t>();
    q.row_a = nullptr;
    q.row_scale = L->dn_row.as<float2>();
    q.h = nullptr;
    q.y16 = L->ypairs.as<uint16_t>();  // (fp16 pair outputs, their rows' true values dn_row[s].x times these)
    PrefillArgs sdn{};  // (the shared down's parts: in dn, or a launch of their own)
    if (sp) {
      const bool merged = shared_dn_merged(L);
      PrefillArgs& into = merged ? dn : sdn;
      prefill_format(L->sdq, into);
      const int n = shared_parts(L, merged);
      // (a launch of its own: tiles of fewer rows where 256-row tiles would leave compute units without an item)
      int tile = 256;
      while (!merged && tile > 64 && (T + tile - 1) / tile * ((H + 255) / 256) * n < L->cus) tile /= 2;
      for (int j = 0; j < n; j++) {
        into.p[into.np] = shared_down_part(L, T, j, n);
        into.p[into.np++].dense_tile = balanced_rows(int(T), tile);
      }
      ys_parts = n;
    }
    ART_TRY(mark());
    ART_TRY(launch_prefill(dn, s));
    if (sdn.np) {
      ART_TRY(mark());
      ART_TRY(launch_prefill(sdn, s));
    }
  } else {
    GemmArgs g{};
    g.w[0] = L->gate.as<uint8_t>();
    g.w[1] = L->up.as<uint8_t>();
    g.expert_bytes = int64_t(F) * L->gate_row;
    g.row_bytes = int(L->gate_row);
    g.N = F;
    g.K = H;
    g.qtype = d.gate_type;
    g.a_hi = ahi;
    g.a_lo = alo;
    g.a_gather = 1;
    g.order = L->order.as<int32_t>();
    g.topk = k;
    g.tiles = L->tiles.as<int32_t>();
    g.n_tiles = L->ctrl.as<int32_t>() + CTRL_TILES;
    g.offsets = L->offsets.as<int32_t>();
    g.max_tiles = tile_bound(P, E, BM);
    g.bm = BM;
    g.h_hi = L->hhi.as<uint16_t>();
    g.h_lo = L->hlo.as<uint16_t>();
    ART_TRY(mark());
    ART_TRY(launch_expert_gemm(g, s));
    GemmArgs dn = g;
    dn.w[0] = L->down.as<uint8_t>();
    dn.w[1] = nullptr;
    dn.expert_bytes = int64_t(H) * L->down_row;
    dn.row_bytes = int(L->down_row);
    dn.N = H;
    dn.K = F;
    dn.qtype = d.down_type;
    dn.a_hi = L->hhi.as<uint16_t>();
    dn.a_lo = L->hlo.as<uint16_t>();
    dn.a_gather = 0;
    dn.y = L->ypairs.as<float>();
    ART_TRY(mark());
    ART_TRY(launch_expert_gemm(dn, s));
  }
  const float* ys = nullptr;
  if (d.shared_ffn && path.shared_gemv) {
    GemvArgs sg{};
    sg.w[0] = L->sgate.as<uint8_t>();
    sg.w[1] = L->sup.as<uint8_t>();
    sg.row_bytes = int(L->sgate_row);
    sg.N = d.shared_ffn;
    sg.K = H;
    sg.qtype = d.shared_type;
    sg.xq = L->xq.as<uint32_t>();
    sg.dense_rows = int(T);
    sg.hq = L->shq.as<uint32_t>();
    ART_TRY(mark());
    ART_TRY(launch_gemv(sg, s));
    GemvArgs sd = sg;
    sd.w[0] = L->sdown.as<uint8_t>();
    sd.w[1] = nullptr;
    sd.row_bytes = int(L->sdown_row);
    sd.N = H;
    sd.K = d.shared_ffn;
    sd.qtype = L->sdq->id;
    sd.xq = L->shq.as<uint32_t>();
    sd.hq = nullptr;
    sd.y = L->ys.as<float>();
    ART_TRY(mark());
    ART_TRY(launch_gemv(sd, s));
    ys = L->ys.as<float>();
  } else if (d.shared_ffn && path.shared_prefill) {  // (with the routed experts' launches)
    ys = L->ys.as<float>();
  } else if (d.shared_ffn) {
    GemmArgs sg{};
    sg.w[0] = L->sgate.as<uint8_t>();
    sg.w[1] = L->sup.as<uint8_t>();
    sg.expert_bytes = 0;
    sg.row_bytes = int(L->sgate_row);
    sg.N = d.shared_ffn;
    sg.K = H;
    sg.qtype = d.shared_type;
    sg.a_hi = ahi;
    sg.a_lo = alo;
    sg.dense_rows = int(T);
    sg.h_hi = L->shhi.as<uint16_t>();
    sg.h_lo = L->shlo.as<uint16_t>();
    ART_TRY(mark());
    ART_TRY(launch_expert_gemm(sg, s));
    GemmArgs sd = sg;
    sd.w[0] = L->sdown.as<uint8_t>();
    sd.w[1] = nullptr;
    sd.row_bytes = int(L->sdown_row);
    sd.N = H;
    sd.K = d.shared_ffn;
    sd.qtype = L->sdq->id;
    sd.a_hi = L->shhi.as<uint16_t>();
    sd.a_lo = L->shlo.as<uint16_t>();
    sd.y = L->ys.as<float>();
    ART_TRY(mark());
    ART_TRY(launch_expert_gemm(sd, s));
    ys = L->ys.as<float>();
  }
  ART_TRY(mark());
  if (path.prefill)
    ART_TRY(launch_combine16(L->ypairs.as<uint16_t>(), L->dn_row.as<float2>(), L->slot.as<int32_t>(), L->w.as<float>(),
                             k, ys, ys_parts, d.shared_gated ? L->sg.as<float>() : nullptr, 1, T, H,
                             d.residual ? L->x.p : nullptr, L->x_dtype, L->y.as<float>(), s));
  else
    ART_TRY(launch_combine(L->ypairs.as<float>(), L->slot.as<int32_t>(), L->w.as<float>(), k, ys,
                           d.shared_gated ? L->sg.as<float>() : nullptr, 1, T, H, d.residual ? L->x.p : nullptr,
                           L->x_dtype, L->y.as<float>(), s));
  ART_TRY(mark());
  L->last_T = T;
  L->last_gemv = path.gemv;
  L->last_prefill = path.prefill;
  L->last_ys_parts = ys_parts;
  return ARTLITE_OK;
}

}  // namespace

extern "C" int artlite_moe_layer_create(const artlite_moe_desc* desc, artlite_moe_layer** out) {
  if (!desc || !out) return fail(ARTLITE_EINVAL, "moe layer: null argument");
  *out = nullptr;
  const artlite_moe_desc& d = *desc;
  if (d.hidden <= 0 || d.n_experts <= 0 || d.expert_ffn <= 0 || d.max_tokens <= 0)
    return fail(ARTLITE_EINVAL, "moe layer: H %d, E %d, F %d, max tokens %d", d.hidden, d.n_experts, d.expert_ffn,
                d.max_tokens);
  ART_TRY(check_route_args(1, d.n_experts, d.n_experts, d.top_k));
  const QType *gq = qtype_by_id(d.gate_type), *dq = qtype_by_id(d.down_type);
  if (!is_expert_type(gq) || !is_expert_type(dq))
    return fail(ARTLITE_EINVAL, "moe layer: expert types %d / %d (not a block format)", d.gate_type, d.down_type);
  if (d.hidden % gq->per || d.expert_ffn % dq->per)
    return fail(ARTLITE_EINVAL, "moe layer: H %d / F %d not multiples of the blocks (%d / %d)", d.hidden,
                d.expert_ffn, gq->per, dq->per);
  if (d.hidden % 4) return fail(ARTLITE_EINVAL, "moe layer: H %d not a multiple of 4", d.hidden);
  const QType *sq = nullptr, *sdq = nullptr;
  if (d.shared_ffn) {
    sq = qtype_by_id(d.shared_type);
    sdq = d.shared_down_type ? qtype_by_id(d.shared_down_type) : sq;
    if (!is_expert_type(sq) || !is_expert_type(sdq) || d.hidden % sq->per || d.shared_ffn % sdq->per)
      return fail(ARTLITE_EINVAL, "moe layer: shared expert types %d / %d, width %d", d.shared_type,
                  d.shared_down_type, d.shared_ffn);
  }
  // the MFMA decode tiles (every product between the GEMV's sizes and the prefill's, and every format the other two
  // do not take) stage an A row's whole K in LDS: K up to 32 MAX_GROUPS
  const int kmax = 32 * MAX_GROUPS;
  if (d.hidden > kmax || d.expert_ffn > kmax || d.shared_ffn > kmax)
    return fail(ARTLITE_EINVAL, "moe layer: H %d, F %d, shared F %d: at most %d each", d.hidden, d.expert_ffn,
                d.shared_ffn, kmax);
  if (d.gating != 0 && d.gating != 1) return fail(ARTLITE_EINVAL, "moe layer: gating %d", d.gating);
  if (!(d.norm_eps >= 0.0f && d.norm_eps < 1.0f) || (d.residual != 0 && d.residual != 1))
    return fail(ARTLITE_EINVAL, "moe layer: norm eps %g, residual %d", double(d.norm_eps), d.residual);
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(ARTLITE_EHIP, "moe layer: no HIP device");
  auto* L = new artlite_moe_layer();
  L->d = d;
  L->gq = gq;
  L->dq = dq;
  L->sq = sq;
  L->sdq = sdq;
  L->gate_row = size_t(d.hidden) / gq->per * gq->dev;
  L->down_row = size_t(d.expert_ffn) / dq->per * dq->dev;
  if (sq) {
    L->sgate_row = size_t(d.hidden) / sq->per * sq->dev;
    L->sdown_row = size_t(d.shared_ffn) / sdq->per * sdq->dev;
  }
  L->gemv_ok = gemv_supported(d.gate_type, d.hidden, d.expert_ffn) && d.expert_ffn % 256 == 0 &&
               gemv_supported(d.down_type, d.expert_ffn, d.hidden);
  // (the prefill tiles address weights and A rows by 32-bit offsets: every expert's bytes, every row of x16 and h16)
  const int64_t maxP = int64_t(d.max_tokens) * d.top_k;
  L->pre_g = prefill_type(gq);
  L->pre_d = prefill_type(dq);
  L->prefill_ok = L->pre_g && L->pre_d && prefill_supported(L->pre_g, d.hidden, d.expert_ffn) &&
                  prefill_supported(L->pre_d, d.expert_ffn, d.hidden) &&
                  prefill_fits(d.n_experts, int64_t(d.expert_ffn) * prefill_row(L->gate_row, d.hidden, L->pre_g),
                               d.max_tokens, d.hidden) &&
                  prefill_fits(d.n_experts, int64_t(d.hidden) * prefill_row(L->down_row, d.expert_ffn, L->pre_d), maxP,
                               d.expert_ffn);
  L->shared_gemv_ok = sq && gemv_supported(sq->id, d.hidden, d.shared_ffn) &&
                      gemv_supported(sdq->id, d.shared_ffn, d.hidden);
  L->pre_sg = prefill_type(sq);
  L->pre_sd = prefill_type(sdq);
  L->shared_prefill_ok = sq && L->pre_sg && L->pre_sd && prefill_supported(L->pre_sg, d.hidden, d.shared_ffn) &&
                         prefill_supported(L->pre_sd, d.shared_ffn, d.hidden) &&
                         prefill_fits(1, int64_t(d.shared_ffn) * prefill_row(L->sgate_row, d.hidden, L->pre_sg),
                                      d.max_tokens, d.hidden) &&
                         prefill_fits(1, int64_t(d.hidden) * prefill_row(L->sdown_row, d.shared_ffn, L->pre_sd),
                                      d.max_tokens, d.shared_ffn);
  hipError_t e = hipGetDevice(&L->device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&L->cus, hipDeviceAttributeMultiprocessorCount, L->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&L->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete L;
    return fail(ARTLITE_EHIP, "moe layer: %s", hipGetErrorString(e));
  }
  // activation buffers for max_tokens
  const int64_t T = d.max_tokens, P = T * d.top_k, H = d.hidden, F = d.expert_ffn, E = d.n_experts;
  int rc = ARTLITE_OK;
  auto res = [&](DevBuf& b, size_t bytes) {
    if (rc == ARTLITE_OK) rc = b.reserve(bytes);
  };
  res(L->x, size_t(T * H) * 4);
  if (d.norm_eps > 0) res(L->xn, size_t(T * H) * 4);
  res(L->xhi, size_t(T * H) * 2);
  res(L->xlo, size_t(T * H) * 2);
  res(L->logits, size_t(T * E) * 4);
  L->rpart_elems = router_part_elems(T, int(E), int(H));
  if (L->rpart_elems) res(L->rpart, L->rpart_elems * 8);
  res(L->ids, size_t(P) * 4);
  res(L->w, size_t(P) * 4);
  res(L->sg, size_t(T) * 4);
  res(L->table, size_t(dispatch_blocks(P) * E) * 4);
  res(L->ctrl, CTRL_WORDS * 4);
  res(L->counts, size_t(E) * 4);
  res(L->offsets, size_t(E + 1) * 4);
  res(L->order, size_t(P) * 4);
  res(L->slot, size_t(P) * 4);
  res(L->tiles, size_t(2 * tile_bound(P, int(E), 1)) * 4);
  res(L->hhi, size_t(P * F) * 2);
  res(L->hlo, size_t(P * F) * 2);
  res(L->ypairs, size_t(P * H) * 4);
  res(L->y, size_t(T * H) * 4);
  res(L->wmax, 10 * 4);
  if (L->prefill_ok) {
    res(L->x16, size_t(T * H) * 2);
    res(L->gu_tok, size_t(T) * 8);
    res(L->dn_tok, size_t(T) * 8);
    res(L->row_a, size_t(P) * 4);
    res(L->gu_row, size_t(P) * 8);
    res(L->dn_row, size_t(P) * 8);
    res(L->h16, size_t(P * F) * 2);
    if (L->shared_prefill_ok) {
      res(L->sgu_tok, size_t(T) * 8);
      res(L->sdn_tok, size_t(T) * 8);
      res(L->sh16, size_t(T) * d.shared_ffn * 2);
    }
  }
  if (L->gemv_ok) {
    res(L->xq, size_t(T * xq_row_dwords(d.hidden)) * 4);
    res(L->hq, size_t(P * xq_row_dwords(d.expert_ffn)) * 4);
    if (L->shared_gemv_ok) res(L->shq, size_t(T * xq_row_dwords(d.shared_ffn)) * 4);
  }
  if (d.shared_ffn) {
    res(L->shhi, size_t(T) * d.shared_ffn * 2);
    res(L->shlo, size_t(T) * d.shared_ffn * 2);
    res(L->ys, size_t(T * H) * 4 * (L->shared_prefill_ok ? PREFILL_MAXP : 1));  // (prefill: the down's K parts)
  }
  if (rc == ARTLITE_OK && hipMemset(L->ctrl.p, 0, CTRL_WORDS * 4) != hipSuccess)
    rc = fail(ARTLITE_EHIP, "moe layer: memset");
  if (rc != ARTLITE_OK) {
    artlite_moe_layer_destroy(L);
    return rc;
  }
  *out = L;
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_destroy(artlite_moe_layer* L) {
  if (!L) return ARTLITE_OK;
  if (L->stream) {
    (void)hipStreamSynchronize(L->stream);
    (void)hipStreamDestroy(L->stream);
  }
  delete L;
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_upload(artlite_moe_layer* L, int t, const void* data, size_t nbytes) {
  if (!L || !data) return fail(ARTLITE_EINVAL, "moe layer upload: null argument");
  DevBuf* b = tensor_buf(L, t);
  const size_t want = tensor_bytes(L, t);
  if (!b || !want) return fail(ARTLITE_EINVAL, "moe layer upload: tensor %d not in this layer", t);
  if (nbytes != want) return fail(ARTLITE_EINVAL, "moe layer upload: tensor %d is %zu bytes, not %zu", t, nbytes, want);
  // blocks whose layer size differs from the file's are padded with zeros, block by block, on the host: Q6_K after
  // the block, IQ4_XS after its 8-byte header (d, the scales), so that its code runs start 16-byte aligned
  const QType* tq = tensor_type(L, t);
  const size_t dev = tq && tq->dev != tq->bytes ? want / tq->bytes * tq->dev : want;
  std::vector<uint8_t> padded;
  const void* src = data;
  if (dev != want) {
    padded.assign(dev, 0);
    const uint8_t* in = static_cast<const uint8_t*>(data);
    const int head = tq->id == ARTLITE_IQ4_XS ? 8 : tq->bytes, gap = tq->dev - tq->bytes;
    for (size_t i = 0; i < want / tq->bytes; i++) {
      uint8_t* o = &padded[i * tq->dev];
      const uint8_t* blk = in + i * tq->bytes;
      std::memcpy(o, blk, head);
      std::memcpy(o + head + gap, blk + head, tq->bytes - head);
    }
    src = padded.data();
  }
  ART_TRY(b->reserve(dev + WEIGHT_TAIL));
  ART_HIP(hipMemcpyAsync(b->p, src, dev, hipMemcpyHostToDevice, L->stream));
  ART_HIP(hipMemsetAsync(static_cast<uint8_t*>(b->p) + dev, 0, WEIGHT_TAIL, L->stream));  // (the loaders' tail)
  // the prefill's bounds on |h| take max |w| of the gate and up matrices, the one on the down's sums that of down
  const int wm = t == ARTLITE_GATE_EXPS ? 0 : t == ARTLITE_UP_EXPS ? 1 : t == ARTLITE_GATE_SHEXP ? 2
               : t == ARTLITE_UP_SHEXP ? 3 : t == ARTLITE_DOWN_EXPS ? 4 : -1;
  const bool pre = wm < 2 || wm == 4 ? L->prefill_ok : L->shared_prefill_ok;
  if (wm >= 0 && pre) {
    const QType* q = wm < 2 ? L->gq : wm == 4 ? L->dq : L->sq;
    ART_TRY(launch_weight_max(static_cast<const uint8_t*>(b->p), q->id, int64_t(want / q->bytes),
                              L->wmax.as<float>() + wm, L->stream));
    const artlite_moe_desc& d = L->d;
    const int cols = wm == 4 ? d.expert_ffn : d.hidden;
    const size_t row = wm < 2 ? L->gate_row : wm == 4 ? L->down_row : L->sgate_row;
    const int64_t rows = wm < 2 ? int64_t(d.n_experts) * d.expert_ffn : wm == 4 ? int64_t(d.n_experts) * d.hidden
                                                                                 : int64_t(d.shared_ffn);
    ART_TRY(launch_weight_l1(static_cast<const uint8_t*>(b->p), q->id, rows, row, cols, L->wmax.as<float>() + 5 + wm,
                             L->stream));
  }
  // the prefill layout of a product the prefill tiles take in it (from the uploaded blocks)
  {
    const artlite_moe_desc& d = L->d;
    DevBuf* pq = nullptr;
    int pre = 0, K = 0;
    int64_t rows = 0;
    size_t row = 0;
    switch (t) {
      case ARTLITE_GATE_EXPS: pq = &L->pq_gate, pre = L->prefill_ok ? L->pre_g : 0; break;
      case ARTLITE_UP_EXPS: pq = &L->pq_up, pre = L->prefill_ok ? L->pre_g : 0; break;
      case ARTLITE_DOWN_EXPS: pq = &L->pq_down, pre = L->prefill_ok ? L->pre_d : 0; break;
      case ARTLITE_GATE_SHEXP: pq = &L->pq_sgate, pre = L->shared_prefill_ok ? L->pre_sg : 0; break;
      case ARTLITE_UP_SHEXP: pq = &L->pq_sup, pre = L->shared_prefill_ok ? L->pre_sg : 0; break;
      case ARTLITE_DOWN_SHEXP: pq = &L->pq_sdown, pre = L->shared_prefill_ok ? L->pre_sd : 0; break;
      default: break;
    }
    if (pre == PREFILL_PQ6) {
      switch (t) {
        case ARTLITE_GATE_EXPS:
        case ARTLITE_UP_EXPS: rows = int64_t(d.n_experts) * d.expert_ffn, K = d.hidden, row = L->gate_row; break;
        case ARTLITE_DOWN_EXPS: rows = int64_t(d.n_experts) * d.hidden, K = d.expert_ffn, row = L->down_row; break;
        case ARTLITE_GATE_SHEXP:
        case ARTLITE_UP_SHEXP: rows = d.shared_ffn, K = d.hidden, row = L->sgate_row; break;
        default: rows = d.hidden, K = d.shared_ffn, row = L->sdown_row; break;
      }
      const size_t bytes = size_t(rows) * size_t(K);
      ART_TRY(pq->reserve(bytes + WEIGHT_TAIL));
      ART_HIP(hipMemsetAsync(pq->as<uint8_t>() + bytes, 0, WEIGHT_TAIL, L->stream));
      ART_TRY(launch_pq6_pack(static_cast<const uint8_t*>(b->p), tq->id, rows, K, row, pq->as<uint8_t>(), L->stream));
    }
  }
  ART_HIP(hipStreamSynchronize(L->stream));
  L->have[t] = true;
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_stage(artlite_moe_layer* L, const void* x, int x_dtype, int64_t T) {
  if (!L || (!x && T)) return fail(ARTLITE_EINVAL, "moe layer stage: null argument");
  if (T < 0 || T > L->d.max_tokens) return fail(ARTLITE_EINVAL, "moe layer: %lld tokens of at most %d", (long long)T,
                                                L->d.max_tokens);
  if (x_dtype != ARTLITE_X_F32 && x_dtype != ARTLITE_X_BF16) return fail(ARTLITE_EINVAL, "moe layer: x dtype %d", x_dtype);
  const size_t bytes = size_t(T) * L->d.hidden * (x_dtype == ARTLITE_X_F32 ? 4 : 2);
  if (bytes) ART_HIP(hipMemcpyAsync(L->x.p, x, bytes, hipMemcpyHostToDevice, L->stream));
  ART_HIP(hipStreamSynchronize(L->stream));
  L->x_dtype = x_dtype;
  L->staged = T;
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_run(artlite_moe_layer* L, int64_t T) {
  if (!L) return fail(ARTLITE_EINVAL, "moe layer run: null layer");
  if (T != L->staged) return fail(ARTLITE_EINVAL, "moe layer run: %lld tokens, %lld staged", (long long)T,
                                  (long long)L->staged);
  ART_TRY(check_ready(L));
  if (T == 0) return ARTLITE_OK;
  return run(L, T, nullptr);
}

extern "C" int artlite_moe_layer_sync(artlite_moe_layer* L) {
  if (!L) return fail(ARTLITE_EINVAL, "moe layer sync: null layer");
  ART_HIP(hipStreamSynchronize(L->stream));
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_output(artlite_moe_layer* L, float* y, int64_t T) {
  if (!L || (!y && T)) return fail(ARTLITE_EINVAL, "moe layer output: null argument");
  if (T != L->last_T && T) return fail(ARTLITE_EINVAL, "moe layer output: %lld tokens, the last run had %lld",
                                       (long long)T, (long long)L->last_T);
  if (T) ART_HIP(hipMemcpyAsync(y, L->y.p, size_t(T) * L->d.hidden * 4, hipMemcpyDeviceToHost, L->stream));
  ART_HIP(hipStreamSynchronize(L->stream));
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_forward(artlite_moe_layer* L, const void* x, int x_dtype, int64_t T, float* y) {
  ART_TRY(artlite_moe_layer_stage(L, x, x_dtype, T));
  ART_TRY(artlite_moe_layer_run(L, T));
  if (T == 0) {
    L->last_T = 0;
    return ARTLITE_OK;
  }
  ART_TRY(artlite_moe_layer_output(L, y, T));
  int32_t ctrl[CTRL_WORDS];
  ART_HIP(hipMemcpy(ctrl, L->ctrl.p, sizeof ctrl, hipMemcpyDeviceToHost));
  if (ctrl[CTRL_BAD]) return fail(ARTLITE_EHIP, "moe layer: the dispatch saw an invalid expert id");
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_tap(artlite_moe_layer* L, int tap, void* out, size_t nbytes) {
  if (!L || !out) return fail(ARTLITE_EINVAL, "moe layer tap: null argument");
  const int64_t T = L->last_T;
  if (T < 0) return fail(ARTLITE_EINVAL, "moe layer tap: no run yet");
  const int64_t P = T * L->d.top_k, E = L->d.n_experts;
  const void* src = nullptr;
  size_t bytes = 0;
  switch (tap) {
    case ARTLITE_TAP_LOGITS: src = L->logits.p, bytes = size_t(T * E) * 4; break;
    case ARTLITE_TAP_IDS: src = L->ids.p, bytes = size_t(P) * 4; break;
    case ARTLITE_TAP_WEIGHTS: src = L->w.p, bytes = size_t(P) * 4; break;
    case ARTLITE_TAP_COUNTS: src = L->counts.p, bytes = size_t(E) * 4; break;
    case ARTLITE_TAP_OFFSETS: src = L->offsets.p, bytes = size_t(E + 1) * 4; break;
    case ARTLITE_TAP_ORDER: src = L->order.p, bytes = size_t(P) * 4; break;
    case ARTLITE_TAP_SLOT: src = L->slot.p, bytes = size_t(P) * 4; break;
    case ARTLITE_TAP_Y:
      if (L->last_prefill) {  // (fp16 pair outputs: row s's true values are dn_row[s].x times them)
        const int H = L->d.hidden;
        const size_t n = size_t(P) * H;
        if (nbytes < n * 4) return fail(ARTLITE_EINVAL, "moe layer tap: %zu bytes, need %zu", nbytes, n * 4);
        ART_HIP(hipStreamSynchronize(L->stream));
        std::vector<uint16_t> y(n);
        std::vector<float2> dn(static_cast<size_t>(P));
        if (n) ART_HIP(hipMemcpy(y.data(), L->ypairs.p, n * 2, hipMemcpyDeviceToHost));
        if (P) ART_HIP(hipMemcpy(dn.data(), L->dn_row.p, size_t(P) * 8, hipMemcpyDeviceToHost));
        float* o = static_cast<float*>(out);
        for (int64_t r = 0; r < P; r++)
          for (int c = 0; c < H; c++)
            o[size_t(r) * H + c] = float(__builtin_bit_cast(_Float16, y[size_t(r) * H + c])) * dn[size_t(r)].x;
        return ARTLITE_OK;
      }
      src = L->ypairs.p, bytes = size_t(P) * L->d.hidden * 4;
      break;
    case ARTLITE_TAP_XN:
      if (!(L->d.norm_eps > 0)) return fail(ARTLITE_EINVAL, "moe layer tap: no norm in this layer");
      src = L->xn.p, bytes = size_t(T) * L->d.hidden * 4;
      break;
    case ARTLITE_TAP_YS: {
      if (!L->d.shared_ffn) return fail(ARTLITE_EINVAL, "moe layer tap: no shared expert in this layer");
      const size_t n = size_t(T) * L->d.hidden;
      if (nbytes < n * 4) return fail(ARTLITE_EINVAL, "moe layer tap: %zu bytes, need %zu", nbytes, n * 4);
      ART_HIP(hipStreamSynchronize(L->stream));
      std::vector<float> part(n * size_t(L->last_ys_parts));
      if (n) ART_HIP(hipMemcpy(part.data(), L->ys.p, part.size() * 4, hipMemcpyDeviceToHost));
      float* o = static_cast<float*>(out);  // (the parts added in order, as the combine adds them)
      for (size_t i = 0; i < n; i++) {
        float v = part[i];
        for (int j = 1; j < L->last_ys_parts; j++) v += part[size_t(j) * n + i];
        o[i] = v;
      }
      return ARTLITE_OK;
    }
    case ARTLITE_TAP_H: {
      const size_t n = size_t(P) * L->d.expert_ffn;
      if (nbytes < n * 4) return fail(ARTLITE_EINVAL, "moe layer tap: %zu bytes, need %zu", nbytes, n * 4);
      ART_HIP(hipStreamSynchronize(L->stream));
      float* o = static_cast<float*>(out);
      if (L->last_gemv) {
        const int64_t rw = xq_row_dwords(L->d.expert_ffn);
        std::vector<uint32_t> q(size_t(P * rw));
        if (P) ART_HIP(hipMemcpy(q.data(), L->hq.p, q.size() * 4, hipMemcpyDeviceToHost));
        for (int64_t r = 0; r < P; r++) xq_dequant_row(q.data() + r * rw, L->d.expert_ffn, o + r * L->d.expert_ffn);
        return ARTLITE_OK;
      }
      if (L->last_prefill) {
        // fp16 h, its row scaled by 2^-he: the down launch's factors dn_row[s] multiply to 2^he
        const int F = L->d.expert_ffn;
        std::vector<uint16_t> h(n);
        std::vector<float2> dn(static_cast<size_t>(P));
        ART_HIP(hipMemcpy(h.data(), L->h16.p, n * 2, hipMemcpyDeviceToHost));
        ART_HIP(hipMemcpy(dn.data(), L->dn_row.p, size_t(P) * 8, hipMemcpyDeviceToHost));
        for (int64_t r = 0; r < P; r++)
          for (int c = 0; c < F; c++)
            o[r * F + c] = float(__builtin_bit_cast(_Float16, h[size_t(r) * F + c])) * (dn[size_t(r)].x * dn[size_t(r)].y);
        return ARTLITE_OK;
      }
      std::vector<uint16_t> hi(n), lo(n);
      ART_HIP(hipMemcpy(hi.data(), L->hhi.p, n * 2, hipMemcpyDeviceToHost));
      ART_HIP(hipMemcpy(lo.data(), L->hlo.p, n * 2, hipMemcpyDeviceToHost));
      for (size_t i = 0; i < n; i++) {
        uint32_t a = uint32_t(hi[i]) << 16, b = uint32_t(lo[i]) << 16;
        float fa, fb;
        std::memcpy(&fa, &a, 4);
        std::memcpy(&fb, &b, 4);
        o[i] = fa + fb;
      }
      return ARTLITE_OK;
    }
    default: return fail(ARTLITE_EINVAL, "moe layer tap: unknown tap %d", tap);
  }
  if (nbytes < bytes) return fail(ARTLITE_EINVAL, "moe layer tap: %zu bytes, need %zu", nbytes, bytes);
  ART_HIP(hipStreamSynchronize(L->stream));
  if (bytes) ART_HIP(hipMemcpy(out, src, bytes, hipMemcpyDeviceToHost));
  return ARTLITE_OK;
}

extern "C" int artlite_moe_kernel_names(artlite_moe_layer* L, int64_t T, char* buf, size_t cap) {
  if (!L || !buf || !cap) return fail(ARTLITE_EINVAL, "kernel names: null argument");
  std::string s;
  for (const std::string& k : kernel_list(L, T)) s += (s.empty() ? "" : ";") + k;
  const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
  std::memcpy(buf, s.data(), n);
  buf[n] = 0;
  return ARTLITE_OK;
}

extern "C" int artlite_moe_layer_time(artlite_moe_layer** layers, int n, int64_t T, int warmup, int iters,
                                      double* ms_per_run, double* run_ms, double* kernel_ms, int kernel_cap,
                                      int* n_kernels) {
  if (!layers || n < 1 || iters < 1 || warmup < 0 || !ms_per_run) return fail(ARTLITE_EINVAL, "layer time: arguments");
  artlite_moe_layer* L0 = layers[0];
  for (int i = 0; i < n; i++) {
    if (!layers[i]) return fail(ARTLITE_EINVAL, "layer time: null layer");
    if (layers[i]->staged != T) return fail(ARTLITE_EINVAL, "layer time: layer %d has %lld tokens staged", i,
                                            (long long)layers[i]->staged);
    if (layers[i]->stream != L0->stream && layers[i]->device != L0->device)
      return fail(ARTLITE_EINVAL, "layer time: layers on different devices");
    ART_TRY(check_ready(layers[i]));
  }
  // one event per kernel of the first layer's sequence: every layer must run the same sequence
  const std::vector<std::string> names = kernel_list(L0, T);
  for (int i = 1; i < n; i++)
    if (kernel_list(layers[i], T) != names)
      return fail(ARTLITE_EINVAL, "layer time: layer %d runs other kernels than layer 0 for %lld tokens", i,
                  (long long)T);
  // every layer runs on the first layer's stream (one ordered sequence)
  std::vector<hipStream_t> own(n);
  for (int i = 0; i < n; i++) {
    own[i] = layers[i]->stream;
    layers[i]->stream = L0->stream;
  }
  int rc = ARTLITE_OK;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  std::vector<hipEvent_t> ev, er;
  const int nk = int(names.size());
  auto done = [&](int code) {
    for (int i = 0; i < n; i++) layers[i]->stream = own[i];
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    for (hipEvent_t x : ev) (void)hipEventDestroy(x);
    for (hipEvent_t x : er) (void)hipEventDestroy(x);
    return code;
  };
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    return done(fail(ARTLITE_EHIP, "layer time: events"));
  if (run_ms) {  // (an event before each run past the first; e0 and e1 bound the region)
    er.resize(size_t(iters > 1 ? iters - 1 : 0), nullptr);
    for (hipEvent_t& x : er)
      if (hipEventCreate(&x) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: events"));
  }
  hipStream_t s = L0->stream;
  for (int i = 0; i < warmup; i++)
    if ((rc = run(layers[i % n], T, nullptr)) != ARTLITE_OK) return done(rc);
  if (hipStreamSynchronize(s) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: sync"));
  // the runs back to back, an event only before the first and after the last (an event between two runs holds the
  // second back by a few microseconds)
  if (hipEventRecord(e0, s) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: record"));
  for (int i = 0; i < iters; i++)
    if ((rc = run(layers[i % n], T, nullptr)) != ARTLITE_OK) return done(rc);
  if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
    return done(fail(ARTLITE_EHIP, "layer time: record"));
  float ms = 0;
  if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: elapsed"));
  *ms_per_run = double(ms) / iters;
  if (run_ms) {  // (a second region: an event before each run past the first)
    if (hipEventRecord(e0, s) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: record"));
    for (int i = 0; i < iters; i++) {
      if (i > 0 && hipEventRecord(er[size_t(i - 1)], s) != hipSuccess)
        return done(fail(ARTLITE_EHIP, "layer time: record"));
      if ((rc = run(layers[i % n], T, nullptr)) != ARTLITE_OK) return done(rc);
    }
    if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
      return done(fail(ARTLITE_EHIP, "layer time: record"));
  }
  if (run_ms)
    for (int i = 0; i < iters; i++) {
      float t = 0;
      if (hipEventElapsedTime(&t, i ? er[size_t(i - 1)] : e0, i + 1 < iters ? er[size_t(i)] : e1) != hipSuccess)
        return done(fail(ARTLITE_EHIP, "layer time: elapsed"));
      run_ms[i] = t;
    }
  if (n_kernels) *n_kernels = nk;
  if (kernel_ms) {
    // a second timed region with an event before each kernel and after the last
    ev.resize(size_t(iters) * (nk + 1), nullptr);
    for (hipEvent_t& x : ev)
      if (hipEventCreate(&x) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: events"));
    for (int i = 0; i < iters; i++)
      if ((rc = run(layers[i % n], T, ev.data() + size_t(i) * (nk + 1))) != ARTLITE_OK) return done(rc);
    if (hipStreamSynchronize(s) != hipSuccess) return done(fail(ARTLITE_EHIP, "layer time: sync"));
    std::vector<double> sum(nk, 0.0);
    for (int i = 0; i < iters; i++)
      for (int j = 0; j < nk; j++) {
        float t = 0;
        if (hipEventElapsedTime(&t, ev[size_t(i) * (nk + 1) + j], ev[size_t(i) * (nk + 1) + j + 1]) != hipSuccess)
          return done(fail(ARTLITE_EHIP, "layer time: elapsed"));
        sum[j] += t;
      }
    for (int j = 0; j < nk && j < kernel_cap; j++) kernel_ms[j] = sum[j] / iters;
  }
  return done(ARTLITE_OK);
}

