/* artlite_moe: an MI355X (gfx950) HIP library for artlite's mixture-of-experts FFN layer over GGUF-quantized experts.
 *
 * A C ABI of plain pointers and sizes. Every function returns an int status (ARTLITE_OK = 0); on failure the
 * calling thread's message is available from artlite_last_error. Host-pointer entry points copy their inputs to the
 * GPU, compute there, and copy the results back before returning (the caller owns every buffer, as with the
 * reference's _native module). A layer handle owns its device memory and a HIP stream; it is safe for one caller at
 * a time.
 */
#ifndef ARTLITE_MOE_H
#define ARTLITE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum artlite_status {
  ARTLITE_OK = 0,
  ARTLITE_EINVAL = 1, /* an argument or shape error (the reference's artlite::Error) */
  ARTLITE_EHIP = 2,   /* a HIP runtime error, or no GPU */
  ARTLITE_ENOMEM = 3,
};

/* ggml tensor type ids of the supported weight formats (src/artlite/gguf_model.py:385-390 of the reference) */
enum artlite_qtype { ARTLITE_F32 = 0, ARTLITE_F16 = 1, ARTLITE_Q4_0 = 2, ARTLITE_Q4_1 = 3, ARTLITE_Q8_0 = 8,
                     ARTLITE_Q3_K = 11, ARTLITE_Q4_K = 12, ARTLITE_Q5_K = 13, ARTLITE_Q6_K = 14, ARTLITE_IQ4_NL = 20,
                     ARTLITE_IQ4_XS = 23, ARTLITE_BF16 = 30 };

/* The calling thread's last error message into buf (NUL-terminated, truncated to cap); returns its full length. */
size_t artlite_last_error(char* buf, size_t cap);

/* The library's version string. */
const char* artlite_version(void);

/* Number of visible GPUs into *n (0 without a GPU; the call itself succeeds). */
int artlite_device_count(int* n);

/* ---- routing: replaces _native.moe_route (reference csrc/bindings/moe.cpp:20-35 -> artlite::moe_route,
 * csrc/artlite/moe_host.h:9-15). The top k of n tokens' E fp32 logits (token t's at logits[t row ..], expert e at
 * (e / per_col) pitch + e % per_col), largest first, ties to the lower id, -0 as +0; weights e^(l - l_max) over the k
 * in double, normalized in numpy's summation order, rounded to fp32; sigmoid != 0: sigmoid(l) over their sum (at
 * least 2^-14). logits_len: the floats readable at logits (the reference's "arrays too small" check). ids, weights:
 * n x k. Errors: k < 1, k > E, E % per_col != 0, a short array. */
int artlite_moe_route(const float* logits, size_t logits_len, int64_t n, int64_t row, int per_col, int64_t pitch,
                      int E, int k, int sigmoid, int32_t* ids, float* weights);

/* ---- the decode cores' top k: replaces the reference's numpy model route.top_k (src/artlite/moe/route.py:69-80).
 * Plain (n, E) logits; the same ids as artlite_moe_route; weights in float64: the softmax over the k (numpy's
 * summation order) or, sigmoid != 0, the sigmoids over their sum (at least 2^-14). */
int artlite_moe_top_k(const float* logits, int64_t n, int E, int k, int sigmoid, int32_t* ids, double* weights);

/* ---- the chunk plan: replaces _native.moe_plan (reference csrc/bindings/moe.cpp:37-58 -> artlite::moe_plan,
 * csrc/artlite/moe_host.h:17-22), same argument order. ids: n x k; experts, sizes: cols x cap; counts: cols;
 * rows: cols x cap x chunk; pos: n x k. An expert's (token, slot) pairs in pair order, in chunks of at most chunk,
 * dealt to the columns in turn (expert by expert); rows hold tokens (padding: the chunk's first); pos the row
 * (c cap + j) chunk + i of each pair. Errors: an id outside [0, E), more than cap chunks in a column. */
int artlite_moe_plan(const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk, int32_t* experts,
                     int32_t* counts, int32_t* sizes, int32_t* rows, int64_t* pos);

/* ---- the chunk plan without allocating: no counterpart in the reference. For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc): artlite_moe_plan's
 * arguments and results, with every device buffer it needs (the staged ids, the per-block histograms, counters,
 * the results before their copy back) carved from one static 8 MiB array per GPU, held until the process ends, and
 * the null stream. It calls no hipMalloc / hipFree. A call needing more than that array returns ARTLITE_EINVAL
 * (about 250000 pairs at E = 128). Calls share the GPU's array: calls that overlap on one GPU (other threads) race;
 * each call clears the counters it needs. Its host copies and synchronization make it unsuitable under HIP graph
 * capture. */
int artlite_moe_plan_static(const int32_t* ids, int64_t n, int k, int E, int cols, int cap, int chunk,
                            int32_t* experts, int32_t* counts, int32_t* sizes, int32_t* rows, int64_t* pos);

/* ---- dequantization: replaces _native.dequant_supported / dequant_rows (reference csrc/bindings/gguf.cpp:62-76 ->
 * artlite::dequant_rows, csrc/artlite/dequant.h:12-17). n rows of qtype (the reference's native types: "F32", "F16",
 * "BF16", "Q4_0", "Q4_1", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS"), row_bytes apart in raw, into
 * out (n x cols fp32): the reference's fp32 values bit for bit. */
int artlite_dequant_supported(const char* qtype);
int artlite_dequant_rows(const char* qtype, const uint8_t* raw, size_t n, size_t row_bytes, size_t cols, float* out);

/* ---- the MoE layer: the device-resident form of the reference's MoE block (src/artlite/moe/prefill.py:33-214, its
 * semantics tests/moe/ref.py:43-60): router logits (x W^T, float64 accumulation, fp32), routing as
 * artlite_moe_route, the stable dispatch of the (token, slot) pairs by expert, the experts' SwiGLU FFNs over the
 * raw GGUF blocks, the weighted combine in slot order, plus an optional shared expert. */
typedef struct artlite_moe_layer artlite_moe_layer;

typedef struct artlite_moe_desc {
  int32_t hidden;       /* H */
  int32_t n_experts;    /* E */
  int32_t top_k;        /* k */
  int32_t expert_ffn;   /* F */
  int32_t gate_type;    /* artlite_qtype of ffn_gate_exps / ffn_up_exps (any quantized type of the enum) */
  int32_t down_type;    /* artlite_qtype of ffn_down_exps */
  int32_t shared_ffn;   /* the shared expert's width, 0: none */
  int32_t shared_type;  /* artlite_qtype of the shared expert's gate / up (and down, see shared_down_type) */
  int32_t shared_gated; /* 1: the shared expert times sigmoid(x . ffn_gate_inp_shexp) */
  int32_t gating;       /* 0: softmax, 1: sigmoid */
  int32_t max_tokens;   /* the most tokens of one call */
  float norm_eps;       /* > 0: x is first RMS-normalised by ffn_norm, x / sqrt(mean(x^2) + eps) * w (the steps
                           before the block's router: llama.cpp's ffn_norm, the reference's tests/np_ops.py:27-32);
                           0: none */
  int32_t residual;     /* 1: y += x (the block's residual add after the combine, x as given, before any norm) */
  int32_t shared_down_type; /* artlite_qtype of ffn_down_shexp when it differs from shared_type (a GGUF file's
                               mixed quantisation, e.g. Q4_K gate / up with a Q6_K down); 0: shared_type */
} artlite_moe_desc;

/* Tensors of artlite_moe_layer_upload, as laid out in a GGUF file. */
enum artlite_tensor {
  ARTLITE_ROUTER = 0,      /* ffn_gate_inp: E x H fp32 */
  ARTLITE_GATE_EXPS = 1,   /* ffn_gate_exps: E F rows of H values, raw blocks */
  ARTLITE_UP_EXPS = 2,     /* ffn_up_exps */
  ARTLITE_DOWN_EXPS = 3,   /* ffn_down_exps: E H rows of F values */
  ARTLITE_GATE_SHEXP = 4,  /* ffn_gate_shexp: Fs rows of H */
  ARTLITE_UP_SHEXP = 5,
  ARTLITE_DOWN_SHEXP = 6,  /* H rows of Fs */
  ARTLITE_GATE_INP_SHEXP = 7, /* H fp32 */
  ARTLITE_FFN_NORM = 8,    /* ffn_norm: H fp32 (with norm_eps > 0) */
};

/* Activation dtypes. */
enum artlite_dtype { ARTLITE_X_F32 = 0, ARTLITE_X_BF16 = 1 };

int artlite_moe_layer_create(const artlite_moe_desc* desc, artlite_moe_layer** out);
int artlite_moe_layer_destroy(artlite_moe_layer* layer);
/* Copy a tensor's bytes (exactly its size) into the layer's device memory. */
int artlite_moe_layer_upload(artlite_moe_layer* layer, int tensor, const void* data, size_t nbytes);
/* y (T x H fp32, host) = the layer of x (T x H, host, x_dtype); synchronous. */
int artlite_moe_layer_forward(artlite_moe_layer* layer, const void* x, int x_dtype, int64_t T, float* y);

/* Device-resident use: stage x into the layer's device input, then run (enqueued on the layer's stream, returns at
 * once), synchronize, and read y. */
int artlite_moe_layer_stage(artlite_moe_layer* layer, const void* x, int x_dtype, int64_t T);
int artlite_moe_layer_run(artlite_moe_layer* layer, int64_t T);
int artlite_moe_layer_sync(artlite_moe_layer* layer);
int artlite_moe_layer_output(artlite_moe_layer* layer, float* y, int64_t T);

/* Intermediate results of the last run, copied to the host (nbytes: the size of out, at least the tap's). */
enum artlite_tap {
  ARTLITE_TAP_LOGITS = 0,  /* T x E fp32 */
  ARTLITE_TAP_IDS = 1,     /* T x k int32 */
  ARTLITE_TAP_WEIGHTS = 2, /* T x k fp32 */
  ARTLITE_TAP_COUNTS = 3,  /* E int32: pairs per expert */
  ARTLITE_TAP_OFFSETS = 4, /* E + 1 int32: exclusive prefix of counts */
  ARTLITE_TAP_ORDER = 5,   /* T k int32: pair indices t k + i sorted by expert, pair order within an expert */
  ARTLITE_TAP_SLOT = 6,    /* T k int32: each pair's position in that order */
  ARTLITE_TAP_H = 7,       /* T k x F fp32: silu(gate) up of each sorted pair (as the run's path holds it) */
  ARTLITE_TAP_Y = 8,       /* T k x H fp32: each sorted pair's expert output (before the weights) */
  ARTLITE_TAP_XN = 9,      /* T x H fp32: the RMS-normalised x (norm_eps > 0) */
  ARTLITE_TAP_YS = 10,     /* T x H fp32: the shared expert's output, before its gate (shared_ffn > 0) */
};
int artlite_moe_layer_tap(artlite_moe_layer* layer, int tap, void* out, size_t nbytes);

/* Timing on the layers' stream with HIP events: warmup then iters runs of T tokens, cycling through the n layers
 * (distinct weight sets, so a working set larger than the GPU's caches is streamed from HBM). ms_per_run: the
 * average over a timed region of back-to-back runs (events only at its ends). run_ms (may be NULL; iters entries):
 * each run's duration, from an event recorded before each run of a second region (those events hold each run back
 * by a few microseconds). kernel_ms (may be NULL): with per-kernel events in a further timed region, each kernel's
 * average duration (artlite_moe_kernel_names order), kernel_cap entries at most; *n_kernels the count. */
int artlite_moe_layer_time(artlite_moe_layer** layers, int n, int64_t T, int warmup, int iters, double* ms_per_run,
                           double* run_ms, double* kernel_ms, int kernel_cap, int* n_kernels);
/* The names of the kernels of a run of T tokens on this layer, ';'-separated, into buf. */
int artlite_moe_kernel_names(artlite_moe_layer* layer, int64_t T, char* buf, size_t cap);

/* Bytes copied per ms by a plain device copy of nbytes (HBM calibration of the profile counters). */
int artlite_hbm_copy(size_t nbytes, int iters, double* ms_per_copy);

#ifdef __cplusplus
}
#endif

#endif /* ARTLITE_MOE_H */
