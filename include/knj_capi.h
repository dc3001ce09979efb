/* include/knj_capi.h -- C ABI of the MI355X (gfx950) MoE decode library.
 *
 * Plain C: pointers, sizes, ints.  Device pointers are addresses in the GPU's
 * memory (from knj_malloc, or any HIP allocation); `stream` is a hipStream_t
 * passed as void* (NULL = the default stream).  Every function returns 0 on
 * success or one of the KNJ_E_* codes below, with a message in knj_last_error().
 *
 * The status codes keep the reference's driver exit codes
 * (/root/reference/tools/bench/q4k_moe_ffn.hip:63, tests/test_gemm_w4.hip:11-19):
 * 5 correctness, 6 arch mismatch, 7 environment, 9 HIP error.
 */
#ifndef KNJ_CAPI_H
#define KNJ_CAPI_H

#include <stdint.h>

#include "knj_model.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KNJ_OK 0
#define KNJ_E_CORRECTNESS 5
#define KNJ_E_ARCH 6
#define KNJ_E_ENV 7
#define KNJ_E_HIP 9
#define KNJ_E_ARG 22
#define KNJ_E_STATE 23

/* ------------------------------------------------------------ device gate
 * Replaces the reference's C2 gate: Backend::create's arch guard and
 * DeviceCaps probe (/root/reference/src/device/backend.cpp:54-62,
 * src/device/device_caps.h:69-157).  The guard compares the device's
 * gcnArchName up to the first ':' with the arch this library was compiled for
 * ("gfx950"); if KNJ_BUILD_ARCH is set in the environment it must name the same
 * arch.  Refusals return KNJ_E_ARCH (mismatch) and leave the device untouched. */
typedef struct knj_device_caps {
  char gcn_arch[32];      /* e.g. "gfx950" (the part before ':') */
  char name[64];
  int32_t wave_size;      /* 64 on CDNA */
  int32_t cu_count;
  int32_t clock_khz;
  int32_t lds_per_block;  /* bytes */
  int32_t l2_bytes;
  int32_t arch_ok;
  int32_t has_mfma_bf16;
  int32_t has_mfma_i8;
  int32_t has_fp8;
  uint64_t vram_total;
  uint64_t vram_free;
} knj_device_caps;

int knj_device_open(int device);
int knj_device_close(void);
int knj_device_caps_get(knj_device_caps* out);
/* Arch guard alone, on strings (host-testable without a GPU): 0 when
 * `device_arch` (full gcnArchName) matches `built_arch` and `env_arch` (may be
 * NULL) agrees, else KNJ_E_ARCH. */
int knj_check_arch(const char* device_arch, const char* built_arch, const char* env_arch);
const char* knj_built_arch(void);
const char* knj_last_error(void);

/* ------------------------------------------------------------ memory */
int knj_malloc(void** dptr, uint64_t bytes);
int knj_free(void* dptr);
int knj_memcpy_h2d(void* dst, const void* src, uint64_t bytes);
int knj_memcpy_d2h(void* dst, const void* src, uint64_t bytes);
int knj_memset_zero(void* dst, uint64_t bytes);
int knj_synchronize(void);

/* ------------------------------------------------------------ format / GEMV
 * knj_dequant: n_weights of `type` at w -> f32, bit-exact with
 *   dequant_row_f32 (/root/reference/src/loader/dequant.cpp:1114-1256).
 * knj_gemv: y[j] = sum_i W[j][i] x[i] for the n_out rows of W, the device
 *   counterpart of Model::matmul at m == 1 (/root/reference/src/model/model.cpp:
 *   326-380) and dequant_dot_f32 (dequant.cpp:1075-1112).  `norm_w` (optional)
 *   applies RMSNorm(x, norm_w, eps) to x first (model.cpp:240-271); `resid`
 *   (optional) makes y = resid + W x (the residual adds at model.cpp:624, 652).
 *   Types: Q4_K, Q6_K (rows of n_in/256 blocks), BF16, F32. */
int knj_dequant(int type, const void* w, uint64_t n_weights, float* out, void* stream);
int knj_gemv(int type, const void* w, int n_in, int n_out, const float* x, const float* norm_w,
             float eps, const float* resid, float* y, void* stream);
int knj_rmsnorm(const float* x, const float* w, int n, float eps, float* out, void* stream);

/* ------------------------------------------------------------ MoE (config 1)
 * knj_moe_router: logits = router_w . RMSNorm(x) (norm skipped when norm_w is
 *   NULL), softmax over all experts, top-k by repeated argmax with ties to the
 *   lower index, weights renormalised over the kept k (model.cpp:420-460).
 *   hx receives the normalised input.  topk in selection order.
 * knj_moe_decode_layer: the whole batch-1 MoE FFN: router as above, then for the
 *   k chosen experts gate/up GEMV, silu(gate)*up, down GEMV, and
 *   out = resid + sum_e w_e * down_e, summed in ascending expert index
 *   (model.cpp:462-509, the moe-router/gate/up/act/down/scatter stages).
 *   `resid` may be NULL (out is then the expert branch alone). */
int knj_moe_router(const float* x, const float* norm_w, float eps, const float* router_w,
                   int n_embd, int n_expert, int k, float* hx, float* logits, int32_t* topk_idx,
                   float* topk_w, void* stream);
int knj_moe_decode_layer(const float* x, const float* norm_w, float eps, const float* router_w,
                         const void* gate, const void* up, const void* down, int type_gate_up,
                         int type_down, int n_embd, int n_ff, int n_expert, int k,
                         const float* resid, float* out, float* logits, int32_t* topk_idx,
                         float* topk_w, void* stream);
/* knj_moe_decode_layer_noalloc: knj_moe_decode_layer computed by the same
 *   kernels, with its scratch (hx, then act: n_embd + k * n_ff floats) in a
 *   fixed device array of 32768 floats (128 KiB per device, held until the
 *   process ends) instead of library-allocated memory: the call allocates and
 *   frees nothing.  No counterpart in the reference; it is for callers that
 *   cannot allocate (code under HIP graph capture, tight serving loops,
 *   harnesses that forbid hipMalloc).  Larger shapes return KNJ_E_ARG.  Every
 *   call on a device shares that device's array, so calls that overlap on one
 *   device (other streams, other threads) race; nothing in the array needs to
 *   start at zero.  The device must have been opened with knj_device_open. */
int knj_moe_decode_layer_noalloc(const float* x, const float* norm_w, float eps,
                                 const float* router_w, const void* gate, const void* up,
                                 const void* down, int type_gate_up, int type_down, int n_embd,
                                 int n_ff, int n_expert, int k, const float* resid, float* out,
                                 float* logits, int32_t* topk_idx, float* topk_w, void* stream);

/* ------------------------------------------------------------ MoE over many tokens (config 2)
 * knj_moe_batch_layer: Model::moe on n_tokens rows at once (model.cpp:399-510
 *   with m > 1, the batched matmul of :354-364): per token RMSNorm(x) (norm
 *   skipped when norm_w is NULL), router logits, softmax and top-k as in
 *   knj_moe_router; the (token, expert) pairs grouped by expert so every
 *   expert's weights are read once for all its tokens; gate/up, silu(gate)*up,
 *   down; out[t] = resid[t] + sum over t's experts in ascending index of
 *   w * down.  x, resid, out: [n_tokens][n_embd]; logits: [n_tokens][n_expert];
 *   topk_idx/topk_w: [n_tokens][k].  Q4_K gate/up, Q4_K or Q6_K down; n_embd
 *   and n_ff multiples of 256, at most 4096; n_expert <= 256; k <= 16. */
int knj_moe_batch_layer(const float* x, const float* norm_w, float eps, const float* router_w,
                        const void* gate, const void* up, const void* down, int type_gate_up,
                        int type_down, int n_tokens, int n_embd, int n_ff, int n_expert, int k,
                        const float* resid, float* out, float* logits, int32_t* topk_idx,
                        float* topk_w, void* stream);

/* ------------------------------------------------------------ attention
 * knj_attention_step: the attention block of one decode token
 *   (/root/reference/src/model/model.cpp:567-616 with an f16 cache): per-head
 *   RMSNorm of the raw projections q [n_head][D] and k [n_head_kv][D] with
 *   q_norm / k_norm, NEOX RoPE at `pos` (pairs (i, i+D/2),
 *   theta = pos*base^(-2i/D)), k and v rounded to f16 and stored at slot `pos`
 *   of the [n_head_kv][n_ctx][D] caches, then GQA attention of every query head
 *   over slots [0, pos]: scores q.k/sqrt(D), softmax, out = sum a*v.
 *   q, k, v are not modified.  D is 64 or 128; the GQA group is at most 8. */
int knj_attention_step(const float* q, const float* k, const float* v, const float* q_norm,
                       const float* k_norm, float eps, float rope_base, int pos, int n_head,
                       int n_head_kv, int head_dim, int n_ctx, uint16_t* k_cache, uint16_t* v_cache,
                       float* out, void* stream);

/* ------------------------------------------------------------ model step
 * The device counterpart of knj::Model (/root/reference/src/model/model.h:55-80):
 * open -> forward(tokens, n) -> logits of the last token, reset(), pos().
 * Weights live in one device image laid out per include/knj_model.h.
 * knj_model_create_synthetic generates the seeded synthetic weights on the GPU
 * (include/knj_synth.h, bit-identical to the host generator);
 * knj_model_create_from_image uploads a host image. */
typedef struct knj_model knj_model;
int knj_model_create_synthetic(const knj_model_config* cfg, uint64_t seed, knj_model** out);
int knj_model_create_from_image(const knj_model_config* cfg, const void* image, uint64_t bytes,
                                knj_model** out);
/* A qwen3moe GGUF file (the reference's Model::open, model.cpp:174-232, and its
 * geometry/tensor checks, :97-172): knj_gguf_probe reads the geometry and the
 * weight types into `out` without a device; knj_model_create_from_gguf also
 * copies every tensor into a device model (Q, K and V rows into one wqkv).
 * Errors: a missing key or tensor, a wrong shape, an unsupported type, n_ctx
 * beyond the trained context -- each with its name in knj_last_error(). */
int knj_gguf_probe(const char* path, int n_ctx, knj_model_config* out);
int knj_model_create_from_gguf(const char* path, int n_ctx, knj_model** out);
int knj_model_config_get(const knj_model* m, knj_model_config* out);
int knj_model_free(knj_model* m);
uint64_t knj_model_image_bytes(const knj_model* m);
const void* knj_model_image_device(const knj_model* m);
/* Fills cache slots [0, n_pos) of every layer with seeded f16 values ~N(0,1)
 * and sets the position to n_pos: a long context without running its prefill
 * (for throughput runs; the decode step's work is the same). */
int knj_model_fill_kv(knj_model* m, int n_pos, uint64_t seed);
/* ------------------------------------------------------------ batched decode (config 4)
 * A knj_batch decodes n_seq sequences in lockstep on one model's weights (the
 * model must outlive it): one step is Model::forward's per-token work
 * (model.cpp:512-672) for n_seq tokens at once, each sequence with its own f16
 * KV cache of n_ctx slots (n_ctx <= the model's) and its own position.  Every
 * weight matrix is read once per step for all sequences (matrix-core GEMMs;
 * the MoE pairs grouped by expert).  Q4_K attention and gate/up, Q4_K or Q6_K
 * expert down, bf16 or Q6_K head.
 * knj_batch_forward: one step on tokens[n_seq]; logits_out [n_seq][n_vocab]
 *   (may be NULL).  knj_batch_decode_greedy: `steps` greedy steps from
 *   first[n_seq]; out_tokens [steps][n_seq].  Hidden states, top-k and caches
 *   of the last step per sequence as for knj_model_*.  No counterpart in the
 *   reference, which decodes one sequence. */
typedef struct knj_batch knj_batch;
int knj_batch_create(knj_model* m, int n_seq, int n_ctx, knj_batch** out);
int knj_batch_free(knj_batch* b);
int knj_batch_pos(const knj_batch* b);
int knj_batch_forward(knj_batch* b, const int32_t* tokens, float* logits_out);
int knj_batch_decode_greedy(knj_batch* b, const int32_t* first, int steps, int32_t* out_tokens);
int knj_batch_fill_kv(knj_batch* b, int n_pos, uint64_t seed);
int knj_batch_hidden(const knj_batch* b, int il, int seq, float* out);
int knj_batch_topk(const knj_batch* b, int il, int seq, int32_t* idx, float* w);
int knj_batch_kv_download(const knj_batch* b, int seq, uint16_t* k, uint16_t* v);
/* One sequence's whole cache ([n_layer][n_head_kv][n_ctx][head_dim] f16, the
 * batch's n_ctx) from the host, e.g. a cache a knj_model prompt pass wrote; and
 * the lockstep position of every sequence. */
int knj_batch_kv_upload(knj_batch* b, int seq, const uint16_t* k, const uint16_t* v);
int knj_batch_set_pos(knj_batch* b, int pos);

/* Byte offsets of layer `il`'s tensors inside the weight image of a model of
 * configuration `c` (the layout of knj_model.h); returns the image size, 0 on a
 * bad argument. */
uint64_t knj_model_layer_offsets(const knj_model_config* c, int il, knj_layer_offsets* out);
int knj_model_download_image(const knj_model* m, void* host, uint64_t bytes);
int knj_model_reset(knj_model* m);
int knj_model_pos(const knj_model* m);
int knj_model_set_pos(knj_model* m, int pos);
/* Model::forward (/root/reference/src/model/model.cpp:512-672): runs n tokens at
 * positions pos .. pos+n-1.  n == 1 is one decode step (the captured graph);
 * n > 1 is the prompt pass: every weight applied to up to 512 rows at once,
 * each row's key and value appended, causal attention (row t over slots
 * 0 .. pos+t), the head on the last row -- for Q4_K attention and gate/up
 * and Q4_K or Q6_K expert down (other tensor types take one decode step per
 * token).  logits_host (n_vocab
 * floats, may be NULL) receives the last token's logits; the per-layer
 * hidden/top-k queries then describe the last token.  Errors: KNJ_E_ARG for
 * token ids out of range or a full context (model.cpp:514-517, 533), nothing
 * run. */
int knj_model_forward(knj_model* m, const int32_t* tokens, int n, float* logits_host);
/* Greedy decode entirely on the device: feeds `first`, then `steps` argmax
 * tokens (first maximum wins, /root/reference/src/cli/main.cpp:126-132) into
 * out_tokens.  Replays one captured HIP graph per step. */
int knj_model_decode_greedy(knj_model* m, int32_t first, int steps, int32_t* out_tokens);
/* Diagnostics of the most recent step: residual stream after layer il
 * (model.cpp:654-658), router choice of layer il, last logits, KV caches. */
int knj_model_hidden(const knj_model* m, int il, float* host_out);
int knj_model_topk(const knj_model* m, int il, int32_t* idx_out, float* w_out);
int knj_model_logits(const knj_model* m, float* host_out);
int knj_model_kv_download(const knj_model* m, uint16_t* k_host, uint16_t* v_host);
int knj_model_kv_upload(knj_model* m, const uint16_t* k_host, const uint16_t* v_host);
/* Times `iters` greedy steps with HIP events on the model's stream (graph
 * replays), returns total milliseconds. */
int knj_model_time_decode(knj_model* m, int iters, float* ms_out);
/* Times the expert GEMV kernels inside real decode steps: `steps` (1..64)
 * greedy tokens from token 0 at the current position, the step's kernels
 * launched directly (no graph); every layer's gate/up and down launch records
 * HIP start/end events of its own execution (hipExtLaunchKernel) on the
 * model's stream, and so does the router launch before them (unused: a launch
 * timed right after one without events reads the earlier launch's drain as
 * its own).  Returns the mean
 * microseconds per launch of each over n_layer * steps launches; advances the
 * position by `steps`. */
int knj_model_time_experts(knj_model* m, int steps, float* us_gateup, float* us_down);

/* ---- device spans for the profiler -------------------------------------------
 * The device event backend of the reference's profiler
 * (/root/reference/src/profiler/profiler.h:98-139: device_span() takes offsets
 * from one epoch event per stream, set_device_floor() a floor measured through
 * the same event path, set_device_dropped() the spans a full ring lost).  One
 * record per kernel launch: the op class it belongs to (the reference's scope
 * names where one kernel does one op -- "embed", "qkv", "attention", "attn-o",
 * "moe-router", "head" -- and joined names for fused kernels:
 * "moe-gate+up+act", "moe-down+scatter", "sample"), the layer (-1 outside the
 * layers), the kernel symbol, and the dispatch's own start/end in nanoseconds
 * after the epoch event. */
typedef struct knj_span {
  char name[32];
  char kernel[40];
  int32_t layer;
  int32_t stream;
  uint64_t start_ns;
  uint64_t end_ns;
} knj_span;

/* Greedy decode exactly as knj_model_decode_greedy (same tokens, same KV
 * writes, position advanced by `steps`), but with the step's kernels launched
 * directly, each with dispatch-recorded start/end events.  Up to `cap` spans
 * are written; *n_dropped counts launches beyond `cap` (a stated loss).
 * cap <= 1 << 20. */
int knj_model_profile(knj_model* m, int32_t first, int steps, int32_t* out_tokens, knj_span* spans,
                      int cap, int* n_spans, uint64_t* n_dropped);

/* Host<->device bytes this model's calls have copied since it was created
 * (weight upload, per-step token state, logits/tokens/diagnostic downloads):
 * the profiler's transfer row. */
int knj_model_transfer_bytes(const knj_model* m, uint64_t* h2d, uint64_t* d2h);

/* The device instrumentation floor: `n` empty kernels (one wave each, after
 * untimed warm-up launches) timed through the same dispatch-event path;
 * *ns_out is their median span. */
int knj_device_floor(int n, uint64_t* ns_out);

#ifdef __cplusplus
}
#endif

#endif /* KNJ_CAPI_H */
