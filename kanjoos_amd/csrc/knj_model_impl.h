// kanjoos_amd/csrc/knj_model_impl.h -- the device model object behind the
// knj_model_* C ABI, shared by the single-sequence step (knj_model.hip) and the
// batched decode step (knj_batch.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/knj_capi.h"
#include "knj_common.h"

// Buffers of the prompt pass (knj::prefill), allocated on its first use for
// chunks of up to `cap` rows.
struct knj_prefill_bufs {
  int cap = 0;
  float *x = nullptr, *hx = nullptr, *qkv = nullptr, *ctx = nullptr;
  float *router_logits = nullptr, *topk_w = nullptr;
  int32_t *topk_idx = nullptr, *tokens = nullptr;
  float* attn_part = nullptr;  // split-KV partials of the prompt-pass attention
  void* scratch = nullptr;
  _Float16* qsplit[4] = {};  // the attn-normalised rows in the QKV product's operand layout
};

struct knj_model {
  knj_model_config c{};
  uint8_t* image = nullptr;
  uint64_t image_bytes = 0;
  std::vector<knj_layer_offsets> lo;
  uint64_t off_embd = 0, off_onorm = 0, off_head = 0;
  hipStream_t stream = nullptr;
  // activations
  float *x = nullptr, *qkv = nullptr, *ctx = nullptr, *hx = nullptr, *act = nullptr;
  // with the router folded into the attention-output launch: that launch's
  // output (the residual stream between attn-o and the MoE), and per layer
  // the folded router rows [n_expert][n_embd + n_head * head_dim]
  float *x2 = nullptr, *router_fold = nullptr;
  bool fold_router = false;
  float *logits = nullptr, *router_logits = nullptr, *hidden = nullptr, *topk_w = nullptr;
  int32_t* topk_idx = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr, *rope_cur = nullptr, *attn_part = nullptr;
  uint16_t *kv_k = nullptr, *kv_v = nullptr;
  knj::StepState* st = nullptr;
  int32_t* out_tokens = nullptr;
  unsigned long long* keys = nullptr;  // LM-head per-workgroup argmax keys
  int max_steps = 0;
  unsigned int* counter = nullptr;
  int pos = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // several decode steps captured back to back (decode loops replay it while
  // at least that many steps remain)
  hipGraph_t graph_multi = nullptr;
  hipGraphExec_t exec_multi = nullptr;
  int multi = 0;
  bool use_graph = true;  // KNJ_NO_GRAPH=1 launches the step's kernels directly
  // prompt pass over several rows at once (KNJ_PROMPT_STEPS=1 feeds prompts
  // one decode step per token instead)
  knj_prefill_bufs pf;
  hipEvent_t* expert_events = nullptr;  // set by knj_model_time_experts: 6 per layer per step
  int expert_slot = 0;
  // host<->device bytes copied by this model's calls (the profiler's transfer row)
  mutable uint64_t h2d_bytes = 0, d2h_bytes = 0;
  std::vector<void*> owned;
};

namespace knj {
// A profiling run: installs a SpanSink (knj_spans.h) of `cap` event pairs on
// the calling thread until stop() or destruction; `epoch` is recorded by the
// caller on the step's stream before the first launch.
struct SpanRun {
  explicit SpanRun(int cap);
  ~SpanRun();
  SpanRun(const SpanRun&) = delete;
  SpanRun& operator=(const SpanRun&) = delete;
  void stop();
  int collect(knj_span* out, int cap, int* n_out, uint64_t* dropped);
  SpanSink sink;
  std::vector<hipEvent_t> events;
  hipEvent_t epoch = nullptr;
  hipError_t err = hipSuccess;
};

// Model::forward over n > 1 tokens as one pass (knj_prefill.hip): every
// weight applied to up to 512 rows at once, causal attention over the cache,
// the last row's hidden states, router choices and logits kept.  `eligible`
// says whether the model's tensor types and shape allow it.
bool prefill_eligible(const knj_model* m);
int prefill(knj_model* m, const int32_t* tokens, int n);

// Slots [0, n_elems / D) of `rows` cache rows of row_elems elements: seeded f16
// values ~N(0, 1) (k_fill_kv).
int fill_kv_rows(uint16_t* k, uint16_t* v, uint64_t rows, uint64_t row_elems, uint64_t n_elems,
                 uint64_t seed, hipStream_t s);
}  // namespace knj
