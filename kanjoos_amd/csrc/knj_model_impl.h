// kanjoos_amd/csrc/knj_model_impl.h -- the device model object behind the
// knj_model_* C ABI, shared by the single-sequence step (knj_model.hip) and the
// batched decode step (knj_batch.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/knj_capi.h"
#include "knj_common.h"

struct knj_model {
  knj_model_config c{};
  uint8_t* image = nullptr;
  uint64_t image_bytes = 0;
  std::vector<knj_layer_offsets> lo;
  uint64_t off_embd = 0, off_onorm = 0, off_head = 0;
  hipStream_t stream = nullptr;
  // activations
  float *x = nullptr, *qkv = nullptr, *ctx = nullptr, *hx = nullptr, *act = nullptr;
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
  bool use_graph = true;  // KNJ_NO_GRAPH=1 launches the step's kernels directly
  hipEvent_t* expert_events = nullptr;  // set by knj_model_time_experts: 4 per layer per step
  int expert_slot = 0;
  std::vector<void*> owned;
};

namespace knj {
// Slots [0, n_elems / D) of `rows` cache rows of row_elems elements: seeded f16
// values ~N(0, 1) (k_fill_kv).
int fill_kv_rows(uint16_t* k, uint16_t* v, uint64_t rows, uint64_t row_elems, uint64_t n_elems,
                 uint64_t seed, hipStream_t s);
}  // namespace knj
