// kanjoos_amd/csrc/knj_common.h -- internal helpers shared by the HIP sources.
#pragma once

#include <hip/hip_runtime.h>

#include "knj_spans.h"

#include <cstdint>
#include <string>

#include "../../include/knj_capi.h"
#include "../../include/knj_format.h"

namespace knj {

// Last error text for knj_last_error(); thread-local so callers on different
// threads do not see each other's messages.
void set_error(const std::string& msg);

// Returns KNJ_E_HIP and records the HIP error text when `e` is not hipSuccess.
int hip_fail(hipError_t e, const char* what);

#define KNJ_HIP(call)                                   \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return knj::hip_fail(e_, #call); \
  } while (0)

#define KNJ_CHECK_ARG(cond, msg)        \
  do {                                  \
    if (!(cond)) {                      \
      knj::set_error(msg);              \
      return KNJ_E_ARG;                 \
    }                                   \
  } while (0)

// Refuses launches before knj_device_open() has passed the arch guard.
int require_open();

// Per-device scratch owned by the library (partials, counters); grown on
// demand, never shrunk, released at knj_device_close().
void* device_scratch(uint64_t bytes, hipStream_t stream);

// 1024 zero-initialised device counters (tickets of last-workgroup-done
// reductions); every kernel that takes one returns it to zero before exiting.
unsigned int* device_counters();

// ---------------------------------------------------------------- kernels
// Launchers return hipError_t of the launch; shapes are validated by callers.
struct GemvArgs {
  int type;                 // KNJ_TYPE_Q4_K / Q6_K / BF16 / F32
  const uint8_t* w;         // n_out rows of n_in weights
  int n_in, n_out;
  const float* x;           // input vector (n_in)
  const float* norm_w;      // optional: RMSNorm weight applied to x first
  float eps;
  const float* resid;       // optional: y = resid + W x
  float* y;                 // output (n_out)
  unsigned long long* argmax_key;  // optional: per-workgroup packed (value, index)
                                   // maxima of y, at most kMaxKeys slots
};
constexpr int kMaxKeys = 4096;
hipError_t launch_gemv(const GemvArgs& a, hipStream_t s);
// The attention-output GEMV (Q4_K, y = resid + W x, one row step per wave)
// with the router's unscaled logits u[e] = R[e] . [resid ; x] in the same
// launch (k_gemv_q4k_router); R [n_router][n_out + n_in] from
// launch_router_fold.  router_fold_ok says whether a shape can take it.
bool router_fold_ok(int type_o, int n_in, int n_out, int n_router);
hipError_t launch_gemv_router(const GemvArgs& a, const float* R, int n_router, float* u,
                              hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
hipError_t launch_router_fold(const float* wr, const float* nw, const float* wd, int H, int QD,
                              int E, float* R, hipStream_t s);

hipError_t launch_dequant(int type, const uint8_t* w, uint64_t n, float* out, hipStream_t s);

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* out, hipStream_t s);

struct RouterArgs {
  const float* x;         // residual stream (n_embd)
  const float* norm_w;    // optional RMSNorm weight (ffn_norm)
  float eps;
  const float* router_w;  // [n_expert][n_embd] f32
  int n_embd, n_expert, k;
  float* hx;              // normalised x written for the expert kernels
  float* logits;          // [n_expert]
  int32_t* topk_idx;      // [k], selection order (null: logits only)
  float* topk_w;          // [k]
  unsigned int* counter;  // zero-initialised ticket, left at zero on exit
};
// t0/t1 as for the expert launches below (timing runs only)
hipError_t launch_router(const RouterArgs& a, hipStream_t s, hipEvent_t t0 = nullptr,
                         hipEvent_t t1 = nullptr);
// Softmax + top-k of n_expert logits by one workgroup (the C-ABI router).
hipError_t launch_topk(const float* logits, int n_expert, int k, int32_t* idx, float* w,
                       hipStream_t s);

struct ExpertArgs {
  const float* hx;        // [n_embd] input of gate/up: RMSNorm(hx, norm_w) when norm_w is
  const float* norm_w;    // set (the residual stream and ffn_norm), else used as is
  float eps;
  const float* logits;    // router logits [n_expert]: when set, gate/up routes itself
                          // (softmax + top-k in every wave) and writes topk_idx/topk_w
  int32_t* topk_idx;      // routing [k], selection order (input when logits is null)
  float* topk_w;
  const uint8_t* gate;    // [n_expert] slabs
  const uint8_t* up;
  const uint8_t* down;
  int type_gate_up, type_down;
  int n_embd, n_ff, n_expert, k;
  float* act;             // [k][n_ff] scratch
  const float* resid;     // optional residual added to the output
  float* out;             // [n_embd]
  float* hidden_copy;     // optional second destination of out
  // logits are W_r' applied to the un-normalised rows (launch_gemv_router):
  // the routed gate/up scales them by 1 / sqrt(mean(hx^2) + eps) first
  bool logits_unscaled = false;
};
hipError_t launch_experts(const ExpertArgs& a, hipStream_t s);
hipError_t expert_kernel_attributes();
// t0/t1, when set, are recorded by the kernel dispatch itself at its start and
// end (hipExtLaunchKernel): the launch's execution time, as a profiler sees it.
hipError_t launch_expert_gateup(const ExpertArgs& a, hipStream_t s, hipEvent_t t0 = nullptr,
                                hipEvent_t t1 = nullptr);
hipError_t launch_expert_down(const ExpertArgs& a, hipStream_t s, hipEvent_t t0 = nullptr,
                              hipEvent_t t1 = nullptr);

// MoE layer over m tokens at once (prefill chunks, batched decode): RMSNorm,
// router, per-token top-k, experts grouped on the matrix cores, combine.
// Q4_K gate/up, Q4_K or Q6_K down, n_embd and n_ff multiples of 256 and <= 4096,
// n_expert <= 256, k <= 16.
struct MoeBatchArgs {
  const float* x;          // [m][n_embd] residual stream
  const float* norm_w;     // ffn_norm (null: x is used as is)
  float eps;
  const float* router_w;   // [n_expert][n_embd] f32
  const uint8_t* gate;     // [n_expert] slabs
  const uint8_t* up;
  const uint8_t* down;
  int m, n_embd, n_ff, n_expert, k;
  const float* resid;      // optional [m][n_embd] added to the output
  float* out;              // [m][n_embd]
  float* logits;           // [m][n_expert]
  int32_t* topk_idx;       // [m][k], selection order
  float* topk_w;           // [m][k]
  float* hidden_copy = nullptr;  // optional second destination of out
  int type_down = KNJ_TYPE_Q4_K;  // Q4_K or Q6_K
  // Optional, the next step's input from the combine's rows: out RMS-normalised
  // with next_norm_w into next_hx (f32, may be
  // null) and/or next_split (k_split_tile's layout: hi, lo, sums hi, sums lo)
  const float* next_norm_w = nullptr;
  float next_eps = 1e-6f;
  float* next_hx = nullptr;
  _Float16* const* next_split = nullptr;
};
uint64_t moe_batch_scratch_bytes(int m, int n_embd, int n_ff, int n_expert, int k);
hipError_t launch_moe_batch(const MoeBatchArgs& a, void* scratch, hipStream_t s);
// Rows of x RMS-normalised with nw into hx (may be null) and/or split (k_split_tile's
// layout); n <= 4096, n % 256 == 0.
hipError_t launch_norm_split(const float* x, const float* nw, float eps, int m, int n, float* hx,
                             _Float16* const* split, hipStream_t s);

// Dense GEMMs over m rows at once (the batched decode step), on the matrix
// cores with split-f16 (Q4_K) or split-bf16 (bf16 weights) activations:
// out[r] (+= resid[r]) = W x_r.  Scratch: dense_scratch_bytes(m, n_in, n_out)
// (Q4_K; the split-f16 operands and, when the reduction is split over several
// workgroups, their partial products), dense_scratch_bytes(m, n_in, 0) for bf16.
uint64_t dense_scratch_bytes(int m, int n_in, int n_out);
hipError_t launch_norm_rows(const float* x, const float* nw, float eps, int m, int n, float* out,
                            hipStream_t s);
hipError_t launch_dense_q4k(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                            const float* resid, float* out, void* scratch, hipStream_t s);
// The same with two fusions a batched layer step uses: `pre` (hi, lo, sums hi,
// sums lo in k_split_tile's layout, or null) is the activation operand already
// split, so x is not read; with `norm_w`, the rows of out are also written
// RMS-normalised with norm_w into norm_out (the next product's input), by the
// launch that adds the reduction ranges when there is one.
struct DenseQ4Extra {
  const _Float16* const* pre = nullptr;  // [4]
  const float* norm_w = nullptr;
  float eps = 1e-6f;
  float* norm_out = nullptr;
};
hipError_t launch_dense_q4k_ex(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                               const float* resid, float* out, void* scratch,
                               const DenseQ4Extra& ex, hipStream_t s);
// Bytes of the split operand of m rows of n floats (k_split_tile's layout:
// hi, lo, sums hi, sums lo, each 256-byte aligned).
uint64_t split_operand_bytes(int m, int n);
hipError_t launch_dense_bf16(const uint16_t* w, int n_in, int n_out, int m, const float* x,
                             float* out, void* scratch, hipStream_t s);
// Q6_K (no residual, no reduction split): scratch dense_scratch_bytes(m, n_in, 0).
hipError_t launch_dense_q6k(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                            float* out, void* scratch, hipStream_t s);
// Greedy token of every row of logits [m][n]; keys: m * argmax_key_count(n) scratch.
int argmax_key_count(int n);
hipError_t launch_argmax_rows(const float* logits, int m, int n, unsigned long long* keys,
                              int32_t* tok, hipStream_t s);

// Fused decode attention of one token (QK-norm, RoPE, f16 append, split-KV
// attention, merge).  q/k/v are the raw projections of this token.
struct AttnArgs {
  const float* q;            // [n_head][D]
  const float* k;            // [n_head_kv][D]
  const float* v;            // [n_head_kv][D]
  const float* q_norm;       // [D]
  const float* k_norm;       // [D]
  float eps;
  const float* rope_cos;     // [D/2] cos of this token's position
  const float* rope_sin;     // [D/2] sin
  const int* pos;            // device position of this token (its cache slot)
  uint16_t* k_cache;         // [n_head_kv][n_ctx][D] of this layer
  uint16_t* v_cache;
  int n_head, n_head_kv, head_dim, n_ctx;
  float scale;
  float* partial;            // [n_seq][n_head][n_split][D + 2] scratch
  float* out;                // [n_head][D]
  // Several sequences in one launch (grid z = sequence): sequence s reads
  // q/k/v + s * qkv_stride, rope rows + s * rope_stride, its position pos[s],
  // the caches + s * kv_stride, and writes out + s * out_stride.
  int n_seq = 1;
  uint64_t qkv_stride = 0, kv_stride = 0, out_stride = 0;
  int rope_stride = 0;
  // With several sequences: the output also (split_hi set) in k_split_tile's
  // layout over the n_seq rows of n_head * D columns (hi, lo, sums hi, sums
  // lo), the next product's operand
  _Float16 *split_hi = nullptr, *split_lo = nullptr, *split_shi = nullptr, *split_slo = nullptr;
};
int attn_splits(int n_ctx);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

// Attention of a prompt chunk (Model::forward with n > 1,
// /root/reference/src/model/model.cpp:560-616): rows t < n_rows at positions
// pos0 + t.  The first launch normalises and rotates every row's query (in
// place) and key, and appends every row's key and value to the cache; the
// second gives row t attention over slots 0 .. pos0 + t.  qkv rows are
// [q | k | v] of qkv_stride floats; out rows are n_head * head_dim floats.
struct PrefillAttnArgs {
  float* qkv;
  int qkv_stride;
  const float* q_norm;
  const float* k_norm;
  float eps;
  const float* rope_cos;     // [n_ctx][D/2] tables
  const float* rope_sin;
  int pos0, n_rows;
  uint16_t* k_cache;         // [n_head_kv][n_ctx][D] of this layer
  uint16_t* v_cache;
  int n_head, n_head_kv, head_dim, n_ctx;
  float scale;
  float* out;
  // scratch for split-KV partials, partial_bytes long
  // (prefill_partial_bytes(n_head, n_head_kv, head_dim, n_rows) suffices)
  float* partial = nullptr;
  uint64_t partial_bytes = 0;
};
// False when the shape is not one the prefill kernels take (64 % group, D).
bool prefill_attention_ok(int n_head, int n_head_kv, int head_dim);
// Scratch the prompt-pass attention needs for up to max_rows rows.
uint64_t prefill_partial_bytes(int n_head, int n_head_kv, int head_dim, int max_rows);
hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t s);

// Decode-step control block in device memory: the token fed to the step, its
// position, the index into the output token ring, and the packed argmax of the
// LM head.
struct StepState {
  int32_t token;
  int32_t pos;
  int32_t step;
  int32_t pad;
  unsigned long long key;
};
hipError_t launch_step_close(StepState* st, const unsigned long long* keys, int nkeys,
                             int32_t* out_tokens, int max_steps, hipStream_t s);
// Workgroups launch_gemv uses for an n_out x n_in GEMV of `type` (the number of
// argmax keys it writes).
int gemv_grid(int type, int n_in, int n_out);

// Embedding row of st->token into x; row st->pos of the RoPE tables into
// rope_cur (cos then sin, `half` each; skipped when rope_cur is null).
hipError_t launch_embed(int type, const uint8_t* table, int n_embd, StepState* st, float* x,
                        const float* rope_cos, const float* rope_sin, int half, float* rope_cur,
                        hipStream_t s);

}  // namespace knj
