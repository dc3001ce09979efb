// kanjoos_amd/csrc/knj_batch.hip -- greedy decode of several sequences at once
// (for example 32 concurrent sequences, each with its own f16 KV cache).
//
// One step runs Model::forward's per-token work (/root/reference/src/model/model.cpp:512-672)
// for n_seq tokens together: every weight matrix is read once for all of them.
// Per layer: RMSNorm + QKV as one matrix-core GEMM over the n_seq rows,
// attention per sequence (grid z = sequence) over its own cache, the output
// projection + residual as a GEMM, the MoE layer over the n_seq rows with the
// (token, expert) pairs grouped by expert, then the final norm, the bf16 LM
// head as a GEMM and the greedy argmax of every row.  The sequences advance in
// lockstep (one position per step); each keeps its own cache and position.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "../../include/knj_capi.h"
#include "knj_common.h"
#include "knj_dev.h"
#include "knj_model_impl.h"

namespace knj {
namespace {

// Embedding rows of tokens[b] and the RoPE cos/sin rows of pos[b] (cos then
// sin, D/2 each) of every sequence b (blockIdx.y).
__global__ void k_embed_batch(int type, const uint8_t* __restrict__ table, int n_embd,
                              const int32_t* __restrict__ tokens, const int32_t* __restrict__ pos,
                              const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
                              int half, float* __restrict__ x, float* __restrict__ rope) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t id = (uint64_t)tokens[b];
  if (i < n_embd) {
    const uint64_t idx = id * n_embd + i;
    x[(uint64_t)b * n_embd + i] =
        type == KNJ_TYPE_BF16
            ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(table)[idx] << 16)
            : reinterpret_cast<const float*>(table)[idx];
  }
  if (blockIdx.x == 0 && threadIdx.x < 2 * half) {
    const int j = threadIdx.x % half;
    const float* tab = threadIdx.x < half ? rope_cos : rope_sin;
    rope[(uint64_t)b * 2 * half + threadIdx.x] = tab[(uint64_t)pos[b] * half + j];
  }
}

// After the argmax: record the step's tokens and advance every position.
__global__ void k_batch_close(int n_seq, const int32_t* __restrict__ next, int32_t* __restrict__ tokens,
                              int32_t* __restrict__ pos, int* __restrict__ step,
                              int32_t* __restrict__ out_tokens, int max_steps) {
  const int b = threadIdx.x;
  const int s = *step;
  if (b < n_seq) {
    tokens[b] = next[b];
    pos[b] += 1;
    if (s < max_steps) out_tokens[(uint64_t)s * n_seq + b] = next[b];
  }
  __syncthreads();
  if (b == 0) *step = s + 1;
}

}  // namespace
}  // namespace knj

using namespace knj;

struct knj_batch {
  knj_model* m = nullptr;  // weights and configuration (not owned)
  int n_seq = 0, n_ctx = 0, max_steps = 0, pos = 0;
  hipStream_t stream = nullptr;
  float *x = nullptr, *hx = nullptr, *qkv = nullptr, *ctx = nullptr, *logits = nullptr;
  float *rope = nullptr, *attn_part = nullptr, *hidden = nullptr, *router_logits = nullptr;
  float* topk_w = nullptr;
  int32_t *topk_idx = nullptr, *tokens = nullptr, *next = nullptr, *dpos = nullptr;
  int32_t* out_tokens = nullptr;
  int* step = nullptr;
  unsigned long long* keys = nullptr;  // argmax partial keys
  uint16_t *kv_k = nullptr, *kv_v = nullptr;
  void* scratch = nullptr;
  _Float16* osplit[4] = {};  // the attention output in the O product's operand layout
  _Float16* qsplit[4] = {};  // the attn-normalised rows in the QKV product's operand layout
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool use_graph = true;
  std::vector<void*> owned;
};

namespace {

int balloc(knj_batch* b, void** p, uint64_t bytes) {
  KNJ_HIP(hipMalloc(p, std::max<uint64_t>(bytes, 256)));
  b->owned.push_back(*p);
  return KNJ_OK;
}

uint64_t kv_seq_elems(const knj_batch* b) {
  const knj_model_config& c = b->m->c;
  return (uint64_t)c.n_layer * c.n_head_kv * b->n_ctx * c.head_dim;
}

int enqueue_batch_step(knj_batch* b, hipStream_t s) {
  const knj_model* m = b->m;
  const knj_model_config& c = m->c;
  const int B = b->n_seq, H = c.n_embd, D = c.head_dim, QD = c.n_head * D, KVD = c.n_head_kv * D;
  const int QKV = QD + 2 * KVD, half = D / 2;
  const uint8_t* img = m->image;
  KNJ_LAUNCH(k_embed_batch, dim3((H + 255) / 256, B), dim3(256), 0, s, c.type_embd,
                     img + m->off_embd, H, b->tokens, b->dpos, m->rope_cos, m->rope_sin, half, b->x,
                     b->rope);
  KNJ_HIP(hipGetLastError());
  // layer 0's QKV operand; every later one comes from the previous layer's
  // combine, and the last combine writes the output-normalised rows
  const bool fused_norms = H <= 4096 && H % 256 == 0;  // (always, for a valid model)
  if (fused_norms)
    KNJ_HIP(launch_norm_split(b->x, reinterpret_cast<const float*>(img + m->lo[0].attn_norm), c.rms_eps,
                              B, H, nullptr, b->qsplit, s));
  for (int il = 0; il < c.n_layer; ++il) {
    const knj_layer_offsets& lo = m->lo[il];
    if (fused_norms) {
      const _Float16* pre[4] = {b->qsplit[0], b->qsplit[1], b->qsplit[2], b->qsplit[3]};
      DenseQ4Extra qx;
      qx.pre = pre;
      KNJ_HIP(launch_dense_q4k_ex(img + lo.wqkv, H, QKV, B, nullptr, nullptr, b->qkv, b->scratch, qx, s));
    } else {
      KNJ_HIP(launch_norm_rows(b->x, reinterpret_cast<const float*>(img + lo.attn_norm), c.rms_eps, B,
                               H, b->hx, s));
      KNJ_HIP(launch_dense_q4k(img + lo.wqkv, H, QKV, B, b->hx, nullptr, b->qkv, b->scratch, s));
    }
    AttnArgs at{b->qkv, b->qkv + QD, b->qkv + QD + KVD,
                reinterpret_cast<const float*>(img + lo.q_norm),
                reinterpret_cast<const float*>(img + lo.k_norm), c.rms_eps, b->rope, b->rope + half,
                b->dpos, b->kv_k + (uint64_t)il * c.n_head_kv * b->n_ctx * D,
                b->kv_v + (uint64_t)il * c.n_head_kv * b->n_ctx * D, c.n_head, c.n_head_kv, D,
                b->n_ctx, 1.0f / std::sqrt((float)D), b->attn_part, b->ctx};
    at.n_seq = B;
    at.qkv_stride = (uint64_t)QKV;
    at.kv_stride = kv_seq_elems(b);
    at.out_stride = (uint64_t)QD;
    at.rope_stride = D;
    // the merge writes the O product's split operand too; the O product's
    // last launch also writes the ffn-normalised rows the MoE takes
    at.split_hi = b->osplit[0];
    at.split_lo = b->osplit[1];
    at.split_shi = b->osplit[2];
    at.split_slo = b->osplit[3];
    KNJ_HIP(launch_attention(at, s));
    const _Float16* pre[4] = {b->osplit[0], b->osplit[1], b->osplit[2], b->osplit[3]};
    DenseQ4Extra ox;
    ox.pre = pre;
    ox.norm_w = reinterpret_cast<const float*>(img + lo.ffn_norm);
    ox.eps = c.rms_eps;
    ox.norm_out = b->hx;
    KNJ_HIP(launch_dense_q4k_ex(img + lo.wo, QD, H, B, b->ctx, b->x, b->x, b->scratch, ox, s));
    MoeBatchArgs ma{b->hx, nullptr, c.rms_eps,
                    reinterpret_cast<const float*>(img + lo.router), img + lo.gate, img + lo.up,
                    img + lo.down, B, H, c.n_ff, c.n_expert, c.n_expert_used, b->x, b->x,
                    b->router_logits + (uint64_t)il * B * c.n_expert,
                    b->topk_idx + (uint64_t)il * B * c.n_expert_used,
                    b->topk_w + (uint64_t)il * B * c.n_expert_used};
    ma.hidden_copy = b->hidden + (uint64_t)il * B * H;
    ma.type_down = c.type_down;
    if (fused_norms) {
      const bool last = il + 1 == c.n_layer;
      ma.next_norm_w = reinterpret_cast<const float*>(img + (last ? m->off_onorm : m->lo[il + 1].attn_norm));
      ma.next_eps = c.rms_eps;
      ma.next_hx = last ? b->hx : nullptr;
      ma.next_split = last ? nullptr : b->qsplit;
    }
    KNJ_HIP(launch_moe_batch(ma, b->scratch, s));
  }
  if (!fused_norms)
    KNJ_HIP(launch_norm_rows(b->x, reinterpret_cast<const float*>(img + m->off_onorm), c.rms_eps, B,
                             H, b->hx, s));
  if (c.type_head == KNJ_TYPE_Q6_K)
    KNJ_HIP(launch_dense_q6k(img + m->off_head, H, c.n_vocab, B, b->hx, b->logits, b->scratch, s));
  else
    KNJ_HIP(launch_dense_bf16(reinterpret_cast<const uint16_t*>(img + m->off_head), H, c.n_vocab, B,
                            b->hx, b->logits, b->scratch, s));
  KNJ_HIP(launch_argmax_rows(b->logits, B, c.n_vocab, b->keys, b->next, s));
  KNJ_LAUNCH(k_batch_close, dim3(1), dim3(std::max(64, (B + 63) / 64 * 64)), 0, s, B,
                     b->next, b->tokens, b->dpos, b->step, b->out_tokens, b->max_steps);
  KNJ_HIP(hipGetLastError());
  return KNJ_OK;
}

int batch_graph(knj_batch* b) {
  const char* ng = std::getenv("KNJ_NO_GRAPH");
  b->use_graph = !(ng && ng[0] == '1');
  if (!b->use_graph || b->exec) return KNJ_OK;
  KNJ_HIP(hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal));
  const int rc = enqueue_batch_step(b, b->stream);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(b->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  b->graph = g;
  KNJ_HIP(hipGraphInstantiate(&b->exec, g, nullptr, nullptr, 0));
  return KNJ_OK;
}

int batch_run_step(knj_batch* b) {
  if (!b->use_graph) return enqueue_batch_step(b, b->stream);
  KNJ_HIP(hipGraphLaunch(b->exec, b->stream));
  return KNJ_OK;
}

// host tokens -> device, every position = b->pos, step counter 0
int batch_set_state(knj_batch* b, const int32_t* tokens) {
  std::vector<int32_t> pos(b->n_seq, b->pos);
  KNJ_HIP(hipMemcpyAsync(b->tokens, tokens, (uint64_t)b->n_seq * 4, hipMemcpyHostToDevice, b->stream));
  KNJ_HIP(hipMemcpyAsync(b->dpos, pos.data(), (uint64_t)b->n_seq * 4, hipMemcpyHostToDevice, b->stream));
  const int zero = 0;
  KNJ_HIP(hipMemcpyAsync(b->step, &zero, 4, hipMemcpyHostToDevice, b->stream));
  KNJ_HIP(hipStreamSynchronize(b->stream));
  return KNJ_OK;
}

}  // namespace

extern "C" {

int knj_batch_free(knj_batch* b) {
  if (!b) return KNJ_OK;
  if (b->exec) (void)hipGraphExecDestroy(b->exec);
  if (b->graph) (void)hipGraphDestroy(b->graph);
  for (void* p : b->owned) (void)hipFree(p);
  if (b->stream) (void)hipStreamDestroy(b->stream);
  delete b;
  return KNJ_OK;
}

int knj_batch_create(knj_model* m, int n_seq, int n_ctx, knj_batch** out) {
  KNJ_CHECK_ARG(m && out, "null pointer");
  const knj_model_config& c = m->c;
  KNJ_CHECK_ARG(n_seq >= 1 && n_seq <= 256, "n_seq must be in [1, 256]");
  KNJ_CHECK_ARG(n_ctx >= 1 && n_ctx <= c.n_ctx,
                "n_ctx must be in [1, the model's n_ctx] (the RoPE tables are the model's)");
  KNJ_CHECK_ARG(c.type_attn == KNJ_TYPE_Q4_K && c.type_gate_up == KNJ_TYPE_Q4_K &&
                    (c.type_down == KNJ_TYPE_Q4_K || c.type_down == KNJ_TYPE_Q6_K) &&
                    (c.type_head == KNJ_TYPE_BF16 || c.type_head == KNJ_TYPE_Q6_K),
                "the batched step takes Q4_K attention and gate/up, Q4_K or Q6_K down and a "
                "bf16 or Q6_K LM head");
  KNJ_CHECK_ARG(c.n_head * c.head_dim <= 4096 && (c.n_head * c.head_dim) % 256 == 0,
                "n_head * head_dim must be a multiple of 256, at most 4096");
  KNJ_CHECK_ARG(c.n_ff <= 4096 && c.n_ff % 256 == 0, "n_ff must be a multiple of 256, at most 4096");
  *out = nullptr;
  knj_batch* b = new knj_batch();
  b->m = m;
  b->n_seq = n_seq;
  b->n_ctx = n_ctx;
  b->max_steps = n_ctx;
  const int B = n_seq, H = c.n_embd, D = c.head_dim, QD = c.n_head * D;
  const int QKV = QD + 2 * c.n_head_kv * D, L = c.n_layer;
  int rc = KNJ_OK;
  auto A = [&](void** p, uint64_t bytes) {
    if (!rc) rc = balloc(b, p, bytes);
  };
  if (hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking) != hipSuccess) rc = KNJ_E_HIP;
  A((void**)&b->x, (uint64_t)B * H * 4);
  A((void**)&b->hx, (uint64_t)B * H * 4);
  A((void**)&b->qkv, (uint64_t)B * QKV * 4);
  A((void**)&b->ctx, (uint64_t)B * QD * 4);
  A((void**)&b->logits, (uint64_t)B * c.n_vocab * 4);
  A((void**)&b->rope, (uint64_t)B * D * 4);
  A((void**)&b->attn_part, (uint64_t)B * c.n_head * attn_splits(n_ctx) * (D + 2) * 4);
  A((void**)&b->hidden, (uint64_t)L * B * H * 4);
  A((void**)&b->router_logits, (uint64_t)L * B * c.n_expert * 4);
  A((void**)&b->topk_idx, (uint64_t)L * B * c.n_expert_used * 4);
  A((void**)&b->topk_w, (uint64_t)L * B * c.n_expert_used * 4);
  A((void**)&b->tokens, (uint64_t)B * 4);
  A((void**)&b->next, (uint64_t)B * 4);
  A((void**)&b->dpos, (uint64_t)B * 4);
  A((void**)&b->out_tokens, (uint64_t)b->max_steps * B * 4);
  A((void**)&b->step, 256);
  A((void**)&b->keys, (uint64_t)B * argmax_key_count(c.n_vocab) * 8);
  const uint64_t kv = (uint64_t)B * L * c.n_head_kv * n_ctx * D * 2;
  A((void**)&b->kv_k, kv);
  A((void**)&b->kv_v, kv);
  const uint64_t scr = std::max({moe_batch_scratch_bytes(B, H, c.n_ff, c.n_expert, c.n_expert_used),
                                 dense_scratch_bytes(B, H, QKV), dense_scratch_bytes(B, QD, H),
                                 dense_scratch_bytes(B, H, 0)});
  A(&b->scratch, scr);
  // [hi | lo | sums hi | sums lo] of B rows x n columns, as split_operand_bytes lays them out
  auto split_buf = [&](int n, _Float16** sp) {
    void* os = nullptr;
    A(&os, split_operand_bytes(B, n));
    if (!rc) {
      uint8_t* q = (uint8_t*)os;
      const uint64_t hb = ((uint64_t)B * n * 2 + 255) & ~255ull, sb = ((uint64_t)B * n / 16 + 255) & ~255ull;
      sp[0] = (_Float16*)q;
      sp[1] = (_Float16*)(q + hb);
      sp[2] = (_Float16*)(q + 2 * hb);
      sp[3] = (_Float16*)(q + 2 * hb + sb);
    }
  };
  split_buf(QD, b->osplit);
  split_buf(H, b->qsplit);
  if (!rc && (hipMemset(b->kv_k, 0, kv) != hipSuccess || hipMemset(b->kv_v, 0, kv) != hipSuccess))
    rc = KNJ_E_HIP;
  if (!rc) rc = batch_graph(b);
  if (rc) {
    knj_batch_free(b);
    return rc;
  }
  *out = b;
  return KNJ_OK;
}

int knj_batch_pos(const knj_batch* b) { return b ? b->pos : -1; }

int knj_batch_forward(knj_batch* b, const int32_t* tokens, float* logits_out) {
  KNJ_CHECK_ARG(b && tokens, "null pointer");
  KNJ_CHECK_ARG(b->pos < b->n_ctx, "context exhausted");
  for (int i = 0; i < b->n_seq; ++i)
    KNJ_CHECK_ARG(tokens[i] >= 0 && tokens[i] < b->m->c.n_vocab, "token id out of range");
  int rc = batch_set_state(b, tokens);
  if (rc) return rc;
  if ((rc = batch_run_step(b))) return rc;
  b->pos += 1;
  if (logits_out)
    KNJ_HIP(hipMemcpyAsync(logits_out, b->logits, (uint64_t)b->n_seq * b->m->c.n_vocab * 4,
                           hipMemcpyDeviceToHost, b->stream));
  KNJ_HIP(hipStreamSynchronize(b->stream));
  return KNJ_OK;
}

int knj_batch_decode_greedy(knj_batch* b, const int32_t* first, int steps, int32_t* out_tokens) {
  KNJ_CHECK_ARG(b && first && out_tokens, "null pointer");
  KNJ_CHECK_ARG(steps > 0 && steps <= b->max_steps, "steps out of range");
  if (b->pos + steps > b->n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  for (int i = 0; i < b->n_seq; ++i)
    KNJ_CHECK_ARG(first[i] >= 0 && first[i] < b->m->c.n_vocab, "token id out of range");
  int rc = batch_set_state(b, first);
  if (rc) return rc;
  for (int i = 0; i < steps; ++i)
    if ((rc = batch_run_step(b))) return rc;
  b->pos += steps;
  KNJ_HIP(hipMemcpyAsync(out_tokens, b->out_tokens, (uint64_t)steps * b->n_seq * 4,
                         hipMemcpyDeviceToHost, b->stream));
  KNJ_HIP(hipStreamSynchronize(b->stream));
  return KNJ_OK;
}

int knj_batch_fill_kv(knj_batch* b, int n_pos, uint64_t seed) {
  KNJ_CHECK_ARG(b && n_pos >= 0 && n_pos <= b->n_ctx, "bad arguments");
  const knj_model_config& c = b->m->c;
  // every (sequence, layer, kv head) row of n_ctx * D elements
  const uint64_t rows = (uint64_t)b->n_seq * c.n_layer * c.n_head_kv;
  int rc = fill_kv_rows(b->kv_k, b->kv_v, rows, (uint64_t)b->n_ctx * c.head_dim,
                        (uint64_t)n_pos * c.head_dim, seed, b->stream);
  if (rc) return rc;
  KNJ_HIP(hipStreamSynchronize(b->stream));
  b->pos = n_pos;
  return KNJ_OK;
}

int knj_batch_hidden(const knj_batch* b, int il, int seq, float* out) {
  KNJ_CHECK_ARG(b && out && il >= 0 && il < b->m->c.n_layer && seq >= 0 && seq < b->n_seq,
                "bad arguments");
  const uint64_t H = b->m->c.n_embd;
  KNJ_HIP(hipMemcpy(out, b->hidden + ((uint64_t)il * b->n_seq + seq) * H, H * 4, hipMemcpyDeviceToHost));
  return KNJ_OK;
}

int knj_batch_topk(const knj_batch* b, int il, int seq, int32_t* idx, float* w) {
  KNJ_CHECK_ARG(b && idx && w && il >= 0 && il < b->m->c.n_layer && seq >= 0 && seq < b->n_seq,
                "bad arguments");
  const uint64_t k = b->m->c.n_expert_used;
  const uint64_t o = ((uint64_t)il * b->n_seq + seq) * k;
  KNJ_HIP(hipMemcpy(idx, b->topk_idx + o, k * 4, hipMemcpyDeviceToHost));
  KNJ_HIP(hipMemcpy(w, b->topk_w + o, k * 4, hipMemcpyDeviceToHost));
  return KNJ_OK;
}

int knj_batch_kv_download(const knj_batch* b, int seq, uint16_t* k, uint16_t* v) {
  KNJ_CHECK_ARG(b && k && v && seq >= 0 && seq < b->n_seq, "bad arguments");
  const uint64_t n = kv_seq_elems(b);
  KNJ_HIP(hipMemcpy(k, b->kv_k + (uint64_t)seq * n, n * 2, hipMemcpyDeviceToHost));
  KNJ_HIP(hipMemcpy(v, b->kv_v + (uint64_t)seq * n, n * 2, hipMemcpyDeviceToHost));
  return KNJ_OK;
}

int knj_batch_kv_upload(knj_batch* b, int seq, const uint16_t* k, const uint16_t* v) {
  KNJ_CHECK_ARG(b && k && v && seq >= 0 && seq < b->n_seq, "bad arguments");
  const uint64_t n = kv_seq_elems(b);
  KNJ_HIP(hipMemcpy(b->kv_k + (uint64_t)seq * n, k, n * 2, hipMemcpyHostToDevice));
  KNJ_HIP(hipMemcpy(b->kv_v + (uint64_t)seq * n, v, n * 2, hipMemcpyHostToDevice));
  return KNJ_OK;
}

int knj_batch_set_pos(knj_batch* b, int pos) {
  KNJ_CHECK_ARG(b && pos >= 0 && pos <= b->n_ctx, "position outside the context");
  b->pos = pos;
  return KNJ_OK;
}

}  // extern "C"
