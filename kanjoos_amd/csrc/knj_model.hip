// kanjoos_amd/csrc/knj_model.hip -- the device decode step behind knj_model_*.
//
// One model = one weight image in HBM (layout of include/knj_model.h), an f16
// KV cache, and a fixed set of activation buffers.  A decode step reads the
// token and the position from device memory, so the whole step is captured
// once as a HIP graph and replayed: greedy decode never returns to the host
// between tokens.
//
// Step (per token):  embed -> 48 x [ qkv GEMV (attn RMSNorm fused) ->
//   q/k norm + RoPE + f16 KV append -> split-KV attention -> merge ->
//   o GEMV + residual -> router (ffn RMSNorm fused, softmax, top-k) ->
//   gate/up GEMV + SwiGLU -> down GEMV + weighted sum + residual ]
//   -> LM head GEMV (final RMSNorm fused) with argmax -> step end.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

#include "../../include/knj_synth.h"
#include "knj_common.h"
#include "knj_gguf.h"
#include "knj_model_impl.h"

namespace knj {
namespace {

// ----------------------------------------------------------- synthetic weights

// One thread per quantised block: 256 draws, then the block quantiser.
__global__ void k_synth_quant(uint64_t seed, int layer, int kind, int type, uint64_t n_in,
                              uint64_t rows_per_expert, int n_expert, int expert_base,
                              float stddev, uint8_t* __restrict__ out) {
  const uint64_t nb_row = n_in / KNJ_QK;
  const uint64_t per_expert = rows_per_expert * nb_row;
  const uint64_t total = per_expert * (uint64_t)n_expert;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint64_t e = i / per_expert, b = i % per_expert;
  const int expert = expert_base < 0 ? -1 : expert_base + (int)e;
  const uint64_t key = knj_tensor_key(seed, layer, kind, expert);
  float tmp[KNJ_QK];
  const uint64_t bb = knj_row_bytes(type, KNJ_QK);
  knj_synth_quant_block(key, type, n_in, b, stddev, tmp, out + i * bb);
}

__global__ void k_synth_plain(uint64_t key, int type, uint64_t n, float stddev,
                              uint8_t* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = knj_synth_value(key, i, stddev);
  if (type == KNJ_TYPE_F32) reinterpret_cast<float*>(out)[i] = v;
  else if (type == KNJ_TYPE_BF16) reinterpret_cast<uint16_t*>(out)[i] = knj_f32_to_bf16(v);
  else reinterpret_cast<uint16_t*>(out)[i] = knj_f32_to_f16(v);
}

// Cache slots [0, n_pos) of every (layer, kv head) row of length n_ctx * D,
// f16 values of N(0, 1) from the seeded generator (a stand-in for a prefill's
// keys and values; the decode step's work does not depend on them).
__global__ void k_fill_kv(uint16_t* __restrict__ k, uint16_t* __restrict__ v, uint64_t rows,
                          uint64_t row_elems, uint64_t n_elems, uint64_t key) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n_elems) return;
  const uint64_t r = i / n_elems, c = i - r * n_elems;
  const uint64_t o = r * row_elems + c;
  k[o] = knj_f32_to_f16(knj_normal(key, 2 * i));
  v[o] = knj_f32_to_f16(knj_normal(key, 2 * i + 1));
}

__global__ void k_fill_ones(float* p, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 1.0f;
}

}  // namespace

int fill_kv_rows(uint16_t* k, uint16_t* v, uint64_t rows, uint64_t row_elems, uint64_t n_elems,
                 uint64_t seed, hipStream_t s) {
  const uint64_t total = rows * n_elems;
  if (!total) return KNJ_OK;
  hipLaunchKernelGGL(k_fill_kv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, k, v, rows,
                     row_elems, n_elems, knj_mix64(seed ^ 0x4B56ull));
  KNJ_HIP(hipGetLastError());
  return KNJ_OK;
}

thread_local SpanSink* tl_span_sink = nullptr;

namespace {
__global__ void k_span_floor(int) {}
}  // namespace

// Installs a span sink of `cap` event pairs on this thread for its lifetime.
SpanRun::SpanRun(int cap) {
  sink.cap = cap;
  events.assign((size_t)2 * cap, nullptr);
  for (auto& e : events)
    if ((err = hipEventCreate(&e)) != hipSuccess) return;
  if ((err = hipEventCreate(&epoch)) != hipSuccess) return;
  sink.ev = events.data();
  sink.tags.reserve((size_t)cap);
  tl_span_sink = &sink;
}

SpanRun::~SpanRun() {
  if (tl_span_sink == &sink) tl_span_sink = nullptr;
  for (auto e : events)
    if (e) (void)hipEventDestroy(e);
  if (epoch) (void)hipEventDestroy(epoch);
}

void SpanRun::stop() {
  if (tl_span_sink == &sink) tl_span_sink = nullptr;
}

// Offsets of every recorded span from the epoch event (the events must have
// completed), written as knj_span records.
int SpanRun::collect(knj_span* out, int cap, int* n_out, uint64_t* dropped) {
  const int n = std::min(sink.used, cap);
  for (int i = 0; i < n; ++i) {
    float a = 0.0f, b = 0.0f;
    hipError_t e = hipEventElapsedTime(&a, epoch, events[2 * i]);
    if (e == hipSuccess) e = hipEventElapsedTime(&b, epoch, events[2 * i + 1]);
    if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
    knj_span& r = out[i];
    std::memset(&r, 0, sizeof(r));
    const SpanTag& t = sink.tags[(size_t)i];
    std::snprintf(r.name, sizeof(r.name), "%s", t.cls);
    // the stringised kernel expression, without wrapping parentheses
    std::string k(t.kernel);
    while (!k.empty() && (k.back() == ')' || k.back() == ' ')) k.pop_back();
    std::snprintf(r.kernel, sizeof(r.kernel), "%s", k.c_str());
    r.layer = t.layer;
    r.stream = 0;
    r.start_ns = (uint64_t)std::llround((double)a * 1e6);
    r.end_ns = std::max(r.start_ns, (uint64_t)std::llround((double)b * 1e6));
  }
  *n_out = n;
  if (dropped) *dropped = sink.dropped + (uint64_t)(sink.used - n);
  return KNJ_OK;
}

}  // namespace knj

using namespace knj;


namespace {

int alloc(knj_model* m, void** p, uint64_t bytes) {
  KNJ_HIP(hipMalloc(p, std::max<uint64_t>(bytes, 256)));
  m->owned.push_back(*p);
  return KNJ_OK;
}

int validate(const knj_model_config* c) {
  KNJ_CHECK_ARG(c, "null config");
  KNJ_CHECK_ARG(c->n_layer > 0 && c->n_embd > 0 && c->n_vocab > 0, "empty model");
  KNJ_CHECK_ARG(c->n_embd % 256 == 0 && c->n_embd <= 4096, "n_embd must be a multiple of 256, <= 4096");
  KNJ_CHECK_ARG(c->head_dim == 64 || c->head_dim == 128, "head_dim must be 64 or 128");
  KNJ_CHECK_ARG(c->n_head_kv > 0 && c->n_head_kv <= 64 && c->n_head % c->n_head_kv == 0 &&
                    c->n_head / c->n_head_kv <= 8,
                "n_head must be a multiple of n_head_kv (<= 64) with a group of at most 8");
  KNJ_CHECK_ARG((int64_t)c->n_head * c->head_dim <= 16384, "q_dim must be at most 16384");
  KNJ_CHECK_ARG(((int64_t)c->n_head * c->head_dim) % 256 == 0, "q_dim must be a multiple of 256");
  KNJ_CHECK_ARG(c->n_ff > 0 && c->n_ff % 256 == 0, "n_ff must be a multiple of 256");
  KNJ_CHECK_ARG(c->n_expert > 0 && c->n_expert <= 256, "n_expert must be in [1, 256]");
  KNJ_CHECK_ARG(c->n_expert_used > 0 && c->n_expert_used <= 16 && c->n_expert_used <= c->n_expert,
                "n_expert_used must be in [1, min(16, n_expert)]");
  KNJ_CHECK_ARG(c->n_ctx > 0, "n_ctx must be positive");
  KNJ_CHECK_ARG(c->type_embd == KNJ_TYPE_BF16 || c->type_embd == KNJ_TYPE_F32, "embeddings must be BF16 or F32");
  KNJ_CHECK_ARG(c->type_attn == KNJ_TYPE_Q4_K || c->type_attn == KNJ_TYPE_Q6_K, "attention weights must be Q4_K or Q6_K");
  KNJ_CHECK_ARG(c->type_gate_up == KNJ_TYPE_Q4_K, "expert gate/up must be Q4_K");
  KNJ_CHECK_ARG(c->type_down == KNJ_TYPE_Q4_K || c->type_down == KNJ_TYPE_Q6_K, "expert down must be Q4_K or Q6_K");
  KNJ_CHECK_ARG(c->type_head == KNJ_TYPE_BF16 || c->type_head == KNJ_TYPE_Q6_K || c->type_head == KNJ_TYPE_Q4_K,
                "LM head must be BF16, Q4_K or Q6_K");
  const uint64_t lds_down = ((uint64_t)c->n_expert_used * c->n_ff * 4) + (uint64_t)c->n_expert_used * (c->n_ff / 32) * 4 +
                            (uint64_t)c->n_expert_used * 8 * 4;
  KNJ_CHECK_ARG(lds_down <= 160 * 1024, "n_expert_used * n_ff too large for LDS staging");
  return KNJ_OK;
}

int setup(knj_model* m) {
  const knj_model_config& c = m->c;
  m->image_bytes = knj_model_layout(&c, 0, nullptr, &m->off_embd, &m->off_onorm, &m->off_head);
  m->lo.resize((size_t)c.n_layer);
  for (int il = 0; il < c.n_layer; ++il) knj_model_layout(&c, il, &m->lo[il], nullptr, nullptr, nullptr);
  KNJ_HIP(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  int rc;
  const uint64_t H = c.n_embd, QD = (uint64_t)c.n_head * c.head_dim, KVD = (uint64_t)c.n_head_kv * c.head_dim;
  if ((rc = alloc(m, (void**)&m->image, m->image_bytes))) return rc;
  if ((rc = alloc(m, (void**)&m->x, H * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->qkv, (QD + 2 * KVD) * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->ctx, QD * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->hx, H * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->x2, H * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->act, (uint64_t)c.n_expert_used * c.n_ff * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->logits, (uint64_t)c.n_vocab * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->router_logits, (uint64_t)c.n_layer * c.n_expert * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->hidden, (uint64_t)c.n_layer * H * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->topk_idx, (uint64_t)c.n_layer * c.n_expert_used * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->topk_w, (uint64_t)c.n_layer * c.n_expert_used * 4))) return rc;
  const int half = c.head_dim / 2;
  if ((rc = alloc(m, (void**)&m->rope_cos, (uint64_t)c.n_ctx * half * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->rope_sin, (uint64_t)c.n_ctx * half * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->rope_cur, (uint64_t)2 * half * 4))) return rc;
  const int n_split = attn_splits(c.n_ctx);
  if ((rc = alloc(m, (void**)&m->attn_part, (uint64_t)c.n_head * n_split * (c.head_dim + 2) * 4))) return rc;
  const uint64_t kv = knj_kv_elems(&c);
  if ((rc = alloc(m, (void**)&m->kv_k, kv * 2))) return rc;
  if ((rc = alloc(m, (void**)&m->kv_v, kv * 2))) return rc;
  if ((rc = alloc(m, (void**)&m->st, sizeof(StepState)))) return rc;
  m->max_steps = std::max(c.n_ctx, 1);
  if ((rc = alloc(m, (void**)&m->out_tokens, (uint64_t)m->max_steps * 4))) return rc;
  if ((rc = alloc(m, (void**)&m->keys, (uint64_t)kMaxKeys * 8))) return rc;
  KNJ_HIP(hipMemset(m->keys, 0, (uint64_t)kMaxKeys * 8));
  // tickets: [0] router, [64 + h] attention of kv head h
  if ((rc = alloc(m, (void**)&m->counter, 4096))) return rc;
  KNJ_HIP(hipMemset(m->counter, 0, 4096));
  KNJ_HIP(hipMemset(m->kv_k, 0, kv * 2));
  KNJ_HIP(hipMemset(m->kv_v, 0, kv * 2));
  KNJ_HIP(hipMemset(m->st, 0, sizeof(StepState)));
  // RoPE table: theta = pos * base^(-2i/D) in f32, cos/sin in f32 on the host,
  // the expressions of model.cpp:227-230 and :278-279
  std::vector<float> inv(half), tc((size_t)c.n_ctx * half), ts((size_t)c.n_ctx * half);
  for (int i = 0; i < half; ++i) inv[i] = std::pow(c.rope_base, -2.0f * (float)i / (float)c.head_dim);
  for (int p = 0; p < c.n_ctx; ++p)
    for (int i = 0; i < half; ++i) {
      const float th = (float)p * inv[i];
      tc[(size_t)p * half + i] = std::cos(th);
      ts[(size_t)p * half + i] = std::sin(th);
    }
  KNJ_HIP(hipMemcpy(m->rope_cos, tc.data(), tc.size() * 4, hipMemcpyHostToDevice));
  m->h2d_bytes += tc.size() * 4;
  KNJ_HIP(hipMemcpy(m->rope_sin, ts.data(), ts.size() * 4, hipMemcpyHostToDevice));
  m->h2d_bytes += ts.size() * 4;
  return KNJ_OK;
}

int synth_quant(knj_model* m, uint64_t seed, int layer, int kind, int type, uint64_t n_in,
                uint64_t rows, int n_expert, int expert_base, uint8_t* dst) {
  const uint64_t total = rows * (n_in / KNJ_QK) * (uint64_t)n_expert;
  const unsigned grid = (unsigned)((total + 127) / 128);
  hipLaunchKernelGGL(k_synth_quant, dim3(grid), dim3(128), 0, m->stream, seed, layer, kind, type,
                     n_in, rows, n_expert, expert_base, m->c.init_std, dst);
  KNJ_HIP(hipGetLastError());
  return KNJ_OK;
}

int synth_plain(knj_model* m, uint64_t key, int type, uint64_t n, uint8_t* dst) {
  const unsigned grid = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(k_synth_plain, dim3(grid), dim3(256), 0, m->stream, key, type, n,
                     m->c.init_std, dst);
  KNJ_HIP(hipGetLastError());
  return KNJ_OK;
}

int ones(knj_model* m, uint64_t off, uint64_t n) {
  hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, m->stream,
                     reinterpret_cast<float*>(m->image + off), n);
  KNJ_HIP(hipGetLastError());
  return KNJ_OK;
}

// Same tensor keys and element order as the host generator (oracle synth_model).
int synth_all(knj_model* m, uint64_t seed) {
  const knj_model_config& c = m->c;
  const uint64_t H = c.n_embd, QD = (uint64_t)c.n_head * c.head_dim, KVD = (uint64_t)c.n_head_kv * c.head_dim;
  const uint64_t F = c.n_ff, V = c.n_vocab;
  int rc;
  auto tensor = [&](int layer, int kind, int type, uint64_t n_in, uint64_t rows, uint8_t* dst) {
    if (type == KNJ_TYPE_Q4_K || type == KNJ_TYPE_Q6_K)
      return synth_quant(m, seed, layer, kind, type, n_in, rows, 1, -1, dst);
    return synth_plain(m, knj_tensor_key(seed, layer, kind, -1), type, n_in * rows, dst);
  };
  if ((rc = tensor(-1, KNJ_T_EMBD, c.type_embd, H, V, m->image + m->off_embd))) return rc;
  for (int il = 0; il < c.n_layer; ++il) {
    const knj_layer_offsets& lo = m->lo[il];
    if ((rc = ones(m, lo.attn_norm, H))) return rc;
    if ((rc = ones(m, lo.ffn_norm, H))) return rc;
    if ((rc = ones(m, lo.q_norm, (uint64_t)c.head_dim))) return rc;
    if ((rc = ones(m, lo.k_norm, (uint64_t)c.head_dim))) return rc;
    const uint64_t rb = knj_row_bytes(c.type_attn, H);
    uint8_t* wqkv = m->image + lo.wqkv;
    if ((rc = tensor(il, KNJ_T_Q, c.type_attn, H, QD, wqkv))) return rc;
    if ((rc = tensor(il, KNJ_T_K, c.type_attn, H, KVD, wqkv + rb * QD))) return rc;
    if ((rc = tensor(il, KNJ_T_V, c.type_attn, H, KVD, wqkv + rb * (QD + KVD)))) return rc;
    if ((rc = tensor(il, KNJ_T_O, c.type_attn, QD, H, m->image + lo.wo))) return rc;
    if ((rc = tensor(il, KNJ_T_ROUTER, KNJ_TYPE_F32, H, (uint64_t)c.n_expert, m->image + lo.router))) return rc;
    if ((rc = synth_quant(m, seed, il, KNJ_T_GATE, c.type_gate_up, H, F, c.n_expert, 0, m->image + lo.gate))) return rc;
    if ((rc = synth_quant(m, seed, il, KNJ_T_UP, c.type_gate_up, H, F, c.n_expert, 0, m->image + lo.up))) return rc;
    if ((rc = synth_quant(m, seed, il, KNJ_T_DOWN, c.type_down, F, H, c.n_expert, 0, m->image + lo.down))) return rc;
  }
  if ((rc = ones(m, m->off_onorm, H))) return rc;
  if ((rc = tensor(-1, KNJ_T_HEAD, c.type_head, H, V, m->image + m->off_head))) return rc;
  KNJ_HIP(hipStreamSynchronize(m->stream));
  return KNJ_OK;
}

// The per-layer launches.  `layer_out` receives the residual after the layer.
int enqueue_layer(knj_model* m, int il, hipStream_t s) {
  const knj_model_config& c = m->c;
  const knj_layer_offsets& lo = m->lo[il];
  const int H = c.n_embd, D = c.head_dim, QD = c.n_head * D, KVD = c.n_head_kv * D;
  const uint8_t* img = m->image;
  GemvArgs qkv{c.type_attn, img + lo.wqkv, H, QD + 2 * KVD, m->x,
               reinterpret_cast<const float*>(img + lo.attn_norm), c.rms_eps, nullptr, m->qkv, nullptr};
  span_scope("qkv", il);
  KNJ_HIP(launch_gemv(qkv, s));
  const uint64_t kv_layer = (uint64_t)il * c.n_head_kv * c.n_ctx * D;
  AttnArgs at{m->qkv, m->qkv + QD, m->qkv + QD + KVD,
              reinterpret_cast<const float*>(img + lo.q_norm),
              reinterpret_cast<const float*>(img + lo.k_norm), c.rms_eps, m->rope_cur, m->rope_cur + D / 2,
              &m->st->pos, m->kv_k + kv_layer, m->kv_v + kv_layer, c.n_head, c.n_head_kv, D, c.n_ctx,
              1.0f / std::sqrt((float)D), m->attn_part, m->ctx};
  span_class("attention");
  KNJ_HIP(launch_attention(at, s));
  // timing runs: the launch before the experts (the router, or attn-o with the
  // router folded in) and each expert launch record start/end events of their
  // own dispatch.  The first pair is not used: an event-timed launch that
  // follows one without events reads ~1.5 us longer (its start event is taken
  // while the launch before it still drains), so the gate/up launch is timed
  // after an event-timed launch as the down launch is.
  hipEvent_t* ev = m->expert_events ? m->expert_events + 6 * m->expert_slot++ : nullptr;
  float* const u = m->router_logits + (uint64_t)il * c.n_expert;
  // with the router folded in, attn-o writes the residual stream into x2 (its
  // router rows still read x) and the MoE goes from x2 back to x
  float* const xm = m->fold_router ? m->x2 : m->x;
  GemvArgs o{c.type_attn, img + lo.wo, QD, H, m->ctx, nullptr, 0.0f, m->x, xm, nullptr};
  if (m->fold_router) {
    span_class("attn-o+moe-router");
    const float* R = m->router_fold + (uint64_t)il * c.n_expert * (H + QD);
    KNJ_HIP(launch_gemv_router(o, R, c.n_expert, u, s, ev ? ev[4] : nullptr, ev ? ev[5] : nullptr));
  } else {
    span_class("attn-o");
    KNJ_HIP(launch_gemv(o, s));
    RouterArgs ra{m->x, reinterpret_cast<const float*>(img + lo.ffn_norm), c.rms_eps,
                  reinterpret_cast<const float*>(img + lo.router), H, c.n_expert, c.n_expert_used,
                  m->hx, u, nullptr, nullptr, m->counter};
    span_class("moe-router");
    KNJ_HIP(launch_router(ra, s, ev ? ev[4] : nullptr, ev ? ev[5] : nullptr));
  }
  // the gate/up launch routes from the logits (softmax + top-k per wave)
  int32_t* ti = m->topk_idx + (uint64_t)il * c.n_expert_used;
  float* tw = m->topk_w + (uint64_t)il * c.n_expert_used;
  ExpertArgs ea{xm, reinterpret_cast<const float*>(img + lo.ffn_norm), c.rms_eps, u, ti, tw,
                img + lo.gate, img + lo.up, img + lo.down,
                c.type_gate_up, c.type_down, H, c.n_ff, c.n_expert, c.n_expert_used, m->act, xm,
                m->x, m->hidden + (uint64_t)il * H};
  ea.logits_unscaled = m->fold_router;
  span_class("moe-gate+up+act");
  KNJ_HIP(launch_expert_gateup(ea, s, ev ? ev[0] : nullptr, ev ? ev[1] : nullptr));
  span_class("moe-down+scatter");
  KNJ_HIP(launch_expert_down(ea, s, ev ? ev[2] : nullptr, ev ? ev[3] : nullptr));
  return KNJ_OK;
}

int enqueue_step(knj_model* m, hipStream_t s) {
  const knj_model_config& c = m->c;
  span_scope("embed", -1);
  KNJ_HIP(launch_embed(c.type_embd, m->image + m->off_embd, c.n_embd, m->st, m->x, m->rope_cos,
                       m->rope_sin, c.head_dim / 2, m->rope_cur, s));
  for (int il = 0; il < c.n_layer; ++il) {
    int rc = enqueue_layer(m, il, s);
    if (rc) return rc;
  }
  if (c.type_head == KNJ_TYPE_Q4_K) {
    set_error("a Q4_K LM head has no fused argmax; use BF16 or Q6_K");
    return KNJ_E_ARG;
  }
  GemvArgs head{c.type_head, m->image + m->off_head, c.n_embd, c.n_vocab, m->x,
                reinterpret_cast<const float*>(m->image + m->off_onorm), c.rms_eps, nullptr,
                m->logits, m->keys};
  span_scope("head", -1);
  KNJ_HIP(launch_gemv(head, s));
  span_class("sample");
  KNJ_HIP(launch_step_close(m->st, m->keys, gemv_grid(c.type_head, c.n_embd, c.n_vocab),
                            m->out_tokens, m->max_steps, s));
  return KNJ_OK;
}

constexpr int kMultiSteps = 8;

int ensure_graph(knj_model* m) {
  const char* ng = std::getenv("KNJ_NO_GRAPH");
  m->use_graph = !(ng && ng[0] == '1');
  if (!m->use_graph || m->exec) return KNJ_OK;
  KNJ_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
  const int rc = enqueue_step(m, m->stream);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(m->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  m->graph = g;
  KNJ_HIP(hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0));
  // decode loops replay kMultiSteps steps per graph launch while at least that
  // many remain: one launch boundary per kMultiSteps tokens (measured 1.684 ->
  // 1.675-1.680 ms/token at config 3 with 8)
  m->multi = kMultiSteps;
  if (m->multi > 1) {
    KNJ_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc2 = KNJ_OK;
    for (int i = 0; i < m->multi && rc2 == KNJ_OK; ++i) rc2 = enqueue_step(m, m->stream);
    hipGraph_t gm = nullptr;
    const hipError_t e2 = hipStreamEndCapture(m->stream, &gm);
    if (rc2) {
      if (gm) (void)hipGraphDestroy(gm);
      return rc2;
    }
    if (e2 != hipSuccess) return hip_fail(e2, "hipStreamEndCapture");
    m->graph_multi = gm;
    KNJ_HIP(hipGraphInstantiate(&m->exec_multi, gm, nullptr, nullptr, 0));
  }
  return KNJ_OK;
}

int run_step(knj_model* m) {
  if (!m->use_graph) return enqueue_step(m, m->stream);
  KNJ_HIP(hipGraphLaunch(m->exec, m->stream));
  return KNJ_OK;
}

// n steps: the multi-step graph while enough remain, then single steps
int run_steps(knj_model* m, int n) {
  if (m->use_graph && m->exec_multi)
    for (; n >= m->multi; n -= m->multi) KNJ_HIP(hipGraphLaunch(m->exec_multi, m->stream));
  for (; n > 0; --n) {
    const int rc = run_step(m);
    if (rc) return rc;
  }
  return KNJ_OK;
}

int set_state(knj_model* m, int32_t token, int step) {
  StepState h{};
  h.token = token;
  h.pos = m->pos;
  h.step = step;
  KNJ_HIP(hipMemcpyAsync(m->st, &h, sizeof(h), hipMemcpyHostToDevice, m->stream));
  m->h2d_bytes += sizeof(h);
  KNJ_HIP(hipStreamSynchronize(m->stream));
  return KNJ_OK;
}

// The router folded into the attention-output launch (k_gemv_q4k_router):
// per layer R = [W_r * ffn_norm | (W_r * ffn_norm) W_o], from the weights in
// the image, computed once when the model is created.
int fold_router(knj_model* m) {
  const knj_model_config& c = m->c;
  const int H = c.n_embd, QD = c.n_head * c.head_dim, E = c.n_expert;
  m->fold_router = router_fold_ok(c.type_attn, QD, H, E) && E <= 128 && H <= 2048 &&
                   c.n_expert_used <= 16 && !std::getenv("KNJ_NO_ROUTER_FOLD");
  if (!m->fold_router) return KNJ_OK;
  const uint64_t NR = (uint64_t)H + QD;
  int rc = alloc(m, (void**)&m->router_fold, (uint64_t)c.n_layer * E * NR * 4);
  if (rc) return rc;
  float* wd = nullptr;
  KNJ_HIP(hipMalloc(&wd, (uint64_t)H * QD * 4));
  hipError_t e = hipSuccess;
  for (int il = 0; il < c.n_layer && e == hipSuccess; ++il) {
    const knj_layer_offsets& lo = m->lo[il];
    e = launch_dequant(c.type_attn, m->image + lo.wo, (uint64_t)H * QD, wd, m->stream);
    if (e == hipSuccess)
      e = launch_router_fold(reinterpret_cast<const float*>(m->image + lo.router),
                             reinterpret_cast<const float*>(m->image + lo.ffn_norm), wd, H, QD, E,
                             m->router_fold + (uint64_t)il * E * NR, m->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  (void)hipFree(wd);
  if (e != hipSuccess) return hip_fail(e, "router fold");
  return KNJ_OK;
}

int finish_create(knj_model* m, knj_model** out) {
  int rc = fold_router(m);
  if (rc) {
    knj_model_free(m);
    return rc;
  }
  rc = ensure_graph(m);
  if (rc) {
    knj_model_free(m);
    return rc;
  }
  *out = m;
  return KNJ_OK;
}

}  // namespace

extern "C" {

int knj_model_create_synthetic(const knj_model_config* cfg, uint64_t seed, knj_model** out) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(out, "null output pointer");
  if ((rc = validate(cfg))) return rc;
  knj_model* m = new knj_model();
  m->c = *cfg;
  if ((rc = setup(m)) || (rc = synth_all(m, seed))) {
    knj_model_free(m);
    return rc;
  }
  return finish_create(m, out);
}

namespace {

// The geometry of a qwen3moe GGUF file (Model::read_geometry and
// bind_tensors, /root/reference/src/model/model.cpp:97-172): metadata, tensor
// names, shapes and the types this path runs.  `n_ctx` must not exceed the
// trained context (model.cpp:180-186).
int gguf_config(const GgufView& g, int n_ctx, knj_model_config* c) {
  const std::string arch = g.meta_string("general.architecture");
  if (arch != "qwen3moe") {
    set_error("model: architecture is '" + gguf_printable(arch) + "', this path implements 'qwen3moe'");
    return KNJ_E_ARG;
  }
  const std::string p = arch + ".";
  int64_t v = 0;
  double f = 0.0;
  auto need_i = [&](const char* key, int32_t& dst) {
    if (!g.meta_int(p + key, v)) {
      set_error(std::string("model: metadata '") + p + key + "' is missing");
      return false;
    }
    dst = (int32_t)v;
    return true;
  };
  *c = knj_model_config{};
  int32_t ctx_train = 0;
  if (!need_i("block_count", c->n_layer) || !need_i("embedding_length", c->n_embd) ||
      !need_i("attention.head_count", c->n_head) || !need_i("attention.key_length", c->head_dim) ||
      !need_i("expert_feed_forward_length", c->n_ff) || !need_i("expert_count", c->n_expert) ||
      !need_i("expert_used_count", c->n_expert_used) || !need_i("context_length", ctx_train))
    return KNJ_E_ARG;
  c->n_head_kv = g.meta_int(p + "attention.head_count_kv", v) ? (int32_t)v : c->n_head;
  if (!g.meta_float(p + "attention.layer_norm_rms_epsilon", f)) {
    set_error("model: metadata '" + p + "attention.layer_norm_rms_epsilon' is missing");
    return KNJ_E_ARG;
  }
  c->rms_eps = (float)f;
  if (!g.meta_float(p + "rope.freq_base", f)) {
    set_error("model: metadata '" + p + "rope.freq_base' is missing");
    return KNJ_E_ARG;
  }
  c->rope_base = (float)f;
  if (n_ctx <= 0 || n_ctx > ctx_train) {
    set_error("model: n_ctx " + std::to_string(n_ctx) + " outside [1, the trained context " +
              std::to_string(ctx_train) + "]");
    return KNJ_E_ARG;
  }
  c->n_ctx = n_ctx;
  const GgufTensor* te = g.find("token_embd.weight");
  if (!te || te->n_dims != 2) {
    set_error("model: tensor 'token_embd.weight' is missing or not 2-D");
    return KNJ_E_ARG;
  }
  c->n_vocab = g.meta_int("vocab_size", v) ? (int32_t)v : (int32_t)te->dims[1];
  // shapes (dims[0] fastest) and types
  const int64_t H = c->n_embd, QD = (int64_t)c->n_head * c->head_dim;
  const int64_t KVD = (int64_t)c->n_head_kv * c->head_dim, F = c->n_ff, E = c->n_expert;
  auto want = [&](const std::string& name, std::initializer_list<int64_t> dims,
                  const GgufTensor** out) {
    const GgufTensor* t = g.find(name);
    if (!t) {
      set_error("model: tensor '" + name + "' is missing");
      return false;
    }
    if (t->n_dims != dims.size()) {
      set_error("model: tensor '" + name + "' has " + std::to_string(t->n_dims) + " dims, expected " +
                std::to_string(dims.size()));
      return false;
    }
    int i = 0;
    for (int64_t d : dims) {
      if ((int64_t)t->dims[i] != d) {
        set_error("model: tensor '" + name + "' dim " + std::to_string(i) + " is " +
                  std::to_string(t->dims[i]) + ", expected " + std::to_string(d));
        return false;
      }
      ++i;
    }
    if (t->bytes == 0) {
      set_error("model: tensor '" + name + "' has unsupported type " + std::to_string(t->type));
      return false;
    }
    if (out) *out = t;
    return true;
  };
  const GgufTensor *ow = nullptr, *on = nullptr;
  if (!want("token_embd.weight", {H, c->n_vocab}, nullptr) ||
      !want("output_norm.weight", {H}, &on) || !want("output.weight", {H, c->n_vocab}, &ow))
    return KNJ_E_ARG;
  c->type_embd = (int32_t)te->type;
  c->type_head = (int32_t)ow->type;
  for (int il = 0; il < c->n_layer; ++il) {
    const std::string b = "blk." + std::to_string(il) + ".";
    const GgufTensor *q, *k, *vv, *o, *gi, *ge, *ue, *de;
    const GgufTensor *n1, *n2, *qn, *kn;
    if (!want(b + "attn_norm.weight", {H}, &n1) || !want(b + "ffn_norm.weight", {H}, &n2) ||
        !want(b + "attn_q.weight", {H, QD}, &q) || !want(b + "attn_k.weight", {H, KVD}, &k) ||
        !want(b + "attn_v.weight", {H, KVD}, &vv) || !want(b + "attn_output.weight", {QD, H}, &o) ||
        !want(b + "attn_q_norm.weight", {c->head_dim}, &qn) ||
        !want(b + "attn_k_norm.weight", {c->head_dim}, &kn) ||
        !want(b + "ffn_gate_inp.weight", {H, E}, &gi) ||
        !want(b + "ffn_gate_exps.weight", {H, F, E}, &ge) ||
        !want(b + "ffn_up_exps.weight", {H, F, E}, &ue) ||
        !want(b + "ffn_down_exps.weight", {F, H, E}, &de))
      return KNJ_E_ARG;
    for (const GgufTensor* t : {n1, n2, qn, kn, gi, on})
      if (t->type != KNJ_TYPE_F32) {
        set_error("model: tensor '" + t->name + "' must be F32 on this path");
        return KNJ_E_ARG;
      }
    if (il == 0) {
      c->type_attn = (int32_t)q->type;
      c->type_gate_up = (int32_t)ge->type;
      c->type_down = (int32_t)de->type;
    }
    if ((int32_t)q->type != c->type_attn || (int32_t)k->type != c->type_attn ||
        (int32_t)vv->type != c->type_attn || (int32_t)o->type != c->type_attn ||
        (int32_t)ge->type != c->type_gate_up || (int32_t)ue->type != c->type_gate_up ||
        (int32_t)de->type != c->type_down) {
      set_error("model: layer " + std::to_string(il) +
                " mixes weight types; this path needs one type per projection kind");
      return KNJ_E_ARG;
    }
  }
  c->init_std = 0.0f;
  return KNJ_OK;
}

}  // namespace

int knj_gguf_probe(const char* path, int n_ctx, knj_model_config* out) {
  KNJ_CHECK_ARG(path && out, "null pointer");
  GgufView g;
  if (!g.open(path)) {
    set_error("gguf: " + g.error());
    return KNJ_E_ARG;
  }
  int rc = gguf_config(g, n_ctx, out);
  if (rc) return rc;
  return validate(out);
}

int knj_model_create_from_gguf(const char* path, int n_ctx, knj_model** out) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(path && out, "null pointer");
  GgufView g;
  if (!g.open(path)) {
    set_error("gguf: " + g.error());
    return KNJ_E_ARG;
  }
  knj_model_config c;
  if ((rc = gguf_config(g, n_ctx, &c)) || (rc = validate(&c))) return rc;
  knj_model* m = new knj_model();
  m->c = c;
  if ((rc = setup(m))) {
    knj_model_free(m);
    return rc;
  }
  // each tensor straight from the mapping to its place in the image; the
  // layer's Q, K and V rows back to back form wqkv
  auto put = [&](const char* name, uint64_t off) -> int {
    const GgufTensor* t = g.find(name);
    if (hipMemcpy(m->image + off, g.data(*t), t->bytes, hipMemcpyHostToDevice) != hipSuccess)
      return hip_fail(hipErrorUnknown, "image upload");
    m->h2d_bytes += t->bytes;
    return KNJ_OK;
  };
  rc = put("token_embd.weight", m->off_embd);
  if (!rc) rc = put("output_norm.weight", m->off_onorm);
  if (!rc) rc = put("output.weight", m->off_head);
  const uint64_t rqkv = knj_row_bytes(c.type_attn, (uint64_t)c.n_embd);
  const uint64_t QD = (uint64_t)c.n_head * c.head_dim, KVD = (uint64_t)c.n_head_kv * c.head_dim;
  for (int il = 0; il < c.n_layer && !rc; ++il) {
    const std::string b = "blk." + std::to_string(il) + ".";
    const knj_layer_offsets& lo = m->lo[il];
    const std::pair<const char*, uint64_t> parts[] = {
        {"attn_norm.weight", lo.attn_norm}, {"ffn_norm.weight", lo.ffn_norm},
        {"attn_q_norm.weight", lo.q_norm},  {"attn_k_norm.weight", lo.k_norm},
        {"attn_q.weight", lo.wqkv},         {"attn_k.weight", lo.wqkv + rqkv * QD},
        {"attn_v.weight", lo.wqkv + rqkv * (QD + KVD)},
        {"attn_output.weight", lo.wo},      {"ffn_gate_inp.weight", lo.router},
        {"ffn_gate_exps.weight", lo.gate},  {"ffn_up_exps.weight", lo.up},
        {"ffn_down_exps.weight", lo.down}};
    for (const auto& pr : parts) {
      if ((rc = put((b + pr.first).c_str(), pr.second))) break;
    }
  }
  if (rc) {
    knj_model_free(m);
    return rc;
  }
  return finish_create(m, out);
}

int knj_model_config_get(const knj_model* m, knj_model_config* out) {
  KNJ_CHECK_ARG(m && out, "null pointer");
  *out = m->c;
  return KNJ_OK;
}

int knj_model_create_from_image(const knj_model_config* cfg, const void* image, uint64_t bytes,
                                knj_model** out) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(out && image, "null pointer");
  if ((rc = validate(cfg))) return rc;
  knj_model* m = new knj_model();
  m->c = *cfg;
  if ((rc = setup(m))) {
    knj_model_free(m);
    return rc;
  }
  if (bytes != m->image_bytes) {
    knj_model_free(m);
    set_error("image size does not match the configuration's layout");
    return KNJ_E_ARG;
  }
  m->h2d_bytes += bytes;
  if (hipMemcpy(m->image, image, bytes, hipMemcpyHostToDevice) != hipSuccess) {
    knj_model_free(m);
    return hip_fail(hipErrorUnknown, "image upload");
  }
  return finish_create(m, out);
}

int knj_model_free(knj_model* m) {
  if (!m) return KNJ_OK;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  if (m->exec) (void)hipGraphExecDestroy(m->exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  if (m->exec_multi) (void)hipGraphExecDestroy(m->exec_multi);
  if (m->graph_multi) (void)hipGraphDestroy(m->graph_multi);
  for (void* p : m->owned) (void)hipFree(p);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
  return KNJ_OK;
}

uint64_t knj_model_image_bytes(const knj_model* m) { return m ? m->image_bytes : 0; }
const void* knj_model_image_device(const knj_model* m) { return m ? m->image : nullptr; }

int knj_model_download_image(const knj_model* m, void* host, uint64_t bytes) {
  KNJ_CHECK_ARG(m && host && bytes == m->image_bytes, "bad image download arguments");
  KNJ_HIP(hipMemcpy(host, m->image, bytes, hipMemcpyDeviceToHost));
  m->d2h_bytes += bytes;
  return KNJ_OK;
}

int knj_model_reset(knj_model* m) {
  KNJ_CHECK_ARG(m, "null model");
  const uint64_t kv = knj_kv_elems(&m->c);
  KNJ_HIP(hipMemsetAsync(m->kv_k, 0, kv * 2, m->stream));
  KNJ_HIP(hipMemsetAsync(m->kv_v, 0, kv * 2, m->stream));
  KNJ_HIP(hipStreamSynchronize(m->stream));
  m->pos = 0;
  return KNJ_OK;
}

int knj_model_pos(const knj_model* m) { return m ? m->pos : -1; }

int knj_model_set_pos(knj_model* m, int pos) {
  KNJ_CHECK_ARG(m && pos >= 0 && pos <= m->c.n_ctx, "position outside the context");
  m->pos = pos;
  return KNJ_OK;
}

int knj_model_forward(knj_model* m, const int32_t* tokens, int n, float* logits_host) {
  KNJ_CHECK_ARG(m && tokens, "null pointer");
  KNJ_CHECK_ARG(n > 0, "forward needs at least one token");
  if (m->pos + n > m->c.n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  for (int t = 0; t < n; ++t) {
    KNJ_CHECK_ARG(tokens[t] >= 0 && tokens[t] < m->c.n_vocab, "token id out of range");
  }
  const char* ps = std::getenv("KNJ_PROMPT_STEPS");
  if (n > 1 && prefill_eligible(m) && !(ps && ps[0] == '1')) {
    const int rc = prefill(m, tokens, n);
    if (rc) return rc;
  } else {
    for (int t = 0; t < n; ++t) {
      int rc = set_state(m, tokens[t], 0);
      if (rc) return rc;
      if ((rc = run_step(m))) return rc;
      m->pos += 1;
    }
  }
  if (logits_host) {
    KNJ_HIP(hipMemcpyAsync(logits_host, m->logits, (uint64_t)m->c.n_vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
    m->d2h_bytes += (uint64_t)m->c.n_vocab * 4;
  }
  KNJ_HIP(hipStreamSynchronize(m->stream));
  return KNJ_OK;
}

int knj_model_fill_kv(knj_model* m, int n_pos, uint64_t seed) {
  KNJ_CHECK_ARG(m && n_pos >= 0 && n_pos <= m->c.n_ctx, "bad arguments");
  const knj_model_config& c = m->c;
  int rc = fill_kv_rows(m->kv_k, m->kv_v, (uint64_t)c.n_layer * c.n_head_kv,
                        (uint64_t)c.n_ctx * c.head_dim, (uint64_t)n_pos * c.head_dim, seed, m->stream);
  if (rc) return rc;
  KNJ_HIP(hipStreamSynchronize(m->stream));
  m->pos = n_pos;
  return KNJ_OK;
}

uint64_t knj_model_layer_offsets(const knj_model_config* c, int il, knj_layer_offsets* out) {
  if (!c || !out || il < 0 || il >= c->n_layer) return 0;
  return knj_model_layout(c, il, out, nullptr, nullptr, nullptr);
}

int knj_model_decode_greedy(knj_model* m, int32_t first, int steps, int32_t* out_tokens) {
  KNJ_CHECK_ARG(m && out_tokens, "null pointer");
  KNJ_CHECK_ARG(steps > 0 && steps <= m->max_steps, "steps out of range");
  KNJ_CHECK_ARG(first >= 0 && first < m->c.n_vocab, "token id out of range");
  if (m->pos + steps > m->c.n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  int rc = set_state(m, first, 0);
  if (rc) return rc;
  if ((rc = run_steps(m, steps))) return rc;
  m->pos += steps;
  KNJ_HIP(hipMemcpyAsync(out_tokens, m->out_tokens, (uint64_t)steps * 4, hipMemcpyDeviceToHost, m->stream));
  m->d2h_bytes += (uint64_t)steps * 4;
  KNJ_HIP(hipStreamSynchronize(m->stream));
  return KNJ_OK;
}

int knj_model_hidden(const knj_model* m, int il, float* host_out) {
  KNJ_CHECK_ARG(m && host_out && il >= 0 && il < m->c.n_layer, "bad arguments");
  KNJ_HIP(hipMemcpy(host_out, m->hidden + (uint64_t)il * m->c.n_embd, (uint64_t)m->c.n_embd * 4,
                    hipMemcpyDeviceToHost));
  m->d2h_bytes += (uint64_t)m->c.n_embd * 4;
  return KNJ_OK;
}

int knj_model_topk(const knj_model* m, int il, int32_t* idx_out, float* w_out) {
  KNJ_CHECK_ARG(m && idx_out && w_out && il >= 0 && il < m->c.n_layer, "bad arguments");
  const uint64_t k = m->c.n_expert_used;
  KNJ_HIP(hipMemcpy(idx_out, m->topk_idx + il * k, k * 4, hipMemcpyDeviceToHost));
  m->d2h_bytes += k * 4;
  KNJ_HIP(hipMemcpy(w_out, m->topk_w + il * k, k * 4, hipMemcpyDeviceToHost));
  m->d2h_bytes += k * 4;
  return KNJ_OK;
}

int knj_model_logits(const knj_model* m, float* host_out) {
  KNJ_CHECK_ARG(m && host_out, "bad arguments");
  KNJ_HIP(hipMemcpy(host_out, m->logits, (uint64_t)m->c.n_vocab * 4, hipMemcpyDeviceToHost));
  m->d2h_bytes += (uint64_t)m->c.n_vocab * 4;
  return KNJ_OK;
}

int knj_model_kv_download(const knj_model* m, uint16_t* k_host, uint16_t* v_host) {
  KNJ_CHECK_ARG(m && k_host && v_host, "bad arguments");
  const uint64_t kv = knj_kv_elems(&m->c) * 2;
  KNJ_HIP(hipMemcpy(k_host, m->kv_k, kv, hipMemcpyDeviceToHost));
  m->d2h_bytes += kv;
  KNJ_HIP(hipMemcpy(v_host, m->kv_v, kv, hipMemcpyDeviceToHost));
  m->d2h_bytes += kv;
  return KNJ_OK;
}

int knj_model_kv_upload(knj_model* m, const uint16_t* k_host, const uint16_t* v_host) {
  KNJ_CHECK_ARG(m && k_host && v_host, "bad arguments");
  const uint64_t kv = knj_kv_elems(&m->c) * 2;
  KNJ_HIP(hipMemcpy(m->kv_k, k_host, kv, hipMemcpyHostToDevice));
  m->h2d_bytes += kv;
  KNJ_HIP(hipMemcpy(m->kv_v, v_host, kv, hipMemcpyHostToDevice));
  m->h2d_bytes += kv;
  return KNJ_OK;
}

int knj_model_time_decode(knj_model* m, int iters, float* ms_out) {
  KNJ_CHECK_ARG(m && ms_out && iters > 0, "bad arguments");
  if (m->pos + iters > m->c.n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  int rc = set_state(m, 0, 0);
  if (rc) return rc;
  hipEvent_t a, b;
  KNJ_HIP(hipEventCreate(&a));
  KNJ_HIP(hipEventCreate(&b));
  KNJ_HIP(hipEventRecord(a, m->stream));
  if ((rc = run_steps(m, iters))) return rc;
  KNJ_HIP(hipEventRecord(b, m->stream));
  KNJ_HIP(hipEventSynchronize(b));
  KNJ_HIP(hipEventElapsedTime(ms_out, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  m->pos += iters;
  return KNJ_OK;
}

int knj_model_time_experts(knj_model* m, int steps, float* us_gateup, float* us_down) {
  KNJ_CHECK_ARG(m && us_gateup && us_down && steps > 0 && steps <= 64, "bad arguments");
  if (m->pos + steps > m->c.n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  const int n = 6 * m->c.n_layer * steps;
  std::vector<hipEvent_t> ev(n, nullptr);
  for (auto& e : ev) KNJ_HIP(hipEventCreate(&e));
  // greedy decode from token 0, the step's kernels launched directly; every
  // expert launch records start/end events of its own execution
  int rc = set_state(m, 0, 0);
  m->expert_events = ev.data();
  m->expert_slot = 0;
  for (int i = 0; i < steps && !rc; ++i) rc = enqueue_step(m, m->stream);
  m->expert_events = nullptr;
  if (!rc) {
    const hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
  }
  double gu = 0.0, dn = 0.0;
  for (int i = 0; i < m->c.n_layer * steps && !rc; ++i) {
    float a = 0.0f, b = 0.0f;
    hipError_t e = hipEventElapsedTime(&a, ev[6 * i], ev[6 * i + 1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&b, ev[6 * i + 2], ev[6 * i + 3]);
    if (e != hipSuccess) rc = hip_fail(e, "hipEventElapsedTime");
    gu += a;
    dn += b;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  if (rc) return rc;
  m->pos += steps;
  const double launches = (double)m->c.n_layer * steps;
  *us_gateup = (float)(gu * 1000.0 / launches);
  *us_down = (float)(dn * 1000.0 / launches);
  return KNJ_OK;
}

int knj_model_profile(knj_model* m, int32_t first, int steps, int32_t* out_tokens, knj_span* spans,
                      int cap, int* n_spans, uint64_t* n_dropped) {
  KNJ_CHECK_ARG(m && out_tokens && spans && n_spans, "null pointer");
  KNJ_CHECK_ARG(cap > 0 && cap <= (1 << 20), "span capacity out of range");
  KNJ_CHECK_ARG(steps > 0 && steps <= m->max_steps, "steps out of range");
  KNJ_CHECK_ARG(first >= 0 && first < m->c.n_vocab, "token id out of range");
  if (m->pos + steps > m->c.n_ctx) {
    set_error("context exhausted");
    return KNJ_E_ARG;
  }
  int rc = set_state(m, first, 0);
  if (rc) return rc;
  SpanRun run(cap);
  if (run.err != hipSuccess) return hip_fail(run.err, "hipEventCreate");
  KNJ_HIP(hipEventRecord(run.epoch, m->stream));
  for (int i = 0; i < steps && !rc; ++i) rc = enqueue_step(m, m->stream);
  run.stop();
  if (rc) return rc;
  KNJ_HIP(hipStreamSynchronize(m->stream));
  m->pos += steps;
  KNJ_HIP(hipMemcpy(out_tokens, m->out_tokens, (uint64_t)steps * 4, hipMemcpyDeviceToHost));
  m->d2h_bytes += (uint64_t)steps * 4;
  return run.collect(spans, cap, n_spans, n_dropped);
}

int knj_model_transfer_bytes(const knj_model* m, uint64_t* h2d, uint64_t* d2h) {
  KNJ_CHECK_ARG(m && h2d && d2h, "null pointer");
  *h2d = m->h2d_bytes;
  *d2h = m->d2h_bytes;
  return KNJ_OK;
}

int knj_device_floor(int n, uint64_t* ns_out) {
  KNJ_CHECK_ARG(ns_out && n > 0 && n <= 4096, "bad arguments");
  hipStream_t s = nullptr;
  KNJ_HIP(hipStreamCreate(&s));
  std::vector<knj_span> sp((size_t)n);
  int got = 0, rc = KNJ_OK;
  // the first launches of a kernel pay for loading its code object; they are
  // not part of the floor
  for (int i = 0; i < 8 && !rc; ++i) {
    hipLaunchKernelGGL(k_span_floor, dim3(1), dim3(64), 0, s, 0);
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = hip_fail(e, "k_span_floor");
  }
  {
    SpanRun run(n);
    if (run.err != hipSuccess) rc = hip_fail(run.err, "hipEventCreate");
    if (!rc) {
      const hipError_t e = hipEventRecord(run.epoch, s);
      if (e != hipSuccess) rc = hip_fail(e, "hipEventRecord");
    }
    for (int i = 0; i < n && !rc; ++i) {
      KNJ_LAUNCH(k_span_floor, dim3(1), dim3(64), 0, s, 0);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) rc = hip_fail(e, "k_span_floor");
    }
    run.stop();
    if (!rc) {
      const hipError_t e = hipStreamSynchronize(s);
      if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    if (!rc) rc = run.collect(sp.data(), n, &got, nullptr);
  }
  (void)hipStreamDestroy(s);
  if (rc) return rc;
  // the median span: robust to the odd launch delayed by the host
  std::vector<uint64_t> d((size_t)got);
  for (int i = 0; i < got; ++i) d[(size_t)i] = sp[(size_t)i].end_ns - sp[(size_t)i].start_ns;
  std::sort(d.begin(), d.end());
  *ns_out = got ? d[(size_t)got / 2] : 0;
  return KNJ_OK;
}

}  // extern "C"
