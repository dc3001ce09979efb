/* include/knj_model.h -- geometry of the Qwen3-MoE decode model and the byte
 * layout of its weights, shared by the GPU library and the CPU oracle.
 *
 * Geometry fields mirror the reference's ModelGeometry
 * (/root/reference/src/model/model.h:32-53); the weights are the tensors that
 * Model::bind_tensors requires (/root/reference/src/model/model.cpp:129-172),
 * each stored as ggml stores it: a 2-D [n_in, n_out] tensor is n_out rows of
 * n_in weights, a 3-D expert tensor is n_expert such slabs back to back.
 *
 * Layout in one contiguous weight image (every tensor 256-byte aligned):
 *
 *   token_embd   [n_vocab][n_embd]                       type_embd
 *   per layer il = 0 .. n_layer-1:
 *     attn_norm [n_embd] f32, ffn_norm [n_embd] f32,
 *     q_norm [head_dim] f32, k_norm [head_dim] f32
 *     wqkv      [q_dim + 2*kv_dim][n_embd]                type_attn
 *               (attn_q rows, then attn_k rows, then attn_v rows, so the
 *                three projections are one row-contiguous matrix)
 *     wo        [n_embd][q_dim]                           type_attn
 *     router    [n_expert][n_embd] f32                    (ffn_gate_inp)
 *     gate      [n_expert][n_ff][n_embd]                  type_gate_up
 *     up        [n_expert][n_ff][n_embd]                  type_gate_up
 *     down      [n_expert][n_embd][n_ff]                  type_down
 *   output_norm  [n_embd] f32
 *   output       [n_vocab][n_embd]                        type_head
 *
 * The KV cache is f16, [n_layer][n_head_kv][n_ctx][head_dim] for K and the same
 * for V: one head's history is contiguous, which is what a decode-attention
 * pass streams.
 */
#ifndef KNJ_MODEL_H
#define KNJ_MODEL_H

#include <stdint.h>

#include "knj_format.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct knj_model_config {
  int32_t n_layer;
  int32_t n_embd;
  int32_t n_head;
  int32_t n_head_kv;
  int32_t head_dim;
  int32_t n_ff;          /* per-expert intermediate width */
  int32_t n_expert;
  int32_t n_expert_used;
  int32_t n_vocab;
  int32_t n_ctx;         /* KV capacity in tokens */
  float rms_eps;
  float rope_base;
  int32_t type_embd;     /* KNJ_TYPE_BF16 or KNJ_TYPE_F32 */
  int32_t type_attn;     /* KNJ_TYPE_Q4_K or KNJ_TYPE_Q6_K */
  int32_t type_gate_up;  /* KNJ_TYPE_Q4_K or KNJ_TYPE_Q6_K */
  int32_t type_down;     /* KNJ_TYPE_Q4_K or KNJ_TYPE_Q6_K */
  int32_t type_head;     /* KNJ_TYPE_BF16, KNJ_TYPE_Q4_K or KNJ_TYPE_Q6_K */
  float init_std;        /* stddev of the synthetic weights */
} knj_model_config;

typedef struct knj_layer_offsets {
  uint64_t attn_norm, ffn_norm, q_norm, k_norm;
  uint64_t wqkv, wo, router, gate, up, down;
} knj_layer_offsets;

static inline uint64_t knj_align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

/* Byte offsets of the global tensors and of layer `il` inside the weight image;
 * returns the total image size. */
static inline uint64_t knj_model_layout(const knj_model_config* c, int il, knj_layer_offsets* lo,
                                        uint64_t* off_embd, uint64_t* off_out_norm,
                                        uint64_t* off_head) {
  const uint64_t H = (uint64_t)c->n_embd;
  const uint64_t QD = (uint64_t)c->n_head * (uint64_t)c->head_dim;
  const uint64_t KVD = (uint64_t)c->n_head_kv * (uint64_t)c->head_dim;
  const uint64_t F = (uint64_t)c->n_ff, E = (uint64_t)c->n_expert, V = (uint64_t)c->n_vocab;
  uint64_t p = 0;
  if (off_embd) *off_embd = p;
  p = knj_align256(p + knj_row_bytes(c->type_embd, H) * V);
  uint64_t layer_bytes = 0;
  for (int l = 0; l < c->n_layer; ++l) {
    knj_layer_offsets t;
    const uint64_t start = p;
    t.attn_norm = p; p = knj_align256(p + 4 * H);
    t.ffn_norm = p;  p = knj_align256(p + 4 * H);
    t.q_norm = p;    p = knj_align256(p + 4 * (uint64_t)c->head_dim);
    t.k_norm = p;    p = knj_align256(p + 4 * (uint64_t)c->head_dim);
    t.wqkv = p;      p = knj_align256(p + knj_row_bytes(c->type_attn, H) * (QD + 2 * KVD));
    t.wo = p;        p = knj_align256(p + knj_row_bytes(c->type_attn, QD) * H);
    t.router = p;    p = knj_align256(p + 4 * H * E);
    t.gate = p;      p = knj_align256(p + knj_row_bytes(c->type_gate_up, H) * F * E);
    t.up = p;        p = knj_align256(p + knj_row_bytes(c->type_gate_up, H) * F * E);
    t.down = p;      p = knj_align256(p + knj_row_bytes(c->type_down, F) * H * E);
    layer_bytes = p - start;
    if (l == il && lo) *lo = t;
  }
  (void)layer_bytes;
  if (off_out_norm) *off_out_norm = p;
  p = knj_align256(p + 4 * H);
  if (off_head) *off_head = p;
  p = knj_align256(p + knj_row_bytes(c->type_head, H) * V);
  return p;
}

/* Elements of one K (or V) cache: n_layer * n_head_kv * n_ctx * head_dim. */
static inline uint64_t knj_kv_elems(const knj_model_config* c) {
  return (uint64_t)c->n_layer * (uint64_t)c->n_head_kv * (uint64_t)c->n_ctx * (uint64_t)c->head_dim;
}

#ifdef __cplusplus
}
#endif

#endif /* KNJ_MODEL_H */
