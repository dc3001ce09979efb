// kanjoos_amd/csrc/knj_prefill.hip -- Model::forward over a prompt of n > 1
// tokens in one pass (/root/reference/src/model/model.cpp:512-672).
//
// The reference feeds all n rows through each weight matrix together
// (matmul with m = n), appends every row's key and value before any
// attention, lets row t attend over slots 0 .. pos + t, runs the MoE over the
// n rows and applies the final norm and the head to the last row only.  Here
// the prompt is cut into chunks of up to kRows rows (each row's result does
// not depend on which rows share its chunk), and per chunk and layer:
//   RMSNorm rows -> QKV GEMM (matrix cores) -> q/k norm + RoPE + f16 append of
//   every row -> causal attention (64 query columns per workgroup) -> O GEMM +
//   residual -> MoE over the rows (router, top-k, grouped experts, combine +
//   residual),
// then the final RMSNorm + LM head GEMV of the prompt's last row.  The last
// row's per-layer residual, router logits and top-k are copied where the
// decode step keeps them, so the model reads the same after a prompt pass as
// after single steps.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "knj_common.h"
#include "knj_model_impl.h"

namespace knj {
namespace {

constexpr int kRows = 512;

__global__ void k_embed_rows(int type, const uint8_t* __restrict__ table, int n_embd,
                             const int32_t* __restrict__ tokens, float* __restrict__ x) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_embd) return;
  const uint64_t idx = (uint64_t)tokens[t] * n_embd + i;
  x[(uint64_t)t * n_embd + i] =
      type == KNJ_TYPE_BF16
          ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(table)[idx] << 16)
          : reinterpret_cast<const float*>(table)[idx];
}

// The last row's residual, router logits and routing into the decode step's
// per-layer slots (one launch instead of four copies).
__global__ void k_keep_last(const float* __restrict__ x, const float* __restrict__ logits,
                            const int32_t* __restrict__ idx, const float* __restrict__ w, int H,
                            int E, int K, float* __restrict__ hidden, float* __restrict__ rlog,
                            int32_t* __restrict__ tk_idx, float* __restrict__ tk_w) {
  for (int i = threadIdx.x; i < H; i += blockDim.x) hidden[i] = x[i];
  for (int i = threadIdx.x; i < E; i += blockDim.x) rlog[i] = logits[i];
  if ((int)threadIdx.x < K) {
    tk_idx[threadIdx.x] = idx[threadIdx.x];
    tk_w[threadIdx.x] = w[threadIdx.x];
  }
}

int palloc(knj_model* m, void** p, uint64_t bytes) {
  KNJ_HIP(hipMalloc(p, std::max<uint64_t>(bytes, 256)));
  m->owned.push_back(*p);
  return KNJ_OK;
}

int ensure_bufs(knj_model* m) {
  knj_prefill_bufs& b = m->pf;
  if (b.cap) return KNJ_OK;
  const knj_model_config& c = m->c;
  const int R = kRows, H = c.n_embd, QD = c.n_head * c.head_dim;
  const int QKV = QD + 2 * c.n_head_kv * c.head_dim;
  int rc = KNJ_OK;
  auto A = [&](void** p, uint64_t bytes) {
    if (!rc) rc = palloc(m, p, bytes);
  };
  A((void**)&b.x, (uint64_t)R * H * 4);
  A((void**)&b.hx, (uint64_t)R * H * 4);
  A((void**)&b.qkv, (uint64_t)R * QKV * 4);
  A((void**)&b.ctx, (uint64_t)R * QD * 4);
  A((void**)&b.router_logits, (uint64_t)R * c.n_expert * 4);
  A((void**)&b.topk_idx, (uint64_t)R * c.n_expert_used * 4);
  A((void**)&b.topk_w, (uint64_t)R * c.n_expert_used * 4);
  A((void**)&b.tokens, (uint64_t)R * 4);
  A((void**)&b.attn_part, prefill_partial_bytes(c.n_head, c.n_head_kv, c.head_dim, R));
  A(&b.scratch, std::max({moe_batch_scratch_bytes(R, H, c.n_ff, c.n_expert, c.n_expert_used),
                          dense_scratch_bytes(R, H, QKV), dense_scratch_bytes(R, QD, H)}));
  {
    // [hi | lo | sums hi | sums lo] as split_operand_bytes lays them out
    void* os = nullptr;
    A(&os, split_operand_bytes(R, H));
    if (!rc) {
      uint8_t* q = (uint8_t*)os;
      const uint64_t hb = ((uint64_t)R * H * 2 + 255) & ~255ull, sb = ((uint64_t)R * H / 16 + 255) & ~255ull;
      b.qsplit[0] = (_Float16*)q;
      b.qsplit[1] = (_Float16*)(q + hb);
      b.qsplit[2] = (_Float16*)(q + 2 * hb);
      b.qsplit[3] = (_Float16*)(q + 2 * hb + sb);
    }
  }
  if (!rc) b.cap = R;
  return rc;
}

// One chunk of n <= kRows rows at positions m->pos ...
int prefill_chunk(knj_model* m, const int32_t* tokens, int n, bool last) {
  const knj_model_config& c = m->c;
  knj_prefill_bufs& b = m->pf;
  const hipStream_t s = m->stream;
  const int H = c.n_embd, D = c.head_dim, QD = c.n_head * D, KVD = c.n_head_kv * D;
  const int QKV = QD + 2 * KVD, E = c.n_expert, K = c.n_expert_used;
  const uint8_t* img = m->image;
  KNJ_HIP(hipMemcpyAsync(b.tokens, tokens, (uint64_t)n * 4, hipMemcpyHostToDevice, s));
  m->h2d_bytes += (uint64_t)n * 4;
  k_embed_rows<<<dim3((H + 255) / 256, n), dim3(256), 0, s>>>(c.type_embd, img + m->off_embd, H,
                                                             b.tokens, b.x);
  KNJ_HIP(hipGetLastError());
  const float* lastx = b.x + (uint64_t)(n - 1) * H;
  // layer 0's QKV operand; every later one comes from the previous layer's
  // MoE combine (split operand of the split rows, in place of x's norm and split)
  KNJ_HIP(launch_norm_split(b.x, reinterpret_cast<const float*>(img + m->lo[0].attn_norm), c.rms_eps,
                            n, H, nullptr, b.qsplit, s));
  for (int il = 0; il < c.n_layer; ++il) {
    const knj_layer_offsets& lo = m->lo[il];
    const uint64_t kv_layer = (uint64_t)il * c.n_head_kv * c.n_ctx * D;
    {
      const _Float16* pre[4] = {b.qsplit[0], b.qsplit[1], b.qsplit[2], b.qsplit[3]};
      DenseQ4Extra qx;
      qx.pre = pre;
      KNJ_HIP(launch_dense_q4k_ex(img + lo.wqkv, H, QKV, n, nullptr, nullptr, b.qkv, b.scratch, qx, s));
    }
    PrefillAttnArgs pa{b.qkv, QKV,
                       reinterpret_cast<const float*>(img + lo.q_norm),
                       reinterpret_cast<const float*>(img + lo.k_norm), c.rms_eps, m->rope_cos,
                       m->rope_sin, m->pos, n, m->kv_k + kv_layer, m->kv_v + kv_layer, c.n_head,
                       c.n_head_kv, D, c.n_ctx, 1.0f / std::sqrt((float)D), b.ctx, b.attn_part,
                       prefill_partial_bytes(c.n_head, c.n_head_kv, D, b.cap)};
    KNJ_HIP(launch_prefill_attention(pa, s));
    // the O product's last launch also writes the ffn-normalised rows the MoE takes
    DenseQ4Extra ox;
    ox.norm_w = reinterpret_cast<const float*>(img + lo.ffn_norm);
    ox.eps = c.rms_eps;
    ox.norm_out = b.hx;
    KNJ_HIP(launch_dense_q4k_ex(img + lo.wo, QD, H, n, b.ctx, b.x, b.x, b.scratch, ox, s));
    MoeBatchArgs ma{b.hx, nullptr, c.rms_eps,
                    reinterpret_cast<const float*>(img + lo.router), img + lo.gate, img + lo.up,
                    img + lo.down, n, H, c.n_ff, E, K, b.x, b.x, b.router_logits, b.topk_idx,
                    b.topk_w};
    ma.type_down = c.type_down;
    if (il + 1 < c.n_layer) {
      ma.next_norm_w = reinterpret_cast<const float*>(img + m->lo[il + 1].attn_norm);
      ma.next_eps = c.rms_eps;
      ma.next_split = b.qsplit;
    }
    KNJ_HIP(launch_moe_batch(ma, b.scratch, s));
    if (last) {
      const uint64_t r = (uint64_t)(n - 1);
      k_keep_last<<<1, 256, 0, s>>>(lastx, b.router_logits + r * E, b.topk_idx + r * K,
                                    b.topk_w + r * K, H, E, K, m->hidden + (uint64_t)il * H,
                                    m->router_logits + (uint64_t)il * E,
                                    m->topk_idx + (uint64_t)il * K, m->topk_w + (uint64_t)il * K);
      KNJ_HIP(hipGetLastError());
    }
  }
  if (last) {
    // final RMSNorm + head of the last row (model.cpp:662-667), the decode
    // step's fused GEMV
    GemvArgs head{c.type_head, img + m->off_head, H, c.n_vocab, lastx,
                  reinterpret_cast<const float*>(img + m->off_onorm), c.rms_eps, nullptr,
                  m->logits, nullptr};
    KNJ_HIP(launch_gemv(head, s));
  }
  m->pos += n;
  return KNJ_OK;
}

}  // namespace

bool prefill_eligible(const knj_model* m) {
  const knj_model_config& c = m->c;
  const int QD = c.n_head * c.head_dim;
  return c.type_attn == KNJ_TYPE_Q4_K && c.type_gate_up == KNJ_TYPE_Q4_K &&
         (c.type_down == KNJ_TYPE_Q4_K || c.type_down == KNJ_TYPE_Q6_K) &&
         c.type_head != KNJ_TYPE_Q4_K &&
         c.n_embd % 256 == 0 && c.n_embd <= 4096 && QD % 256 == 0 && QD <= 4096 &&
         c.n_ff % 256 == 0 && c.n_ff <= 4096 && c.n_expert <= 256 && c.n_expert_used <= 16 &&
         prefill_attention_ok(c.n_head, c.n_head_kv, c.head_dim);
}

int prefill(knj_model* m, const int32_t* tokens, int n) {
  int rc = ensure_bufs(m);
  for (int i = 0; !rc && i < n; i += kRows) {
    const int cnt = std::min(kRows, n - i);
    rc = prefill_chunk(m, tokens + i, cnt, i + cnt == n);  // stream-ordered: chunks share buffers
  }
  return rc;
}

}  // namespace knj
