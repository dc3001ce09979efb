// oracle/knj_oracle.cpp -- CPU restatement of Kanjoos's qwen3moe forward pass.
//
// TEST INFRASTRUCTURE: the checker for the GPU path and the CPU baseline of the
// benchmark.  Nothing in the product links it.
//
// Every function states the reference lines it follows.  The order of
// floating-point operations is the reference's (sequential f32 sums in the
// loops' order, the same association of each expression); the build uses
// -ffp-contract=off so no a*b+c is fused that the reference's own x86-64 build
// (no -mfma, no -march) would not fuse either.
#include "knj_oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../include/knj_format.h"
#include "../include/knj_synth.h"

namespace {

thread_local std::string g_err;

// ---------------------------------------------------------------- thread pool
// Persistent workers; for_each(count, fn) hands out indices from a shared
// counter and the calling thread takes part, as the reference's
// ThreadPool::for_each does (/root/reference/src/util/parallel.cpp:54-86).
class Pool {
 public:
  explicit Pool(int threads) {
    int n = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
    if (n < 1) n = 1;
    total_ = n;
    for (int i = 1; i < n; ++i) workers_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  int total() const { return total_; }

  void for_each(int count, const std::function<void(int)>& fn) {
    if (count <= 0) return;
    if (total_ == 1 || count == 1) {
      for (int i = 0; i < count; ++i) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> g(mu_);
      fn_ = &fn;
      count_ = count;
      next_.store(0);
      busy_ = (int)workers_.size();
      ++gen_;
    }
    cv_.notify_all();
    run();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [this] { return busy_ == 0; });
    fn_ = nullptr;
  }

 private:
  void run() {
    for (;;) {
      const int i = next_.fetch_add(1);
      if (i >= count_) break;
      (*fn_)(i);
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
      }
      run();
      {
        std::lock_guard<std::mutex> g(mu_);
        if (--busy_ == 0) done_cv_.notify_all();
      }
    }
  }

  int total_ = 1;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int count_ = 0;
  std::atomic<int> next_{0};
  int busy_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

Pool& shared_pool(int threads) {
  static std::mutex mu;
  static std::unique_ptr<Pool> pool;
  std::lock_guard<std::mutex> g(mu);
  const int want = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
  if (!pool || pool->total() != want) pool.reset(new Pool(want));
  return *pool;
}

// ---------------------------------------------------------------- fused dots
// dot_q4_k (/root/reference/src/loader/dequant.cpp:954-984): per 64-weight
// group, four sequential sums (codes*x and x for both sub-blocks), then
// acc += (d1*sq0 - dm1*sx0) + (d2*sq1 - dm2*sx1).
float dot_q4k(const uint8_t* src, const float* x, uint64_t nb) {
  float acc = 0.0f;
  for (uint64_t b = 0; b < nb; ++b, src += KNJ_Q4K_BLOCK, x += KNJ_QK) {
    const float d = knj_f16_to_f32(knj_rd_u16(src + KNJ_Q4K_D));
    const float dmin = knj_f16_to_f32(knj_rd_u16(src + KNJ_Q4K_DMIN));
    for (int g = 0; g < 4; ++g) {
      uint32_t sc, mn;
      knj_q4k_sub_scale(src + KNJ_Q4K_SCALES, 2 * g, &sc, &mn);
      const float d1 = d * (float)sc, dm1 = dmin * (float)mn;
      knj_q4k_sub_scale(src + KNJ_Q4K_SCALES, 2 * g + 1, &sc, &mn);
      const float d2 = d * (float)sc, dm2 = dmin * (float)mn;
      const uint8_t* q = src + KNJ_Q4K_QS + 32 * g;
      const float* xg = x + 64 * g;
      float sq0 = 0.0f, sx0 = 0.0f, sq1 = 0.0f, sx1 = 0.0f;
      for (int l = 0; l < 32; ++l) {
        sq0 += (float)(q[l] & 0x0F) * xg[l];
        sx0 += xg[l];
        sq1 += (float)(q[l] >> 4) * xg[l + 32];
        sx1 += xg[l + 32];
      }
      acc += (d1 * sq0 - dm1 * sx0) + (d2 * sq1 - dm2 * sx1);
    }
  }
  return acc;
}

// dot_q6_k (dequant.cpp:986-1022): per 32-weight quarter, two sequential sums
// split at position 16, acc += d * (sc_a*s0 + sc_b*s1).
float dot_q6k(const uint8_t* src, const float* x, uint64_t nb) {
  float acc = 0.0f;
  for (uint64_t b = 0; b < nb; ++b, src += KNJ_Q6K_BLOCK, x += KNJ_QK) {
    const float d = knj_f16_to_f32(knj_rd_u16(src + KNJ_Q6K_D));
    const int8_t* sc = reinterpret_cast<const int8_t*>(src + KNJ_Q6K_SC);
    for (int h = 0; h < 2; ++h) {
      for (int t = 0; t < 4; ++t) {
        const float* xg = x + 128 * h + 32 * t;
        float s0 = 0.0f, s1 = 0.0f;
        for (int l = 0; l < 32; ++l) {
          const float v = (float)knj_q6k_code(src, 128 * h + 32 * t + l) * xg[l];
          if (l < 16) s0 += v;
          else s1 += v;
        }
        acc += d * ((float)sc[8 * h + 2 * t] * s0 + (float)sc[8 * h + 2 * t + 1] * s1);
      }
    }
  }
  return acc;
}

float dot_plain(int type, const uint8_t* src, const float* x, uint64_t n) {
  float acc = 0.0f;
  if (type == KNJ_TYPE_F32) {
    const float* w = reinterpret_cast<const float*>(src);
    for (uint64_t i = 0; i < n; ++i) acc += w[i] * x[i];
  } else if (type == KNJ_TYPE_F16) {
    for (uint64_t i = 0; i < n; ++i) acc += knj_f16_to_f32(knj_rd_u16(src + 2 * i)) * x[i];
  } else {
    for (uint64_t i = 0; i < n; ++i) acc += knj_bf16_to_f32(knj_rd_u16(src + 2 * i)) * x[i];
  }
  return acc;
}

void dequant_row(int type, const uint8_t* src, float* dst, uint64_t n) {
  switch (type) {
    case KNJ_TYPE_F32:
      std::memcpy(dst, src, n * 4);
      return;
    case KNJ_TYPE_F16:
      for (uint64_t i = 0; i < n; ++i) dst[i] = knj_f16_to_f32(knj_rd_u16(src + 2 * i));
      return;
    case KNJ_TYPE_BF16:
      for (uint64_t i = 0; i < n; ++i) dst[i] = knj_bf16_to_f32(knj_rd_u16(src + 2 * i));
      return;
    case KNJ_TYPE_Q4_K:
      // dequant_q4_k (dequant.cpp:102-125): d1*q - dm1 per weight
      for (uint64_t b = 0; b < n / KNJ_QK; ++b, src += KNJ_Q4K_BLOCK, dst += KNJ_QK) {
        for (int r = 0; r < KNJ_QK; ++r) dst[r] = knj_q4k_weight(src, r);
      }
      return;
    case KNJ_TYPE_Q6_K:
      // dequant_q6_k (dequant.cpp:164-191): d*sc*q, left to right
      for (uint64_t b = 0; b < n / KNJ_QK; ++b, src += KNJ_Q6K_BLOCK, dst += KNJ_QK) {
        for (int r = 0; r < KNJ_QK; ++r) dst[r] = knj_q6k_weight(src, r);
      }
      return;
    default:
      throw std::runtime_error("oracle: unsupported type " + std::to_string(type));
  }
}

// dequant_dot_f32 (dequant.cpp:1075-1112)
float dequant_dot(int type, const uint8_t* src, const float* x, uint64_t n) {
  if (type == KNJ_TYPE_Q4_K) return dot_q4k(src, x, n / KNJ_QK);
  if (type == KNJ_TYPE_Q6_K) return dot_q6k(src, x, n / KNJ_QK);
  return dot_plain(type, src, x, n);
}

// Model::matmul_plain (model.cpp:308-324): single-threaded, column decoded
// into a staging row, then a sequential dot per input row.
void matmul_plain(int type, const uint8_t* w, int n_in, int n_out, const float* x, int m, int ldx,
                  float* y, int ldy, std::vector<float>& col) {
  const uint64_t stride = knj_row_bytes(type, (uint64_t)n_in);
  col.resize((size_t)n_in);
  for (int j = 0; j < n_out; ++j) {
    dequant_row(type, w + (uint64_t)j * stride, col.data(), (uint64_t)n_in);
    for (int r = 0; r < m; ++r) {
      const float* xr = x + (size_t)r * ldx;
      float acc = 0.0f;
      for (int i = 0; i < n_in; ++i) acc += col[i] * xr[i];
      y[(size_t)r * ldy + j] = acc;
    }
  }
}

// Model::matmul (model.cpp:326-380): block-quantised weights; m == 1 is the
// fused decode-and-dot, m > 1 dequantises each 256-block once and dots every
// row with it, accumulating per block.  Columns are split over the pool in
// min(n_out, 4*threads) chunks once the work reaches 2^16.
void matmul(Pool& pool, int type, const uint8_t* w, int n_in, int n_out, const float* x, int m,
            int ldx, float* y, int ldy, std::vector<float>& col) {
  if (knj_block_weights(type) == 1) {
    matmul_plain(type, w, n_in, n_out, x, m, ldx, y, ldy, col);
    return;
  }
  const uint64_t stride = knj_row_bytes(type, (uint64_t)n_in);
  const uint64_t bb = knj_row_bytes(type, KNJ_QK);
  auto body = [&](int j0, int j1) {
    float buf[KNJ_QK];
    for (int j = j0; j < j1; ++j) {
      const uint8_t* src = w + (uint64_t)j * stride;
      if (m == 1) {
        y[j] = dequant_dot(type, src, x, (uint64_t)n_in);
        continue;
      }
      for (int r = 0; r < m; ++r) y[(size_t)r * ldy + j] = 0.0f;
      const int nblk = n_in / KNJ_QK;
      for (int b = 0; b < nblk; ++b) {
        dequant_row(type, src + (uint64_t)b * bb, buf, KNJ_QK);
        for (int r = 0; r < m; ++r) {
          const float* xr = x + (size_t)r * ldx + (size_t)b * KNJ_QK;
          float acc = 0.0f;
          for (int l = 0; l < KNJ_QK; ++l) acc += buf[l] * xr[l];
          y[(size_t)r * ldy + j] += acc;
        }
      }
    }
  };
  const uint64_t work = (uint64_t)n_in * (uint64_t)n_out * (uint64_t)m;
  if (work < (1ull << 16) || pool.total() <= 1) {
    body(0, n_out);
    return;
  }
  const int nt = std::min<int>(n_out, pool.total() * 4);
  const int per = (n_out + nt - 1) / nt;
  pool.for_each(nt, [&](int t) { body(t * per, std::min(n_out, (t + 1) * per)); });
}

// Model::rmsnorm / rmsnorm_rows (model.cpp:240-271): sequential sum of squares,
// scale = 1/sqrt(ss/width + eps), out = x*scale*w.
void rmsnorm(const float* x, const float* w, float* out, int width, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < width; ++i) ss += x[i] * x[i];
  const float scale = 1.0f / std::sqrt(ss / (float)width + eps);
  for (int i = 0; i < width; ++i) out[i] = x[i] * scale * w[i];
}

// Model::softmax (model.cpp:296-306)
void softmax(float* v, int n) {
  float mx = v[0];
  for (int i = 1; i < n; ++i) mx = std::max(mx, v[i]);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    v[i] = std::exp(v[i] - mx);
    sum += v[i];
  }
  const float inv = 1.0f / sum;
  for (int i = 0; i < n; ++i) v[i] *= inv;
}

// silu (model.cpp:47)
inline float silu(float x) { return x / (1.0f + std::exp(-x)); }

struct MoeScratch {
  std::vector<float> probs, gat, yg, yu, yd, col;
  std::vector<int> chosen;
  std::vector<std::vector<int32_t>> tok;
  std::vector<std::vector<float>> wt;
};

// Model::moe (model.cpp:399-510)
void moe(Pool& pool, const float* hx, int m, int H, int F, int E, int K, const float* router_w,
         const uint8_t* gate, const uint8_t* up, const uint8_t* down, int tgu, int tdn, float* out,
         float* logits, int32_t* topk_idx, float* topk_w, MoeScratch& s) {
  // router: F32 weights take the plain path (model.cpp:421-423)
  matmul(pool, KNJ_TYPE_F32, reinterpret_cast<const uint8_t*>(router_w), H, E, hx, m, H, logits, E,
         s.col);
  s.tok.assign((size_t)E, {});
  s.wt.assign((size_t)E, {});
  s.probs.resize((size_t)E);
  s.chosen.resize((size_t)K);
  for (int t = 0; t < m; ++t) {
    const float* lg = logits + (size_t)t * E;
    float mx = lg[0];
    for (int e = 1; e < E; ++e) mx = std::max(mx, lg[e]);
    float sum = 0.0f;
    for (int e = 0; e < E; ++e) {
      s.probs[e] = std::exp(lg[e] - mx);
      sum += s.probs[e];
    }
    for (int e = 0; e < E; ++e) s.probs[e] /= sum;
    // repeated strict-'>' argmax: ties keep the lower index (model.cpp:442-451)
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        bool taken = false;
        for (int q = 0; q < k; ++q) taken = taken || s.chosen[q] == e;
        if (taken) continue;
        if (best < 0 || s.probs[e] > s.probs[best]) best = e;
      }
      s.chosen[k] = best;
    }
    float keep = 0.0f;
    for (int k = 0; k < K; ++k) keep += s.probs[s.chosen[k]];
    const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
    for (int k = 0; k < K; ++k) {
      const int e = s.chosen[k];
      s.tok[e].push_back(t);
      s.wt[e].push_back(s.probs[e] * inv);
      if (topk_idx) topk_idx[(size_t)t * K + k] = e;
      if (topk_w) topk_w[(size_t)t * K + k] = s.probs[e] * inv;
    }
  }

  std::fill(out, out + (size_t)m * H, 0.0f);
  const uint64_t slab_gu = knj_row_bytes(tgu, (uint64_t)H) * (uint64_t)F;
  const uint64_t slab_dn = knj_row_bytes(tdn, (uint64_t)F) * (uint64_t)H;
  s.gat.resize((size_t)m * H);
  s.yg.resize((size_t)m * F);
  s.yu.resize((size_t)m * F);
  s.yd.resize((size_t)m * H);
  for (int e = 0; e < E; ++e) {
    const int cnt = (int)s.tok[e].size();
    if (cnt == 0) continue;
    for (int r = 0; r < cnt; ++r) {
      std::memcpy(s.gat.data() + (size_t)r * H, hx + (size_t)s.tok[e][r] * H, sizeof(float) * H);
    }
    matmul(pool, tgu, gate + (uint64_t)e * slab_gu, H, F, s.gat.data(), cnt, H, s.yg.data(), F,
           s.col);
    matmul(pool, tgu, up + (uint64_t)e * slab_gu, H, F, s.gat.data(), cnt, H, s.yu.data(), F, s.col);
    for (size_t i = 0, n = (size_t)cnt * F; i < n; ++i) s.yg[i] = silu(s.yg[i]) * s.yu[i];
    matmul(pool, tdn, down + (uint64_t)e * slab_dn, F, H, s.yg.data(), cnt, F, s.yd.data(), H,
           s.col);
    for (int r = 0; r < cnt; ++r) {
      const float w = s.wt[e][r];
      float* dst = out + (size_t)s.tok[e][r] * H;
      const float* src = s.yd.data() + (size_t)r * H;
      for (int i = 0; i < H; ++i) dst[i] += w * src[i];
    }
  }
}

void synth_serial(uint64_t key, int type, uint64_t n_in, uint64_t n_rows, float sd, uint8_t* out) {
  float tmp[KNJ_QK];
  const uint64_t nblk = n_rows * (n_in / KNJ_QK);
  const uint64_t bb = knj_row_bytes(type, KNJ_QK);
  for (uint64_t b = 0; b < nblk; ++b) knj_synth_quant_block(key, type, n_in, b, sd, tmp, out + b * bb);
}

void synth_tensor(Pool& pool, uint64_t key, int type, uint64_t n_in, uint64_t n_rows, float sd,
                  uint8_t* out) {
  if (type == KNJ_TYPE_Q4_K || type == KNJ_TYPE_Q6_K) {
    const uint64_t nblk = n_rows * (n_in / KNJ_QK);
    const uint64_t bb = knj_row_bytes(type, KNJ_QK);
    const uint64_t chunk = 4096;
    const int nchunks = (int)((nblk + chunk - 1) / chunk);
    pool.for_each(nchunks, [&](int c) {
      float tmp[KNJ_QK];
      const uint64_t b0 = (uint64_t)c * chunk, b1 = std::min(nblk, b0 + chunk);
      for (uint64_t b = b0; b < b1; ++b) knj_synth_quant_block(key, type, n_in, b, sd, tmp, out + b * bb);
    });
    return;
  }
  const uint64_t n = n_rows * n_in;
  const uint64_t chunk = 1 << 16;
  const int nchunks = (int)((n + chunk - 1) / chunk);
  pool.for_each(nchunks, [&](int c) {
    const uint64_t i0 = (uint64_t)c * chunk, i1 = std::min(n, i0 + chunk);
    for (uint64_t i = i0; i < i1; ++i) {
      const float v = knj_synth_value(key, i, sd);
      if (type == KNJ_TYPE_F32) std::memcpy(out + 4 * i, &v, 4);
      else {
        const uint16_t b = type == KNJ_TYPE_BF16 ? knj_f32_to_bf16(v) : knj_f32_to_f16(v);
        std::memcpy(out + 2 * i, &b, 2);
      }
    }
  });
}

void fill_ones(uint8_t* p, uint64_t n) {
  const float one = 1.0f;
  for (uint64_t i = 0; i < n; ++i) std::memcpy(p + 4 * i, &one, 4);
}

void synth_model(Pool& pool, const knj_model_config* c, uint64_t seed, uint8_t* img) {
  uint64_t off_embd, off_onorm, off_head;
  const uint64_t H = c->n_embd, QD = (uint64_t)c->n_head * c->head_dim,
                 KVD = (uint64_t)c->n_head_kv * c->head_dim, F = c->n_ff, V = c->n_vocab;
  const float sd = c->init_std;
  knj_model_layout(c, 0, nullptr, &off_embd, &off_onorm, &off_head);
  synth_tensor(pool, knj_tensor_key(seed, -1, KNJ_T_EMBD, -1), c->type_embd, H, V, sd, img + off_embd);
  for (int il = 0; il < c->n_layer; ++il) {
    knj_layer_offsets lo;
    knj_model_layout(c, il, &lo, nullptr, nullptr, nullptr);
    fill_ones(img + lo.attn_norm, H);
    fill_ones(img + lo.ffn_norm, H);
    fill_ones(img + lo.q_norm, (uint64_t)c->head_dim);
    fill_ones(img + lo.k_norm, (uint64_t)c->head_dim);
    const uint64_t rb = knj_row_bytes(c->type_attn, H);
    synth_tensor(pool, knj_tensor_key(seed, il, KNJ_T_Q, -1), c->type_attn, H, QD, sd, img + lo.wqkv);
    synth_tensor(pool, knj_tensor_key(seed, il, KNJ_T_K, -1), c->type_attn, H, KVD, sd,
                 img + lo.wqkv + rb * QD);
    synth_tensor(pool, knj_tensor_key(seed, il, KNJ_T_V, -1), c->type_attn, H, KVD, sd,
                 img + lo.wqkv + rb * (QD + KVD));
    synth_tensor(pool, knj_tensor_key(seed, il, KNJ_T_O, -1), c->type_attn, QD, H, sd, img + lo.wo);
    synth_tensor(pool, knj_tensor_key(seed, il, KNJ_T_ROUTER, -1), KNJ_TYPE_F32, H,
                 (uint64_t)c->n_expert, sd, img + lo.router);
    const uint64_t sgu = knj_row_bytes(c->type_gate_up, H) * F;
    const uint64_t sdn = knj_row_bytes(c->type_down, F) * H;
    // one task per (expert, tensor): the expert slabs are the bulk of the image
    pool.for_each(3 * c->n_expert, [&](int task) {
      const int e = task / 3, which = task % 3;
      if (which == 0)
        synth_serial(knj_tensor_key(seed, il, KNJ_T_GATE, e), c->type_gate_up, H, F, sd,
                     img + lo.gate + e * sgu);
      else if (which == 1)
        synth_serial(knj_tensor_key(seed, il, KNJ_T_UP, e), c->type_gate_up, H, F, sd,
                     img + lo.up + e * sgu);
      else
        synth_serial(knj_tensor_key(seed, il, KNJ_T_DOWN, e), c->type_down, F, H, sd,
                     img + lo.down + e * sdn);
    });
  }
  fill_ones(img + off_onorm, H);
  synth_tensor(pool, knj_tensor_key(seed, -1, KNJ_T_HEAD, -1), c->type_head, H, V, sd, img + off_head);
}

// One query head over slots 0..n_slots-1 of its KV head (model.cpp:591-616):
// scores q.k * scale in slot order, softmax, then out = sum_s a_s * v_s in slot
// order, K and V read back from the f16 cache.  The scores live in a buffer of
// the calling thread, so heads (and rows) can run on different threads with the
// same arithmetic per head.
void attend_head(const float* qh, const uint16_t* kh0, const uint16_t* vh0, int n_slots, int D,
                 float attn_scale, float* out) {
  thread_local std::vector<float> scores;
  if ((int)scores.size() < n_slots) scores.resize((size_t)n_slots);
  for (int s = 0; s < n_slots; ++s) {
    const uint16_t* kh = kh0 + (size_t)s * D;
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc += qh[d] * knj_f16_to_f32(kh[d]);
    scores[s] = acc * attn_scale;
  }
  softmax(scores.data(), n_slots);
  std::fill(out, out + D, 0.0f);
  for (int s = 0; s < n_slots; ++s) {
    const uint16_t* vh = vh0 + (size_t)s * D;
    const float a = scores[s];
    for (int d = 0; d < D; ++d) out[d] += a * knj_f16_to_f32(vh[d]);
  }
}

}  // namespace

// ======================================================================= model
struct knjo_model;
static uint16_t adopt_kv(knjo_model* m, float v, const uint16_t* src, size_t idx);

struct knjo_model {
  knj_model_config c;
  std::unique_ptr<Pool> pool;
  std::vector<uint8_t> own;
  const uint8_t* img = nullptr;
  uint64_t img_bytes = 0;
  std::vector<knj_layer_offsets> lo;
  uint64_t off_embd = 0, off_onorm = 0, off_head = 0;
  int pos = 0;
  std::vector<float> x, xn, q, k, v, ctx, ao, hx, ffn_out, rlog, logits, inv_freq, head_tmp;
  std::vector<uint16_t> kv_k, kv_v;
  // optional f16 values to adopt for each newly written slot (see
  // knjo_model_set_kv_source) and the statistics of that adoption
  const uint16_t* src_k = nullptr;
  const uint16_t* src_v = nullptr;
  int64_t kv_adopted = 0, kv_diff = 0;
  int kv_max_ulp = 0;
  float kv_max_mid = 0.0f;
  double kv_sum_d2 = 0.0, kv_sum_v2 = 0.0;  // squared distances, squared values
  std::vector<float> hidden;     // [n_layer][H], last token
  std::vector<int32_t> topk_idx; // [n_layer][K]
  std::vector<float> topk_w;     // [n_layer][K]
  std::vector<int32_t> tk_tmp;
  std::vector<float> tw_tmp;
  MoeScratch ms;
  std::vector<float> col;
};

// f16 of one new cache element.  Without a source this is the oracle's own
// round-to-nearest-even.  With a source (the GPU's cache), the source's value
// is adopted; when it differs from the oracle's own rounding, the distance from
// `v` to the set of f32 values that round to the source's value is recorded
// (zero would mean the source rounded `v` itself differently, which RNE never
// does; a tiny distance means an f32 value a few ulps from `v` was rounded).  This separates the
// single rounding decision an f32 difference in the last bits can flip from
// every other operation of the step.
static uint16_t adopt_kv(knjo_model* m, float v, const uint16_t* src, size_t idx) {
  const uint16_t own = knj_f32_to_f16(v);
  if (!src) return own;
  const uint16_t got = src[idx];
  m->kv_adopted += 1;
  m->kv_sum_v2 += (double)v * (double)v;
  if (got == own) return own;
  m->kv_diff += 1;
  const int ulp = std::abs((int)(own & 0x7FFF) - (int)(got & 0x7FFF)) +
                  (((own ^ got) & 0x8000) ? 1 : 0);
  m->kv_max_ulp = std::max(m->kv_max_ulp, ulp);
  // the interval of f32 values that round to `got` lies between the midpoints
  // to its two f16 neighbours; record how far `v` is from that interval
  auto ord = [](uint16_t h) { return (h & 0x8000) ? 0x8000 - (int)(h & 0x7FFF) : 0x8000 + (int)h; };
  auto unord = [](int k) {
    return (uint16_t)(k >= 0x8000 ? (k - 0x8000) : (0x8000 | (0x8000 - k)));
  };
  const float g = knj_f16_to_f32(got);
  const float below = knj_f16_to_f32(unord(ord(got) - 1));
  const float above = knj_f16_to_f32(unord(ord(got) + 1));
  const double lo = 0.5 * ((double)g + (double)below), hi = 0.5 * ((double)g + (double)above);
  const double dist = v < lo ? lo - v : (v > hi ? v - hi : 0.0);
  m->kv_max_mid = std::max(m->kv_max_mid, (float)dist);
  m->kv_sum_d2 += dist * dist;
  return got;
}

extern "C" {

void knjo_model_set_kv_source(knjo_model* m, const uint16_t* k, const uint16_t* v) {
  m->src_k = k;
  m->src_v = v;
  m->kv_adopted = m->kv_diff = 0;
  m->kv_max_ulp = 0;
  m->kv_max_mid = 0.0f;
  m->kv_sum_d2 = m->kv_sum_v2 = 0.0;
}

void knjo_model_kv_rms(knjo_model* m, double* sum_d2, double* sum_v2) {
  *sum_d2 = m->kv_sum_d2;
  *sum_v2 = m->kv_sum_v2;
}

void knjo_model_kv_stats(knjo_model* m, int64_t* adopted, int64_t* differing, int* max_ulp,
                         float* max_mid_dist) {
  *adopted = m->kv_adopted;
  *differing = m->kv_diff;
  *max_ulp = m->kv_max_ulp;
  *max_mid_dist = m->kv_max_mid;
}

float knjo_f16_to_f32(uint16_t h) { return knj_f16_to_f32(h); }
uint16_t knjo_f32_to_f16(float f) { return knj_f32_to_f16(f); }
float knjo_bf16_to_f32(uint16_t b) { return knj_bf16_to_f32(b); }

void knjo_dequant_row_f32(int type, const uint8_t* src, float* dst, uint64_t n) {
  dequant_row(type, src, dst, n);
}

float knjo_dequant_dot_f32(int type, const uint8_t* src, const float* x, uint64_t n) {
  return dequant_dot(type, src, x, n);
}

uint64_t knjo_tensor_key(uint64_t seed, int layer, int kind, int expert) {
  return knj_tensor_key(seed, layer, kind, expert);
}

void knjo_synth_tensor(uint64_t key, int type, uint64_t n_in, uint64_t n_rows, float stddev,
                       uint8_t* out, int threads) {
  synth_tensor(shared_pool(threads), key, type, n_in, n_rows, stddev, out);
}

void knjo_synth_model(const knj_model_config* cfg, uint64_t seed, uint8_t* image, int threads) {
  synth_model(shared_pool(threads), cfg, seed, image);
}

void knjo_matmul(int type, const uint8_t* w, int n_in, int n_out, const float* x, int m, float* y,
                 int threads) {
  std::vector<float> col;
  matmul(shared_pool(threads), type, w, n_in, n_out, x, m, n_in, y, n_out, col);
}

void knjo_moe(const float* hx, int m, int n_embd, int n_ff, int n_expert, int k,
              const float* router_w, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
              int type_gate_up, int type_down, float* out, float* logits, int32_t* topk_idx,
              float* topk_w, int threads) {
  MoeScratch s;
  moe(shared_pool(threads), hx, m, n_embd, n_ff, n_expert, k, router_w, gate, up, down,
      type_gate_up, type_down, out, logits, topk_idx, topk_w, s);
}

void knjo_rmsnorm(const float* x, const float* w, float* out, int width, float eps) {
  rmsnorm(x, w, out, width, eps);
}

const char* knjo_last_error(void) { return g_err.c_str(); }

knjo_model* knjo_model_create(const knj_model_config* cfg, uint64_t seed, const uint8_t* image,
                              int threads) {
  try {
    std::unique_ptr<knjo_model> m(new knjo_model());
    m->c = *cfg;
    const knj_model_config& c = m->c;
    if (c.n_head % c.n_head_kv) throw std::runtime_error("n_head is not a multiple of n_head_kv");
    if (c.n_expert_used > c.n_expert) throw std::runtime_error("n_expert_used exceeds n_expert");
    if (c.n_ctx <= 0) throw std::runtime_error("n_ctx must be positive");
    m->pool.reset(new Pool(threads));
    m->img_bytes = knj_model_layout(&c, 0, nullptr, &m->off_embd, &m->off_onorm, &m->off_head);
    m->lo.resize((size_t)c.n_layer);
    for (int il = 0; il < c.n_layer; ++il) knj_model_layout(&c, il, &m->lo[il], nullptr, nullptr, nullptr);
    if (image) {
      m->img = image;
    } else {
      m->own.assign(m->img_bytes, 0);
      synth_model(*m->pool, &c, seed, m->own.data());
      m->img = m->own.data();
    }
    const size_t H = c.n_embd, QD = (size_t)c.n_head * c.head_dim,
                 KVD = (size_t)c.n_head_kv * c.head_dim;
    m->x.assign(H, 0.f);
    m->xn.assign(H, 0.f);
    m->q.assign(QD, 0.f);
    m->k.assign(KVD, 0.f);
    m->v.assign(KVD, 0.f);
    m->ctx.assign(QD, 0.f);
    m->ao.assign(H, 0.f);
    m->hx.assign(H, 0.f);
    m->ffn_out.assign(H, 0.f);
    m->rlog.assign((size_t)c.n_expert, 0.f);
    m->logits.assign((size_t)c.n_vocab, 0.f);
    m->head_tmp.assign((size_t)c.head_dim, 0.f);
    m->kv_k.assign(knj_kv_elems(&c), 0);
    m->kv_v.assign(knj_kv_elems(&c), 0);
    m->hidden.assign((size_t)c.n_layer * H, 0.f);
    m->topk_idx.assign((size_t)c.n_layer * c.n_expert_used, 0);
    m->topk_w.assign((size_t)c.n_layer * c.n_expert_used, 0.f);
    // inv_freq[i] = base^(-2i/d) (model.cpp:227-230)
    m->inv_freq.resize((size_t)c.head_dim / 2);
    for (int i = 0; i < c.head_dim / 2; ++i) {
      m->inv_freq[i] = std::pow(c.rope_base, -2.0f * (float)i / (float)c.head_dim);
    }
    return m.release();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void knjo_model_free(knjo_model* m) { delete m; }
const uint8_t* knjo_model_image(knjo_model* m) { return m->img; }
uint64_t knjo_model_image_bytes(knjo_model* m) { return m->img_bytes; }
void knjo_model_reset(knjo_model* m) {
  m->pos = 0;
  std::fill(m->kv_k.begin(), m->kv_k.end(), (uint16_t)0);
  std::fill(m->kv_v.begin(), m->kv_v.end(), (uint16_t)0);
}
int knjo_model_pos(knjo_model* m) { return m->pos; }
int knjo_model_threads(knjo_model* m) { return m->pool->total(); }
const float* knjo_model_hidden(knjo_model* m, int il) { return m->hidden.data() + (size_t)il * m->c.n_embd; }
const int32_t* knjo_model_topk_idx(knjo_model* m, int il) {
  return m->topk_idx.data() + (size_t)il * m->c.n_expert_used;
}
const float* knjo_model_topk_w(knjo_model* m, int il) {
  return m->topk_w.data() + (size_t)il * m->c.n_expert_used;
}
uint16_t* knjo_model_kv_k(knjo_model* m) { return m->kv_k.data(); }
uint16_t* knjo_model_kv_v(knjo_model* m) { return m->kv_v.data(); }
int knjo_model_set_pos(knjo_model* m, int pos) {
  if (pos < 0 || pos > m->c.n_ctx) return -1;
  m->pos = pos;
  return 0;
}

// n single-token steps of Model::forward (model.cpp:512-672): what the
// reference computes when a prompt is fed one forward(&tok, 1) call at a time.
// For n == 1 this is exactly Model::forward.
int knjo_model_forward_steps(knjo_model* m, const int32_t* tokens, int n, float* logits) {
  try {
    const knj_model_config& c = m->c;
    if (n <= 0) throw std::runtime_error("forward needs at least one token");
    if (m->pos + n > c.n_ctx) throw std::runtime_error("context exhausted");
    const int H = c.n_embd, D = c.head_dim, QD = c.n_head * D, KVD = c.n_head_kv * D;
    const int E = c.n_expert, K = c.n_expert_used, F = c.n_ff, V = c.n_vocab;
    const float attn_scale = 1.0f / std::sqrt((float)D);
    const uint8_t* img = m->img;
    Pool& pool = *m->pool;
    m->tk_tmp.resize((size_t)K);
    m->tw_tmp.resize((size_t)K);
    for (int t = 0; t < n; ++t) {
      const int32_t id = tokens[t];
      if (id < 0 || id >= V) throw std::runtime_error("token id out of range");
      const int p = m->pos;
      // embed (model.cpp:527-537)
      dequant_row(c.type_embd, img + m->off_embd + (uint64_t)id * knj_row_bytes(c.type_embd, H),
                  m->x.data(), (uint64_t)H);
      for (int il = 0; il < c.n_layer; ++il) {
        const knj_layer_offsets& lo = m->lo[il];
        const float* attn_norm = reinterpret_cast<const float*>(img + lo.attn_norm);
        const float* ffn_norm = reinterpret_cast<const float*>(img + lo.ffn_norm);
        const float* qn = reinterpret_cast<const float*>(img + lo.q_norm);
        const float* kn = reinterpret_cast<const float*>(img + lo.k_norm);
        rmsnorm(m->x.data(), attn_norm, m->xn.data(), H, c.rms_eps);
        const uint64_t rb = knj_row_bytes(c.type_attn, H);
        matmul(pool, c.type_attn, img + lo.wqkv, H, QD, m->xn.data(), 1, H, m->q.data(), QD, m->col);
        matmul(pool, c.type_attn, img + lo.wqkv + rb * QD, H, KVD, m->xn.data(), 1, H, m->k.data(),
               KVD, m->col);
        matmul(pool, c.type_attn, img + lo.wqkv + rb * (QD + KVD), H, KVD, m->xn.data(), 1, H,
               m->v.data(), KVD, m->col);
        // QK-norm, NEOX RoPE, KV append (model.cpp:567-584)
        for (int h = 0; h < c.n_head; ++h) {
          rmsnorm(m->q.data() + (size_t)h * D, qn, m->head_tmp.data(), D, c.rms_eps);
          std::memcpy(m->q.data() + (size_t)h * D, m->head_tmp.data(), sizeof(float) * D);
        }
        for (int h = 0; h < c.n_head_kv; ++h) {
          rmsnorm(m->k.data() + (size_t)h * D, kn, m->head_tmp.data(), D, c.rms_eps);
          std::memcpy(m->k.data() + (size_t)h * D, m->head_tmp.data(), sizeof(float) * D);
        }
        const int half = D / 2;
        for (int pass = 0; pass < 2; ++pass) {
          float* base = pass == 0 ? m->q.data() : m->k.data();
          const int nh = pass == 0 ? c.n_head : c.n_head_kv;
          for (int h = 0; h < nh; ++h) {
            float* pv = base + (size_t)h * D;
            for (int i = 0; i < half; ++i) {
              const float theta = (float)p * m->inv_freq[i];
              const float cs = std::cos(theta), sn = std::sin(theta);
              const float x0 = pv[i], x1 = pv[i + half];
              pv[i] = x0 * cs - x1 * sn;
              pv[i + half] = x0 * sn + x1 * cs;
            }
          }
        }
        for (int h = 0; h < c.n_head_kv; ++h) {
          const size_t off = (((size_t)il * c.n_head_kv + h) * c.n_ctx + p) * D;
          for (int d = 0; d < D; ++d) {
            m->kv_k[off + d] = adopt_kv(m, m->k[(size_t)h * D + d], m->src_k, off + d);
            m->kv_v[off + d] = adopt_kv(m, m->v[(size_t)h * D + d], m->src_v, off + d);
          }
        }
        // attention (model.cpp:591-616), K/V read back from the f16 cache
        const int group = c.n_head / c.n_head_kv;
        pool.for_each(c.n_head, [&](int h) {
          const size_t hb = ((size_t)il * c.n_head_kv + h / group) * c.n_ctx;
          attend_head(m->q.data() + (size_t)h * D, m->kv_k.data() + hb * D, m->kv_v.data() + hb * D,
                      p + 1, D, attn_scale, m->ctx.data() + (size_t)h * D);
        });
        // attn-o + residual (model.cpp:620-625)
        matmul(pool, c.type_attn, img + lo.wo, QD, H, m->ctx.data(), 1, QD, m->ao.data(), H, m->col);
        for (int i = 0; i < H; ++i) m->x[i] += m->ao[i];
        // ffn norm, MoE, residual (model.cpp:628-653)
        rmsnorm(m->x.data(), ffn_norm, m->hx.data(), H, c.rms_eps);
        moe(pool, m->hx.data(), 1, H, F, E, K, reinterpret_cast<const float*>(img + lo.router),
            img + lo.gate, img + lo.up, img + lo.down, c.type_gate_up, c.type_down,
            m->ffn_out.data(), m->rlog.data(), m->tk_tmp.data(), m->tw_tmp.data(), m->ms);
        for (int i = 0; i < H; ++i) m->x[i] += m->ffn_out[i];
        if (t == n - 1) {
          std::memcpy(m->hidden.data() + (size_t)il * H, m->x.data(), sizeof(float) * H);
          std::memcpy(m->topk_idx.data() + (size_t)il * K, m->tk_tmp.data(), sizeof(int32_t) * K);
          std::memcpy(m->topk_w.data() + (size_t)il * K, m->tw_tmp.data(), sizeof(float) * K);
        }
      }
      m->pos += 1;
      if (t == n - 1) {
        // head (model.cpp:662-667)
        rmsnorm(m->x.data(), reinterpret_cast<const float*>(img + m->off_onorm), m->xn.data(), H,
                c.rms_eps);
        matmul(pool, c.type_head, img + m->off_head, H, V, m->xn.data(), 1, H, m->logits.data(), V,
               m->col);
      }
    }
    if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * (size_t)V);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// Model::forward (model.cpp:512-672) over n tokens at once: every weight
// matrix is applied to the n rows together (matmul with m = n, whose m > 1
// branch dequantises each 256-block and dots every row with it), all n keys
// and values are appended before any attention (model.cpp:562-584), row t then
// attends causally over slots 0..pos+t (:591-616), the MoE runs over the n
// rows (:628-653), and only the last row goes through the final norm and the
// head (:662-667).  n == 1 is the single-token step.
int knjo_model_forward(knjo_model* m, const int32_t* tokens, int n, float* logits) {
  if (n == 1) return knjo_model_forward_steps(m, tokens, n, logits);
  try {
    const knj_model_config& c = m->c;
    if (n <= 0) throw std::runtime_error("forward needs at least one token");
    if (m->pos + n > c.n_ctx) throw std::runtime_error("context exhausted");
    const int H = c.n_embd, D = c.head_dim, QD = c.n_head * D, KVD = c.n_head_kv * D;
    const int E = c.n_expert, K = c.n_expert_used, F = c.n_ff, V = c.n_vocab;
    const float attn_scale = 1.0f / std::sqrt((float)D);
    const uint8_t* img = m->img;
    Pool& pool = *m->pool;
    const size_t N = (size_t)n;
    std::vector<float> x(N * H), xn(N * H), q(N * QD), k(N * KVD), v(N * KVD), ctx(N * QD);
    std::vector<float> ao(N * H), hx(N * H), ffn(N * H), rlog(N * E), tw(N * K);
    std::vector<int32_t> tk(N * K);
    // embed (model.cpp:527-537)
    for (int t = 0; t < n; ++t) {
      const int32_t id = tokens[t];
      if (id < 0 || id >= V) throw std::runtime_error("token id out of range");
      dequant_row(c.type_embd, img + m->off_embd + (uint64_t)id * knj_row_bytes(c.type_embd, H),
                  x.data() + (size_t)t * H, (uint64_t)H);
    }
    const int half = D / 2, group = c.n_head / c.n_head_kv;
    const uint64_t rb = knj_row_bytes(c.type_attn, H);
    for (int il = 0; il < c.n_layer; ++il) {
      const knj_layer_offsets& lo = m->lo[il];
      const float* qn = reinterpret_cast<const float*>(img + lo.q_norm);
      const float* kn = reinterpret_cast<const float*>(img + lo.k_norm);
      // rmsnorm_rows + QKV (model.cpp:546-558)
      for (int t = 0; t < n; ++t)
        rmsnorm(x.data() + (size_t)t * H, reinterpret_cast<const float*>(img + lo.attn_norm),
                xn.data() + (size_t)t * H, H, c.rms_eps);
      matmul(pool, c.type_attn, img + lo.wqkv, H, QD, xn.data(), n, H, q.data(), QD, m->col);
      matmul(pool, c.type_attn, img + lo.wqkv + rb * QD, H, KVD, xn.data(), n, H, k.data(), KVD,
             m->col);
      matmul(pool, c.type_attn, img + lo.wqkv + rb * (QD + KVD), H, KVD, xn.data(), n, H, v.data(),
             KVD, m->col);
      // QK-norm, NEOX RoPE and the append of every row (model.cpp:562-584)
      for (int t = 0; t < n; ++t) {
        const int p = m->pos + t;
        float* qt = q.data() + (size_t)t * QD;
        float* kt = k.data() + (size_t)t * KVD;
        for (int h = 0; h < c.n_head; ++h) {
          rmsnorm(qt + (size_t)h * D, qn, m->head_tmp.data(), D, c.rms_eps);
          std::memcpy(qt + (size_t)h * D, m->head_tmp.data(), sizeof(float) * D);
        }
        for (int h = 0; h < c.n_head_kv; ++h) {
          rmsnorm(kt + (size_t)h * D, kn, m->head_tmp.data(), D, c.rms_eps);
          std::memcpy(kt + (size_t)h * D, m->head_tmp.data(), sizeof(float) * D);
        }
        for (int pass = 0; pass < 2; ++pass) {
          float* base = pass == 0 ? qt : kt;
          const int nh = pass == 0 ? c.n_head : c.n_head_kv;
          for (int h = 0; h < nh; ++h) {
            float* pv = base + (size_t)h * D;
            for (int i = 0; i < half; ++i) {
              const float theta = (float)p * m->inv_freq[i];
              const float cs = std::cos(theta), sn = std::sin(theta);
              const float x0 = pv[i], x1 = pv[i + half];
              pv[i] = x0 * cs - x1 * sn;
              pv[i + half] = x0 * sn + x1 * cs;
            }
          }
        }
        for (int h = 0; h < c.n_head_kv; ++h) {
          const size_t off = (((size_t)il * c.n_head_kv + h) * c.n_ctx + p) * D;
          for (int d = 0; d < D; ++d) {
            m->kv_k[off + d] = adopt_kv(m, kt[(size_t)h * D + d], m->src_k, off + d);
            m->kv_v[off + d] = adopt_kv(m, v[(size_t)t * KVD + (size_t)h * D + d], m->src_v, off + d);
          }
        }
      }
      // causal attention, row t over slots 0..pos+t (model.cpp:591-616); the
      // (row, head) pairs are independent, so they are spread over the pool
      pool.for_each(n * c.n_head, [&](int task) {
        const int t = task / c.n_head, h = task - t * c.n_head;
        const size_t hb = ((size_t)il * c.n_head_kv + h / group) * c.n_ctx;
        attend_head(q.data() + (size_t)t * QD + (size_t)h * D, m->kv_k.data() + hb * D,
                    m->kv_v.data() + hb * D, m->pos + t + 1, D, attn_scale,
                    ctx.data() + (size_t)t * QD + (size_t)h * D);
      });
      // attn-o + residual (model.cpp:620-625)
      matmul(pool, c.type_attn, img + lo.wo, QD, H, ctx.data(), n, QD, ao.data(), H, m->col);
      for (size_t i = 0; i < N * H; ++i) x[i] += ao[i];
      // ffn norm, MoE over the n rows, residual (model.cpp:628-653)
      for (int t = 0; t < n; ++t)
        rmsnorm(x.data() + (size_t)t * H, reinterpret_cast<const float*>(img + lo.ffn_norm),
                hx.data() + (size_t)t * H, H, c.rms_eps);
      moe(pool, hx.data(), n, H, F, E, K, reinterpret_cast<const float*>(img + lo.router),
          img + lo.gate, img + lo.up, img + lo.down, c.type_gate_up, c.type_down, ffn.data(),
          rlog.data(), tk.data(), tw.data(), m->ms);
      for (size_t i = 0; i < N * H; ++i) x[i] += ffn[i];
      const size_t last = (size_t)(n - 1);
      std::memcpy(m->hidden.data() + (size_t)il * H, x.data() + last * H, sizeof(float) * H);
      std::memcpy(m->topk_idx.data() + (size_t)il * K, tk.data() + last * K, sizeof(int32_t) * K);
      std::memcpy(m->topk_w.data() + (size_t)il * K, tw.data() + last * K, sizeof(float) * K);
    }
    // final norm + head of the last row (model.cpp:662-667)
    rmsnorm(x.data() + (size_t)(n - 1) * H, reinterpret_cast<const float*>(img + m->off_onorm),
            m->xn.data(), H, c.rms_eps);
    matmul(pool, c.type_head, img + m->off_head, H, V, m->xn.data(), 1, H, m->logits.data(), V,
           m->col);
    m->pos += n;
    if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * (size_t)V);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"
