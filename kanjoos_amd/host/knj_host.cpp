// kanjoos_amd/host/knj_host.cpp -- C++ host classes (Model, Backend) over the C ABI.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/knj/backend.h"
#include "../../include/knj/model.h"

namespace knj {

void check(int rc, const char* what) {
  if (rc != KNJ_OK) {
    throw std::runtime_error(std::string("model: ") + what + ": " + knj_last_error());
  }
}

std::string ModelGeometry::describe() const {
  char buf[512];
  std::snprintf(buf, sizeof(buf),
                "layers=%d hidden=%d heads=%d/%d head_dim=%d q_dim=%d kv_dim=%d\n"
                "  experts=%d top_k=%d expert_ff=%d vocab=%d ctx=%d rms_eps=%.3g rope_base=%.6g",
                n_layer, n_embd, n_head, n_head_kv, head_dim, q_dim(), kv_dim(), n_expert,
                n_expert_used, n_ff_exp, n_vocab, n_ctx_train, rms_eps, rope_base);
  return buf;
}

namespace {
ModelGeometry geometry_of(const knj_model_config& c) {
  ModelGeometry g;
  g.n_layer = c.n_layer;
  g.n_embd = c.n_embd;
  g.n_head = c.n_head;
  g.n_head_kv = c.n_head_kv;
  g.head_dim = c.head_dim;
  g.n_ff_exp = c.n_ff;
  g.n_expert = c.n_expert;
  g.n_expert_used = c.n_expert_used;
  g.n_vocab = c.n_vocab;
  g.n_ctx_train = c.n_ctx;
  g.rms_eps = c.rms_eps;
  g.rope_base = c.rope_base;
  return g;
}
}  // namespace

std::unique_ptr<Model> Model::open_synthetic(const knj_model_config& cfg, uint64_t seed,
                                             const Options& opt) {
  if (opt.n_ctx <= 0) throw std::runtime_error("model: n_ctx must be positive");
  knj_model_config c = cfg;
  c.n_ctx = opt.n_ctx;
  std::unique_ptr<Model> m(new Model());
  check(knj_model_create_synthetic(&c, seed, &m->m_), "open");
  m->g_ = geometry_of(c);
  m->n_ctx_ = c.n_ctx;
  m->logits_.assign((size_t)c.n_vocab, 0.0f);
  return m;
}

std::unique_ptr<Model> Model::open(const std::string& path, const Options& opt) {
  if (opt.n_ctx <= 0) throw std::runtime_error("model: n_ctx must be positive");
  std::unique_ptr<Model> m(new Model());
  check(knj_model_create_from_gguf(path.c_str(), opt.n_ctx, &m->m_), "open");
  knj_model_config c{};
  check(knj_model_config_get(m->m_, &c), "open");
  m->g_ = geometry_of(c);
  m->n_ctx_ = c.n_ctx;
  m->logits_.assign((size_t)c.n_vocab, 0.0f);
  return m;
}

std::unique_ptr<Model> Model::open_image(const knj_model_config& cfg, const void* image,
                                         uint64_t bytes, const Options& opt) {
  if (opt.n_ctx <= 0) throw std::runtime_error("model: n_ctx must be positive");
  knj_model_config c = cfg;
  c.n_ctx = opt.n_ctx;
  std::unique_ptr<Model> m(new Model());
  check(knj_model_create_from_image(&c, image, bytes, &m->m_), "open");
  m->g_ = geometry_of(c);
  m->n_ctx_ = c.n_ctx;
  m->logits_.assign((size_t)c.n_vocab, 0.0f);
  return m;
}

std::vector<int32_t> Model::decode_greedy_profiled(int32_t first, int steps, Profiler& prof) {
  if (steps <= 0) throw std::runtime_error("model: steps must be positive");
  std::vector<int32_t> out;
  out.reserve((size_t)steps);
  // one step's launches: 2 per layer for attention and 5 more per layer, plus
  // embed, head and sample; the ring is sized with room to spare
  const int cap = 8 * g_.n_layer + 16;
  std::vector<knj_span> sp((size_t)cap);
  uint64_t base = 0;
  int32_t tok = first;
  for (int i = 0; i < steps; ++i) {
    int n = 0;
    uint64_t dropped = 0;
    int32_t next = 0;
    check(knj_model_profile(m_, tok, 1, &next, sp.data(), cap, &n, &dropped), "profile");
    const bool kept = prof.steps_kept() + prof.steps_discarded() >= (uint64_t)prof.config().warmup_steps;
    uint64_t last = 0;
    for (int j = 0; j < n; ++j) {
      const knj_span& s = sp[(size_t)j];
      last = std::max(last, s.end_ns);
      if (!kept) continue;
      std::string k(s.kernel);
      const size_t lt = k.find('<');
      if (lt != std::string::npos) k.resize(lt);
      char name[128];
      if (s.layer >= 0)
        std::snprintf(name, sizeof(name), "%s:%d:%s", s.name, s.layer, k.c_str());
      else
        std::snprintf(name, sizeof(name), "%s:-:%s", s.name, k.c_str());
      prof.device_span(name, base + s.start_ns, base + s.end_ns, s.stream);
    }
    if (kept && dropped) prof.set_device_dropped(prof.device_dropped() + dropped);
    base += last;
    prof.step_done();
    out.push_back(next);
    tok = next;
  }
  return out;
}

void Model::fill_kv(int n_pos, uint64_t seed) { check(knj_model_fill_kv(m_, n_pos, seed), "fill_kv"); }

TransferStats Model::transfer_stats() const {
  TransferStats t;
  check(knj_model_transfer_bytes(m_, &t.h2d_bytes, &t.d2h_bytes), "transfer stats");
  t.measured = true;
  return t;
}

Model::~Model() {
  if (m_) knj_model_free(m_);
}

int Model::pos() const { return knj_model_pos(m_); }

void Model::reset() { check(knj_model_reset(m_), "reset"); }

const float* Model::forward(const int32_t* tokens, int n) {
  if (n <= 0) throw std::runtime_error("model: forward needs at least one token");
  if (pos() + n > n_ctx_) {
    throw std::runtime_error("model: context exhausted (" + std::to_string(pos()) + " + " +
                             std::to_string(n) + " > " + std::to_string(n_ctx_) + ")");
  }
  for (int t = 0; t < n; ++t)
    if (tokens[t] < 0 || tokens[t] >= g_.n_vocab) throw std::runtime_error("model: token id out of range");
  check(knj_model_forward(m_, tokens, n, logits_.data()), "forward");
  return logits_.data();
}

std::vector<int32_t> Model::decode_greedy(int32_t first, int steps) {
  std::vector<int32_t> out((size_t)steps);
  check(knj_model_decode_greedy(m_, first, steps, out.data()), "decode");
  return out;
}

// ------------------------------------------------------------------ Backend
namespace {
thread_local char g_refusal[256] = "";

bool plan_is_empty(const ExpertPlan& p) { return p.out == nullptr; }

// The one concrete backend: gfx950 through the C ABI.
class Gfx950Backend final : public Backend {
 public:
  using Backend::Backend;

  bool launch_expert_gemm_wmma(const ExpertPlan& p) override {
    if (!would_instantiate(KnjCap::WmmaF16)) return false;
    if (plan_is_empty(p)) return true;
    return knj_moe_batch_layer(p.x, p.norm_w, p.eps, p.router_w, p.gate, p.up, p.down,
                               p.type_gate_up, p.type_down, p.n_tokens, p.n_embd, p.n_ff,
                               p.n_expert, p.k, p.resid, p.out, p.logits, p.topk_idx, p.topk_w,
                               p.stream) == KNJ_OK;
  }

  bool launch_expert_gemm_simt(const ExpertPlan& p) override {
    if (!would_instantiate(KnjCap::Wave64)) return false;
    if (plan_is_empty(p)) return true;
    if (p.n_tokens != 1) return launch_expert_gemm_wmma(p);
    return knj_moe_decode_layer(p.x, p.norm_w, p.eps, p.router_w, p.gate, p.up, p.down,
                                p.type_gate_up, p.type_down, p.n_embd, p.n_ff, p.n_expert, p.k,
                                p.resid, p.out, p.logits, p.topk_idx, p.topk_w,
                                p.stream) == KNJ_OK;
  }

  bool launch_attention(const AttentionPlan& p) override {
    if (!would_instantiate(KnjCap::Wave64)) return false;
    if (p.out == nullptr) return true;
    return knj_attention_step(p.q, p.k, p.v, p.q_norm, p.k_norm, p.eps, p.rope_base, p.pos,
                              p.n_head, p.n_head_kv, p.head_dim, p.n_ctx, p.k_cache, p.v_cache,
                              p.out, p.stream) == KNJ_OK;
  }

  // The reference's KvWritePlan has no output buffer: without one, the step's
  // attention output goes to a device buffer this backend owns.  A failed
  // launch is recorded where knj_last_refusal() reads it (the method returns
  // nothing, as the reference's does).
  void launch_kv_write(const KvWritePlan& p) override {
    if (p.attn.q == nullptr || !would_instantiate(KnjCap::Wave64)) return;  // an empty plan
    AttentionPlan a = p.attn;
    a.out = p.scratch_out;
    if (a.out == nullptr) {
      const uint64_t need = (uint64_t)std::max(a.n_head, 1) * (uint64_t)std::max(a.head_dim, 1) * 4;
      if (need > kv_out_bytes_) {
        if (kv_out_) knj_free(kv_out_);
        kv_out_ = nullptr;
        kv_out_bytes_ = 0;
        if (knj_malloc(&kv_out_, need) != KNJ_OK) {
          std::snprintf(g_refusal, sizeof(g_refusal), "launch_kv_write: %s", knj_last_error());
          return;
        }
        kv_out_bytes_ = need;
      }
      a.out = static_cast<float*>(kv_out_);
    }
    if (!launch_attention(a))
      std::snprintf(g_refusal, sizeof(g_refusal), "launch_kv_write: %s", knj_last_error());
  }

  ~Gfx950Backend() override {
    if (kv_out_) knj_free(kv_out_);
  }

 private:
  void* kv_out_ = nullptr;
  uint64_t kv_out_bytes_ = 0;
};

void copy_arch(char (&dst)[16], const char* src) {
  size_t i = 0;
  for (; i + 1 < sizeof(dst) && src[i] != '\0'; ++i) dst[i] = src[i];
  dst[i] = '\0';
}
}  // namespace

const char* Backend::knj_last_refusal() { return g_refusal; }

std::unique_ptr<Backend> Backend::create() {
  const char* env = std::getenv("KNJ_DEVICE");
  const int device = (env && *env) ? std::atoi(env) : 0;
  DeviceCaps c;
  if (knj_device_open(device) != KNJ_OK || knj_device_caps_get(&c.device) != KNJ_OK) {
    std::snprintf(g_refusal, sizeof(g_refusal), "%s", knj_last_error());
    return nullptr;
  }
  copy_arch(c.gcn_arch, c.device.gcn_arch);
  c.has_wmma = c.device.has_mfma_bf16 != 0;
  c.has_fp8 = c.device.has_fp8 != 0;
  c.has_dot_builtin = knj_cap_available(c.gcn_arch, KnjCap::Sdot4Builtin);
  c.wave_size = c.device.wave_size;
  c.vram_total = c.device.vram_total;
  c.vram_usable = c.device.vram_free;
  c.rebar_full_aperture = false;
  c.sms = (uint32_t)c.device.cu_count;
  c.clock_khz = (uint32_t)c.device.clock_khz;
  c.max_streams = 4;  // hardware queues per process (GPU_MAX_HW_QUEUES default)
  c.num_queue_groups = 1;
  c.arch_ok = c.device.arch_ok != 0;
  c.arch_reason = "";
  g_refusal[0] = '\0';
  return std::unique_ptr<Backend>(new Gfx950Backend(c));
}

std::unique_ptr<Backend> Backend::from_caps(const DeviceCaps& caps) {
  g_refusal[0] = '\0';
  return std::unique_ptr<Backend>(new Gfx950Backend(caps));
}

bool Backend::would_instantiate(KnjCap cap) const noexcept {
  if (!caps_.arch_ok || !knj_cap_available(caps_.gcn_arch, cap)) return false;
  // probed caps can be absent where the arch nominally has them
  switch (cap) {
    case KnjCap::WmmaF16:
    case KnjCap::MfmaBf16: return caps_.has_wmma;
    case KnjCap::Fp8: return caps_.has_fp8;
    case KnjCap::Wave64: return caps_.wave_size == 64;
    default: return true;
  }
}

}  // namespace knj

bool knj_cap_available(const char* arch, KnjCap cap) {
  if (arch == nullptr || std::strcmp(arch, knj_built_arch()) != 0) return false;
  switch (cap) {
    case KnjCap::Dot4I32I8:
    case KnjCap::Dot8I32I4:
    case KnjCap::PkFmaF16:
    case KnjCap::WmmaF16:
    case KnjCap::Fp8:
    case KnjCap::Sdot4Builtin:
    case KnjCap::Wave64:
    case KnjCap::MfmaBf16:
    case KnjCap::MfmaI8: return true;
  }
  return false;
}

const char* knj_cap_label(KnjCap cap) {
  switch (cap) {
    case KnjCap::Dot4I32I8: return "dot4_i32_i8";
    case KnjCap::Dot8I32I4: return "dot8_i32_i4";
    case KnjCap::PkFmaF16: return "pk_fma_f16";
    case KnjCap::WmmaF16: return "mfma_f16";
    case KnjCap::Fp8: return "fp8";
    case KnjCap::Sdot4Builtin: return "sdot4";
    case KnjCap::Wave64: return "wave64";
    case KnjCap::MfmaBf16: return "mfma_bf16";
    case KnjCap::MfmaI8: return "mfma_i8";
  }
  return "unknown";
}
