// A caller written against the reference's C2 interface
// (/root/reference/src/device/backend.h:37-76): unqualified Backend,
// ExpertPlan, AttentionPlan and KvWritePlan; the argument-less create(); the
// virtual launch_expert_gemm_wmma / launch_expert_gemm_simt / launch_attention
// / launch_kv_write; from_caps() with injected DeviceCaps fields.  No GPU is
// touched: every plan is empty, so each launch answers only the gate question.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "knj/backend.h"
#include "knj_capi.h"

static int failures = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);    \
      ++failures;                                                     \
    }                                                                 \
  } while (0)

// Anything a caller of the reference could write against the abstract class.
static bool run_plans(Backend& b) {
  ExpertPlan ep{};
  AttentionPlan ap{};
  KvWritePlan kp{};
  const bool w = b.launch_expert_gemm_wmma(ep);
  const bool s = b.launch_expert_gemm_simt(ep);
  const bool a = b.launch_attention(ap);
  b.launch_kv_write(kp);
  return w && s && a;
}

static void* upload(const std::vector<float>& h) {
  void* d = nullptr;
  CHECK(knj_malloc(&d, h.size() * 4) == KNJ_OK);
  CHECK(knj_memcpy_h2d(d, h.data(), h.size() * 4) == KNJ_OK);
  return d;
}

static void device_kv_write() {
  std::unique_ptr<Backend> dev = Backend::create();
  CHECK(dev != nullptr);
  if (!dev) return;
  const int n_head = 8, n_kv = 2, D = 64, n_ctx = 64, pos = 5;
  std::vector<float> q(n_head * D), k(n_kv * D), v(n_kv * D), norm(D, 1.0f);
  for (size_t i = 0; i < q.size(); ++i) q[i] = 0.01f * (float)((i * 7) % 23) - 0.1f;
  for (size_t i = 0; i < k.size(); ++i) k[i] = 0.02f * (float)((i * 5) % 17) - 0.15f;
  for (size_t i = 0; i < v.size(); ++i) v[i] = 0.03f * (float)((i * 3) % 19) - 0.2f;
  void *dq = upload(q), *dk = upload(k), *dv = upload(v), *dn = upload(norm);
  const uint64_t cache = (uint64_t)n_kv * n_ctx * D * 2;
  void *kc[2] = {nullptr, nullptr}, *vc[2] = {nullptr, nullptr}, *out = nullptr;
  for (int i = 0; i < 2; ++i) {
    CHECK(knj_malloc(&kc[i], cache) == KNJ_OK && knj_memset_zero(kc[i], cache) == KNJ_OK);
    CHECK(knj_malloc(&vc[i], cache) == KNJ_OK && knj_memset_zero(vc[i], cache) == KNJ_OK);
  }
  CHECK(knj_malloc(&out, (uint64_t)n_head * D * 4) == KNJ_OK);
  auto plan = [&](int i) {
    AttentionPlan a{};
    a.q = (const float*)dq;
    a.k = (const float*)dk;
    a.v = (const float*)dv;
    a.q_norm = a.k_norm = (const float*)dn;
    a.pos = pos;
    a.n_head = n_head;
    a.n_head_kv = n_kv;
    a.head_dim = D;
    a.n_ctx = n_ctx;
    a.k_cache = (uint16_t*)kc[i];
    a.v_cache = (uint16_t*)vc[i];
    return a;
  };
  KvWritePlan kp{};
  kp.attn = plan(0);  // scratch_out stays null, as the reference's plan has none
  dev->launch_kv_write(kp);
  CHECK(std::strcmp(Backend::knj_last_refusal(), "") == 0);
  AttentionPlan ap = plan(1);
  ap.out = (float*)out;
  CHECK(dev->launch_attention(ap));
  CHECK(knj_synchronize() == KNJ_OK);
  std::vector<uint16_t> h[4];
  for (int i = 0; i < 4; ++i) {
    h[i].resize(cache / 2);
    CHECK(knj_memcpy_d2h(h[i].data(), i < 2 ? kc[i] : vc[i - 2], cache) == KNJ_OK);
  }
  CHECK(h[0] == h[1]);
  CHECK(h[2] == h[3]);
  int written = 0;
  for (int c = 0; c < n_kv; ++c)
    for (int d = 0; d < D; ++d) written += h[0][((size_t)c * n_ctx + pos) * D + d] != 0 ? 1 : 0;
  CHECK(written > n_kv * D / 2);
  // a plan the launch refuses (head_dim 48) is reported through the refusal
  KvWritePlan bad{};
  bad.attn = plan(0);
  bad.attn.head_dim = 48;
  dev->launch_kv_write(bad);
  CHECK(std::strlen(Backend::knj_last_refusal()) > 0);
  std::printf("device KV write: %d of %d slot elements written, caches identical\n", written, n_kv * D);
  for (void* p : {dq, dk, dv, dn, kc[0], kc[1], vc[0], vc[1], out}) knj_free(p);
}

int main() {
  // 1) create() on a machine without the device refuses with a reason
  if (std::getenv("KNJ_EXPECT_NO_DEVICE")) {
    std::unique_ptr<Backend> none = Backend::create();
    CHECK(none == nullptr);
    CHECK(std::strlen(Backend::knj_last_refusal()) > 0);
    std::printf("create() refused: %s\n", Backend::knj_last_refusal());
  }

  // 2) injected caps for the built arch: every gate open
  DeviceCaps caps{};
  std::strncpy(caps.gcn_arch, "gfx950", sizeof(caps.gcn_arch) - 1);
  caps.has_wmma = true;
  caps.has_fp8 = true;
  caps.wave_size = 64;
  caps.arch_ok = true;
  std::unique_ptr<Backend> b = Backend::from_caps(caps);
  CHECK(b != nullptr);
  CHECK(std::strcmp(Backend::knj_last_refusal(), "") == 0);
  CHECK(b->would_instantiate(KnjCap::WmmaF16));
  CHECK(b->would_instantiate(KnjCap::Fp8));
  CHECK(b->would_instantiate(KnjCap::Dot4I32I8));
  CHECK(b->would_instantiate(KnjCap::Wave64));
  CHECK(run_plans(*b));

  // 3) a probed cap can be absent although the arch has it
  DeviceCaps no_mc = caps;
  no_mc.has_wmma = false;
  no_mc.has_fp8 = false;
  std::unique_ptr<Backend> b2 = Backend::from_caps(no_mc);
  CHECK(!b2->would_instantiate(KnjCap::WmmaF16));
  CHECK(!b2->would_instantiate(KnjCap::Fp8));
  CHECK(b2->would_instantiate(KnjCap::Dot4I32I8));
  CHECK(!b2->launch_expert_gemm_wmma(ExpertPlan{}));
  CHECK(b2->launch_expert_gemm_simt(ExpertPlan{}));

  // 4) another arch: nothing is instantiated, every launch refuses
  DeviceCaps other = caps;
  std::strncpy(other.gcn_arch, "gfx1201", sizeof(other.gcn_arch) - 1);
  std::unique_ptr<Backend> b3 = Backend::from_caps(other);
  CHECK(!b3->would_instantiate(KnjCap::WmmaF16));
  CHECK(!b3->would_instantiate(KnjCap::Dot4I32I8));
  CHECK(!run_plans(*b3));

  // 5) the arch guard refused: nothing either
  DeviceCaps refused = caps;
  refused.arch_ok = false;
  CHECK(!run_plans(*Backend::from_caps(refused)));

  // 6) wave32 caps (a wave32 part): the wave64 kernels are not instantiated
  DeviceCaps w32 = caps;
  w32.wave_size = 32;
  std::unique_ptr<Backend> b4 = Backend::from_caps(w32);
  CHECK(!b4->launch_expert_gemm_simt(ExpertPlan{}));
  CHECK(!b4->launch_attention(AttentionPlan{}));

  CHECK(std::strcmp(knj_cap_label(KnjCap::WmmaF16), "mfma_f16") == 0);

  // 7) on a device (KNJ_DEVICE_CHECKS=1): a KV write with the reference's
  // plan, which has no output buffer, writes the same cache slot as an
  // attention launch given an explicit output
  if (std::getenv("KNJ_DEVICE_CHECKS")) device_kv_write();
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
