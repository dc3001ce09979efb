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

#include "knj/backend.h"

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
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
