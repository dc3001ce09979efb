// include/knj/backend.h -- C++ device gate over the gfx950 library.
//
// Keeps the shape of the reference's C2 device layer
// (/root/reference/src/device/backend.h:35-76, device_caps.h:53-85): an
// arch-guarded factory that returns nullptr plus a thread-local refusal reason,
// a caps-injection factory for host tests, would_instantiate(KnjCap), and
// launch_* methods that return false when the kernel is not available on this
// device.  The plans carry real device pointers and map onto the C ABI
// (include/knj_capi.h); the reference's plans are empty placeholders.
#pragma once

#include <cstdint>
#include <memory>

#include "../knj_capi.h"

namespace knj {

// Capabilities a kernel may need.  gfx950 (CDNA4, wave64) has all of them.
enum class KnjCap {
  Wave64,        // 64-lane wavefronts (the kernels' lane mappings assume it)
  MfmaBf16,      // v_mfma_f32_*_bf16
  MfmaI8,        // v_mfma_i32_*_i8
  Fp8,           // fp8 MFMA
  Dot4I32I8,     // v_dot4_i32_i8
};

// Batch-1 MoE FFN of one layer (knj_moe_decode_layer).
struct ExpertPlan {
  const float* x = nullptr;        // residual stream [n_embd]
  const float* norm_w = nullptr;   // ffn_norm (may be null: x already normalised)
  float eps = 1e-6f;
  const float* router_w = nullptr; // [n_expert][n_embd]
  const void* gate = nullptr;
  const void* up = nullptr;
  const void* down = nullptr;
  int type_gate_up = KNJ_TYPE_Q4_K, type_down = KNJ_TYPE_Q4_K;
  int n_embd = 0, n_ff = 0, n_expert = 0, k = 0;
  const float* resid = nullptr;
  float* out = nullptr;
  float* logits = nullptr;
  int32_t* topk_idx = nullptr;
  float* topk_w = nullptr;
  void* stream = nullptr;
};

// Attention block of one decode token (knj_attention_step).
struct AttentionPlan {
  const float *q = nullptr, *k = nullptr, *v = nullptr;
  const float *q_norm = nullptr, *k_norm = nullptr;
  float eps = 1e-6f, rope_base = 1e6f;
  int pos = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ctx = 0;
  uint16_t *k_cache = nullptr, *v_cache = nullptr;
  float* out = nullptr;
  void* stream = nullptr;
};

// The attention step writes the new KV slot itself; a standalone KV write
// (f16 rounding of k/v into slot `pos`) is the same call with the output
// discarded, so the plan only needs the attention fields.
struct KvWritePlan {
  AttentionPlan attn;
  float* scratch_out = nullptr;  // [n_head][head_dim]
};

struct DeviceCaps {
  knj_device_caps caps{};
  bool arch_ok = false;
  const char* arch_reason = "";
};

class Backend {
 public:
  // Opens device `device` through the arch guard; nullptr (and a reason in
  // knj_last_refusal()) when the device is not gfx950 or KNJ_BUILD_ARCH names
  // another arch.
  static std::unique_ptr<Backend> create(int device = 0);
  // Test hook: a backend over injected caps, no device touched.
  static std::unique_ptr<Backend> from_caps(const DeviceCaps& caps);
  static const char* knj_last_refusal();

  const DeviceCaps& caps() const noexcept { return caps_; }
  bool would_instantiate(KnjCap cap) const noexcept;

  bool launch_expert_gemv(const ExpertPlan& p);   // batch-1 MoE layer
  bool launch_attention(const AttentionPlan& p);
  void launch_kv_write(const KvWritePlan& p);

 private:
  explicit Backend(const DeviceCaps& c) : caps_(c) {}
  DeviceCaps caps_;
};

}  // namespace knj
