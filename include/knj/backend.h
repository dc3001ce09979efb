// include/knj/backend.h -- C++ device gate over the gfx950 library.
//
// The shape of the reference's C2 device layer
// (/root/reference/src/device/backend.h:37-76, device_caps.h:53-85, 160-178):
//   * Backend::create() takes no argument; it returns nullptr plus a
//     thread-local refusal reason (knj_last_refusal()) when the device is not
//     the arch this library was built for, or KNJ_BUILD_ARCH names another;
//   * Backend::from_caps() is the test injection point (no device touched);
//   * would_instantiate(KnjCap) answers the cap-gating question;
//   * the launch_* methods are virtual; a false return means "not
//     instantiated for this device".
// The device that create() opens is KNJ_DEVICE (default 0).  The plans carry
// real device pointers and map onto the C ABI (include/knj_capi.h); a plan
// left empty (no output pointer) asks only the gate question, which is what
// the reference's empty stand-in plans (backend.h:26-33) do.
#pragma once

#include <cstdint>
#include <memory>

#include "../knj_capi.h"

// Instruction capabilities a kernel may need.  The first six are the
// reference's spellings (device_caps.h:57-64); the last three are the CDNA
// features this build's kernels are written against.
enum class KnjCap {
  Dot4I32I8,     // v_dot4_i32_i8
  Dot8I32I4,     // v_dot8_i32_i4
  PkFmaF16,      // v_pk_fma_f16
  WmmaF16,       // f16 matrix-core tiles (on CDNA: v_mfma_f32_*_f16)
  Fp8,           // fp8 matrix cores
  Sdot4Builtin,  // the __builtin_amdgcn_sdot4 spelling of the int8 dot
  Wave64,        // 64-lane wavefronts (the kernels' lane mappings assume it)
  MfmaBf16,      // v_mfma_f32_*_bf16
  MfmaI8,        // v_mfma_i32_*_i8
};

// Capability table by arch string: every cap above on gfx950, nothing on an
// arch this library does not target.
bool knj_cap_available(const char* arch, KnjCap cap);
const char* knj_cap_label(KnjCap cap);

// The reference's DeviceCaps field names (device_caps.h:69-85), filled from
// the device by create(), plus the full record of the C ABI.
struct DeviceCaps {
  char gcn_arch[16] = {};
  bool has_wmma = false;         // matrix cores (MFMA on CDNA)
  bool has_fp8 = false;
  bool has_dot_builtin = false;  // the sdot4 builtin compiles for this arch
  int wave_size = 0;
  uint64_t vram_total = 0, vram_usable = 0;
  bool rebar_full_aperture = false;
  uint32_t sms = 0, clock_khz = 0;  // sms: compute units
  uint32_t max_streams = 0, num_queue_groups = 0;
  bool arch_ok = false;
  const char* arch_reason = "";
  knj_device_caps device{};      // everything the C ABI reports
};

namespace knj {

using ::DeviceCaps;
using ::KnjCap;

// MoE FFN of n_tokens rows (knj_moe_decode_layer at one row,
// knj_moe_batch_layer above).
struct ExpertPlan {
  const float* x = nullptr;        // residual stream [n_tokens][n_embd]
  const float* norm_w = nullptr;   // ffn_norm (may be null: x already normalised)
  float eps = 1e-6f;
  const float* router_w = nullptr; // [n_expert][n_embd]
  const void* gate = nullptr;
  const void* up = nullptr;
  const void* down = nullptr;
  int type_gate_up = KNJ_TYPE_Q4_K, type_down = KNJ_TYPE_Q4_K;
  int n_tokens = 1;
  int n_embd = 0, n_ff = 0, n_expert = 0, k = 0;
  const float* resid = nullptr;
  float* out = nullptr;            // null: the plan only asks the gate question
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
  float* out = nullptr;            // null: the plan only asks the gate question
  void* stream = nullptr;
};

// The attention step writes the new KV slot itself; a stand-alone KV write
// (f16 rounding of the normalised, rotated k and of v into slot `pos`) is the
// same call with its output sent to scratch_out.
struct KvWritePlan {
  AttentionPlan attn;
  float* scratch_out = nullptr;  // [n_head][head_dim]; null: a device buffer the backend owns
};

class Backend {
 public:
  // Opens device KNJ_DEVICE (default 0) through the arch guard.
  static std::unique_ptr<Backend> create();
  // Test hook: a backend over injected caps, no device touched.
  static std::unique_ptr<Backend> from_caps(const DeviceCaps& caps);
  static const char* knj_last_refusal();

  const DeviceCaps& caps() const noexcept { return caps_; }
  bool would_instantiate(KnjCap cap) const noexcept;

  // The matrix-core path: the grouped f16-MFMA expert GEMMs
  // (knj_moe_batch_layer) at any n_tokens.
  virtual bool launch_expert_gemm_wmma(const ExpertPlan& p) = 0;
  // The vector path: the fused Q4_K/Q6_K GEMVs at n_tokens == 1
  // (knj_moe_decode_layer); larger batches go to the matrix-core path.
  virtual bool launch_expert_gemm_simt(const ExpertPlan& p) = 0;
  virtual bool launch_attention(const AttentionPlan& p) = 0;
  virtual void launch_kv_write(const KvWritePlan& p) = 0;

  virtual ~Backend() = default;

 protected:
  explicit Backend(const DeviceCaps& c) : caps_(c) {}
  DeviceCaps caps_;
};

}  // namespace knj

// The reference declares these at global scope; callers written against it
// name them unqualified.
using knj::AttentionPlan;
using knj::Backend;
using knj::ExpertPlan;
using knj::KvWritePlan;
