// kanjoos_amd/csrc/knj_device.hip -- device gate, errors, memory, primitive entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "knj_common.h"

namespace knj {

namespace {
thread_local std::string g_error;
std::mutex g_mu;
bool g_open = false;
int g_device = -1;
void* g_scratch = nullptr;
uint64_t g_scratch_bytes = 0;
unsigned int* g_counters = nullptr;  // zeroed once at open; every user leaves them at zero
constexpr const char* kBuiltArch = "gfx950";
// Device address of `scratch` (below) per device, taken at knj_device_open.
constexpr int kMaxDevices = 64;
float* g_fixed_scratch[kMaxDevices] = {};
}  // namespace

// Fixed scratch of knj_moe_decode_layer_noalloc: hx [n_embd] then act
// [k][n_ff], at most kFixedScratchFloats floats.  Each device holds its own
// copy for the life of the process.  Host code never passes the array's name
// to a kernel: it is a host-side stand-in, and the device address comes from
// hipGetSymbolAddress at knj_device_open.
constexpr uint64_t kFixedScratchFloats = 32768;  // 128 KiB
static __device__ __align__(256) float scratch[kFixedScratchFloats];

void set_error(const std::string& msg) { g_error = msg; }

int hip_fail(hipError_t e, const char* what) {
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return KNJ_E_HIP;
}

unsigned int* device_counters() { return g_counters; }

int require_open() {
  if (!g_open) {
    set_error("device not open: call knj_device_open() first (arch guard)");
    return KNJ_E_STATE;
  }
  return KNJ_OK;
}

void* device_scratch(uint64_t bytes, hipStream_t stream) {
  std::lock_guard<std::mutex> g(g_mu);
  if (bytes > g_scratch_bytes) {
    if (g_scratch) {
      // the previous buffer may still be read by queued work
      if (hipStreamSynchronize(stream) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return nullptr;
      (void)hipFree(g_scratch);
      g_scratch = nullptr;
    }
    const uint64_t want = std::max<uint64_t>(bytes, 1u << 20);
    if (hipMalloc(&g_scratch, want) != hipSuccess) {
      g_scratch_bytes = 0;
      return nullptr;
    }
    g_scratch_bytes = want;
  }
  return g_scratch;
}

}  // namespace knj

using namespace knj;

extern "C" {

const char* knj_last_error(void) { return g_error.c_str(); }
const char* knj_built_arch(void) { return kBuiltArch; }

int knj_check_arch(const char* device_arch, const char* built_arch, const char* env_arch) {
  if (!device_arch || !built_arch || !built_arch[0]) {
    set_error("arch guard: missing arch string");
    return KNJ_E_ARCH;
  }
  // gcnArchName carries target features after ':' (e.g. gfx950:sramecc+:xnack-)
  const char* colon = std::strchr(device_arch, ':');
  const size_t n = colon ? (size_t)(colon - device_arch) : std::strlen(device_arch);
  if (n != std::strlen(built_arch) || std::strncmp(device_arch, built_arch, n) != 0) {
    set_error(std::string("arch mismatch: library built for ") + built_arch + ", device is " +
              std::string(device_arch, n));
    return KNJ_E_ARCH;
  }
  if (env_arch && env_arch[0] && std::strcmp(env_arch, built_arch) != 0) {
    set_error(std::string("arch mismatch: KNJ_BUILD_ARCH=") + env_arch + " but library built for " +
              built_arch);
    return KNJ_E_ARCH;
  }
  return KNJ_OK;
}

int knj_device_open(int device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    set_error("no HIP device visible");
    return KNJ_E_ENV;
  }
  if (device < 0 || device >= count) {
    set_error("device index out of range");
    return KNJ_E_ARG;
  }
  hipDeviceProp_t p;
  KNJ_HIP(hipGetDeviceProperties(&p, device));
  const int rc = knj_check_arch(p.gcnArchName, kBuiltArch, std::getenv("KNJ_BUILD_ARCH"));
  if (rc != KNJ_OK) return rc;
  KNJ_HIP(hipSetDevice(device));
  KNJ_HIP(expert_kernel_attributes());
  std::lock_guard<std::mutex> g(g_mu);
  if (device < kMaxDevices && !g_fixed_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "address of the fixed scratch");
    g_fixed_scratch[device] = (float*)p;
  }
  if (!g_counters) {
    KNJ_HIP(hipMalloc(&g_counters, 4096));
    KNJ_HIP(hipMemset(g_counters, 0, 4096));
  }
  g_open = true;
  g_device = device;
  return KNJ_OK;
}

int knj_device_close(void) {
  std::lock_guard<std::mutex> g(g_mu);
  if (g_scratch) {
    (void)hipDeviceSynchronize();
    (void)hipFree(g_scratch);
    g_scratch = nullptr;
    g_scratch_bytes = 0;
  }
  if (g_counters) {
    (void)hipDeviceSynchronize();
    (void)hipFree(g_counters);
    g_counters = nullptr;
  }
  g_open = false;
  return KNJ_OK;
}

int knj_device_caps_get(knj_device_caps* out) {
  KNJ_CHECK_ARG(out, "null caps pointer");
  int rc = require_open();
  if (rc) return rc;
  hipDeviceProp_t p;
  KNJ_HIP(hipGetDeviceProperties(&p, g_device));
  std::memset(out, 0, sizeof(*out));
  const char* colon = std::strchr(p.gcnArchName, ':');
  const size_t n = std::min<size_t>(colon ? (size_t)(colon - p.gcnArchName) : std::strlen(p.gcnArchName),
                                    sizeof(out->gcn_arch) - 1);
  std::memcpy(out->gcn_arch, p.gcnArchName, n);
  std::strncpy(out->name, p.name, sizeof(out->name) - 1);
  out->wave_size = p.warpSize;
  out->cu_count = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->lds_per_block = (int32_t)p.sharedMemPerBlock;
  out->l2_bytes = p.l2CacheSize;
  out->arch_ok = 1;
  // CDNA3/4 matrix cores: bf16 and int8 MFMA; gfx950 adds fp8/fp6/fp4 MFMA
  out->has_mfma_bf16 = 1;
  out->has_mfma_i8 = 1;
  out->has_fp8 = 1;
  size_t fr = 0, tot = 0;
  KNJ_HIP(hipMemGetInfo(&fr, &tot));
  out->vram_total = tot;
  out->vram_free = fr;
  return KNJ_OK;
}

int knj_malloc(void** dptr, uint64_t bytes) {
  KNJ_CHECK_ARG(dptr, "null pointer");
  int rc = require_open();
  if (rc) return rc;
  KNJ_HIP(hipMalloc(dptr, std::max<uint64_t>(bytes, 256)));
  return KNJ_OK;
}

int knj_free(void* dptr) {
  if (dptr) KNJ_HIP(hipFree(dptr));
  return KNJ_OK;
}

int knj_memcpy_h2d(void* dst, const void* src, uint64_t bytes) {
  KNJ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return KNJ_OK;
}

int knj_memcpy_d2h(void* dst, const void* src, uint64_t bytes) {
  KNJ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return KNJ_OK;
}

int knj_memset_zero(void* dst, uint64_t bytes) {
  KNJ_HIP(hipMemset(dst, 0, bytes));
  return KNJ_OK;
}

int knj_synchronize(void) {
  KNJ_HIP(hipDeviceSynchronize());
  return KNJ_OK;
}

static bool type_ok(int t) {
  return t == KNJ_TYPE_F32 || t == KNJ_TYPE_F16 || t == KNJ_TYPE_BF16 || t == KNJ_TYPE_Q4_K ||
         t == KNJ_TYPE_Q6_K;
}

int knj_dequant(int type, const void* w, uint64_t n_weights, float* out, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(type_ok(type), "unsupported weight type");
  KNJ_CHECK_ARG(w && out, "null pointer");
  KNJ_CHECK_ARG(n_weights % knj_block_weights(type) == 0, "run is not a whole number of blocks");
  KNJ_HIP(launch_dequant(type, (const uint8_t*)w, n_weights, out, (hipStream_t)stream));
  return KNJ_OK;
}

int knj_gemv(int type, const void* w, int n_in, int n_out, const float* x, const float* norm_w,
             float eps, const float* resid, float* y, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(type == KNJ_TYPE_Q4_K || type == KNJ_TYPE_Q6_K || type == KNJ_TYPE_BF16 ||
                    type == KNJ_TYPE_F32,
                "knj_gemv: type must be Q4_K, Q6_K, BF16 or F32");
  KNJ_CHECK_ARG(w && x && y, "null pointer");
  KNJ_CHECK_ARG(n_in > 0 && n_out > 0, "empty GEMV");
  KNJ_CHECK_ARG(n_in % 256 == 0, "n_in must be a multiple of 256");
  KNJ_CHECK_ARG(n_in <= 16384, "n_in above the LDS staging limit (16384)");
  GemvArgs a{type, (const uint8_t*)w, n_in, n_out, x, norm_w, eps, resid, y, nullptr};
  KNJ_HIP(launch_gemv(a, (hipStream_t)stream));
  return KNJ_OK;
}

int knj_rmsnorm(const float* x, const float* w, int n, float eps, float* out, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(x && w && out && n > 0, "bad rmsnorm arguments");
  KNJ_HIP(launch_rmsnorm(x, w, n, eps, out, (hipStream_t)stream));
  return KNJ_OK;
}

static int check_moe_shape(int n_embd, int n_ff, int n_expert, int k) {
  KNJ_CHECK_ARG(n_embd > 0 && n_embd % 256 == 0 && n_embd <= 16384,
                "n_embd must be a positive multiple of 256, at most 16384");
  KNJ_CHECK_ARG(n_ff > 0 && n_ff % 256 == 0, "n_ff must be a positive multiple of 256");
  KNJ_CHECK_ARG(n_expert > 0 && n_expert <= 256, "n_expert must be in [1, 256]");
  KNJ_CHECK_ARG(k > 0 && k <= 16 && k <= n_expert, "k must be in [1, min(16, n_expert)]");
  KNJ_CHECK_ARG((size_t)k * n_ff * 4 + (size_t)k * (n_ff / 32) * 4 + (size_t)k * 8 * 4 <= 160 * 1024,
                "k * n_ff too large for the down kernel's LDS staging");
  return KNJ_OK;
}

int knj_moe_router(const float* x, const float* norm_w, float eps, const float* router_w,
                   int n_embd, int n_expert, int k, float* hx, float* logits, int32_t* topk_idx,
                   float* topk_w, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  rc = check_moe_shape(n_embd, 256, n_expert, k);
  if (rc) return rc;
  KNJ_CHECK_ARG(n_embd <= 4096, "router: n_embd must be at most 4096");
  if (rc) return rc;
  KNJ_CHECK_ARG(x && router_w && hx && logits && topk_idx && topk_w, "null pointer");
  RouterArgs a{x, norm_w, eps, router_w, n_embd, n_expert, k, hx, logits, topk_idx, topk_w,
               device_counters()};
  KNJ_HIP(launch_router(a, (hipStream_t)stream));
  return KNJ_OK;
}

// The batch-1 MoE layer on a given scratch of n_embd + k * n_ff floats.
static int moe_decode_layer_on(float* scratch_ptr, const float* x, const float* norm_w, float eps,
                               const float* router_w, const void* gate, const void* up,
                               const void* down, int type_gate_up, int type_down, int n_embd,
                               int n_ff, int n_expert, int k, const float* resid, float* out,
                               float* logits, int32_t* topk_idx, float* topk_w, hipStream_t s) {
  float* hx = scratch_ptr;
  float* act = hx + n_embd;
  // logits only: the gate/up launch routes from them and writes topk_idx/topk_w
  RouterArgs ra{x, norm_w, eps, router_w, n_embd, n_expert, k, hx, logits, nullptr, nullptr,
                device_counters()};
  KNJ_HIP(launch_router(ra, s));
  ExpertArgs ea{x, norm_w, eps, logits, topk_idx, topk_w, (const uint8_t*)gate,
                (const uint8_t*)up, (const uint8_t*)down, type_gate_up, type_down, n_embd, n_ff,
                n_expert, k, act, resid, out, nullptr};
  KNJ_HIP(launch_experts(ea, s));
  return KNJ_OK;
}

static int check_moe_decode_args(const float* x, const float* router_w, const void* gate,
                                 const void* up, const void* down, int type_gate_up, int type_down,
                                 int n_embd, int n_ff, int n_expert, int k, float* out,
                                 float* logits, int32_t* topk_idx, float* topk_w) {
  int rc = require_open();
  if (rc) return rc;
  rc = check_moe_shape(n_embd, n_ff, n_expert, k);
  if (rc) return rc;
  KNJ_CHECK_ARG(n_embd <= 4096, "router: n_embd must be at most 4096");
  KNJ_CHECK_ARG(type_gate_up == KNJ_TYPE_Q4_K, "gate/up experts must be Q4_K");
  KNJ_CHECK_ARG(type_down == KNJ_TYPE_Q4_K || type_down == KNJ_TYPE_Q6_K,
                "down experts must be Q4_K or Q6_K");
  KNJ_CHECK_ARG(x && router_w && gate && up && down && out && logits && topk_idx && topk_w,
                "null pointer");
  return KNJ_OK;
}

int knj_moe_decode_layer(const float* x, const float* norm_w, float eps, const float* router_w,
                         const void* gate, const void* up, const void* down, int type_gate_up,
                         int type_down, int n_embd, int n_ff, int n_expert, int k,
                         const float* resid, float* out, float* logits, int32_t* topk_idx,
                         float* topk_w, void* stream) {
  int rc = check_moe_decode_args(x, router_w, gate, up, down, type_gate_up, type_down, n_embd,
                                 n_ff, n_expert, k, out, logits, topk_idx, topk_w);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const uint64_t bytes = (uint64_t)n_embd * 4 + (uint64_t)k * n_ff * 4;
  float* buf = (float*)device_scratch(bytes, s);
  if (!buf) return hip_fail(hipErrorOutOfMemory, "scratch");
  return moe_decode_layer_on(buf, x, norm_w, eps, router_w, gate, up, down, type_gate_up,
                             type_down, n_embd, n_ff, n_expert, k, resid, out, logits, topk_idx,
                             topk_w, s);
}

int knj_moe_decode_layer_noalloc(const float* x, const float* norm_w, float eps,
                                 const float* router_w, const void* gate, const void* up,
                                 const void* down, int type_gate_up, int type_down, int n_embd,
                                 int n_ff, int n_expert, int k, const float* resid, float* out,
                                 float* logits, int32_t* topk_idx, float* topk_w, void* stream) {
  int rc = check_moe_decode_args(x, router_w, gate, up, down, type_gate_up, type_down, n_embd,
                                 n_ff, n_expert, k, out, logits, topk_idx, topk_w);
  if (rc) return rc;
  const uint64_t need = (uint64_t)n_embd + (uint64_t)k * n_ff;
  if (need > kFixedScratchFloats) {
    set_error("knj_moe_decode_layer_noalloc: n_embd + k * n_ff = " + std::to_string(need) +
              " floats exceeds the fixed scratch of " + std::to_string(kFixedScratchFloats) +
              " floats (use knj_moe_decode_layer)");
    return KNJ_E_ARG;
  }
  int dev = -1;
  KNJ_HIP(hipGetDevice(&dev));
  float* fixed = (dev >= 0 && dev < kMaxDevices) ? g_fixed_scratch[dev] : nullptr;
  if (!fixed) {
    set_error("knj_moe_decode_layer_noalloc: the current device was not opened with knj_device_open");
    return KNJ_E_STATE;
  }
  return moe_decode_layer_on(fixed, x, norm_w, eps, router_w, gate, up, down, type_gate_up,
                             type_down, n_embd, n_ff, n_expert, k, resid, out, logits, topk_idx,
                             topk_w, (hipStream_t)stream);
}

int knj_moe_batch_layer(const float* x, const float* norm_w, float eps, const float* router_w,
                        const void* gate, const void* up, const void* down, int type_gate_up,
                        int type_down, int n_tokens, int n_embd, int n_ff, int n_expert, int k,
                        const float* resid, float* out, float* logits, int32_t* topk_idx,
                        float* topk_w, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(n_tokens > 0 && n_tokens <= 65536, "n_tokens must be in [1, 65536]");
  KNJ_CHECK_ARG(n_embd > 0 && n_embd % 256 == 0 && n_embd <= 4096,
                "n_embd must be a positive multiple of 256, at most 4096");
  KNJ_CHECK_ARG(n_ff > 0 && n_ff % 256 == 0 && n_ff <= 4096,
                "n_ff must be a positive multiple of 256, at most 4096");
  KNJ_CHECK_ARG(n_expert > 0 && n_expert <= 256, "n_expert must be in [1, 256]");
  KNJ_CHECK_ARG(k > 0 && k <= 16 && k <= n_expert, "k must be in [1, min(16, n_expert)]");
  KNJ_CHECK_ARG(type_gate_up == KNJ_TYPE_Q4_K &&
                    (type_down == KNJ_TYPE_Q4_K || type_down == KNJ_TYPE_Q6_K),
                "the batched expert path takes Q4_K gate/up and Q4_K or Q6_K down");
  KNJ_CHECK_ARG(x && router_w && gate && up && down && out && logits && topk_idx && topk_w,
                "null pointer");
  hipStream_t s = (hipStream_t)stream;
  void* scr = device_scratch(moe_batch_scratch_bytes(n_tokens, n_embd, n_ff, n_expert, k), s);
  if (!scr) return hip_fail(hipErrorOutOfMemory, "scratch");
  MoeBatchArgs a{x, norm_w, eps, router_w, (const uint8_t*)gate, (const uint8_t*)up,
                 (const uint8_t*)down, n_tokens, n_embd, n_ff, n_expert, k, resid, out, logits,
                 topk_idx, topk_w};
  a.type_down = type_down;
  KNJ_HIP(launch_moe_batch(a, scr, s));
  return KNJ_OK;
}

int knj_attention_step(const float* q, const float* k, const float* v, const float* q_norm,
                       const float* k_norm, float eps, float rope_base, int pos, int n_head,
                       int n_head_kv, int head_dim, int n_ctx, uint16_t* k_cache, uint16_t* v_cache,
                       float* out, void* stream) {
  int rc = require_open();
  if (rc) return rc;
  KNJ_CHECK_ARG(q && k && v && q_norm && k_norm && k_cache && v_cache && out, "null pointer");
  KNJ_CHECK_ARG(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
  KNJ_CHECK_ARG(n_head_kv > 0 && n_head_kv <= 64 && n_head % n_head_kv == 0 &&
                    n_head / n_head_kv <= 8,
                "n_head must be a multiple of n_head_kv (<= 64) with a group of at most 8");
  KNJ_CHECK_ARG(pos >= 0 && pos < n_ctx, "position outside the cache");
  hipStream_t s = (hipStream_t)stream;
  // cos/sin of this position, computed like the model's table (model.cpp:227-230, 278-279)
  const int half = head_dim / 2;
  std::vector<float> tab(2 * (size_t)half + 64);
  for (int i = 0; i < half; ++i) {
    const float inv = std::pow(rope_base, -2.0f * (float)i / (float)head_dim);
    const float th = (float)pos * inv;
    tab[i] = std::cos(th);
    tab[half + i] = std::sin(th);
  }
  std::memcpy(&tab[2 * half], &pos, sizeof(int));
  const int n_split = attn_splits(n_ctx);
  const uint64_t part_bytes = (uint64_t)n_head * n_split * (head_dim + 2) * 4;
  uint8_t* scr = (uint8_t*)device_scratch(1024 + part_bytes, s);
  if (!scr) return hip_fail(hipErrorOutOfMemory, "scratch");
  float* dtab = (float*)scr;
  int* dpos = (int*)(scr + 2 * half * 4);
  KNJ_HIP(hipMemcpyAsync(scr, tab.data(), 2 * half * 4 + 4, hipMemcpyHostToDevice, s));
  AttnArgs a{q, k, v, q_norm, k_norm, eps, dtab, dtab + half, dpos, k_cache, v_cache, n_head, n_head_kv,
             head_dim, n_ctx, 1.0f / std::sqrt((float)head_dim), (float*)(scr + 1024), out};
  KNJ_HIP(launch_attention(a, s));
  KNJ_HIP(hipStreamSynchronize(s));  // the host table must outlive the copy
  return KNJ_OK;
}

}  // extern "C"
