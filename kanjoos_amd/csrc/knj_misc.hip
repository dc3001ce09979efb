// kanjoos_amd/csrc/knj_misc.hip -- small kernels: dequant, RMSNorm, embedding.
#include "knj_common.h"
#include "knj_dev.h"

namespace knj {
namespace {

using namespace dev;

// Bit-exact block decode through the shared format header (dequant_row_f32,
// /root/reference/src/loader/dequant.cpp:1114-1256).
__global__ void k_dequant(int type, const uint8_t* __restrict__ w, uint64_t n,
                          float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t b = i / KNJ_QK;
  const int r = (int)(i % KNJ_QK);
  switch (type) {
    case KNJ_TYPE_Q4_K: out[i] = knj_q4k_weight(w + b * KNJ_Q4K_BLOCK, r); break;
    case KNJ_TYPE_Q6_K: out[i] = knj_q6k_weight(w + b * KNJ_Q6K_BLOCK, r); break;
    case KNJ_TYPE_BF16: out[i] = knj_bf16_to_f32(knj_rd_u16(w + 2 * i)); break;
    case KNJ_TYPE_F16: out[i] = knj_f16_to_f32(knj_rd_u16(w + 2 * i)); break;
    default: out[i] = reinterpret_cast<const float*>(w)[i]; break;
  }
}

// RMSNorm of one row (model.cpp:240-271): out = x * (1/sqrt(mean(x^2)+eps)) * w.
__global__ __launch_bounds__(kBlock) void k_rmsnorm(const float* __restrict__ x,
                                                    const float* __restrict__ w, int n, float eps,
                                                    float* __restrict__ out) {
  __shared__ float red[8];
  float ss = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
  ss = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * scale * w[i];
}

// Embedding row of the step's token (model.cpp:527-537).  Workgroup 0 also
// copies the RoPE cos/sin row of the step's position into `rope_cur`, so the
// attention launches of every layer read it without a position-dependent load.
__global__ void k_embed(int type, const uint8_t* __restrict__ table, int n_embd, StepState* st,
                        float* __restrict__ x, const float* __restrict__ rope_cos,
                        const float* __restrict__ rope_sin, int half, float* __restrict__ rope_cur) {
  const int id = st->token;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && rope_cur && threadIdx.x < 2 * half) {
    const int pos = st->pos, j = threadIdx.x % half;
    const float* tab = threadIdx.x < half ? rope_cos : rope_sin;
    rope_cur[threadIdx.x] = tab[(uint64_t)pos * half + j];
  }
  if (i >= n_embd) return;
  const uint64_t idx = (uint64_t)id * n_embd + i;
  if (type == KNJ_TYPE_BF16)
    x[i] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(table)[idx] << 16);
  else
    x[i] = reinterpret_cast<const float*>(table)[idx];
}

}  // namespace

hipError_t launch_dequant(int type, const uint8_t* w, uint64_t n, float* out, hipStream_t s) {
  const uint64_t blocks = (n + 255) / 256;
  KNJ_LAUNCH(k_dequant, dim3((unsigned)blocks), dim3(256), 0, s, type, w, n, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* out,
                          hipStream_t s) {
  KNJ_LAUNCH(k_rmsnorm, dim3(1), dim3(kBlock), 0, s, x, w, n, eps, out);
  return hipGetLastError();
}

hipError_t launch_embed(int type, const uint8_t* table, int n_embd, StepState* st, float* x,
                        const float* rope_cos, const float* rope_sin, int half, float* rope_cur,
                        hipStream_t s) {
  if (2 * half > 256) return hipErrorInvalidValue;
  KNJ_LAUNCH(k_embed, dim3((n_embd + 255) / 256), dim3(256), 0, s, type, table, n_embd, st,
                     x, rope_cos, rope_sin, half, rope_cur);
  return hipGetLastError();
}

}  // namespace knj
