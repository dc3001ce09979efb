// kanjoos_amd/csrc/knj_kernels.hip -- gfx950 kernels of the batch-1 MoE decode step.
//
// Wave64 throughout.  Weights stay in their GGUF block formats in HBM and are
// decoded in registers; activations are staged in LDS once per workgroup.
//
// Q4_K GEMV lane mapping: a "slice" is one 32-byte code group of a super-block
// (sub-blocks 2g and 2g+1, 64 weights).  A row of n_in weights has 4*n_in/256
// slices; LPR lanes share a row (LPR = slices rounded up to a power of two,
// capped at 64), so a wave covers 64/LPR consecutive rows per step and every
// lane issues 16-byte loads: the block header and its two 16-byte code chunks.
// Per slice the lane forms the two code sums q.x and applies the factored form
// d1*sum(q.x) - dmin1*sum(x) (the reference's dot_q4_k, dequant.cpp:954-984),
// with sum(x) per 32-weight sub-block precomputed once in LDS.
#include "knj_common.h"

#include "../../include/knj_synth.h"

namespace knj {
namespace {

constexpr int kBlock = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits16 & 0xFFFFu));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over the workgroup in a fixed order: wave trees, then waves 0..3.
__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  const int nw = (blockDim.x + 63) >> 6;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage x (optionally RMS-normalised: x * (1/sqrt(mean(x^2)+eps)) * w) into LDS,
// plus the 32-weight sub-block sums of the staged values.
__device__ void stage_x(const float* __restrict__ x, const float* __restrict__ norm_w, float eps,
                        int n, float* xs, float* sx, float* red) {
  if (norm_w) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = x[i] * scale * norm_w[i];
  } else {
    for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = x[i];
  }
  __syncthreads();
  if (sx) {
    for (int sb = threadIdx.x; sb < n / 32; sb += blockDim.x) {
      float s = 0.0f;
#pragma unroll 8
      for (int l = 0; l < 32; ++l) s += xs[32 * sb + l];
      sx[sb] = s;
    }
    __syncthreads();
  }
}

// 6-bit scale and min of sub-block s from the header words (bytes 4..15 of the
// block are w1, w2, w3), same packing as knj_q4k_sub_scale.
__device__ __forceinline__ void q4k_scale_min(uint32_t w1, uint32_t w2, uint32_t w3, int s,
                                              uint32_t& sc, uint32_t& mn) {
  if (s < 4) {
    sc = (w1 >> (8 * s)) & 63u;
    mn = (w2 >> (8 * s)) & 63u;
  } else {
    const int t = s - 4;
    const uint32_t lo = (w3 >> (8 * t)) & 0xFFu;
    sc = (lo & 15u) | (((w1 >> (8 * t + 6)) & 3u) << 4);
    mn = (lo >> 4) | (((w2 >> (8 * t + 6)) & 3u) << 4);
  }
}

// Sums of codes*x for 16 code bytes: low nibbles against xlo[0..16), high
// nibbles against xhi[0..16).
__device__ __forceinline__ void q4k_dot16(const uint4 q, const float* xlo, const float* xhi,
                                          float& slo, float& shi) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 a = *reinterpret_cast<const float4*>(xlo + 4 * k);
    const float4 b = *reinterpret_cast<const float4*>(xhi + 4 * k);
    const uint32_t lo = w[k] & 0x0F0F0F0Fu;
    const uint32_t hi = (w[k] >> 4) & 0x0F0F0F0Fu;
    slo += (float)(lo & 0xFFu) * a.x;
    slo += (float)((lo >> 8) & 0xFFu) * a.y;
    slo += (float)((lo >> 16) & 0xFFu) * a.z;
    slo += (float)(lo >> 24) * a.w;
    shi += (float)(hi & 0xFFu) * b.x;
    shi += (float)((hi >> 8) & 0xFFu) * b.y;
    shi += (float)((hi >> 16) & 0xFFu) * b.z;
    shi += (float)(hi >> 24) * b.w;
  }
}

// Contribution of slice g (0..3) of one Q4_K block to a row dot product.
// xb: the 256 staged activations of this block, sxb: its 8 sub-block sums.
__device__ __forceinline__ float q4k_slice(const uint8_t* __restrict__ blk, int g,
                                           const float* xb, const float* sxb) {
  const uint4 h = *reinterpret_cast<const uint4*>(blk);
  const uint4 qa = *reinterpret_cast<const uint4*>(blk + KNJ_Q4K_QS + 32 * g);
  const uint4 qb = *reinterpret_cast<const uint4*>(blk + KNJ_Q4K_QS + 32 * g + 16);
  const float d = h2f(h.x), dmin = h2f(h.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(h.y, h.z, h.w, 2 * g, sc0, m0);
  q4k_scale_min(h.y, h.z, h.w, 2 * g + 1, sc1, m1);
  const float* x0 = xb + 64 * g;
  float s0 = 0.0f, s1 = 0.0f;
  q4k_dot16(qa, x0, x0 + 32, s0, s1);
  q4k_dot16(qb, x0 + 16, x0 + 48, s0, s1);
  const float d0 = d * (float)sc0, dm0 = dmin * (float)m0;
  const float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
  return (d0 * s0 - dm0 * sxb[2 * g]) + (d1 * s1 - dm1 * sxb[2 * g + 1]);
}

// Contribution of quarter t (0..3) of half hf (0..1) of one Q6_K block: 32
// weights, two 16-weight scale groups.  Q6_K blocks are 210 bytes, so only
// 2-byte alignment is guaranteed; the codes are read as bytes.
__device__ __forceinline__ float q6k_slice(const uint8_t* __restrict__ blk, int hf, int t,
                                           const float* xb) {
  const float d = h2f((uint32_t)blk[KNJ_Q6K_D] | ((uint32_t)blk[KNJ_Q6K_D + 1] << 8));
  const uint8_t* ql = blk + KNJ_Q6K_QL + 64 * hf + 32 * (t & 1);
  const uint8_t* qh = blk + KNJ_Q6K_QH + 32 * hf;
  const float* xq = xb + 128 * hf + 32 * t;
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll 8
  for (int l = 0; l < 32; ++l) {
    const uint32_t lb = ql[l];
    const uint32_t lo4 = (t < 2) ? (lb & 15u) : (lb >> 4);
    const uint32_t hi2 = ((uint32_t)qh[l] >> (2 * t)) & 3u;
    const float v = (float)((int)(lo4 | (hi2 << 4)) - 32) * xq[l];
    if (l < 16) s0 += v;
    else s1 += v;
  }
  const int8_t* sc = reinterpret_cast<const int8_t*>(blk + KNJ_Q6K_SC) + 8 * hf + 2 * t;
  return d * ((float)sc[0] * s0 + (float)sc[1] * s1);
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// ------------------------------------------------------------------ GEMV

template <int LPR>
__global__ __launch_bounds__(kBlock) void k_gemv_q4k(const uint8_t* __restrict__ w, int n_in,
                                                     int n_out, const float* __restrict__ x,
                                                     const float* __restrict__ norm_w, float eps,
                                                     const float* __restrict__ resid,
                                                     float* __restrict__ y) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* sx = xs + n_in;
  float* red = sx + n_in / 32;
  stage_x(x, norm_w, eps, n_in, xs, sx, red);
  const int nb = n_in / KNJ_QK, nslices = 4 * nb;
  const uint64_t rbytes = (uint64_t)nb * KNJ_Q4K_BLOCK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rsub = lane / LPR;
  constexpr int RPW = 64 / LPR;
  const int stride = gridDim.x * (kBlock / 64) * RPW;
  for (int row0 = (blockIdx.x * (kBlock / 64) + wave) * RPW; row0 < n_out; row0 += stride) {
    const int row = row0 + rsub;
    float acc = 0.0f;
    if (row < n_out) {
      const uint8_t* rp = w + (uint64_t)row * rbytes;
      for (int s = sub; s < nslices; s += LPR) {
        const int b = s >> 2;
        acc += q4k_slice(rp + (uint64_t)b * KNJ_Q4K_BLOCK, s & 3, xs + b * KNJ_QK, sx + 8 * b);
      }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (sub == 0 && row < n_out) y[row] = resid ? resid[row] + acc : acc;
  }
}

template <int LPR>
__global__ __launch_bounds__(kBlock) void k_gemv_q6k(const uint8_t* __restrict__ w, int n_in,
                                                     int n_out, const float* __restrict__ x,
                                                     const float* __restrict__ norm_w, float eps,
                                                     const float* __restrict__ resid,
                                                     float* __restrict__ y,
                                                     unsigned long long* argmax) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* red = xs + n_in;
  stage_x(x, norm_w, eps, n_in, xs, nullptr, red);
  const int nb = n_in / KNJ_QK, nslices = 8 * nb;
  const uint64_t rbytes = (uint64_t)nb * KNJ_Q6K_BLOCK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rsub = lane / LPR;
  constexpr int RPW = 64 / LPR;
  const int stride = gridDim.x * (kBlock / 64) * RPW;
  unsigned long long best = 0;
  for (int row0 = (blockIdx.x * (kBlock / 64) + wave) * RPW; row0 < n_out; row0 += stride) {
    const int row = row0 + rsub;
    float acc = 0.0f;
    if (row < n_out) {
      const uint8_t* rp = w + (uint64_t)row * rbytes;
      for (int s = sub; s < nslices; s += LPR) {
        const int b = s >> 3, hf = (s >> 2) & 1, t = s & 3;
        acc += q6k_slice(rp + (uint64_t)b * KNJ_Q6K_BLOCK, hf, t, xs + b * KNJ_QK);
      }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (sub == 0 && row < n_out) {
      const float v = resid ? resid[row] + acc : acc;
      y[row] = v;
      if (argmax) {
        const unsigned long long k = argmax_key(v, row);
        best = k > best ? k : best;
      }
    }
  }
  if (argmax) {
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long t = __shfl_xor(best, o, 64);
      best = t > best ? t : best;
    }
    if (lane == 0 && best) atomicMax(argmax, best);
  }
}

// BF16 / F32 rows: one wave per row, 8 (bf16) or 4 (f32) weights per lane per
// step, 16-byte loads.
template <bool BF16>
__global__ __launch_bounds__(kBlock) void k_gemv_plain(const uint8_t* __restrict__ w, int n_in,
                                                       int n_out, const float* __restrict__ x,
                                                       const float* __restrict__ norm_w, float eps,
                                                       const float* __restrict__ resid,
                                                       float* __restrict__ y,
                                                       unsigned long long* argmax) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* red = xs + n_in;
  stage_x(x, norm_w, eps, n_in, xs, nullptr, red);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int PER = BF16 ? 8 : 4;
  const uint64_t rbytes = (uint64_t)n_in * (BF16 ? 2 : 4);
  const int stride = gridDim.x * (kBlock / 64);
  unsigned long long best = 0;
  for (int row = blockIdx.x * (kBlock / 64) + wave; row < n_out; row += stride) {
    const uint8_t* rp = w + (uint64_t)row * rbytes;
    float acc = 0.0f;
    for (int i0 = lane * PER; i0 < n_in; i0 += 64 * PER) {
      const uint4 v = *reinterpret_cast<const uint4*>(rp + (uint64_t)i0 * (BF16 ? 2 : 4));
      const float4 xa = *reinterpret_cast<const float4*>(xs + i0);
      if (BF16) {
        const float4 xb = *reinterpret_cast<const float4*>(xs + i0 + 4);
        acc += __uint_as_float(v.x << 16) * xa.x;
        acc += __uint_as_float(v.x & 0xFFFF0000u) * xa.y;
        acc += __uint_as_float(v.y << 16) * xa.z;
        acc += __uint_as_float(v.y & 0xFFFF0000u) * xa.w;
        acc += __uint_as_float(v.z << 16) * xb.x;
        acc += __uint_as_float(v.z & 0xFFFF0000u) * xb.y;
        acc += __uint_as_float(v.w << 16) * xb.z;
        acc += __uint_as_float(v.w & 0xFFFF0000u) * xb.w;
      } else {
        acc += __uint_as_float(v.x) * xa.x;
        acc += __uint_as_float(v.y) * xa.y;
        acc += __uint_as_float(v.z) * xa.z;
        acc += __uint_as_float(v.w) * xa.w;
      }
    }
    acc = wave_sum(acc);
    const float out = resid ? resid[row] + acc : acc;
    if (lane == 0) y[row] = out;
    if (argmax) {
      const unsigned long long k = argmax_key(out, row);
      best = k > best ? k : best;
    }
  }
  if (argmax && lane == 0 && best) atomicMax(argmax, best);
}

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

// ------------------------------------------------------------------ router
// Workgroups of 4 waves, one wave per expert row.  Every workgroup normalises x
// itself (same order, same result); workgroup 0 also publishes hx.  The last
// workgroup to finish (ticket) does softmax and top-k over all logits.
__global__ __launch_bounds__(kBlock) void k_router(RouterArgs a) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* red = xs + a.n_embd;
  __shared__ unsigned int ticket;
  stage_x(a.x, a.norm_w, a.eps, a.n_embd, xs, nullptr, red);
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < a.n_embd; i += blockDim.x) a.hx[i] = xs[i];
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * (kBlock / 64) + wave;
  if (e < a.n_expert) {
    const float* wr = a.router_w + (uint64_t)e * a.n_embd;
    float acc = 0.0f;
    for (int i = lane * 4; i < a.n_embd; i += 256) {
      const float4 wv = *reinterpret_cast<const float4*>(wr + i);
      const float4 xv = *reinterpret_cast<const float4*>(xs + i);
      acc += wv.x * xv.x;
      acc += wv.y * xv.y;
      acc += wv.z * xv.z;
      acc += wv.w * xv.w;
    }
    acc = wave_sum(acc);
    if (lane == 0) a.logits[e] = acc;
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) ticket = atomicAdd(a.counter, 1u);
  __syncthreads();
  if (ticket != gridDim.x - 1) return;
  __threadfence();
  if (wave != 0) return;
  // softmax over all experts (up to 4 per lane), then top-k
  constexpr int kMaxPer = 4;
  float p[kMaxPer];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int ex = lane + 64 * j;
    p[j] = ex < a.n_expert ? ld_coherent(a.logits + ex) : -INFINITY;
    mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int ex = lane + 64 * j;
    p[j] = ex < a.n_expert ? expf(p[j] - mx) : 0.0f;
    sum += p[j];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) p[j] = p[j] / sum;
  bool taken[kMaxPer] = {false, false, false, false};
  float keep = 0.0f;
  int chosen_idx[16];
  float chosen_p[16];
  for (int k = 0; k < a.k; ++k) {
    // best untaken: larger probability, ties to the lower index
    float bv = -1.0f;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
      const int ex = lane + 64 * j;
      if (ex < a.n_expert && !taken[j] && (p[j] > bv || (p[j] == bv && ex < bi))) {
        bv = p[j];
        bi = ex;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j)
      if (lane + 64 * j == bi) taken[j] = true;
    chosen_idx[k] = bi;
    chosen_p[k] = bv;
    keep += bv;
  }
  const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
  if (lane == 0) {
    for (int k = 0; k < a.k; ++k) {
      a.topk_idx[k] = chosen_idx[k];
      a.topk_w[k] = chosen_p[k] * inv;
    }
    __threadfence();
    atomicExch(a.counter, 0u);
  }
}

// ------------------------------------------------------------------ experts
// Gate and up of one chosen expert: lanes [0,32) run a gate row, lanes [32,64)
// the matching up row (n_in = 8 super-blocks gives exactly 32 slices), then
// act = silu(g) * u.
__global__ __launch_bounds__(kBlock) void k_expert_gateup(ExpertArgs a) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* sx = xs + a.n_embd;
  float* red = sx + a.n_embd / 32;
  stage_x(a.hx, nullptr, 0.0f, a.n_embd, xs, sx, red);
  const int kk = blockIdx.y;
  const int e = a.topk_idx[kk];
  const int nb = a.n_embd / KNJ_QK, nslices = 4 * nb;
  const uint64_t rbytes = (uint64_t)nb * KNJ_Q4K_BLOCK;
  const uint64_t slab = rbytes * (uint64_t)a.n_ff;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, sub = lane & 31;
  const uint8_t* base = (half ? a.up : a.gate) + (uint64_t)e * slab;
  const int stride = gridDim.x * (kBlock / 64);
  for (int row = blockIdx.x * (kBlock / 64) + wave; row < a.n_ff; row += stride) {
    const uint8_t* rp = base + (uint64_t)row * rbytes;
    float acc = 0.0f;
    for (int s = sub; s < nslices; s += 32) {
      const int b = s >> 2;
      acc += q4k_slice(rp + (uint64_t)b * KNJ_Q4K_BLOCK, s & 3, xs + b * KNJ_QK, sx + 8 * b);
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    const float u = __shfl(acc, 32, 64);
    if (lane == 0) {
      const float g = acc;
      const float silu = g / (1.0f + expf(-g));
      a.act[(uint64_t)kk * a.n_ff + row] = silu * u;
    }
  }
}

// Down projection of all k chosen experts for a tile of output rows, then the
// weighted sum in ascending expert index (the reference's scatter order) and
// the residual add.  Tasks are (expert slot, row) pairs, LPR lanes each.
template <int LPR, bool Q6>
__global__ __launch_bounds__(kBlock) void k_expert_down(ExpertArgs a, int rows_per_block) {
  extern __shared__ float smem[];
  const int F = a.n_ff, K = a.k;
  float* acts = smem;                       // [K][F]
  float* sx = acts + K * F;                 // [K][F/32]
  float* dots = sx + K * (F / 32);          // [K][rows_per_block]
  for (int i = threadIdx.x; i < K * F; i += blockDim.x) acts[i] = a.act[i];
  __syncthreads();
  if (!Q6) {
    for (int sb = threadIdx.x; sb < K * (F / 32); sb += blockDim.x) {
      float s = 0.0f;
#pragma unroll 8
      for (int l = 0; l < 32; ++l) s += acts[32 * sb + l];
      sx[sb] = s;
    }
  }
  __syncthreads();
  const int row_base = blockIdx.x * rows_per_block;
  const int nb = F / KNJ_QK;
  const int nslices = (Q6 ? 8 : 4) * nb;
  const uint64_t rbytes = (uint64_t)nb * (Q6 ? KNJ_Q6K_BLOCK : KNJ_Q4K_BLOCK);
  const uint64_t slab = rbytes * (uint64_t)a.n_embd;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, tsub = lane / LPR;
  constexpr int TPW = 64 / LPR;
  const int ntasks = K * rows_per_block;
  for (int t0 = wave * TPW; t0 < ntasks; t0 += (kBlock / 64) * TPW) {
    const int t = t0 + tsub;
    float acc = 0.0f;
    const int kk = t / rows_per_block, r = t % rows_per_block;
    const int row = row_base + r;
    if (t < ntasks && row < a.n_embd) {
      const int e = a.topk_idx[kk];
      const uint8_t* rp = a.down + (uint64_t)e * slab + (uint64_t)row * rbytes;
      const float* xk = acts + kk * F;
      for (int s = sub; s < nslices; s += LPR) {
        if (Q6) {
          const int b = s >> 3;
          acc += q6k_slice(rp + (uint64_t)b * KNJ_Q6K_BLOCK, (s >> 2) & 1, s & 3, xk + b * KNJ_QK);
        } else {
          const int b = s >> 2;
          acc += q4k_slice(rp + (uint64_t)b * KNJ_Q4K_BLOCK, s & 3, xk + b * KNJ_QK,
                           sx + kk * (F / 32) + 8 * b);
        }
      }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (sub == 0 && t < ntasks) dots[kk * rows_per_block + r] = acc;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < rows_per_block; r += blockDim.x) {
    const int row = row_base + r;
    if (row >= a.n_embd) break;
    // ascending expert index; k is small, so rank by counting
    float o = 0.0f;
    for (int rank = 0; rank < K; ++rank) {
      int pick = 0;
      for (int kk = 0; kk < K; ++kk) {
        int cnt = 0;
        const int ek = a.topk_idx[kk];
        for (int j = 0; j < K; ++j) cnt += (a.topk_idx[j] < ek) ? 1 : 0;
        if (cnt == rank) pick = kk;
      }
      o = __fadd_rn(o, __fmul_rn(a.topk_w[pick], dots[pick * rows_per_block + r]));
    }
    const float v = a.resid ? __fadd_rn(a.resid[row], o) : o;
    a.out[row] = v;
    if (a.hidden_copy) a.hidden_copy[row] = v;
  }
}

// ------------------------------------------------------------------ attention prep
// One workgroup per head (q heads first, then kv heads), head_dim threads:
// per-head RMSNorm, NEOX rotation of (i, i + D/2) from the precomputed cos/sin
// table, f16 append of k and v at the current position.
__global__ void k_qk_rope_append(QkRopeArgs a) {
  __shared__ float vals[512];
  __shared__ float red[8];
  const int D = a.head_dim, half = D / 2;
  const int hidx = blockIdx.x;
  const bool is_q = hidx < a.n_head;
  const int h = is_q ? hidx : hidx - a.n_head;
  const int d = threadIdx.x;
  const int pos = *a.pos;
  const float* src = is_q ? a.q + (uint64_t)h * D : a.k + (uint64_t)h * D;
  const float* nw = is_q ? a.q_norm : a.k_norm;
  const float xv = d < D ? src[d] : 0.0f;
  const float ss = block_sum(xv * xv, red);
  const float scale = 1.0f / sqrtf(ss / (float)D + a.eps);
  if (d < D) vals[d] = xv * scale * nw[d];
  __syncthreads();
  if (d < half) {
    const float c = a.rope_cos[(uint64_t)pos * half + d];
    const float s = a.rope_sin[(uint64_t)pos * half + d];
    const float x0 = vals[d], x1 = vals[d + half];
    const float y0 = x0 * c - x1 * s;
    const float y1 = x0 * s + x1 * c;
    if (is_q) {
      a.q[(uint64_t)h * D + d] = y0;
      a.q[(uint64_t)h * D + d + half] = y1;
    } else {
      uint16_t* kc = a.k_cache + ((uint64_t)h * a.n_ctx + pos) * D;
      kc[d] = knj_f32_to_f16(y0);
      kc[d + half] = knj_f32_to_f16(y1);
    }
  }
  if (!is_q && d < D) {
    a.v_cache[((uint64_t)h * a.n_ctx + pos) * D + d] = knj_f32_to_f16(a.v[(uint64_t)h * D + d]);
  }
}

// ------------------------------------------------------------------ attention
// Split-KV decode attention.  Workgroup (kv head, split) owns positions
// [split*kChunk, +kChunk) for all `group` query heads of that kv head: scores in
// LDS, per-head chunk max / sum / weighted V, written as a partial record
// {m, l, acc[D]}.  The merge workgroup combines the splits of one head in
// ascending split order.
constexpr int kChunk = 64;
constexpr int kMaxGroup = 8;
constexpr int kMaxD = 128;

__global__ __launch_bounds__(kBlock) void k_attn_partial(AttnArgs a) {
  __shared__ float qs[kMaxGroup * kMaxD];
  __shared__ float sc[kMaxGroup * kChunk];
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int D = a.head_dim, G = a.n_head / a.n_head_kv;
  const int n_kv = a.n_kv_dev ? (*a.n_kv_dev + a.n_kv_add) : a.n_kv_host;
  const int n_split = gridDim.y;
  const int p0 = split * kChunk;
  const int cnt = min(kChunk, n_kv - p0);
  float* part = a.partial + ((uint64_t)(kvh * G) * n_split + split) * (D + 2);
  const uint64_t hstride = (uint64_t)n_split * (D + 2);
  if (cnt <= 0) {
    for (int i = threadIdx.x; i < G * (D + 2); i += blockDim.x) {
      const int g = i / (D + 2), j = i % (D + 2);
      part[g * hstride + j] = (j == 0) ? -INFINITY : 0.0f;
    }
    return;
  }
  for (int i = threadIdx.x; i < G * D; i += blockDim.x) qs[i] = a.q[(uint64_t)(kvh * G) * D + i];
  __syncthreads();
  const uint16_t* kb = a.k_cache + ((uint64_t)kvh * a.n_ctx + p0) * D;
  const uint16_t* vb = a.v_cache + ((uint64_t)kvh * a.n_ctx + p0) * D;
  // scores: 16 lanes per position, 8 dims per lane (one 16-byte load)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pl = lane >> 4, dl = lane & 15;
  for (int p = wave * 4 + pl; p < kChunk; p += 16) {
    float part_s[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) part_s[g] = 0.0f;
    if (p < cnt && dl * 8 < D) {
      const uint4 kv4 = *reinterpret_cast<const uint4*>(kb + (uint64_t)p * D + dl * 8);
      const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
      float kf[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kf[2 * i] = h2f(kw[i]);
        kf[2 * i + 1] = h2f(kw[i] >> 16);
      }
      for (int g = 0; g < G; ++g) {
        const float* qg = qs + g * D + dl * 8;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += qg[i] * kf[i];
        part_s[g] = s;
      }
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      float s = part_s[g];
      for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      part_s[g] = s;
    }
    if (dl == 0) {
      for (int g = 0; g < G; ++g) sc[g * kChunk + p] = p < cnt ? part_s[g] * a.scale : -INFINITY;
    }
  }
  __syncthreads();
  // per head: chunk max and exp; wave w handles heads w, w+4
  for (int g = wave; g < G; g += kBlock / 64) {
    const float v = lane < cnt ? sc[g * kChunk + lane] : -INFINITY;
    const float m = wave_max(v);
    const float e = lane < cnt ? expf(v - m) : 0.0f;
    const float l = wave_sum(e);
    sc[g * kChunk + lane] = e;
    if (lane == 0) {
      part[g * hstride + 0] = m;
      part[g * hstride + 1] = l;
    }
  }
  __syncthreads();
  // weighted V: thread owns dim pair (2*dp, 2*dp+1) for heads hg, hg+4
  const int dp = threadIdx.x & 63, hg = threadIdx.x >> 6;
  if (dp * 2 < D) {
    float acc0[2] = {0.0f, 0.0f}, acc1[2] = {0.0f, 0.0f};
    for (int p = 0; p < cnt; ++p) {
      const uint32_t vv = *reinterpret_cast<const uint32_t*>(vb + (uint64_t)p * D + 2 * dp);
      const float v0 = h2f(vv), v1 = h2f(vv >> 16);
      const float e0 = sc[hg * kChunk + p];
      acc0[0] += e0 * v0;
      acc0[1] += e0 * v1;
      if (hg + 4 < G) {
        const float e1 = sc[(hg + 4) * kChunk + p];
        acc1[0] += e1 * v0;
        acc1[1] += e1 * v1;
      }
    }
    if (hg < G) {
      part[hg * hstride + 2 + 2 * dp] = acc0[0];
      part[hg * hstride + 3 + 2 * dp] = acc0[1];
    }
    if (hg + 4 < G) {
      part[(hg + 4) * hstride + 2 + 2 * dp] = acc1[0];
      part[(hg + 4) * hstride + 3 + 2 * dp] = acc1[1];
    }
  }
}

__global__ void k_attn_merge(AttnArgs a, int n_split) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int D = a.head_dim;
  const float* part = a.partial + (uint64_t)h * n_split * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, part[(uint64_t)s * (D + 2)]);
  float L = 0.0f, acc = 0.0f;
  for (int s = 0; s < n_split; ++s) {
    const float m = part[(uint64_t)s * (D + 2)];
    if (m == -INFINITY) continue;
    const float f = expf(m - M);
    L += part[(uint64_t)s * (D + 2) + 1] * f;
    if (d < D) acc += part[(uint64_t)s * (D + 2) + 2 + d] * f;
  }
  if (d < D) a.out[(uint64_t)h * D + d] = acc / L;
}

__global__ void k_embed(int type, const uint8_t* __restrict__ table, int n_embd,
                        const int32_t* __restrict__ tok, float* __restrict__ x) {
  const int id = *tok;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_embd) return;
  const uint64_t idx = (uint64_t)id * n_embd + i;
  if (type == KNJ_TYPE_BF16) x[i] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(table)[idx] << 16);
  else x[i] = reinterpret_cast<const float*>(table)[idx];
}

}  // namespace

// ====================================================================== launchers

static int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t s) {
  const size_t lds_x = (size_t)a.n_in * 4;
  if (a.type == KNJ_TYPE_Q4_K) {
    const int lpr = std::min(64, pow2_at_least(4 * (a.n_in / KNJ_QK)));
    const size_t lds = lds_x + (size_t)(a.n_in / 32) * 4 + 64;
    const int rows_per_block = 4 * (64 / lpr);
    const int grid = std::max(1, std::min(4096, (a.n_out + rows_per_block - 1) / rows_per_block));
#define GQ4(L)                                                                                 \
  case L:                                                                                      \
    hipLaunchKernelGGL(k_gemv_q4k<L>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out, \
                       a.x, a.norm_w, a.eps, a.resid, a.y);                                    \
    break;
    switch (lpr) { GQ4(4) GQ4(8) GQ4(16) GQ4(32) GQ4(64) default: return hipErrorInvalidValue; }
#undef GQ4
    return hipGetLastError();
  }
  if (a.type == KNJ_TYPE_Q6_K) {
    const int lpr = std::min(64, pow2_at_least(8 * (a.n_in / KNJ_QK)));
    const size_t lds = lds_x + 64;
    const int rows_per_block = 4 * (64 / lpr);
    const int grid = std::max(1, std::min(4096, (a.n_out + rows_per_block - 1) / rows_per_block));
#define GQ6(L)                                                                                 \
  case L:                                                                                      \
    hipLaunchKernelGGL(k_gemv_q6k<L>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out, \
                       a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);                      \
    break;
    switch (lpr) { GQ6(8) GQ6(16) GQ6(32) GQ6(64) default: return hipErrorInvalidValue; }
#undef GQ6
    return hipGetLastError();
  }
  const size_t lds = lds_x + 64;
  const int grid = std::max(1, std::min(4096, (a.n_out + 3) / 4));
  if (a.type == KNJ_TYPE_BF16) {
    hipLaunchKernelGGL(k_gemv_plain<true>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out,
                       a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);
  } else {
    hipLaunchKernelGGL(k_gemv_plain<false>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in,
                       a.n_out, a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);
  }
  return hipGetLastError();
}

hipError_t launch_dequant(int type, const uint8_t* w, uint64_t n, float* out, hipStream_t s) {
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(256), 0, s, type, w, n, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* out,
                          hipStream_t s) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kBlock), 0, s, x, w, n, eps, out);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs& a, hipStream_t s) {
  const int grid = (a.n_expert + 3) / 4;
  const size_t lds = (size_t)a.n_embd * 4 + 64;
  hipLaunchKernelGGL(k_router, dim3(grid), dim3(kBlock), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_experts(const ExpertArgs& a, hipStream_t s) {
  const hipError_t e = launch_expert_gateup(a, s);
  if (e != hipSuccess) return e;
  return launch_expert_down(a, s);
}

hipError_t launch_expert_gateup(const ExpertArgs& a, hipStream_t s) {
  const size_t lds = (size_t)a.n_embd * 4 + (size_t)(a.n_embd / 32) * 4 + 64;
  const int rows_per_block = 16;  // 4 waves x 4 row pairs
  dim3 grid((a.n_ff + rows_per_block - 1) / rows_per_block, a.k);
  hipLaunchKernelGGL(k_expert_gateup, grid, dim3(kBlock), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_expert_down(const ExpertArgs& a, hipStream_t s) {
  const bool q6 = a.type_down == KNJ_TYPE_Q6_K;
  const int nb = a.n_ff / KNJ_QK;
  const int lpr = std::min(64, pow2_at_least((q6 ? 8 : 4) * nb));
  const int rows_per_block = 8;
  const size_t lds = ((size_t)a.k * a.n_ff + (size_t)a.k * (a.n_ff / 32) +
                      (size_t)a.k * rows_per_block) * 4;
  const int grid = (a.n_embd + rows_per_block - 1) / rows_per_block;
#define GD(L, Q)                                                                           \
  if (lpr == L && q6 == Q) {                                                               \
    hipLaunchKernelGGL((k_expert_down<L, Q>), dim3(grid), dim3(kBlock), lds, s, a,         \
                       rows_per_block);                                                    \
    return hipGetLastError();                                                              \
  }
  GD(4, false) GD(8, false) GD(16, false) GD(32, false) GD(64, false)
  GD(8, true) GD(16, true) GD(32, true) GD(64, true)
#undef GD
  return hipErrorInvalidValue;
}

hipError_t launch_qk_rope_append(const QkRopeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_qk_rope_append, dim3(a.n_head + a.n_head_kv), dim3(a.head_dim), 0, s, a);
  return hipGetLastError();
}

int attn_splits(int n_ctx) { return (n_ctx + kChunk - 1) / kChunk; }

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
  const int n_split = attn_splits(a.n_ctx);
  hipLaunchKernelGGL(k_attn_partial, dim3(a.n_head_kv, n_split), dim3(kBlock), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_merge, dim3(a.n_head), dim3(a.head_dim), 0, s, a, n_split);
  return hipGetLastError();
}

hipError_t launch_embed(int type, const uint8_t* table, int n_embd, const int32_t* tok, float* x,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3((n_embd + 255) / 256), dim3(256), 0, s, type, table, n_embd,
                     tok, x);
  return hipGetLastError();
}

}  // namespace knj
