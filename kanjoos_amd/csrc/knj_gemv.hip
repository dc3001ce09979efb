// kanjoos_amd/csrc/knj_gemv.hip -- batch-1 GEMV kernels (Q4_K, Q6_K, BF16, F32).
//
// y[j] = sum_i W[j][i] * x[i] over rows j of a ggml 2-D weight (one row per
// output, n_in weights each), the device side of Model::matmul at m == 1
// (/root/reference/src/model/model.cpp:326-380).  Optional fused RMSNorm of x
// and residual add.
//
// Q4_K rows: LPR lanes per row, one 64-weight slice per lane (n_in <= 64*LPR),
// RS row-steps per wave.  Every lane issues the 16-byte loads of all its rows
// before the activation staging starts, keeps its 64 activations in registers
// and reuses them for each row.
#include "knj_common.h"
#include "knj_dev.h"

namespace knj {
namespace {

using namespace dev;

constexpr int kRouterF4 = 8;  // float4 per lane of a router quarter row: n_embd + n_in <= 8192

template <int LPR, int RS>
__device__ __forceinline__ void gemv_q4k_body(const uint8_t* __restrict__ w, int n_in, int n_out,
                                              const float* __restrict__ x,
                                              const float* __restrict__ nw, float eps,
                                              const float* __restrict__ resid,
                                              float* __restrict__ y) {
  __shared__ float xs[xpad_size(4096)];
  __shared__ float xsum[128];
  __shared__ float red[8];
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rsub = lane / LPR;
  const int nslices = n_in >> 6;
  const uint64_t rb = (uint64_t)(n_in >> 8) * KNJ_Q4K_BLOCK;
  const int row0 = (blockIdx.x * (kBlock / 64) + wave) * (RS * RPW);
  const bool active = sub < nslices;
  const int b = active ? (sub >> 2) : 0, g = sub & 3;
  // loads in the order they are needed: x (and its norm weight) first, so the
  // staging waits only for them; then the weights and the residual
  XRegs xr;
  stage_x_load(x, nw, n_in, xr);
  Q4Slice q[RS];
  float rv[RS];
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int row = min(row0 + st * RPW + rsub, n_out - 1);  // valid address; extra rows dropped
    q[st] = q4k_load(w + (uint64_t)row * rb + (uint64_t)b * KNJ_Q4K_BLOCK, g);
  }
#pragma unroll
  for (int st = 0; st < RS; ++st)
    rv[st] = resid ? resid[min(row0 + st * RPW + rsub, n_out - 1)] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  stage_x_store(xr, nw != nullptr, eps, n_in, xs, red, xsum);
  XSlice xv;
  const int sl = active ? sub : 0;
  xslice_load_sums(xs, sl, xsum[2 * sl], xsum[2 * sl + 1], xv);
  float res[RS];
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int row = row0 + st * RPW + rsub;
    float acc = (active && row < n_out) ? q4k_dot(q[st], g, xv) : 0.0f;
    res[st] = group_sum<LPR>(acc);
  }
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int row = row0 + st * RPW + rsub;
    if (sub == 0 && row < n_out) y[row] = resid ? rv[st] + res[st] : res[st];
  }
}

template <int LPR, int RS>
__global__ __launch_bounds__(kBlock) void k_gemv_q4k(const uint8_t* __restrict__ w, int n_in,
                                                     int n_out, const float* __restrict__ x,
                                                     const float* __restrict__ nw, float eps,
                                                     const float* __restrict__ resid,
                                                     float* __restrict__ y) {
  gemv_q4k_body<LPR, RS>(w, n_in, n_out, x, nw, eps, resid, y);
}

// The attention-output GEMV y = resid + W x (one row step per wave) with the
// router's logits computed in the same launch, before the normalisation of
// y.  The router applies W_r to RMSNorm(y) with y = resid + W x
// (/root/reference/src/model/model.cpp:420-423, 620-628); regrouped,
//   logit_e = scale * (sum_i R[e][i] resid[i] + sum_j R[e][H + j] x[j]),
//   R[e][i] = W_r[e][i] nw[i],  R[e][H + j] = sum_i R[e][i] W[i][j],
// with scale = 1 / sqrt(mean(y^2) + eps), which needs all of y and is applied
// by the gate/up launch (the ranking does not depend on it, the weights do).
// Workgroups past the GEMV's take one row e of R each, a quarter row per
// wave (the 8 KB resid and the x inputs read as they are), and write the
// unscaled logit u[e]; they do not depend on the GEMV's rows, so the two
// run side by side.  R is precomputed per layer from the weights
// (launch_router_fold).
template <int LPR>
__global__ __launch_bounds__(kBlock) void k_gemv_q4k_router(const uint8_t* __restrict__ w, int n_in,
                                                            int n_out, const float* __restrict__ x,
                                                            const float* __restrict__ resid,
                                                            float* __restrict__ y,
                                                            const float* __restrict__ R, int n_router,
                                                            int n_gemv_blocks, float* __restrict__ u) {
  if ((int)blockIdx.x < n_gemv_blocks) {
    gemv_q4k_body<LPR, 1>(w, n_in, n_out, x, nullptr, 0.0f, resid, y);
    return;
  }
  __shared__ float part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x - n_gemv_blocks, H = n_out, NR = n_out + n_in, Q = NR >> 2;
  const float* rr = R + (uint64_t)e * NR;
  float4 wv[kRouterF4], iv[kRouterF4];
#pragma unroll
  for (int j = 0; j < kRouterF4; ++j) {
    const int i = Q * wave + 4 * lane + 256 * j;
    if (4 * lane + 256 * j < Q) {
      wv[j] = *reinterpret_cast<const float4*>(rr + i);
      iv[j] = i < H ? *reinterpret_cast<const float4*>(resid + i)
                    : *reinterpret_cast<const float4*>(x + (i - H));
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kRouterF4; ++j)
    if (4 * lane + 256 * j < Q) {
      acc += wv[j].x * iv[j].x;
      acc += wv[j].y * iv[j].y;
      acc += wv[j].z * iv[j].z;
      acc += wv[j].w * iv[j].w;
    }
  acc = group_sum<64>(acc);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0 && e < n_router) u[e] = ((part[0] + part[1]) + part[2]) + part[3];
}

// R (see k_gemv_q4k_router) from the router weights W_r [E][H], the norm
// weight nw [H] and the dequantised attention-output matrix Wd [H][QD]:
// thread (column j, 8 rows e) accumulates sum_i R[e][i] Wd[i][j] in double
// and rounds once to f32; the first H columns are the products W_r nw.
__global__ __launch_bounds__(kBlock) void k_router_fold(const float* __restrict__ wr,
                                                        const float* __restrict__ nw,
                                                        const float* __restrict__ wd, int H, int QD,
                                                        int E, float* __restrict__ R) {
  const int j = blockIdx.x * kBlock + threadIdx.x, e0 = 8 * blockIdx.y;
  const int NR = H + QD;
  if (j < H) {
    for (int e = e0; e < min(E, e0 + 8); ++e) R[(uint64_t)e * NR + j] = wr[(uint64_t)e * H + j] * nw[j];
  }
  if (j >= QD) return;
  double acc[8] = {};
  for (int i = 0; i < H; ++i) {
    const double wdv = (double)wd[(uint64_t)i * QD + j];
    const float nwi = nw[i];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (e0 + q < E) acc[q] += (double)(wr[(uint64_t)(e0 + q) * H + i] * nwi) * wdv;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q)
    if (e0 + q < E) R[(uint64_t)(e0 + q) * NR + H + j] = (float)acc[q];
}

// Q4_K rows wider than 64 slices (n_in > 4096, up to 16384): the activations
// stay in LDS and each lane walks several slices per row.
__global__ __launch_bounds__(kBlock) void k_gemv_q4k_wide(const uint8_t* __restrict__ w, int n_in,
                                                          int n_out, const float* __restrict__ x,
                                                          const float* __restrict__ nw, float eps,
                                                          const float* __restrict__ resid,
                                                          float* __restrict__ y) {
  extern __shared__ float xsw[];
  __shared__ float red[8];
  float* xs = xsw;
  // stage (up to 16384 floats, padded), optional RMSNorm
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    *reinterpret_cast<float4*>(xs + xpad(i)) = v;
  }
  if (nw) {
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n_in + eps);
    for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
      float4 v = *reinterpret_cast<float4*>(xs + xpad(i));
      const float4 wv = *reinterpret_cast<const float4*>(nw + i);
      v.x = v.x * scale * wv.x;
      v.y = v.y * scale * wv.y;
      v.z = v.z * scale * wv.z;
      v.w = v.w * scale * wv.w;
      *reinterpret_cast<float4*>(xs + xpad(i)) = v;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nslices = n_in >> 6;
  const uint64_t rb = (uint64_t)(n_in >> 8) * KNJ_Q4K_BLOCK;
  for (int row = blockIdx.x * (kBlock / 64) + wave; row < n_out; row += gridDim.x * (kBlock / 64)) {
    float acc = 0.0f;
    for (int s = lane; s < nslices; s += 64) {
      XSlice xv;
      xslice_load(xs, s, xv);
      const Q4Slice q = q4k_load(w + (uint64_t)row * rb + (uint64_t)(s >> 2) * KNJ_Q4K_BLOCK, s & 3);
      acc += q4k_dot(q, s & 3, xv);
    }
    acc = group_sum<64>(acc);
    if (lane == 0) y[row] = resid ? resid[row] + acc : acc;
  }
}

// Q6_K rows of n_in <= 2048 (at most 64 units of 32 weights): lane = unit, so
// every lane's x (32 values and 4 run sums) is the same for every row and
// stays in registers; RS rows per wave step, all their loads issued first;
// rows walked grid-stride (the argmax variant keeps the grid <= kMaxKeys).
template <int RS>
__global__ __launch_bounds__(kBlock) void k_gemv_q6k_u(const uint8_t* __restrict__ w, int n_in,
                                                       int n_out, const float* __restrict__ x,
                                                       const float* __restrict__ nw, float eps,
                                                       const float* __restrict__ resid,
                                                       float* __restrict__ y,
                                                       unsigned long long* argmax) {
  __shared__ float xs[xpad_size(2048)];
  __shared__ float xs8[256];
  __shared__ float red[8];
  stage_x(x, nw, eps, n_in, xs, red);
  for (int g = threadIdx.x; 8 * g < n_in; g += kBlock) {
    const float4 a = *reinterpret_cast<const float4*>(xs + xpad(8 * g));
    const float4 b = *reinterpret_cast<const float4*>(xs + xpad(8 * g) + 4);
    xs8[g] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = n_in / KNJ_QK, nunits = 8 * nb;
  const bool active = lane < nunits;
  const int u = active ? lane : 0;
  const int b = u >> 3, hf = (u >> 2) & 1, o = u & 3;
  float4 x8[4][2];
  float sx[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = 256 * b + 128 * hf + 32 * t + 8 * o;
    x8[t][0] = *reinterpret_cast<const float4*>(xs + xpad(i));
    x8[t][1] = *reinterpret_cast<const float4*>(xs + xpad(i) + 4);
    sx[t] = xs8[i >> 3];
  }
  const uint64_t rb = (uint64_t)nb * KNJ_Q6K_BLOCK;
  const uint8_t* wu = w + (uint64_t)b * KNJ_Q6K_BLOCK;
  unsigned long long best = 0;
  const int stride = gridDim.x * (kBlock / 64) * RS;
  for (int r0 = (blockIdx.x * (kBlock / 64) + wave) * RS; r0 < n_out; r0 += stride) {
    Q6Unit q[RS];
#pragma unroll
    for (int st = 0; st < RS; ++st) q[st] = q6_unit_load(wu + (uint64_t)min(r0 + st, n_out - 1) * rb, hf, o);
    float rv[RS];
#pragma unroll
    for (int st = 0; st < RS; ++st) rv[st] = resid ? resid[min(r0 + st, n_out - 1)] : 0.0f;
#pragma unroll
    for (int st = 0; st < RS; ++st) {
      const float acc = group_sum<64>(active ? q6_unit_dot(q[st], x8, sx) : 0.0f);
      const int row = r0 + st;
      if (lane == 0 && row < n_out) {
        const float v = resid ? rv[st] + acc : acc;
        y[row] = v;
        if (argmax) {
          const unsigned long long k = argmax_key(v, row);
          best = k > best ? k : best;
        }
      }
    }
  }
  if (argmax) block_argmax_store(best, argmax);
}

// Q6_K rows: 8 quarters per block, LPR lanes per row, activations in LDS.
template <int LPR>
__global__ __launch_bounds__(kBlock) void k_gemv_q6k(const uint8_t* __restrict__ w, int n_in,
                                                     int n_out, const float* __restrict__ x,
                                                     const float* __restrict__ nw, float eps,
                                                     const float* __restrict__ resid,
                                                     float* __restrict__ y,
                                                     unsigned long long* argmax) {
  extern __shared__ float xsq[];
  __shared__ float red[8];
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    *reinterpret_cast<float4*>(xsq + i) = v;
  }
  if (nw) {
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n_in + eps);
    for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
      float4 v = *reinterpret_cast<float4*>(xsq + i);
      const float4 wv = *reinterpret_cast<const float4*>(nw + i);
      v.x = v.x * scale * wv.x;
      v.y = v.y * scale * wv.y;
      v.z = v.z * scale * wv.z;
      v.w = v.w * scale * wv.w;
      *reinterpret_cast<float4*>(xsq + i) = v;
    }
  }
  __syncthreads();
  const int nb = n_in / KNJ_QK, nq = 8 * nb;
  const uint64_t rb = (uint64_t)nb * KNJ_Q6K_BLOCK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rsub = lane / LPR;
  constexpr int RPW = 64 / LPR;
  const int stride = gridDim.x * (kBlock / 64) * RPW;
  unsigned long long best = 0;
  for (int row0 = (blockIdx.x * (kBlock / 64) + wave) * RPW; row0 < n_out; row0 += stride) {
    const int row = row0 + rsub;
    float acc = 0.0f;
    if (row < n_out) {
      const uint8_t* rp = w + (uint64_t)row * rb;
      for (int s = sub; s < nq; s += LPR) {
        const int bb = s >> 3;
        acc += q6k_quarter(rp + (uint64_t)bb * KNJ_Q6K_BLOCK, (s >> 2) & 1, s & 3,
                           xsq + bb * KNJ_QK + 128 * ((s >> 2) & 1) + 32 * (s & 3));
      }
    }
    acc = group_sum<LPR>(acc);
    if (sub == 0 && row < n_out) {
      const float v = resid ? resid[row] + acc : acc;
      y[row] = v;
      if (argmax) {
        const unsigned long long k = argmax_key(v, row);
        best = k > best ? k : best;
      }
    }
  }
  if (argmax) block_argmax_store(best, argmax);
}

// BF16 rows (the LM head): 8 weights per lane per 16-byte load, NJ loads per
// row (n_in = 512*NJ); the lane's 8*NJ activations live in registers; RS rows
// per step with the next step's loads issued before the current rows are
// reduced.  Optional packed argmax of y.
template <int NJ, int RS>
__global__ __launch_bounds__(kBlock) void k_gemv_bf16(const uint8_t* __restrict__ w, int n_in,
                                                      int n_out, const float* __restrict__ x,
                                                      const float* __restrict__ nw, float eps,
                                                      const float* __restrict__ resid,
                                                      float* __restrict__ y,
                                                      unsigned long long* argmax) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = gridDim.x * (kBlock / 64);
  const int wave_g = blockIdx.x * (kBlock / 64) + wave;
  const uint64_t rb = (uint64_t)n_in * 2;
  uint4 cur[RS][NJ];
  int base = wave_g * RS;
#pragma unroll
  for (int r = 0; r < RS; ++r)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int row = min(base + r, n_out - 1);
      cur[r][j] = *reinterpret_cast<const uint4*>(w + (uint64_t)row * rb + 16 * (lane + 64 * j));
    }
  // the lane's 8*NJ activations straight into registers; the wave holds all of
  // x, so the RMSNorm sum is a wave reduction
  float xv[NJ][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = 8 * lane + 512 * j;
    const float4 a = *reinterpret_cast<const float4*>(x + i);
    const float4 c = *reinterpret_cast<const float4*>(x + i + 4);
    xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
    xv[j][4] = c.x; xv[j][5] = c.y; xv[j][6] = c.z; xv[j][7] = c.w;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += xv[j][k] * xv[j][k];
  }
  if (nw) {
    ss = group_sum<64>(ss);
    const float scale = 1.0f / sqrtf(ss / (float)n_in + eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = 8 * lane + 512 * j;
      const float4 a = *reinterpret_cast<const float4*>(nw + i);
      const float4 c = *reinterpret_cast<const float4*>(nw + i + 4);
      const float wv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) xv[j][k] = xv[j][k] * scale * wv[k];
    }
  }
  unsigned long long best = 0;
  for (; base < n_out; base += nwaves * RS) {
    const int nbase = base + nwaves * RS;
    uint4 nxt[RS][NJ];
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (nbase + r < n_out)
          nxt[r][j] = *reinterpret_cast<const uint4*>(w + (uint64_t)(nbase + r) * rb + 16 * (lane + 64 * j));
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint4 v = cur[r][j];
        acc += __uint_as_float(v.x << 16) * xv[j][0];
        acc += __uint_as_float(v.x & 0xFFFF0000u) * xv[j][1];
        acc += __uint_as_float(v.y << 16) * xv[j][2];
        acc += __uint_as_float(v.y & 0xFFFF0000u) * xv[j][3];
        acc += __uint_as_float(v.z << 16) * xv[j][4];
        acc += __uint_as_float(v.z & 0xFFFF0000u) * xv[j][5];
        acc += __uint_as_float(v.w << 16) * xv[j][6];
        acc += __uint_as_float(v.w & 0xFFFF0000u) * xv[j][7];
      }
      acc = group_sum<64>(acc);
      const int row = base + r;
      if (row < n_out) {
        const float o = resid ? resid[row] + acc : acc;
        if (lane == 0) y[row] = o;
        if (argmax) {
          const unsigned long long k = argmax_key(o, row);
          best = k > best ? k : best;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int j = 0; j < NJ; ++j) cur[r][j] = nxt[r][j];
  }
  if (argmax) block_argmax_store(best, argmax);
}

// BF16 / F32 rows of any width (multiple of 8 / 4): one wave per row.
template <bool BF16>
__global__ __launch_bounds__(kBlock) void k_gemv_plain(const uint8_t* __restrict__ w, int n_in,
                                                       int n_out, const float* __restrict__ x,
                                                       const float* __restrict__ nw, float eps,
                                                       const float* __restrict__ resid,
                                                       float* __restrict__ y,
                                                       unsigned long long* argmax) {
  extern __shared__ float xsp[];
  __shared__ float red[8];
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    *reinterpret_cast<float4*>(xsp + i) = v;
  }
  if (nw) {
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n_in + eps);
    for (int i = 4 * threadIdx.x; i < n_in; i += 4 * kBlock) {
      float4 v = *reinterpret_cast<float4*>(xsp + i);
      const float4 wv = *reinterpret_cast<const float4*>(nw + i);
      v.x = v.x * scale * wv.x;
      v.y = v.y * scale * wv.y;
      v.z = v.z * scale * wv.z;
      v.w = v.w * scale * wv.w;
      *reinterpret_cast<float4*>(xsp + i) = v;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int PER = BF16 ? 8 : 4;
  const uint64_t rb = (uint64_t)n_in * (BF16 ? 2 : 4);
  unsigned long long best = 0;
  for (int row = blockIdx.x * (kBlock / 64) + wave; row < n_out; row += gridDim.x * (kBlock / 64)) {
    const uint8_t* rp = w + (uint64_t)row * rb;
    float acc = 0.0f;
    for (int i0 = lane * PER; i0 < n_in; i0 += 64 * PER) {
      const uint4 v = *reinterpret_cast<const uint4*>(rp + (uint64_t)i0 * (BF16 ? 2 : 4));
      const float4 xa = *reinterpret_cast<const float4*>(xsp + i0);
      if (BF16) {
        const float4 xb = *reinterpret_cast<const float4*>(xsp + i0 + 4);
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
    acc = group_sum<64>(acc);
    const float out = resid ? resid[row] + acc : acc;
    if (lane == 0) y[row] = out;
    if (argmax) {
      const unsigned long long k = argmax_key(out, row);
      best = k > best ? k : best;
    }
  }
  if (argmax) block_argmax_store(best, argmax);
}

// The decode step's last launch closes the step: the per-workgroup argmax keys
// of the LM head (kMaxKeys slots, unused ones zero) are reduced to the next
// token (first maximum wins, /root/reference/src/cli/main.cpp:126-132) and the
// device-side position advances.
__global__ __launch_bounds__(kBlock) void k_step_close(StepState* st, const unsigned long long* keys,
                                                       int nkeys, int32_t* out_tokens, int max_steps) {
  unsigned long long best = 0;
#pragma unroll
  for (int j = 0; j < kMaxKeys / kBlock; ++j) {
    const int i = threadIdx.x + kBlock * j;
    const unsigned long long k = i < nkeys ? keys[i] : 0ull;
    best = k > best ? k : best;
  }
  __shared__ unsigned long long wb[4];
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < 4; ++w) best = wb[w] > best ? wb[w] : best;
  best = wb[0] > best ? wb[0] : best;
  const int tok = argmax_index(best);
  st->key = best;
  if (st->step < max_steps) out_tokens[st->step] = tok;
  st->step += 1;
  st->token = tok;
  st->pos += 1;
}

int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// The bf16 fast path is instantiated for 512, 1024, 2048 and 4096 inputs only;
// gemv_grid and launch_gemv both decide through this one predicate, so the
// number of argmax keys the step reads always matches the launch.
constexpr int kBf16Rows = 2;  // rows per wave step of the bf16 fast path

bool bf16_fast(int n_in) {
  if (n_in % 512 != 0) return false;
  const int nj = n_in / 512;
  return nj == 1 || nj == 2 || nj == 4 || nj == 8;
}

}  // namespace

// Grids of the argmax-capable GEMVs (Q6_K, BF16, F32); one key per workgroup.
int gemv_grid(int type, int n_in, int n_out) {
  if (type == KNJ_TYPE_Q6_K && n_in <= 2048) {
    constexpr int RS = 4;
    return std::max(1, std::min(2048, (n_out + 4 * RS - 1) / (4 * RS)));
  }
  if (type == KNJ_TYPE_Q6_K) {
    const int lpr = std::min(64, pow2_at_least(8 * (n_in / KNJ_QK)));
    const int rows_per_block = 4 * (64 / lpr);
    return std::max(1, std::min(kMaxKeys, (n_out + rows_per_block - 1) / rows_per_block));
  }
  if (type == KNJ_TYPE_BF16 && bf16_fast(n_in)) {
    // two rows per wave step, up to kMaxKeys workgroups: the 151,936-row
    // head measured 112.5 us at 512 workgroups of four rows per step, 103.5
    // at 4096 of two (a graph of back-to-back launches)
    const int waves_needed = (n_out + kBf16Rows - 1) / kBf16Rows;
    return std::max(1, std::min(kMaxKeys, (waves_needed + 3) / 4));
  }
  return std::max(1, std::min(kMaxKeys, (n_out + 3) / 4));
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t s) {
  if (a.type == KNJ_TYPE_Q4_K) {
    const int nslices = a.n_in / 64;
    if (nslices <= 64) {
      const int lpr = pow2_at_least(nslices);
      const int rpw = 64 / lpr;
      const int steps_total = (a.n_out + rpw - 1) / rpw;  // wave-steps
      const int rs = steps_total <= 4 * 1024 ? 1 : (steps_total <= 4 * 2048 ? 2 : 4);
      const int grid = (steps_total + 4 * rs - 1) / (4 * rs);
#define GQ(L, R)                                                                            \
  if (lpr == L && rs == R) {                                                                \
    KNJ_LAUNCH((k_gemv_q4k<L, R>), dim3(grid), dim3(kBlock), 0, s, a.w, a.n_in,    \
                       a.n_out, a.x, a.norm_w, a.eps, a.resid, a.y);                        \
    return hipGetLastError();                                                               \
  }
      GQ(4, 1) GQ(4, 2) GQ(4, 4) GQ(8, 1) GQ(8, 2) GQ(8, 4) GQ(16, 1) GQ(16, 2) GQ(16, 4)
      GQ(32, 1) GQ(32, 2) GQ(32, 4) GQ(64, 1) GQ(64, 2) GQ(64, 4)
#undef GQ
      return hipErrorInvalidValue;
    }
    const size_t lds = (size_t)xpad_size(a.n_in) * 4;
    const int grid = std::max(1, std::min(2048, (a.n_out + 3) / 4));
    KNJ_LAUNCH(k_gemv_q4k_wide, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out, a.x,
                       a.norm_w, a.eps, a.resid, a.y);
    return hipGetLastError();
  }
  if (a.type == KNJ_TYPE_Q6_K && a.n_in <= 2048) {
    KNJ_LAUNCH(k_gemv_q6k_u<4>, dim3(gemv_grid(a.type, a.n_in, a.n_out)), dim3(kBlock), 0, s,
                       a.w, a.n_in, a.n_out, a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);
    return hipGetLastError();
  }
  if (a.type == KNJ_TYPE_Q6_K) {
    const int lpr = std::min(64, pow2_at_least(8 * (a.n_in / KNJ_QK)));
    const size_t lds = (size_t)a.n_in * 4;
    const int grid = gemv_grid(a.type, a.n_in, a.n_out);
#define G6(L)                                                                                 \
  if (lpr == L) {                                                                             \
    KNJ_LAUNCH(k_gemv_q6k<L>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out, \
                       a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);                     \
    return hipGetLastError();                                                                 \
  }
    G6(8) G6(16) G6(32) G6(64)
#undef G6
    return hipErrorInvalidValue;
  }
  if (a.type == KNJ_TYPE_BF16 && bf16_fast(a.n_in)) {
    const int nj = a.n_in / 512;
    constexpr int RS = kBf16Rows;
    const int grid = gemv_grid(a.type, a.n_in, a.n_out);
#define GB(J)                                                                                   \
  if (nj == J) {                                                                                \
    KNJ_LAUNCH((k_gemv_bf16<J, RS>), dim3(grid), dim3(kBlock), 0, s, a.w, a.n_in,     \
                       a.n_out, a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);             \
    return hipGetLastError();                                                                   \
  }
    GB(1) GB(2) GB(4) GB(8)
#undef GB
  }
  const size_t lds = (size_t)a.n_in * 4;
  const int grid = gemv_grid(KNJ_TYPE_F32, a.n_in, a.n_out);
  if (a.type == KNJ_TYPE_BF16) {
    KNJ_LAUNCH(k_gemv_plain<true>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in, a.n_out,
                       a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);
  } else {
    KNJ_LAUNCH(k_gemv_plain<false>, dim3(grid), dim3(kBlock), lds, s, a.w, a.n_in,
                       a.n_out, a.x, a.norm_w, a.eps, a.resid, a.y, a.argmax_key);
  }
  return hipGetLastError();
}

hipError_t launch_step_close(StepState* st, const unsigned long long* keys, int nkeys,
                             int32_t* out_tokens, int max_steps, hipStream_t s) {
  KNJ_LAUNCH(k_step_close, dim3(1), dim3(kBlock), 0, s, st, keys, nkeys, out_tokens,
                     max_steps);
  return hipGetLastError();
}

bool router_fold_ok(int type_o, int n_in, int n_out, int n_router) {
  if (type_o != KNJ_TYPE_Q4_K || n_router <= 0) return false;
  if (n_in % 256 || n_out % 256 || n_in / 64 > 64) return false;  // one row step per wave below
  const int lpr = pow2_at_least(n_in / 64), rpw = 64 / lpr;
  const int steps_total = (n_out + rpw - 1) / rpw;
  return steps_total <= 4 * 1024 && (n_in + n_out) / 4 <= 256 * kRouterF4 && lpr >= 4;
}

hipError_t launch_gemv_router(const GemvArgs& a, const float* R, int n_router, float* u,
                              hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  if (!router_fold_ok(a.type, a.n_in, a.n_out, n_router) || a.norm_w || !a.resid || a.y == a.resid)
    return hipErrorInvalidValue;
  const int lpr = pow2_at_least(a.n_in / 64), rpw = 64 / lpr;
  const int nob = ((a.n_out + rpw - 1) / rpw + 3) / 4;
  const dim3 grid(nob + n_router);
#define GR(L)                                                                                  \
  if (lpr == L) {                                                                              \
    if (t0) /* a timing run: dispatch events of its own */                                     \
      hipExtLaunchKernelGGL(k_gemv_q4k_router<L>, grid, dim3(kBlock), 0u, s, t0, t1, 0u, a.w,  \
                            a.n_in, a.n_out, a.x, a.resid, a.y, R, n_router, nob, u);          \
    else                                                                                       \
      KNJ_LAUNCH(k_gemv_q4k_router<L>, grid, dim3(kBlock), 0, s, a.w, a.n_in, a.n_out, a.x,     \
                 a.resid, a.y, R, n_router, nob, u);                                           \
    return hipGetLastError();                                                                  \
  }
  GR(4) GR(8) GR(16) GR(32) GR(64)
#undef GR
  return hipErrorInvalidValue;
}

hipError_t launch_router_fold(const float* wr, const float* nw, const float* wd, int H, int QD,
                              int E, float* R, hipStream_t s) {
  const dim3 grid((std::max(H, QD) + kBlock - 1) / kBlock, (E + 7) / 8);
  hipLaunchKernelGGL(k_router_fold, grid, dim3(kBlock), 0, s, wr, nw, wd, H, QD, E, R);
  return hipGetLastError();
}

}  // namespace knj
