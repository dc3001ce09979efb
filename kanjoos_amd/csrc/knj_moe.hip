// kanjoos_amd/csrc/knj_moe.hip -- router and expert FFN kernels of the batch-1 MoE layer.
//
// Device side of Model::moe (/root/reference/src/model/model.cpp:399-510):
//   router     logits = W_r . RMSNorm(x), softmax over all experts, top-k by
//              probability with ties to the lower index, weights renormalised
//              over the kept k (model.cpp:420-460);
//   gate/up    g = W_gate[e] . hx, u = W_up[e] . hx, act = silu(g) * u
//              (model.cpp:477-493);
//   down       y_e = W_down[e] . act_e, out = resid + sum_e w_e * y_e with the
//              experts summed in ascending index (the scatter order of
//              model.cpp:464-508).
#include <hip/hip_ext.h>

#include "knj_common.h"
#include "knj_dev.h"

namespace knj {
namespace {

using namespace dev;

// Softmax over the n_expert logits and the top-k by rank: rank(e) = #{e' :
// p' > p or (p' == p and e' < e)}, which is exactly the reference's repeated
// strict-'>' argmax order (model.cpp:442-451); the kept weights are
// renormalised by their sum in selection order (model.cpp:452-458).  All 256
// threads of the workgroup take part; results land in LDS.
template <bool COHERENT>
__device__ __forceinline__ void router_topk(const float* __restrict__ logits, int n_expert, int k, int* sel_idx,
                            float* sel_w, float* probs, float* red) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float lg = t < n_expert ? (COHERENT ? ld_acquire_f(logits + t) : logits[t]) : -INFINITY;
  float mx = group_max<64>(lg);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  const float ex = t < n_expert ? expf(lg - mx) : 0.0f;
  const float sum = block_sum(ex, red);
  const float p = t < n_expert ? ex / sum : -1.0f;
  probs[t] = p;
  __syncthreads();
  // rank(e) = #{e' : key(e') > key(e)} with key = (probability bits << 8) |
  // (255 - e): probabilities are non-negative, so their bit patterns order like
  // the values, and the low byte breaks ties toward the lower index.  Two
  // threads per expert (n_expert <= 128) each count half of the candidates,
  // with every LDS read of a pass issued before its compares.
  __shared__ int rank_half[256];
  __shared__ unsigned long long keys[256];
  const int E2 = n_expert <= 128 ? 2 : 1;
  const int e = E2 == 2 ? (t & 127) : t;
  const int part = E2 == 2 ? (t >> 7) : 0;
  if (t < n_expert) keys[t] = ((unsigned long long)__float_as_uint(p) << 8) | (unsigned)(255 - t);
  __syncthreads();
  int rank = 0;
  if (e < n_expert) {
    const unsigned long long me = keys[e];
    const int per = (n_expert + E2 - 1) / E2;
    const int lo = part * per, hi = min(n_expert, lo + per);
    for (int base = lo; base < hi; base += 64) {
      unsigned long long kv[64];
#pragma unroll
      for (int j = 0; j < 64; ++j) kv[j] = keys[min(base + j, 255)];
#pragma unroll
      for (int j = 0; j < 64; ++j) rank += (base + j < hi && kv[j] > me) ? 1 : 0;
    }
  }
  rank_half[t] = rank;
  __syncthreads();
  if (t < n_expert) {
    const int r = E2 == 2 ? rank_half[t] + rank_half[t + 128] : rank_half[t];
    if (r < k) {
      sel_idx[r] = t;
      sel_w[r] = p;
    }
  }
  __syncthreads();
  if (t == 0) {
    float keep = 0.0f;
    for (int q = 0; q < k; ++q) keep += sel_w[q];
    const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
    for (int q = 0; q < k; ++q) sel_w[q] = sel_w[q] * inv;
  }
  __syncthreads();
}

// ------------------------------------------------------------------ router
// One wave per expert row (4 per workgroup).  Each wave normalises x itself
// (no workgroup barrier before the dot); workgroup 0 writes hx.  The logits
// are published (agent-scope stores) and, when a routing output is given, the
// last workgroup to finish computes softmax and top-k (router_topk).
__global__ __launch_bounds__(kBlock) void k_router(RouterArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * (blockDim.x / 64) + wave;
  const int H = a.n_embd;
  const int nj = H / 256;  // float4 per lane
  float4 wv[16];
  if (e < a.n_expert) {
    const float* wr = a.router_w + (uint64_t)e * H;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < nj) wv[j] = *reinterpret_cast<const float4*>(wr + 4 * lane + 256 * j);
  }
  float4 xv[16], nw[16];
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (j < nj) {
      xv[j] = *reinterpret_cast<const float4*>(a.x + 4 * lane + 256 * j);
      if (a.norm_w) nw[j] = *reinterpret_cast<const float4*>(a.norm_w + 4 * lane + 256 * j);
    }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (j < nj) ss += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
  if (a.norm_w) {
    ss = group_sum<64>(ss);
    const float scale = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < nj) {
        xv[j].x = xv[j].x * scale * nw[j].x;
        xv[j].y = xv[j].y * scale * nw[j].y;
        xv[j].z = xv[j].z * scale * nw[j].z;
        xv[j].w = xv[j].w * scale * nw[j].w;
      }
  }
  if (blockIdx.x == 0 && wave == 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < nj) *reinterpret_cast<float4*>(a.hx + 4 * lane + 256 * j) = xv[j];
  }
  if (e < a.n_expert) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < nj) {
        acc += wv[j].x * xv[j].x;
        acc += wv[j].y * xv[j].y;
        acc += wv[j].z * xv[j].z;
        acc += wv[j].w * xv[j].w;
      }
    acc = group_sum<64>(acc);
    if (lane == 0) publish(a.logits + e, acc);
  }
  if (!a.topk_idx) return;
  // the last workgroup to finish turns the logits into the routing
  __shared__ unsigned int flag;
  __shared__ __align__(16) float probs[256];
  __shared__ float red[8];
  __shared__ int sel_idx[16];
  __shared__ float sel_w[16];
  if (!last_block_done(a.counter, gridDim.x, &flag)) return;
  router_topk<true>(a.logits, a.n_expert, a.k, sel_idx, sel_w, probs, red);
  if (threadIdx.x < a.k) {
    a.topk_idx[threadIdx.x] = sel_idx[threadIdx.x];
    a.topk_w[threadIdx.x] = sel_w[threadIdx.x];
  }
}

// Logits only (the router of the decode step): workgroup = one expert row,
// wave q = quarter q of the row (n_embd <= 4096: at most four float4 per lane,
// elements 4 lane + 256 j of the quarter).  Each wave loads its quarter of the
// row, of x and of the norm weight; the quarters' sums of squares and then
// their dot products meet in LDS and are added in quarter order.  Against one
// wave per row (48 16-byte loads per lane issued one after another on a CU of
// its own): 3.7 -> 2.1 us per launch in a graph of back-to-back launches.
// Workgroup 0 also writes the normalised x (hx).
__global__ __launch_bounds__(kBlock) void k_router_q(RouterArgs a) {
  __shared__ float red[4], part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x, H = a.n_embd, Q = H >> 2;
  // float4 j of a lane: element 4 lane + 256 j of the quarter (Q is a multiple of 64)
  auto in_q = [&](int j) { return 4 * lane + 256 * j < Q; };
  const int base = Q * wave + 4 * lane;
  const float* wr = a.router_w + (uint64_t)e * H;
  float4 wv[4], xv[4], nv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (in_q(j)) wv[j] = *reinterpret_cast<const float4*>(wr + base + 256 * j);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (in_q(j)) {
      xv[j] = *reinterpret_cast<const float4*>(a.x + base + 256 * j);
      nv[j] = a.norm_w ? *reinterpret_cast<const float4*>(a.norm_w + base + 256 * j)
                       : make_float4(1.f, 1.f, 1.f, 1.f);
    }
  if (a.norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (in_q(j)) ss += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
    ss = group_sum<64>(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float sst = ((red[0] + red[1]) + red[2]) + red[3];
    const float scale = 1.0f / sqrtf(sst / (float)H + a.eps);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (in_q(j)) {
        xv[j].x = xv[j].x * scale * nv[j].x;
        xv[j].y = xv[j].y * scale * nv[j].y;
        xv[j].z = xv[j].z * scale * nv[j].z;
        xv[j].w = xv[j].w * scale * nv[j].w;
      }
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (in_q(j)) {
      acc += wv[j].x * xv[j].x;
      acc += wv[j].y * xv[j].y;
      acc += wv[j].z * xv[j].z;
      acc += wv[j].w * xv[j].w;
    }
  acc = group_sum<64>(acc);
  if (lane == 0) part[wave] = acc;
  if (e == 0 && a.hx) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (in_q(j)) *reinterpret_cast<float4*>(a.hx + base + 256 * j) = xv[j];
  }
  __syncthreads();
  if (threadIdx.x == 0) a.logits[e] = ((part[0] + part[1]) + part[2]) + part[3];
}

// Stand-alone top-k (the C-ABI router): one workgroup.
__global__ __launch_bounds__(kBlock) void k_topk(const float* __restrict__ logits, int n_expert,
                                                 int k, int32_t* topk_idx, float* topk_w) {
  __shared__ __align__(16) float probs[256];
  __shared__ float red[8];
  __shared__ int sel_idx[16];
  __shared__ float sel_w[16];
  router_topk<false>(logits, n_expert, k, sel_idx, sel_w, probs, red);
  if (threadIdx.x < k) {
    topk_idx[threadIdx.x] = sel_idx[threadIdx.x];
    topk_w[threadIdx.x] = sel_w[threadIdx.x];
  }
}

// ------------------------------------------------------------------ gate/up
// Wave = one (expert slot, row) pair: lanes [0,32) the gate row, [32,64) the
// up row, one 64-weight slice per lane (n_embd <= 2048).  RS pairs per wave,
// their weights requested as soon as the expert index is known.
template <int RS>
__global__ __launch_bounds__(kBlock) void k_expert_gateup(ExpertArgs a) {
  static_assert(RS == 1 || RS == 2 || RS == 4, "one, two or four row pairs per wave");
  __shared__ float xs[xpad_size(2048)];
  __shared__ float xsum[64];  // sums of the 32-element sub-blocks of the normalised x
  __shared__ int sel[16];
  __shared__ float selp[16];
  __shared__ unsigned long long ckey[256];  // candidate keys
  __shared__ uint32_t gmax[32];
  __shared__ uint32_t gthr;
  __shared__ int ncand;
  __shared__ float red[3][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  KNJ_STAMP(0);
  // 1) the whole workgroup routes and stages x before any weight is loaded.
  // Loads first: thread t holds the logit of expert t and float4s t, t + 256
  // of x and of its norm weight (n_embd <= 2048, n_expert <= 256).
  const bool route = a.logits != nullptr;
  const int H = a.n_embd, E = a.n_expert;
  float4 x4[2], w4[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i4 = t + kBlock * j;
    x4[j] = 4 * i4 < H ? *reinterpret_cast<const float4*>(a.hx + 4 * i4) : make_float4(0.f, 0.f, 0.f, 0.f);
    w4[j] = (a.norm_w && 4 * i4 < H) ? *reinterpret_cast<const float4*>(a.norm_w + 4 * i4)
                                      : make_float4(1.f, 1.f, 1.f, 1.f);
  }
  const float lg = (route && t < E) ? a.logits[t] : -INFINITY;
  if (t == 0) ncand = 0;
  const int given = (!route && t < a.k) ? a.topk_idx[t] : 0;
  // softmax max and the sum of squares of x: one reduction round
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) ss += x4[j].x * x4[j].x + x4[j].y * x4[j].y + x4[j].z * x4[j].z + x4[j].w * x4[j].w;
  ss = group_sum<64>(ss);
  const float wmax = group_max<64>(lg);
  if (lane == 0) {
    red[0][wave] = wmax;
    red[1][wave] = ss;
  }
  __syncthreads();
  const float mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float ex = (route && t < E) ? expf(lg - mx) : 0.0f;
  const float wsum = group_sum<64>(ex);
  if (lane == 0) red[2][wave] = wsum;
  // x normalised into LDS meanwhile, with the 32-element sub-block sums
  {
    const float sst = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
    const float scale = 1.0f / sqrtf(sst / (float)H + a.eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i4 = t + kBlock * j;
      float4 o = x4[j];
      if (a.norm_w) {
        o.x = x4[j].x * scale * w4[j].x;
        o.y = x4[j].y * scale * w4[j].y;
        o.z = x4[j].z * scale * w4[j].z;
        o.w = x4[j].w * scale * w4[j].w;
      }
      // eight consecutive threads hold one sub-block
      const float sb = group_sum<8>((o.x + o.y) + (o.z + o.w));
      if (4 * i4 < H) {
        *reinterpret_cast<float4*>(xs + xpad(4 * i4)) = o;
        if ((lane & 7) == 0) xsum[(4 * i4) >> 5] = sb;
      }
    }
  }
  __syncthreads();
  // Selection of the k largest probabilities, ties to the lower index
  // (strict > over ascending experts, model.cpp:442-451).  A key is the bits
  // of p (non-negative, so they order like the values) above the complement
  // of the index.  Candidates first: the maxima of the n_group groups of 8
  // experts are n_group distinct experts, so when n_group >= k the k-th
  // largest of them is at most the k-th largest probability, and every
  // selected expert is at or above it.  Only the candidates are ranked.
  const float sum = ((red[2][0] + red[2][1]) + red[2][2]) + red[2][3];
  const float p = (route && t < E) ? ex / sum : 0.0f;
  if (route) {
    const unsigned long long key =
        t < E ? ((unsigned long long)__float_as_uint(p) << 32) | (0xFFFFFFFFu - (unsigned)t) : 0ull;
    const uint32_t pb = t < E ? __float_as_uint(p) + 1u : 0u;  // 0: no expert
    uint32_t gm = max(pb, dpp_u32<kDppXor1>(pb));
    gm = max(gm, dpp_u32<kDppXor2>(gm));
    gm = max(gm, dpp_u32<kDppHalfMirror>(gm));
    const int n_group = (E + 7) >> 3;
    if ((t & 7) == 0 && (t >> 3) < n_group) gmax[t >> 3] = gm;
    __syncthreads();
    // the k-th largest group maximum (ties by group order), or 0 (everyone)
    if (t < n_group && n_group >= a.k) {
      const uint32_t mine = gmax[t];
      int r = 0;
      for (int g2 = 0; g2 < n_group; ++g2) {
        const uint32_t o = gmax[g2];
        r += (o > mine || (o == mine && g2 < t)) ? 1 : 0;
      }
      if (r == a.k - 1) gthr = mine;
    }
    __syncthreads();
    const uint32_t thr = n_group >= a.k ? gthr : 0u;
    if (t < E && pb >= thr) ckey[atomicAdd(&ncand, 1)] = key;
    __syncthreads();
    // each candidate counts the larger candidate keys (order of the list is
    // immaterial), sixteen loads in flight per pass
    const int n_cand = ncand;
    if (t < E && pb >= thr) {
      int rank = 0;
      for (int b0 = 0; b0 < n_cand; b0 += 16) {
        unsigned long long kv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) kv[j] = ckey[min(b0 + j, n_cand - 1)];
#pragma unroll
        for (int j = 0; j < 16; ++j) rank += (b0 + j < n_cand && kv[j] > key) ? 1 : 0;
      }
      if (rank < a.k) {
        sel[rank] = t;
        selp[rank] = p;
      }
    }
  } else if (t < a.k) {
    sel[t] = given;
  }
  __syncthreads();
  KNJ_STAMP(1);
  // 2) the expert rows: wave = RS (slot, row) pairs, lanes [0,32) the gate
  // row and [32,64) the up row, one 64-weight slice per lane
  const int half = lane >> 5, sub = lane & 31;
  const int nslices = a.n_embd >> 6;
  const bool active = sub < nslices;
  const uint64_t rb = (uint64_t)(a.n_embd >> 8) * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_ff;
  const int npairs = a.k * a.n_ff;
  const int pair0 = (blockIdx.x * (kBlock / 64) + wave) * RS;
  const int b = sub >> 2, g = sub & 3;
  const uint8_t* base = half ? a.up : a.gate;
  // named registers (an indexed array was placed in scratch memory here)
  Q4Slice q0, q1, q2, q3;
  auto load_pair = [&](int pr, Q4Slice& q) {
    const int prc = min(pr, npairs - 1);  // always a valid row; unused results are dropped
    const int kk = prc / a.n_ff, row = prc - kk * a.n_ff;
    const int e = sel[kk];
    q = q4k_load(base + (uint64_t)e * slab + (uint64_t)row * rb + (uint64_t)(active ? b : 0) * KNJ_Q4K_BLOCK, g);
  };
  load_pair(pair0, q0);
  if constexpr (RS >= 2) load_pair(pair0 + 1, q1);
  if constexpr (RS == 4) {
    load_pair(pair0 + 2, q2);
    load_pair(pair0 + 3, q3);
  }
  __builtin_amdgcn_sched_barrier(0);  // every weight load is issued before any wait
  XSlice xv;
  const int sl = active ? sub : 0;
  xslice_load_sums(xs, sl, xsum[2 * sl], xsum[2 * sl + 1], xv);
  KNJ_STAMP(2);
  // all dot products before any store: a store counts in the same in-order
  // completion counter as the loads, so a wait for a later load would also
  // wait for the store
  float res[RS];
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int pr = pair0 + st;
    const Q4Slice& q = st == 0 ? q0 : st == 1 ? q1 : st == 2 ? q2 : q3;
    float acc = (active && pr < npairs) ? q4k_dot(q, g, xv) : 0.0f;
    acc = group_sum<32>(acc);
    const float u = lane_bcast(acc, 32);
    res[st] = (acc / (1.0f + expf(-acc))) * u;
    if (st == 0) KNJ_STAMP(3);
  }
  if (lane == 0) {
#pragma unroll
    for (int st = 0; st < RS; ++st)
      if (pair0 + st < npairs) a.act[pair0 + st] = res[st];  // act is [k][n_ff]
  }
  // the routing, for the down launch and the caller (kept until now so no
  // wave waits on these stores before its loads)
  if (route && blockIdx.x == 0 && t < a.k) {
    // weights renormalised over the kept probabilities, summed in selection
    // order (model.cpp:452-458)
    float keep = 0.0f;
    for (int q = 0; q < a.k; ++q) keep += selp[q];
    const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
    a.topk_idx[t] = sel[t];
    a.topk_w[t] = selp[t] * inv;
  }
  KNJ_STAMP(4);
}

// ------------------------------------------------------------------ gate/up, one routing wave
// The routed gate/up for n_expert <= 128, n_embd <= 2048, as one workgroup of
// kGuWaves waves per CU.  Wave 0 routes alone while waves 1-4 load x and form
// its sum of squares; after one barrier every wave issues its weight loads,
// and waves 1-4 normalise x into LDS while the weights are in flight.
//
// Routing (the same selection as k_expert_gateup, bit for bit): lane l holds
// experts l and l + 64.  The softmax max is a wave maximum; the denominator is
// the sum of the two 64-expert halves, each a wave tree, added in order (the
// workgroup sum of k_expert_gateup).  Candidates: the maxima of the 16 groups
// of 8 consecutive experts are 16 distinct experts, so the k-th largest of
// them bounds the k-th largest probability from below and every selected
// expert is at or above it.  Lane 8g + j compares groups g and 8 + g with
// groups j and 8 + j (one LDS permute each) and the group's 8 lanes add the
// counts.  Each candidate then counts the larger candidate keys (probability,
// then the lower index; model.cpp:442-451) by a scalar walk over the ~10
// candidates.  A single wave keeps the routing off the other waves' SIMD time;
// every wave routing for itself measured slower (8.3 vs 8.0 us), this form
// ~7.0 us against 8.0 for the workgroup-cooperative routing.
constexpr int kGuWaves = 12;

__global__ __launch_bounds__(64 * kGuWaves) void k_expert_gateup_r(ExpertArgs a) {
  constexpr int RS = 2;
  __shared__ float xs[xpad_size(2048)];
  __shared__ float xsum[64];
  __shared__ float red[4];
  __shared__ int sel[16];
  __shared__ float selp[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int H = a.n_embd, E = a.n_expert;
  const int tx = t - 64;  // waves 1-4 stage x as the 256 threads of k_expert_gateup
  const bool xw = wave >= 1 && wave <= 4;
  float4 x4[2], w4[2];
  // wave 0's logits and selection, kept for the softmax weights of
  // unscaled logits (workgroup 0, after the first barrier)
  float lg0 = -INFINITY, lg1 = -INFINITY;
  int r0 = 0, r1 = 0;
  bool c0 = false, c1 = false;
  if (wave == 0) {
    lg0 = lane < E ? a.logits[lane] : -INFINITY;
    lg1 = lane + 64 < E ? a.logits[lane + 64] : -INFINITY;
    uint32_t pb0, pb1;  // selection keys, 0: no expert
    float p0 = 0.0f, p1 = 0.0f;
    if (a.logits_unscaled) {
      // the softmax of s * logit with s > 0 ranks as the logits do: select on
      // order-preserving keys of the logits themselves (-0 taken as +0)
      auto okey = [](float v) {
        const uint32_t b = __float_as_uint(v + 0.0f);
        return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
      };
      pb0 = lane < E ? okey(lg0) + 1u : 0u;
      pb1 = lane + 64 < E ? okey(lg1) + 1u : 0u;
    } else {
      const float mx = group_max<64>(fmaxf(lg0, lg1));
      const float ex0 = lane < E ? expf(lg0 - mx) : 0.0f;
      const float ex1 = lane + 64 < E ? expf(lg1 - mx) : 0.0f;
      const float sum = group_sum<64>(ex0) + group_sum<64>(ex1);
      p0 = ex0 / sum;
      p1 = ex1 / sum;
      pb0 = lane < E ? __float_as_uint(p0) + 1u : 0u;
      pb1 = lane + 64 < E ? __float_as_uint(p1) + 1u : 0u;
    }
    auto gmax8 = [](uint32_t v) {
      v = max(v, dpp_u32<kDppXor1>(v));
      v = max(v, dpp_u32<kDppXor2>(v));
      return max(v, dpp_u32<kDppHalfMirror>(v));
    };
    const uint32_t gm0 = gmax8(pb0), gm1 = gmax8(pb1);  // groups g, 8 + g in lanes 8g..8g+7
    const int n_group = (E + 7) >> 3;
    const int g = lane >> 3, j = lane & 7;
    const uint32_t mj0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (8 * j), (int)gm0);
    const uint32_t mj1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (8 * j), (int)gm1);
    auto beats = [&](uint32_t o, int go, uint32_t me, int gme) {
      return (go < n_group && (o > me || (o == me && go < gme))) ? 1 : 0;
    };
    int ra = beats(mj0, j, gm0, g) + beats(mj1, 8 + j, gm0, g);
    int rb = beats(mj0, j, gm1, 8 + g) + beats(mj1, 8 + j, gm1, 8 + g);
    ra += __builtin_amdgcn_update_dpp(ra, ra, kDppXor1, 0xF, 0xF, false);
    rb += __builtin_amdgcn_update_dpp(rb, rb, kDppXor1, 0xF, 0xF, false);
    ra += __builtin_amdgcn_update_dpp(ra, ra, kDppXor2, 0xF, 0xF, false);
    rb += __builtin_amdgcn_update_dpp(rb, rb, kDppXor2, 0xF, 0xF, false);
    ra += __builtin_amdgcn_update_dpp(ra, ra, kDppHalfMirror, 0xF, 0xF, false);
    rb += __builtin_amdgcn_update_dpp(rb, rb, kDppHalfMirror, 0xF, 0xF, false);
    const unsigned long long ta = __ballot(g < n_group && ra == a.k - 1);
    const unsigned long long tb = __ballot(8 + g < n_group && rb == a.k - 1);
    uint32_t thr = 0u;  // fewer groups than k: every expert is a candidate
    if (n_group >= a.k)
      thr = ta ? (uint32_t)__builtin_amdgcn_readlane((int)gm0, (int)__builtin_ctzll(ta))
               : (uint32_t)__builtin_amdgcn_readlane((int)gm1, (int)__builtin_ctzll(tb));
    c0 = lane < E && pb0 >= thr;
    c1 = lane + 64 < E && pb1 >= thr;
    unsigned long long m0 = __ballot(c0), m1 = __ballot(c1);
    while (m0 | m1) {
      const bool hi = m0 == 0;
      const int l = (int)__builtin_ctzll(hi ? m1 : m0);
      const uint32_t pc = (uint32_t)__builtin_amdgcn_readlane((int)(hi ? pb1 : pb0), l);
      const int ec = l + (hi ? 64 : 0);
      r0 += (pc > pb0 || (pc == pb0 && ec < lane)) ? 1 : 0;
      r1 += (pc > pb1 || (pc == pb1 && ec < lane + 64)) ? 1 : 0;
      if (hi) m1 &= m1 - 1;
      else m0 &= m0 - 1;
    }
    if (c0 && r0 < a.k) {
      sel[r0] = lane;
      selp[r0] = p0;
    }
    if (c1 && r1 < a.k) {
      sel[r1] = lane + 64;
      selp[r1] = p1;
    }
  } else if (xw) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int i4 = tx + kBlock * jj;
      x4[jj] = 4 * i4 < H ? *reinterpret_cast<const float4*>(a.hx + 4 * i4) : make_float4(0.f, 0.f, 0.f, 0.f);
      w4[jj] = (a.norm_w && 4 * i4 < H) ? *reinterpret_cast<const float4*>(a.norm_w + 4 * i4)
                                         : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      ss += x4[jj].x * x4[jj].x + x4[jj].y * x4[jj].y + x4[jj].z * x4[jj].z + x4[jj].w * x4[jj].w;
    ss = group_sum<64>(ss);
    if (lane == 0) red[wave - 1] = ss;
  }
  __syncthreads();
  // the weights of this wave's RS (slot, row) pairs: lanes [0,32) the gate
  // row, [32,64) the up row, one 64-weight slice per lane
  const int half = lane >> 5, sub = lane & 31;
  const int nslices = H >> 6;
  const bool active = sub < nslices;
  const uint64_t rb = (uint64_t)(H >> 8) * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_ff;
  const int npairs = a.k * a.n_ff;
  const int pair0 = (blockIdx.x * kGuWaves + wave) * RS;
  const int b = sub >> 2, g = sub & 3;
  const uint8_t* base = half ? a.up : a.gate;
  Q4Slice q0, q1;
  auto load_pair = [&](int pr, Q4Slice& q) {
    const int prc = min(pr, npairs - 1);  // always a valid row; unused results are dropped
    const int kk = prc / a.n_ff, row = prc - kk * a.n_ff;
    q = q4k_load(base + (uint64_t)sel[kk] * slab + (uint64_t)row * rb + (uint64_t)(active ? b : 0) * KNJ_Q4K_BLOCK, g);
  };
  load_pair(pair0, q0);
  load_pair(pair0 + 1, q1);
  __builtin_amdgcn_sched_barrier(0);
  if (a.logits_unscaled && blockIdx.x == 0 && wave == 0) {
    // the routing weights (written by workgroup 0 only): softmax of the
    // logits times the RMSNorm scale of hx (model.cpp:240-271, 438-441), the
    // scale from waves 1-4's sum of squares of the same hx
    const float sst = ((red[0] + red[1]) + red[2]) + red[3];
    const float scale = 1.0f / sqrtf(sst / (float)H + a.eps);
    const float l0 = lg0 * scale, l1 = lg1 * scale;
    const float mx = group_max<64>(fmaxf(l0, l1));
    const float ex0 = lane < E ? expf(l0 - mx) : 0.0f;
    const float ex1 = lane + 64 < E ? expf(l1 - mx) : 0.0f;
    const float sum = group_sum<64>(ex0) + group_sum<64>(ex1);
    if (c0 && r0 < a.k) selp[r0] = ex0 / sum;
    if (c1 && r1 < a.k) selp[r1] = ex1 / sum;
  }
  // x normalised into LDS with its 32-element sub-block sums (as k_expert_gateup)
  if (xw) {
    const float sst = ((red[0] + red[1]) + red[2]) + red[3];
    const float scale = 1.0f / sqrtf(sst / (float)H + a.eps);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int i4 = tx + kBlock * jj;
      float4 o = x4[jj];
      if (a.norm_w) {
        o.x = x4[jj].x * scale * w4[jj].x;
        o.y = x4[jj].y * scale * w4[jj].y;
        o.z = x4[jj].z * scale * w4[jj].z;
        o.w = x4[jj].w * scale * w4[jj].w;
      }
      const float sb = group_sum<8>((o.x + o.y) + (o.z + o.w));
      if (4 * i4 < H) {
        *reinterpret_cast<float4*>(xs + xpad(4 * i4)) = o;
        if ((lane & 7) == 0) xsum[(4 * i4) >> 5] = sb;
      }
    }
  }
  // barrier on the LDS writes only: the weight loads stay in flight
  __builtin_amdgcn_s_waitcnt(kWaitLdsOnly);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  XSlice xv;
  const int sl = active ? sub : 0;
  xslice_load_sums(xs, sl, xsum[2 * sl], xsum[2 * sl + 1], xv);
  float res[RS];
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int pr = pair0 + st;
    float acc = (active && pr < npairs) ? q4k_dot(st == 0 ? q0 : q1, g, xv) : 0.0f;
    acc = group_sum<32>(acc);
    const float u = lane_bcast(acc, 32);
    res[st] = (acc / (1.0f + expf(-acc))) * u;
  }
  if (lane == 0) {
#pragma unroll
    for (int st = 0; st < RS; ++st)
      if (pair0 + st < npairs) a.act[pair0 + st] = res[st];  // act is [k][n_ff]
  }
  if (blockIdx.x == 0 && t < a.k) {
    // weights renormalised over the kept probabilities, summed in selection
    // order (model.cpp:452-458)
    float keep = 0.0f;
    for (int q = 0; q < a.k; ++q) keep += selp[q];
    const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
    a.topk_idx[t] = sel[t];
    a.topk_w[t] = selp[t] * inv;
  }
}

// Reference-shaped fallback for n_embd > 2048: 32 lanes per row, loop.
__global__ __launch_bounds__(kBlock) void k_expert_gateup_wide(ExpertArgs a) {
  extern __shared__ float xw[];
  __shared__ float red[8];
  int my_idx;
  if (a.logits) {
    float my_w;
    wave_route(a.logits, a.n_expert, a.k, my_idx, my_w);
    if (blockIdx.x == 0 && threadIdx.x < a.k) {
      a.topk_idx[threadIdx.x] = my_idx;
      a.topk_w[threadIdx.x] = my_w;
    }
  } else {
    my_idx = (threadIdx.x & 63) < a.k ? a.topk_idx[threadIdx.x & 63] : 0;
  }
  const int H = a.n_embd;
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < H; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(a.hx + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    *reinterpret_cast<float4*>(xw + xpad(i)) = v;
  }
  if (a.norm_w) {
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)H + a.eps);
    for (int i = 4 * threadIdx.x; i < H; i += 4 * kBlock) {
      float4 v = *reinterpret_cast<float4*>(xw + xpad(i));
      const float4 w = *reinterpret_cast<const float4*>(a.norm_w + i);
      v.x = v.x * scale * w.x;
      v.y = v.y * scale * w.y;
      v.z = v.z * scale * w.z;
      v.w = v.w * scale * w.w;
      *reinterpret_cast<float4*>(xw + xpad(i)) = v;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, sub = lane & 31;
  const int nslices = H >> 6;
  const uint64_t rb = (uint64_t)(H >> 8) * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_ff;
  const int npairs = a.k * a.n_ff;
  for (int pr = blockIdx.x * (kBlock / 64) + wave; pr < npairs; pr += gridDim.x * (kBlock / 64)) {
    const int kk = pr / a.n_ff, row = pr - kk * a.n_ff;
    const int e = lane_bcast(my_idx, kk);
    const uint8_t* rp = (half ? a.up : a.gate) + (uint64_t)e * slab + (uint64_t)row * rb;
    float acc = 0.0f;
    for (int s = sub; s < nslices; s += 32) {
      XSlice xv;
      xslice_load(xw, s, xv);
      acc += q4k_dot(q4k_load(rp + (uint64_t)(s >> 2) * KNJ_Q4K_BLOCK, s & 3), s & 3, xv);
    }
    acc = group_sum<32>(acc);
    const float u = lane_bcast(acc, 32);
    if (lane == 0) a.act[pr] = (acc / (1.0f + expf(-acc))) * u;
  }
}

// Ordered weighted sum of the k expert outputs of one row (ascending expert
// index) plus the residual.  dots[kk] and the expert ids are per slot.
__device__ __forceinline__ float combine_sorted(const float* dots, const int32_t* idx,
                                                const float* wts, int k) {
  float o = 0.0f;
  int prev = -1;
  for (int r = 0; r < k; ++r) {
    int pick = -1, best = 0x7FFFFFFF;
    for (int kk = 0; kk < k; ++kk) {
      const int ek = idx[kk];
      if (ek > prev && ek < best) {
        best = ek;
        pick = kk;
      }
    }
    prev = best;
    o = __fadd_rn(o, __fmul_rn(wts[pick], dots[pick]));
  }
  return o;
}

// ------------------------------------------------------------------ down (Q4_K)
// Wave = one output row for all k experts: 16-lane group gi takes expert slots
// gi, gi+4, ...; one 64-weight slice per lane (n_ff <= 1024).  The k activation
// vectors are staged in LDS once per workgroup.  Slot order is then folded
// into ascending expert order by lane 0.
template <int KPG>
__global__ __launch_bounds__(kBlock) void k_expert_down(ExpertArgs a) {
  extern __shared__ float acts[];  // [k][xpad_size(n_ff)], then [k * n_ff / 32] sub-block sums
  constexpr int KMAX = 4 * KPG;    // k <= KMAX
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gi = lane >> 4, sub = lane & 15;
  const int F = a.n_ff, K = a.k, n = K * F;
  const int fpad = xpad_size(F);
  float* sums = acts + K * fpad;
  const int nslices = F >> 6;
  const bool active = sub < nslices;
  const uint64_t rb = (uint64_t)(F >> 8) * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_embd;
  KNJ_STAMP(8);
  KNJ_WG_STAMP(0);
  const int row = min((int)(blockIdx.x * (kBlock / 64) + wave), a.n_embd - 1);
  const bool row_ok = (int)(blockIdx.x * (kBlock / 64) + wave) < a.n_embd;
  const int b = active ? (sub >> 2) : 0, g = sub & 3;
  // 1) the routing (the same for every row), the first 8192 activations and
  // this row's residual; the expert weights follow, so staging the
  // activations waits only for the activations
  int ids[KMAX];
  float wts[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) {
    ids[kk] = kk < K ? a.topk_idx[kk] : 0x7FFFFFFF;
    wts[kk] = kk < K ? a.topk_w[kk] : 0.0f;
  }
  const float resid = a.resid ? a.resid[row] : 0.0f;
  // (named registers: an indexed array was placed in scratch memory)
  float4 v0, v1, v2, v3, v4, v5, v6, v7;
  auto ld = [&](int base, float4& v0, float4& v1, float4& v2, float4& v3, float4& v4, float4& v5,
                float4& v6, float4& v7) {
    auto one = [&](int j, float4& v) {
      const int i = base + 4 * kBlock * j;
      v = *reinterpret_cast<const float4*>(a.act + (i < n ? i : 0));
    };
    one(0, v0); one(1, v1); one(2, v2); one(3, v3);
    one(4, v4); one(5, v5); one(6, v6); one(7, v7);
  };
  ld(4 * threadIdx.x, v0, v1, v2, v3, v4, v5, v6, v7);
  Q4Slice q[KPG];
#pragma unroll
  for (int j = 0; j < KPG; ++j) {
    const int kk = min(gi + 4 * j, K - 1);
    int e = ids[0];
#pragma unroll
    for (int t = 1; t < KMAX; ++t) e = kk == t ? ids[t] : e;
    q[j] = q4k_load(a.down + (uint64_t)e * slab + (uint64_t)row * rb + (uint64_t)b * KNJ_Q4K_BLOCK, g);
  }
  __builtin_amdgcn_sched_barrier(0);  // every weight load is issued before any wait
  // 2) activations to LDS, with the sum of every 32-element sub-block (eight
  // consecutive threads hold one sub-block)
  auto put = [&](int base, const float4& v0, const float4& v1, const float4& v2, const float4& v3,
                 const float4& v4, const float4& v5, const float4& v6, const float4& v7) {
    auto one = [&](int j, const float4& v) {
      const int i = base + 4 * kBlock * j;
      if (i < n) {  // uniform over each group of eight lanes (n is a multiple of 32)
        const int kk = i / F, c = i - kk * F;
        *reinterpret_cast<float4*>(acts + kk * fpad + xpad(c)) = v;
        const float t = group_sum<8>((v.x + v.y) + (v.z + v.w));
        if ((threadIdx.x & 7) == 0) sums[i >> 5] = t;
      }
    };
    one(0, v0); one(1, v1); one(2, v2); one(3, v3);
    one(4, v4); one(5, v5); one(6, v6); one(7, v7);
  };
  put(4 * threadIdx.x, v0, v1, v2, v3, v4, v5, v6, v7);
  for (int base = 4 * threadIdx.x + 32 * kBlock; base < n; base += 32 * kBlock) {
    ld(base, v0, v1, v2, v3, v4, v5, v6, v7);
    put(base, v0, v1, v2, v3, v4, v5, v6, v7);
  }
  // slot order by ascending expert index (ids are distinct): rank[kk] =
  // #{t : ids[t] < ids[kk]}
  int rank[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) {
    int r = 0;
#pragma unroll
    for (int t = 0; t < KMAX; ++t) r += ids[t] < ids[kk] ? 1 : 0;
    rank[kk] = r;
  }
  __syncthreads();
  KNJ_STAMP(9);
  float dot[KPG];
#pragma unroll
  for (int j = 0; j < KPG; ++j) {
    const int kk = min(gi + 4 * j, K - 1);
    const int sl = active ? sub : 0;
    XSlice xv;
    xslice_load_sums(acts + kk * fpad, sl, sums[(kk * F >> 5) + 2 * sl], sums[(kk * F >> 5) + 2 * sl + 1], xv);
    const float acc = (active && gi + 4 * j < K) ? q4k_dot(q[j], g, xv) : 0.0f;
    dot[j] = group_sum<16>(acc);
  }
  KNJ_STAMP(10);
  // every lane folds the k products in ascending expert order:
  // o = ((w_a d_a + w_b d_b) + ...) with d of slot kk in lane 16 (kk % 4)
  float dk[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) dk[kk] = lane_bcast(dot[kk / 4], 16 * (kk % 4));
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    float wr = 0.0f, dr = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KMAX; ++kk) {
      const bool hit = rank[kk] == r;
      wr = hit ? wts[kk] : wr;
      dr = hit ? dk[kk] : dr;
    }
    if (r < K) o = __fadd_rn(o, __fmul_rn(wr, dr));
  }
  KNJ_STAMP(11);
  if (row_ok && lane == 0) {
    const float v = a.resid ? __fadd_rn(resid, o) : o;
    a.out[row] = v;
    if (a.hidden_copy) a.hidden_copy[row] = v;
  }
  KNJ_STAMP(12);
  KNJ_WG_STAMP(1);
}

// Rank of slot kk's expert in ascending expert index among the k <= KMAX
// slots (unused slots hold 0x7FFFFFFF and rank last; ids are distinct).
template <int KMAX>
__device__ __forceinline__ int expert_rank(const int (&ids)[KMAX], int kk) {
  int me = ids[0];
#pragma unroll
  for (int q = 1; q < KMAX; ++q) me = kk == q ? ids[q] : me;
  int rk = 0;
#pragma unroll
  for (int q = 0; q < KMAX; ++q) rk += ids[q] < me ? 1 : 0;
  return rk;
}

// ------------------------------------------------------------------ down (Q4_K, k <= 8)
// Workgroup = 8 waves x 8 output rows; wave w takes expert slot w for all 8
// rows (16-lane row groups, one 64-weight slice per lane, two rows per lane
// so each staged activation slice serves two rows).  The loads are ordered so
// no wait covers more than it needs: first the routing (the expert rows'
// addresses wait on it alone), then the k activation vectors and the
// residuals, then this wave's expert rows; the activations are staged in LDS
// while the weights are in flight.  Each wave files its products under its
// expert's rank in ascending index, and one thread per row adds them in that
// order (a search of the slot order per row cost ~2 us of the launch).
constexpr int kDownRows = 8;

__global__ __launch_bounds__(512) void k_expert_down8(ExpertArgs a) {
  constexpr int KMAX = 8;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int rg = lane >> 4, sub = lane & 15;
  const int F = a.n_ff, K = a.k, n = K * F;
  const int nslices = F >> 6;
  const bool active = sub < nslices && wave < K;
  const uint64_t rb = (uint64_t)(F >> 8) * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_embd;
  const int r0 = blockIdx.x * kDownRows;
  const int kk = min(wave, K - 1);
  __shared__ float acts[KMAX * xpad_size(1024)];
  __shared__ float sums[KMAX * 32];
  __shared__ float dots[KMAX][kDownRows];
  __shared__ float wsr[KMAX];
  const int fpad = xpad_size(F);
  // 1) the routing first (the weight addresses wait on it alone), then the
  // activations (k * n_ff <= 8192 floats: four float4 per thread) and residuals
  int ids[KMAX];
  float wts[KMAX];
#pragma unroll
  for (int q = 0; q < KMAX; ++q) {
    ids[q] = q < K ? a.topk_idx[q] : 0x7FFFFFFF;
    wts[q] = q < K ? a.topk_w[q] : 0.0f;
  }
  float4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * (t + 512 * j);
    v[j] = *reinterpret_cast<const float4*>(a.act + (i < n ? i : 0));
  }
  const bool own_row = t < kDownRows && r0 + t < a.n_embd;
  const float resid = (own_row && a.resid) ? a.resid[r0 + t] : 0.0f;
  // 2) this wave's expert rows (valid rows only; rows past n_embd read row n_embd - 1)
  int e = ids[0];
#pragma unroll
  for (int q = 1; q < KMAX; ++q) e = kk == q ? ids[q] : e;
  const int sl = active ? sub : 0;
  const int b = sl >> 2, g = sl & 3;
  const int ra = min(r0 + rg, a.n_embd - 1), rb2 = min(r0 + rg + 4, a.n_embd - 1);
  const uint8_t* ex = a.down + (uint64_t)e * slab + (uint64_t)b * KNJ_Q4K_BLOCK;
  const Q4Slice q0 = q4k_load(ex + (uint64_t)ra * rb, g);
  const Q4Slice q1 = q4k_load(ex + (uint64_t)rb2 * rb, g);
  __builtin_amdgcn_sched_barrier(0);
  // 3) stage the activations with their 32-element sums (eight threads per sub-block)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * (t + 512 * j);
    const float sb = group_sum<8>((v[j].x + v[j].y) + (v[j].z + v[j].w));
    if (i < n) {
      const int k2 = i / F, c = i - k2 * F;
      *reinterpret_cast<float4*>(acts + k2 * fpad + xpad(c)) = v[j];
      if ((t & 7) == 0) sums[i >> 5] = sb;
    }
  }
  __syncthreads();
  // 4) the two rows of this lane's group
  XSlice xv;
  const int sb0 = kk * (F >> 5) + 2 * sl;
  xslice_load_sums(acts + kk * fpad, sl, sums[sb0], sums[sb0 + 1], xv);
  const float d0 = group_sum<16>(active ? q4k_dot(q0, g, xv) : 0.0f);
  const float d1 = group_sum<16>(active ? q4k_dot(q1, g, xv) : 0.0f);
  // 5) each wave files its products and weight under its expert's rank in
  // ascending index (rank = #{slots with a lower expert}; ids are distinct),
  // so one thread per row folds them in that order with no search
  const int rk = expert_rank<KMAX>(ids, kk);
  if (sub == 0 && wave < K) {
    dots[rk][rg] = d0;
    dots[rk][rg + 4] = d1;
  }
  if (lane == 0 && wave < K) wsr[rk] = wts[kk];
  __syncthreads();
  if (!own_row) return;
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < KMAX; ++r)
    if (r < K) o = __fadd_rn(o, __fmul_rn(wsr[r], dots[r][t]));
  const int row = r0 + t;
  const float out = a.resid ? __fadd_rn(resid, o) : o;
  a.out[row] = out;
  if (a.hidden_copy) a.hidden_copy[row] = out;
}

// ------------------------------------------------------------------ down (Q6_K, k <= 8)
// As k_expert_down8 for Q6_K experts: wave w takes expert slot w for the
// workgroup's 8 rows; lane = one 32-weight unit of a row (32-lane halves take
// rows 2i and 2i + 1, four rounds), read with q6_unit_load as in the one-row
// kernel; activations and their 8-element sums staged once per workgroup.
// STAGED: the 8 rows of a wave's expert are one contiguous, 16-byte aligned
// run (8 x 630 bytes at n_ff = 768), fetched with 16-byte loads into LDS and
// decoded from there, instead of three unaligned 8-byte runs, four scale
// bytes and d per 32-weight unit straight from memory.
constexpr int kQ6StageLoads = 7;  // 16-byte loads per lane: 8 rows of n_ff <= 1024

// q6_unit_load from a Q6_K block at byte `blk` of an LDS region (2-byte
// aligned blocks): the 8-byte runs as three aligned words and a funnel shift
__device__ __forceinline__ void lds_ld8(const uint32_t* w4, uint32_t off, uint32_t& x, uint32_t& y) {
  const uint32_t* w = w4 + (off >> 2);
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
  const uint32_t sh = (off & 3) * 8;
  x = sh ? __builtin_amdgcn_alignbit(w1, w0, sh) : w0;
  y = sh ? __builtin_amdgcn_alignbit(w2, w1, sh) : w1;
}
__device__ __forceinline__ Q6Unit q6_unit_load_lds(const uint8_t* region, uint32_t blk, int hf, int o) {
  const uint32_t* w4 = reinterpret_cast<const uint32_t*>(region);
  Q6Unit u;
  lds_ld8(w4, blk + KNJ_Q6K_QL + 64 * hf + 8 * o, u.l0a, u.l0b);
  lds_ld8(w4, blk + KNJ_Q6K_QL + 64 * hf + 32 + 8 * o, u.l1a, u.l1b);
  lds_ld8(w4, blk + KNJ_Q6K_QH + 32 * hf + 8 * o, u.ha, u.hb);
  const int8_t* sp = reinterpret_cast<const int8_t*>(region + blk + KNJ_Q6K_SC + 8 * hf + (o >> 1));
#pragma unroll
  for (int t = 0; t < 4; ++t) u.sc[t] = sp[2 * t];
  u.d = *reinterpret_cast<const uint16_t*>(region + blk + KNJ_Q6K_D);
  return u;
}
template <bool STAGED>
__global__ __launch_bounds__(512) void k_expert_down8_q6(ExpertArgs a) {
  constexpr int KMAX = 8;
  extern __shared__ uint4 wstage[];  // STAGED: [wave][8 rows x rb / 16]
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int F = a.n_ff, K = a.k, n = K * F;
  const int nunits = F / 32;
  const int half = lane >> 5, u = lane & 31;
  const bool active = u < nunits && wave < K;
  const int uu = u < nunits ? u : 0;
  const int b = uu >> 3, hf = (uu >> 2) & 1, o = uu & 3;
  const uint64_t rb = (uint64_t)(F / KNJ_QK) * KNJ_Q6K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_embd;
  const int r0 = blockIdx.x * kDownRows;
  const int kk = min(wave, K - 1);
  __shared__ float acts[KMAX * 1024];
  __shared__ float s8[KMAX * 1024 / 8];
  __shared__ float dots[KMAX][kDownRows];
  __shared__ float wsr[KMAX];
  // the routing first, then the activations (named registers: an array here
  // was placed in scratch memory)
  int ids[KMAX];
  float wts[KMAX];
#pragma unroll
  for (int q = 0; q < KMAX; ++q) {
    ids[q] = q < K ? a.topk_idx[q] : 0x7FFFFFFF;
    wts[q] = q < K ? a.topk_w[q] : 0.0f;
  }
  auto act4 = [&](int j) {
    const int i = 4 * (t + 512 * j);
    return *reinterpret_cast<const float4*>(a.act + (i < n ? i : 0));
  };
  const float4 v0 = act4(0), v1 = act4(1), v2 = act4(2), v3 = act4(3);
  const bool own_row = t < kDownRows && r0 + t < a.n_embd;
  const float resid = (own_row && a.resid) ? a.resid[r0 + t] : 0.0f;
  int e = ids[0];
#pragma unroll
  for (int q = 1; q < KMAX; ++q) e = kk == q ? ids[q] : e;
  const uint8_t* ex = a.down + (uint64_t)e * slab + (uint64_t)b * KNJ_Q6K_BLOCK;
  Q6Unit qu[kDownRows / 2];
  const int nch = (int)(kDownRows * rb / 16);  // 16-byte chunks of the 8 rows
  uint4 w0, w1, w2, w3, w4, w5, w6;  // (named registers, as above)
  if constexpr (STAGED) {
    const uint4* src = reinterpret_cast<const uint4*>(a.down + (uint64_t)e * slab + (uint64_t)r0 * rb);
    auto ldc = [&](int j) { return src[min(lane + 64 * j, nch - 1)]; };
    w0 = ldc(0); w1 = ldc(1); w2 = ldc(2); w3 = ldc(3); w4 = ldc(4); w5 = ldc(5); w6 = ldc(6);
  } else {
#pragma unroll
    for (int it = 0; it < kDownRows / 2; ++it) {
      const int row = min(r0 + 2 * it + half, a.n_embd - 1);
      qu[it] = q6_unit_load(ex + (uint64_t)row * rb, hf, o);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  auto stage4 = [&](int j, const float4& v) {
    const int i = 4 * (t + 512 * j);
    if (i < n) *reinterpret_cast<float4*>(acts + i) = v;
  };
  stage4(0, v0);
  stage4(1, v1);
  stage4(2, v2);
  stage4(3, v3);
  __syncthreads();
  for (int g = t; 8 * g < n; g += 512) {
    const float4 x0 = *reinterpret_cast<const float4*>(acts + 8 * g);
    const float4 x1 = *reinterpret_cast<const float4*>(acts + 8 * g + 4);
    s8[g] = ((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w));
  }
  __syncthreads();
  if constexpr (STAGED) {
    // this wave's rows into its own LDS range and back: one wave's LDS
    // accesses complete in order, so no barrier
    uint4* mine = wstage + wave * nch;
    auto stc = [&](int j, const uint4& v) {
      if (lane + 64 * j < nch) mine[lane + 64 * j] = v;
    };
    stc(0, w0); stc(1, w1); stc(2, w2); stc(3, w3); stc(4, w4); stc(5, w5); stc(6, w6);
    asm volatile("" ::: "memory");
    const uint8_t* wl = reinterpret_cast<const uint8_t*>(mine);
#pragma unroll
    for (int it = 0; it < kDownRows / 2; ++it)
      qu[it] = q6_unit_load_lds(wl, (uint32_t)((2 * it + half) * rb + b * KNJ_Q6K_BLOCK), hf, o);
  }
  float4 x8[4][2];
  float sx[4];
#pragma unroll
  for (int tq = 0; tq < 4; ++tq) {
    const int i = kk * F + 256 * b + 128 * hf + 32 * tq + 8 * o;
    x8[tq][0] = *reinterpret_cast<const float4*>(acts + i);
    x8[tq][1] = *reinterpret_cast<const float4*>(acts + i + 4);
    sx[tq] = s8[i >> 3];
  }
  // products and weight filed under the expert's rank in ascending index,
  // folded in that order by one thread per row (as k_expert_down8)
  const int rk = expert_rank<KMAX>(ids, kk);
#pragma unroll
  for (int it = 0; it < kDownRows / 2; ++it) {
    const float acc = group_sum<32>(active ? q6_unit_dot(qu[it], x8, sx) : 0.0f);
    if (u == 0 && wave < K) dots[rk][2 * it + half] = acc;
  }
  if (lane == 0 && wave < K) wsr[rk] = wts[kk];
  __syncthreads();
  if (!own_row) return;
  float o_ = 0.0f;
#pragma unroll
  for (int r = 0; r < KMAX; ++r)
    if (r < K) o_ = __fadd_rn(o_, __fmul_rn(wsr[r], dots[r][t]));
  const int row = r0 + t;
  const float out = a.resid ? __fadd_rn(resid, o_) : o_;
  a.out[row] = out;
  if (a.hidden_copy) a.hidden_copy[row] = out;
}

// ------------------------------------------------------------------ down (Q6_K, n_ff <= 1024)
// Wave = one output row for all k experts: 32-lane group gi takes expert slots
// gi, gi+2, ..; lane = one 32-weight Q6_K unit of the row (n_ff / 32 <= 32
// units).  The k activation vectors and their 8-run sums are staged in LDS once
// per workgroup; slots are folded in ascending expert order as in the Q4_K
// kernel.
template <int KPG>
__global__ __launch_bounds__(kBlock) void k_expert_down_q6u(ExpertArgs a) {
  extern __shared__ float acts[];  // [k][n_ff], then [k * n_ff / 8] run sums
  constexpr int KMAX = 2 * KPG;    // k <= KMAX
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gi = lane >> 5, u = lane & 31;
  const int F = a.n_ff, K = a.k, n = K * F;
  float* s8 = acts + n;
  const int nunits = F / 32;
  const bool active = u < nunits;
  const int uu = active ? u : 0;
  const int b = uu >> 3, hf = (uu >> 2) & 1, o = uu & 3;
  const uint64_t rb = (uint64_t)(F / KNJ_QK) * KNJ_Q6K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_embd;
  const int row = min((int)(blockIdx.x * (kBlock / 64) + wave), a.n_embd - 1);
  const bool row_ok = (int)(blockIdx.x * (kBlock / 64) + wave) < a.n_embd;
  int ids[KMAX];
  float wts[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) {
    ids[kk] = kk < K ? a.topk_idx[kk] : 0x7FFFFFFF;
    wts[kk] = kk < K ? a.topk_w[kk] : 0.0f;
  }
  const float resid = a.resid ? a.resid[row] : 0.0f;
  // activations first (their staging waits only for them), 8 loads in flight
  // per thread per round; then the weights
  for (int base = 4 * threadIdx.x; base < n; base += 32 * kBlock) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = base + 4 * kBlock * j;
      v[j] = *reinterpret_cast<const float4*>(a.act + (i < n ? i : 0));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = base + 4 * kBlock * j;
      if (i < n) *reinterpret_cast<float4*>(acts + i) = v[j];
    }
  }
  Q6Unit q[KPG];
#pragma unroll
  for (int j = 0; j < KPG; ++j) {
    const int kk = min(gi + 2 * j, K - 1);
    int e = ids[0];
#pragma unroll
    for (int t = 1; t < KMAX; ++t) e = kk == t ? ids[t] : e;
    q[j] = q6_unit_load(a.down + (uint64_t)e * slab + (uint64_t)row * rb + (uint64_t)b * KNJ_Q6K_BLOCK,
                        hf, o);
  }
  __syncthreads();
  for (int g = threadIdx.x; 8 * g < n; g += kBlock) {
    const float4 x0 = *reinterpret_cast<const float4*>(acts + 8 * g);
    const float4 x1 = *reinterpret_cast<const float4*>(acts + 8 * g + 4);
    s8[g] = ((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w));
  }
  int rank[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) {
    int r = 0;
#pragma unroll
    for (int t = 0; t < KMAX; ++t) r += ids[t] < ids[kk] ? 1 : 0;
    rank[kk] = r;
  }
  __syncthreads();
  float dot[KPG];
#pragma unroll
  for (int j = 0; j < KPG; ++j) {
    const int kk = min(gi + 2 * j, K - 1);
    float4 x8[4][2];
    float sx[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = kk * F + 256 * b + 128 * hf + 32 * t + 8 * o;
      x8[t][0] = *reinterpret_cast<const float4*>(acts + i);
      x8[t][1] = *reinterpret_cast<const float4*>(acts + i + 4);
      sx[t] = s8[i >> 3];
    }
    const float acc = (active && gi + 2 * j < K) ? q6_unit_dot(q[j], x8, sx) : 0.0f;
    dot[j] = group_sum<32>(acc);
  }
  // every lane folds the k products in ascending expert order (slot kk's
  // product is in lane 32 (kk % 2), register kk / 2)
  float dk[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) dk[kk] = lane_bcast(dot[kk / 2], 32 * (kk % 2));
  float o_ = 0.0f;
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    float wr = 0.0f, dr = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KMAX; ++kk) {
      const bool hit = rank[kk] == r;
      wr = hit ? wts[kk] : wr;
      dr = hit ? dk[kk] : dr;
    }
    if (r < K) o_ = __fadd_rn(o_, __fmul_rn(wr, dr));
  }
  if (!row_ok || lane != 0) return;
  const float v = a.resid ? __fadd_rn(resid, o_) : o_;
  a.out[row] = v;
  if (a.hidden_copy) a.hidden_copy[row] = v;
}

// ------------------------------------------------------------------ down (Q6_K)
// Tasks (expert slot, row), LPR lanes each over the 8 quarters per block.
template <int LPR>
__global__ __launch_bounds__(kBlock) void k_expert_down_q6k(ExpertArgs a, int rows_per_block) {
  extern __shared__ float smem[];
  const int F = a.n_ff, K = a.k;
  float* acts = smem;                  // [K][F]
  float* dots = acts + K * F;          // [K][rows_per_block]
  for (int i = threadIdx.x; i < K * F; i += blockDim.x) acts[i] = a.act[i];
  __syncthreads();
  const int row_base = blockIdx.x * rows_per_block;
  const int nb = F / KNJ_QK;
  const int nq = 8 * nb;
  const uint64_t rbytes = (uint64_t)nb * KNJ_Q6K_BLOCK;
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
      for (int s = sub; s < nq; s += LPR) {
        const int bb = s >> 3, hf = (s >> 2) & 1, tq = s & 3;
        acc += q6k_quarter(rp + (uint64_t)bb * KNJ_Q6K_BLOCK, hf, tq, xk + bb * KNJ_QK + 128 * hf + 32 * tq);
      }
    }
    acc = group_sum<LPR>(acc);
    if (sub == 0 && t < ntasks) dots[kk * rows_per_block + r] = acc;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < rows_per_block; r += blockDim.x) {
    const int row = row_base + r;
    if (row >= a.n_embd) break;
    float d[16], w[16];
    int32_t ids[16];
    for (int kk = 0; kk < K; ++kk) {
      d[kk] = dots[kk * rows_per_block + r];
      ids[kk] = a.topk_idx[kk];
      w[kk] = a.topk_w[kk];
    }
    const float o = combine_sorted(d, ids, w, K);
    const float v = a.resid ? __fadd_rn(a.resid[row], o) : o;
    a.out[row] = v;
    if (a.hidden_copy) a.hidden_copy[row] = v;
  }
}

int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// hipLaunchKernelGGL, or the timed launch when start/stop events are given or
// a span sink is installed (knj_spans.h)
template <class F>
void launch_maybe_timed(F kernel, const char* name, dim3 grid, size_t lds, hipStream_t s,
                        hipEvent_t t0, hipEvent_t t1, const ExpertArgs& a, int block = kBlock) {
  if (t0 || span_take(name, &t0, &t1))
    hipExtLaunchKernelGGL(kernel, grid, dim3(block), (uint32_t)lds, s, t0, t1, 0u, a);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(block), lds, s, a);
}

}  // namespace


hipError_t launch_router(const RouterArgs& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  if (a.topk_idx) {
    // four rows (waves) per workgroup; the last workgroup also ranks the experts
    if (t0)  // a timing run: dispatch events of its own
      hipExtLaunchKernelGGL(k_router, dim3((a.n_expert + 3) / 4), dim3(kBlock), 0u, s, t0, t1, 0u, a);
    else
      KNJ_LAUNCH(k_router, dim3((a.n_expert + 3) / 4), dim3(kBlock), 0, s, a);
  } else if (t0) {
    hipExtLaunchKernelGGL(k_router_q, dim3(a.n_expert), dim3(kBlock), 0u, s, t0, t1, 0u, a);
  } else {
    // logits only: one row per workgroup, a quarter of it per wave
    KNJ_LAUNCH(k_router_q, dim3(a.n_expert), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int n_expert, int k, int32_t* idx, float* w,
                       hipStream_t s) {
  KNJ_LAUNCH(k_topk, dim3(1), dim3(kBlock), 0, s, logits, n_expert, k, idx, w);
  return hipGetLastError();
}

hipError_t launch_expert_gateup(const ExpertArgs& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  const int npairs = a.k * a.n_ff;
  // unscaled logits: only the one-routing-wave kernel applies the scale
  if (a.logits_unscaled && !(a.logits && a.n_embd <= 2048 && a.n_expert <= 128 && a.k <= 16))
    return hipErrorInvalidValue;
  if (a.logits && a.n_embd <= 2048 && a.n_expert <= 128 && a.k <= 16) {
    const int grid = (npairs + 2 * kGuWaves - 1) / (2 * kGuWaves);
    launch_maybe_timed(k_expert_gateup_r, "k_expert_gateup", dim3(grid), 0, s, t0, t1, a, 64 * kGuWaves);
    return hipGetLastError();
  }
  if (a.n_embd <= 2048) {
    constexpr int RS = 2;
    const int grid = (npairs + 4 * RS - 1) / (4 * RS);
    launch_maybe_timed(k_expert_gateup<RS>, "k_expert_gateup", dim3(grid), 0, s, t0, t1, a);
    return hipGetLastError();
  }
  const size_t lds = (size_t)xpad_size(a.n_embd) * 4;
  const int grid = std::min(2048, (npairs + 3) / 4);
  launch_maybe_timed(k_expert_gateup_wide, "k_expert_gateup_wide", dim3(grid), lds, s, t0, t1, a);
  return hipGetLastError();
}

hipError_t launch_expert_down(const ExpertArgs& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  if (a.type_down == KNJ_TYPE_Q4_K && a.n_ff <= 1024 && a.k <= 8) {
    const int grid = (a.n_embd + kDownRows - 1) / kDownRows;
    if (t0 || span_take("k_expert_down8", &t0, &t1))
      hipExtLaunchKernelGGL(k_expert_down8, dim3(grid), dim3(512), 0u, s, t0, t1, 0u, a);
    else
      hipLaunchKernelGGL(k_expert_down8, dim3(grid), dim3(512), 0, s, a);
    return hipGetLastError();
  }
  if (a.type_down == KNJ_TYPE_Q4_K && a.n_ff <= 1024) {
    const int kpg = (a.k + 3) / 4;
    const int grid = (a.n_embd + 3) / 4;
    const size_t lds = ((size_t)a.k * xpad_size(a.n_ff) + (size_t)a.k * a.n_ff / 32) * 4;
#define GD(J)                                                                                \
  if (kpg == J) {                                                                            \
    if (lds > 65536)                                                                         \
      (void)hipFuncSetAttribute((const void*)k_expert_down<J>,                               \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);       \
    launch_maybe_timed(k_expert_down<J>, "k_expert_down", dim3(grid), lds, s, t0, t1, a);                     \
    return hipGetLastError();                                                                \
  }
    GD(1) GD(2) GD(3) GD(4)
#undef GD
    return hipErrorInvalidValue;
  }
  if (a.type_down != KNJ_TYPE_Q6_K) return hipErrorInvalidValue;
  if (a.n_ff <= 1024 && a.k <= 8) {
    const int grid = (a.n_embd + kDownRows - 1) / kDownRows;
    const uint64_t rb = (uint64_t)(a.n_ff / KNJ_QK) * KNJ_Q6K_BLOCK;
    const bool staged = a.n_embd % kDownRows == 0 && (kDownRows * rb) % 16 == 0 &&
                        (rb * a.n_embd) % 16 == 0 && (reinterpret_cast<uintptr_t>(a.down) & 15) == 0;
    if (staged) {
      const unsigned lds = (unsigned)(8 * kDownRows * rb);  // 8 waves x 8 rows
      if (t0 || span_take("k_expert_down8_q6", &t0, &t1))
        hipExtLaunchKernelGGL(k_expert_down8_q6<true>, dim3(grid), dim3(512), lds, s, t0, t1, 0u, a);
      else
        hipLaunchKernelGGL(k_expert_down8_q6<true>, dim3(grid), dim3(512), lds, s, a);
    } else if (t0 || span_take("k_expert_down8_q6", &t0, &t1)) {
      hipExtLaunchKernelGGL(k_expert_down8_q6<false>, dim3(grid), dim3(512), 0u, s, t0, t1, 0u, a);
    } else {
      hipLaunchKernelGGL(k_expert_down8_q6<false>, dim3(grid), dim3(512), 0, s, a);
    }
    return hipGetLastError();
  }
  if (a.n_ff <= 1024 && a.k <= 16) {
    const int kpg = (a.k + 1) / 2;
    const int grid = (a.n_embd + 3) / 4;
    const size_t lds = ((size_t)a.k * a.n_ff + (size_t)a.k * a.n_ff / 8) * 4;
#define GU(J)                                                                                 \
  if (kpg <= J) {                                                                             \
    if (lds > 65536)                                                                          \
      (void)hipFuncSetAttribute((const void*)k_expert_down_q6u<J>,                            \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);        \
    launch_maybe_timed(k_expert_down_q6u<J>, "k_expert_down_q6u", dim3(grid), lds, s, t0, t1, a);                  \
    return hipGetLastError();                                                                 \
  }
    GU(2) GU(4) GU(8)
#undef GU
  }
  const int lpr = std::min(64, pow2_at_least(8 * (a.n_ff / KNJ_QK)));
  const int rows_per_block = 8;
  const size_t lds = ((size_t)a.k * a.n_ff + (size_t)a.k * rows_per_block) * 4;
  const int grid = (a.n_embd + rows_per_block - 1) / rows_per_block;
#define GQ(L)                                                                                   \
  if (lpr == L) {                                                                               \
    if (t0 || span_take("k_expert_down_q6k", &t0, &t1))                                         \
      hipExtLaunchKernelGGL(k_expert_down_q6k<L>, dim3(grid), dim3(kBlock), (uint32_t)lds, s, t0, \
                            t1, 0u, a, rows_per_block);                                         \
    else                                                                                        \
      hipLaunchKernelGGL(k_expert_down_q6k<L>, dim3(grid), dim3(kBlock), lds, s, a, rows_per_block); \
    return hipGetLastError();                                                                   \
  }
  GQ(8) GQ(16) GQ(32) GQ(64)
#undef GQ
  return hipErrorInvalidValue;
}

// Kernel attributes the batch-1 expert launches rely on, set once per device
// when it is opened (knj_device_open), so no launch path (possibly under graph
// capture) sets them lazily: the staged Q6_K down's dynamic LDS (8 waves x 8
// rows of up to n_ff = 1024) exceeds the 64 KiB default.
hipError_t expert_kernel_attributes() {
  return hipFuncSetAttribute((const void*)k_expert_down8_q6<true>,
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)(8 * kDownRows * 4 * KNJ_Q6K_BLOCK));
}

hipError_t launch_experts(const ExpertArgs& a, hipStream_t s) {
  const hipError_t e = launch_expert_gateup(a, s);
  if (e != hipSuccess) return e;
  return launch_expert_down(a, s);
}

}  // namespace knj
