// kanjoos_amd/csrc/knj_moe_batch.hip -- the MoE layer over many tokens at once
// (prefill chunks, batched decode).
//
// Device side of Model::moe with m > 1 (/root/reference/src/model/model.cpp:399-510):
// router logits for every token, softmax + top-k per token, the (token, expert)
// pairs bucketed by expert so each expert's weights are read once for all of
// its tokens (model.cpp:456-457, 462-477), gate/up + SwiGLU, down, and the
// weighted sum of each token's k expert outputs in ascending expert order plus
// the residual.
//
// The expert GEMMs run on the matrix cores with f32-equivalent operands.  A
// Q4_K weight is d*sc*q - dmin*m; per 32-weight sub-block
//   sum_i w_i x_i = d * sum_i (sc*q_i) x_i - dmin * m * sum_i x_i.
// sc*q_i (<= 63*15) is an exact f16 integer; x is split into an f16 high part
// and an f16 remainder, so every product is exact in the f32 accumulator and x
// keeps ~22 significant bits.  The min term is one more matrix-core step over
// the per-sub-block sums of x (also split hi/lo) against the 6-bit mins.  d and
// dmin scale the two accumulators once per 256-weight super-block.
#include "knj_common.h"
#include "knj_dev.h"

namespace knj {
namespace {

using namespace dev;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTok = 32;      // pairs (A rows) per work item
constexpr int kRowsWG = 128;  // weight rows per workgroup (32 per wave)

// Order of the 8 weights a lane unpacks from 8 code bytes (low halves of bytes
// 0, 2, then 1, 3, ...): position j holds weight perm8(j).  The A operand (x)
// is stored in the same order.
__host__ __device__ constexpr int perm8(int j) { return (j & 4) | ((j & 1) << 1) | ((j & 2) >> 1); }

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// 8 weights sc*q from two code words (bytes c0..c7), nibble `shift` (0 low, 4
// high), in perm8 order.  (0x6400 | q) is the f16 1024 + q; fma with sc and
// -1024*sc leaves q*sc exactly.
__device__ __forceinline__ half8 q4_unpack(uint32_t w0, uint32_t w1, int shift, half2v sc2,
                                           half2v nc2) {
  auto cv = [&](uint32_t w) {
    return __builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | 0x64006400u), sc2, nc2);
  };
  const half2v a = cv(w0 >> shift), b = cv(w0 >> (shift + 8));
  const half2v c = cv(w1 >> shift), d = cv(w1 >> (shift + 8));
  return half8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// (w & m) | c in one instruction (with the masks in registers; the
// compiler splits it when they are literals)
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(m), "v"(c));
  return r;
}
__device__ __forceinline__ half2v cvt_h2(float v) {
  const _Float16 h = (_Float16)v;
  return half2v{h, h};
}
constexpr uint32_t kNib = 0x000F000Fu;      // low nibbles of bytes 0 and 2
constexpr uint32_t kF16Base = 0x64006400u;  // f16 1024 in both halves

// The 16 weights of 8 code bytes (words wa, wb): low nibbles sc_lo q and high
// nibbles sc_hi q, each in perm8 order.  Low: (1024 + q) sc - 1024 sc; high,
// unshifted: (1024 + 16 q) sc / 16 - 64 sc (every value exact in f16); the
// byte shift is shared by both halves.  s_lo/n_lo = sc_lo, -1024 sc_lo;
// s_hi/n_hi = sc_hi / 16, -64 sc_hi.
__device__ __forceinline__ void q4_unpack2(uint32_t wa, uint32_t wb, half2v s_lo, half2v n_lo,
                                           half2v s_hi, half2v n_hi, half8& lo, half8& hi) {
  const uint32_t mlo = kNib, mhi = kNib << 4, sa = wa >> 8, sb = wb >> 8;
  auto cv = [&](uint32_t w, uint32_t m, half2v sc, half2v nc) {
    return __builtin_elementwise_fma(as_h2(and_or(w, m, kF16Base)), sc, nc);
  };
  const half2v l0 = cv(wa, mlo, s_lo, n_lo), l1 = cv(sa, mlo, s_lo, n_lo);
  const half2v l2 = cv(wb, mlo, s_lo, n_lo), l3 = cv(sb, mlo, s_lo, n_lo);
  const half2v h0 = cv(wa, mhi, s_hi, n_hi), h1 = cv(sa, mhi, s_hi, n_hi);
  const half2v h2 = cv(wb, mhi, s_hi, n_hi), h3 = cv(sb, mhi, s_hi, n_hi);
  lo = half8{l0.x, l0.y, l1.x, l1.y, l2.x, l2.y, l3.x, l3.y};
  hi = half8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

__device__ __forceinline__ half8 ld_h8(const _Float16* p) {
  return __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ f32x16 mfma32(half8 a, half8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ operand prep
// Row r of src (n floats): RMS-normalised with w (model.cpp:240-271) into dst.
__global__ __launch_bounds__(kBlock) void k_norm_rows(const float* __restrict__ src,
                                                      const float* __restrict__ nw, float eps,
                                                      int n, float* __restrict__ dst) {
  __shared__ float xs[4096];
  __shared__ float red[8];
  const float* s = src + (uint64_t)blockIdx.x * n;
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < n; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(s + i);
    *reinterpret_cast<float4*>(xs + i) = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  float* d = dst + (uint64_t)blockIdx.x * n;
  for (int i = 4 * threadIdx.x; i < n; i += 4 * kBlock) {
    const float4 v = *reinterpret_cast<const float4*>(xs + i);
    const float4 w = *reinterpret_cast<const float4*>(nw + i);
    *reinterpret_cast<float4*>(d + i) =
        make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
  }
}

// The A operand of the grouped GEMM: for each pair p, row row_of[p] of src
// (row p when row_of is null), n floats, as f16 high parts and remainders in
// perm8 order and as per-32 sums split the same way.  Layouts interleave the
// pairs so that a wave's 32 pairs read one contiguous run:
// hi/lo[(q * P + p) * 8 + j] for 8-group q; sums[((b / 8) * P + p) * 8 + b % 8]
// for 32-sub-block b.  Workgroup = a tile of 32 pairs x 64 elements
// (blockIdx.x, blockIdx.y; 64-element tiles give the launch four times the
// workgroups of 256-element ones, which left it short of work): each pair's
// row segment is read whole (8 consecutive threads, 256 bytes), the
// 8-element groups pass through LDS, and each output row [group][pairs] is
// written as 32 consecutive 16-byte records.  n % 64 == 0.
__global__ __launch_bounds__(kBlock) void k_split_tile(const float* __restrict__ src,
                                                       const int* __restrict__ row_of, int n,
                                                       int P, _Float16* __restrict__ hi,
                                                       _Float16* __restrict__ lo,
                                                       _Float16* __restrict__ shi,
                                                       _Float16* __restrict__ slo) {
  __shared__ uint4 th[8][33], tl[8][33];  // [group][pair] (+1 against bank conflicts)
  __shared__ __align__(16) _Float16 sh_h[32][2], sh_l[32][2];  // [pair][sub-block]
  const int t = threadIdx.x, p0 = blockIdx.x * 32, c0 = blockIdx.y * 64;
  {
    const int pr = t >> 3, g = t & 7;  // 8 consecutive threads: one pair
    const int p = min(p0 + pr, P - 1);
    const float* s = src + (uint64_t)(row_of ? row_of[p] : p) * n + c0 + 8 * g;
    const float4 a = *reinterpret_cast<const float4*>(s);
    const float4 b = *reinterpret_cast<const float4*>(s + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    half8 h, l;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = v[perm8(j)];
      h[j] = (_Float16)x;
      l[j] = (_Float16)(x - (float)h[j]);
      sum += v[j];
    }
    th[g][pr] = __builtin_bit_cast(uint4, h);
    tl[g][pr] = __builtin_bit_cast(uint4, l);
    sum = group_sum<4>(sum);  // sub-block g / 4: four consecutive threads
    if ((t & 3) == 0) {
      const _Float16 sv = (_Float16)sum;
      sh_h[pr][g >> 2] = sv;
      sh_l[pr][g >> 2] = (_Float16)(sum - (float)sv);
    }
  }
  __syncthreads();
  {
    const int g = t >> 5, pr = t & 31;  // 32 consecutive threads: one group
    if (p0 + pr < P) {
      const uint64_t o = ((uint64_t)(c0 / 8 + g) * P + p0 + pr) * 8;
      *reinterpret_cast<uint4*>(hi + o) = th[g][pr];
      *reinterpret_cast<uint4*>(lo + o) = tl[g][pr];
    }
  }
  if (t < 64) {
    const int pr = t & 31;
    if (p0 + pr < P) {
      // the tile's two sub-blocks b, b + 1 (b even: one 4-byte pair of the record)
      const int b = c0 / 32;
      const uint64_t so = ((uint64_t)(b / 8) * P + p0 + pr) * 8 + (b % 8);
      *reinterpret_cast<uint32_t*>((t < 32 ? shi : slo) + so) =
          *reinterpret_cast<const uint32_t*>(t < 32 ? sh_h[pr] : sh_l[pr]);
    }
  }
}

// ------------------------------------------------------------------ router
// logits[t][e] = sum_i hx[t][i] W[e][i] on the f32 matrix cores.  The
// reduction is cut into 16 slices of n_embd / 16 (n_embd % 256 == 0); tile
// (16 tokens x 16 experts) x slice-group z (blockIdx.z, kz groups of 16 / kz
// consecutive slices): one wave per slice, the group's waves added in slice
// order into out[z][t][e].  With kz = 1 out is the logits; with kz > 1 the
// routing below adds the kz groups in order, so the sum is the same
// sequence of additions either way.  Lane (r, kq) takes the float4 at
// 16 s + 4 kq of its slice, so a row's four lanes read 64 contiguous bytes,
// eight float4 of each operand in flight per round, and four accumulation
// chains (one per float4 component) are added at the end.
constexpr int kRouterSlices = 16;
__global__ __launch_bounds__(64 * kRouterSlices) void k_router_batch(const float* __restrict__ hx,
                                                                     const float* __restrict__ w,
                                                                     int m, int n, int n_expert,
                                                                     float* __restrict__ out) {
  __shared__ float part[kRouterSlices][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  const int tok = min(t0 + r, m - 1), ex = min(e0 + r, n_expert - 1);
  const int q = n / kRouterSlices, slice = blockIdx.z * W + wave;
  const float* ap = hx + (uint64_t)tok * n + slice * q + 4 * kq;
  const float* bp = w + (uint64_t)ex * n + slice * q + 4 * kq;
  f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0, c2 = c0, c3 = c0;
  for (int s = 0; s < q; s += 128) {
    float4 a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool in = s + 16 * u < q;
      a[u] = in ? *reinterpret_cast<const float4*>(ap + s + 16 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
      b[u] = in ? *reinterpret_cast<const float4*>(bp + s + 16 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u].x, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u].y, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u].z, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u].w, c3, 0, 0, 0);
    }
  }
  // c[i] = C[token 4kq+i][expert r]
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave][(4 * kq + i) * 16 + r] = (c0[i] + c1[i]) + (c2[i] + c3[i]);
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {  // the 16 x 16 tile
    const int tt = i >> 4, ee = i & 15;
    if (t0 + tt < m && e0 + ee < n_expert) {
      float v = part[0][i];
      for (int ww = 1; ww < W; ++ww) v += part[ww][i];
      out[((uint64_t)blockIdx.z * m + t0 + tt) * n_expert + e0 + ee] = v;
    }
  }
}

// Slice groups of the router: enough workgroups to spread its loads over
// the chip at decode batch sizes (a power of two <= 16).
int router_groups(int m, int n_expert) {
  const int tiles = ((m + 15) / 16) * ((n_expert + 15) / 16);
  int kz = 1;
  while (kz < kRouterSlices && tiles * kz * 2 <= 256) kz *= 2;
  return kz;
}

// Softmax + top-k of every token: one wave per token.  With kz > 1 the
// router's slice groups are added first, in order, and written as the logits.
__global__ __launch_bounds__(kBlock) void k_route_batch(const float* __restrict__ part, int kz,
                                                        int m, int n_expert, int k,
                                                        float* __restrict__ logits,
                                                        int32_t* __restrict__ topk_idx,
                                                        float* __restrict__ topk_w) {
  const int t = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= m) return;
  // every group's value is loaded before the first addition
  float pv[4][kRouterSlices];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = min(lane + 64 * j, n_expert - 1);
#pragma unroll
    for (int z = 0; z < kRouterSlices; ++z)
      pv[j][z] = z < kz ? part[((uint64_t)z * m + t) * n_expert + e] : 0.0f;
  }
  float lg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    float v = pv[j][0];
#pragma unroll
    for (int z = 1; z < kRouterSlices; ++z)
      if (z < kz) v += pv[j][z];
    if (e < n_expert && kz > 1) logits[(uint64_t)t * n_expert + e] = v;
    lg[j] = e < n_expert ? v : -INFINITY;
  }
  int idx;
  float wt;
  wave_route_lg(lg, n_expert, k, idx, wt);
  if (lane < k) {
    topk_idx[(uint64_t)t * k + lane] = idx;
    topk_w[(uint64_t)t * k + lane] = wt;
  }
}

// ------------------------------------------------------------------ bucketing
// One workgroup: pairs (token, slot) grouped by expert.  offsets[e] is the
// first pair of expert e (offsets[E] = m*k); pair_tok[q] the token of pair q;
// pair_of[t*k + s] the pair of token t's slot s; items the (expert, first
// pair) of every tile of `tile` pairs.  The order of pairs within an expert does
// not change any result: each pair's outputs depend only on its own row.
constexpr int kBucketThreads = 1024;  // (the counting and scattering atomics spread wider)
__global__ __launch_bounds__(kBucketThreads) void k_bucket(const int32_t* __restrict__ topk_idx, int m,
                                                   int k, int n_expert, int* __restrict__ offsets,
                                                   int* __restrict__ pair_tok,
                                                   int* __restrict__ pair_of,
                                                   int2* __restrict__ items,
                                                   int* __restrict__ n_items, int tile) {
  __shared__ int cnt[256], cur[256];
  __shared__ int wsum[2][kBucketThreads / 64];
  const int t = threadIdx.x, P = m * k, lane = t & 63, wave = t >> 6;
  if (t < n_expert) cnt[t] = 0;
  __syncthreads();
  for (int p = t; p < P; p += kBucketThreads) atomicAdd(&cnt[topk_idx[p]], 1);
  __syncthreads();
  // exclusive prefix sums over the experts (thread t = expert t) of the pair
  // counts and the tile counts: a scan within each wave, then the wave totals
  const int c = t < n_expert ? cnt[t] : 0, ct = (c + tile - 1) / tile;
  int sc = c, st = ct;
  for (int d = 1; d < 64; d <<= 1) {
    const int yc = __shfl_up(sc, d, 64), yt = __shfl_up(st, d, 64);
    if (lane >= d) {
      sc += yc;
      st += yt;
    }
  }
  if (lane == 63) {
    wsum[0][wave] = sc;
    wsum[1][wave] = st;
  }
  __syncthreads();
  int oc = sc - c, ot = st - ct;
  for (int w = 0; w < wave; ++w) {
    oc += wsum[0][w];
    ot += wsum[1][w];
  }
  if (t < n_expert) {
    offsets[t] = oc;
    cur[t] = oc;
    for (int i = 0; i < ct; ++i) items[ot + i] = make_int2(t, i * tile);
    if (t == n_expert - 1) {
      offsets[n_expert] = oc + c;
      *n_items = ot + ct;
    }
  }
  __syncthreads();
  for (int p = t; p < P; p += kBucketThreads) {
    const int q = atomicAdd(&cur[topk_idx[p]], 1);
    pair_tok[q] = p / k;
    pair_of[p] = q;
  }
}

// ------------------------------------------------------------------ grouped expert GEMM
struct GroupArgs {
  const uint8_t* w0;        // [E] Q4_K slabs of n_out rows x n_in (gate, or down)
  const uint8_t* w1;        // up slabs (gate/up only)
  int n_in, n_out;
  const _Float16* ah;       // A operand of every pair (k_split_tile layout), high parts
  const _Float16* al;       // f16 remainders
  const _Float16* sh;       // sub-block sums, high parts
  const _Float16* sl;
  int P;                    // pairs
  const int* offsets;       // [E + 1]; null: dense, the P rows are one expert
  const int2* items;
  const int* n_items;
  float* out;               // [pairs][n_out]
  const float* resid = nullptr;  // optional [pairs][n_out] added to out (may alias out)
  // Split over the reduction (dense, not gate/up): blockIdx.z = k-range of
  // super-blocks [z * nsb / ksplit, (z + 1) * nsb / ksplit); with ksplit > 1
  // the workgroup writes its product to partial[z][pairs][n_out] (no
  // residual) and k_ksum adds the ranges in order.
  int ksplit = 1;
  float* partial = nullptr;
  int tile = kTok;          // pairs per work item of the list (<= kTok)
  // gate/up of the few-pair kernel with 32 rows per workgroup: the output in
  // k_split_tile's layout (f16 high parts, remainders, per-32 sums) instead
  // of f32 rows, when oh is set
  _Float16 *oh = nullptr, *ol = nullptr, *osh = nullptr, *osl = nullptr;
};

// Workgroup = one tile of kTok pairs of one expert x kRowsWG weight rows; wave
// = 32 rows.  C[token][row] of the 32x32x16 matrix-core steps: lane l owns
// weight row l % 32, so its row's d/dmin/scales are its own; A = the pair rows
// (token l % 32), B = the unpacked weights.  Per 256-weight super-block the
// workgroup stages the tile's A operand (32 pairs x 256 x hi/lo, and the
// sub-block sums) in LDS once for its four waves; the next super-block's A and
// this lane's next weight block are loaded while the current one is computed
// (double-buffered LDS, one barrier per super-block).  Per code group: 8 steps
// per matrix (hi/lo x and the two nibble sub-blocks x 2); one min-term step
// per matrix per super-block.
constexpr int kQStride = 32;                   // uint4 per 8-group row of 32 pairs
constexpr int kPart = 32 * kQStride;           // uint4 per hi (or lo) part of a super-block
constexpr int kBuf = 2 * kPart + 64;           // + the sums (hi 32, lo 32)
constexpr size_t kGroupLds = 2 * kBuf * 16;    // double-buffered bytes

struct WBlock {
  uint4 h, c[4];
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations are outstanding and does not wait on the other counters
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// ... and that also waits for every LDS access of this wave
constexpr int vm_lds_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// Workgroup barrier once at most N vector memory operations of this wave
// remain outstanding (and no LDS access).  __syncthreads() is a release fence
// plus the barrier, and the fence waits for every outstanding load (the
// LDS-DMA staging makes them count as LDS writes), which would empty the
// weight look-ahead at every barrier; the staging a barrier hands over is
// covered by the explicit count instead.  The asm's memory clobber keeps the
// compiler from moving memory accesses across it.
#define KNJ_BARRIER_VM(N)                      \
  do {                                         \
    __builtin_amdgcn_s_waitcnt(vm_lds_imm(N)); \
    __builtin_amdgcn_sched_barrier(0);         \
    asm volatile("s_barrier" ::: "memory");    \
    __builtin_amdgcn_sched_barrier(0);         \
  } while (0)

// XCD-aware work mapping of a grouped launch (grid nrb row blocks x at least
// 8 * ceil(n_items / 8) items): workgroups are dispatched to the eight XCDs
// in turn by linear index, so XCD x runs linear indices x, x + 8, ...; this
// gives XCD x the contiguous run of items [x * ipx, (x + 1) * ipx) with all
// their row blocks.  The row blocks of one item share its activation tile,
// and an expert's items are adjacent in the list and share its weight rows:
// both are then read once into that XCD's L2 instead of once per XCD.
// False: no work for this workgroup.
__device__ __forceinline__ bool xcd_item(int nrb, int n_items, int& rblock, int& item) {
  const int L = blockIdx.x + nrb * blockIdx.y;
  const int xcd = L & 7, k = L >> 3;
  const int ipx = (n_items + 7) >> 3;
  const int ii = k / nrb;
  rblock = k - ii * nrb;
  item = xcd * ipx + ii;
  return ii < ipx && item < n_items;
}

// NSBT > 0: the super-block range of every workgroup is exactly NSBT long
// (the fully unrolled form below).
template <bool GATEUP, int NSBT = 0>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2))) void k_group_q4k(GroupArgs a) {
  extern __shared__ uint4 lds[];
  // grouped: a work item of the list and a row block (xcd_item); dense (no
  // offsets): the m rows are one expert, tile blockIdx.y, row block blockIdx.x
  int e = 0, p0 = blockIdx.y * kTok, cnt = min(kTok, a.P - p0), rblock = blockIdx.x;
  if (a.offsets) {
    int item;
    if (!xcd_item(gridDim.x, *a.n_items, rblock, item)) return;  // uniform over the workgroup
    const int2 it = a.items[item];
    e = it.x;
    p0 = a.offsets[e] + it.y;
    cnt = min(a.tile, a.offsets[e + 1] - p0);
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int rbase = rblock * kRowsWG + wave * 32;
  const bool rows_ok = rbase < a.n_out;  // waves past the last row still stage and sync
  const int row = min(rbase + (lane & 31), a.n_out - 1), kh = lane >> 5;
  const int j = lane & 31;
  const int nsb_all = a.n_in >> 8;
  const int kz = GATEUP ? 0 : (int)blockIdx.z;
  const int sbb = kz * nsb_all / a.ksplit, nsb = (kz + 1) * nsb_all / a.ksplit;  // [sbb, nsb)
  const uint64_t P = (uint64_t)a.P;
  const uint64_t rb = (uint64_t)nsb_all * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_out;
  const uint8_t* wr0 = a.w0 + (uint64_t)e * slab + (uint64_t)row * rb;
  const uint8_t* wr1 = GATEUP ? a.w1 + (uint64_t)e * slab + (uint64_t)row * rb : wr0;
  // staging by LDS DMA (no registers): wave w's instruction u fills entries
  // e = (8 w + u) 64 + lane of the buffer's hi/lo parts ([part][8-group q]
  // [pair]); wave 0 also fills the 64 sums entries (hi 32, lo 32), and in the
  // unrolled form every wave does, the same bytes, so that all waves issue
  // the same number of loads and the compiler's count of outstanding loads
  // stays exact along the straight line
  // (entry e = 512 w + 64 u + lane: part w / 2, 8-group 16 (w & 1) + 2 u +
  // lane / 32, pair lane % 32; so the source is a part base the wave shares,
  // plus a per-lane byte offset that does not change, plus 2 u P 16 bytes)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>((wv >> 1) ? a.al : a.ah);
  const uint32_t soff =
      (uint32_t)(((uint64_t)(16 * (wv & 1) + (lane >> 5)) * P + p0 + min(lane & 31, cnt - 1)) * 16);
  auto stage = [&](int sb, int buf) {
    const uint8_t* b = sbase + (uint64_t)sb * 32 * P * 16;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e0 = (8 * wave + u) * 64;
      const uint8_t* src = b + (uint64_t)u * 2 * P * 16 + soff;
      __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(lds + buf * kBuf + e0), 16, 0, 0);
    }
    if (NSBT > 0 || wave == 0) {
      const _Float16* src = ((lane >> 5) ? a.sl : a.sh) + ((uint64_t)sb * P + p0 + min(lane & 31, cnt - 1)) * 8;
      __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(lds + buf * kBuf + 2 * kPart), 16, 0, 0);
    }
  };
  auto w_load = [&](const uint8_t* wr, int sb, WBlock& w) {
    const uint8_t* b = wr + (uint64_t)sb * KNJ_Q4K_BLOCK;
    w.h = *reinterpret_cast<const uint4*>(b);
#pragma unroll
    for (int g = 0; g < 4; ++g) w.c[g] = *reinterpret_cast<const uint4*>(b + KNJ_Q4K_QS + 32 * g + 16 * kh);
  };
  f32x16 acc0 = {}, acc1 = {};
  constexpr int WN = GATEUP ? 10 : 5;  // weight loads of one super-block
  // Weight register sets.  Fixed range (NSBT > 0, fully unrolled): three sets
  // in rotation, the weights of super-block i + 2 loaded while i is computed;
  // a straight line, so no register copies wait for loads and the compiler's
  // wait counts are exact.  Any range: the weights of i + 1 go to the other
  // of two sets while one is computed.
  WBlock w0s[3], w1s[3];
  const int n_it = NSBT > 0 ? NSBT : nsb - sbb;
  stage(sbb, 0);
  w_load(wr0, sbb, w0s[0]);
  if constexpr (GATEUP) w_load(wr1, sbb, w1s[0]);
  if constexpr (NSBT > 1) {
    w_load(wr0, sbb + 1, w0s[1]);
    if constexpr (GATEUP) w_load(wr1, sbb + 1, w1s[1]);
    KNJ_BARRIER_VM(WN);
  } else {
    KNJ_BARRIER_VM(0);
  }
  // super-block i on register set ci, the next weights into set ni
  auto step = [&](int i, int ci, int ni) __attribute__((always_inline)) {
    const int buf = i & 1;
    // every load of a later super-block is issued before this one's
    // arithmetic, the staging first: the memory counter is in order, so
    // the wait for the staging at the end leaves the weights in flight
    if (i + 1 < n_it) stage(sbb + i + 1, buf ^ 1);
    const bool load_next = NSBT == 0 || i + 2 < NSBT;
    if (load_next) {
      // any range: the last iteration reloads its own block, unused
      const int nx = NSBT > 0 ? sbb + i + 2 : min(sbb + i + 1, nsb - 1);
      w_load(wr0, nx, w0s[ni]);
      if constexpr (GATEUP) w_load(wr1, nx, w1s[ni]);
    }
    __builtin_amdgcn_sched_barrier(0);
    const WBlock& w0c = w0s[ci];
    const WBlock& w1c = w1s[ci];
    const uint4* L = lds + buf * kBuf;
    const half8 am = __builtin_bit_cast(half8, L[2 * kPart + kh * 32 + j]);
    // the scales and mins of this lane's row, decoded byte-parallel (small
    // integers: every f16 below is exact, the same values as a per-sub-block
    // decode), and the min-term step
    const Q4Scales8 q0 = q4k_scales8(w0c.h.y, w0c.h.z, w0c.h.w);
    Q4Scales8 q1 = {};
    if constexpr (GATEUP) q1 = q4k_scales8(w1c.h.y, w1c.h.z, w1c.h.w);
    auto pk = [](float x, float y) { return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(x, y)); };
    auto mins = [&](const Q4Scales8& q) {
      const half2v m01 = pk(ub0(q.m[0]), ub1(q.m[0])), m23 = pk(ub2(q.m[0]), ub3(q.m[0]));
      const half2v m45 = pk(ub0(q.m[1]), ub1(q.m[1])), m67 = pk(ub2(q.m[1]), ub3(q.m[1]));
      const half8 bm = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
      return mfma32(am, bm, f32x16{});
    };
    auto scales = [&](const Q4Scales8& q, int g, half2v& sl, half2v& nl, half2v& sh, half2v& nh) {
      const uint32_t sw = q.s[g >> 1];
      const float f0 = ubn(sw, (2 * g) & 3), f1 = ubn(sw, (2 * g + 1) & 3);
      sl = pk(f0, f0);
      nl = sl * half2v{(_Float16)-1024.0f, (_Float16)-1024.0f};
      const half2v s1 = pk(f1, f1);
      sh = s1 * half2v{(_Float16)0.0625f, (_Float16)0.0625f};
      nh = s1 * half2v{(_Float16)-64.0f, (_Float16)-64.0f};
    };
    const f32x16 cm0 = mins(q0);
    f32x16 cm1 = {};
    if constexpr (GATEUP) cm1 = mins(q1);
    f32x16 cqa = {}, cqb = {};  // gate (or even groups), up (or odd groups)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      half2v sl0, nl0, sh0, nh0, sl1, nl1, sh1, nh1;
      scales(q0, g, sl0, nl0, sh0, nh0);
      if constexpr (GATEUP) scales(q1, g, sl1, nl1, sh1, nh1);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int q = 8 * g + 2 * kh + kk;
        const half8 xh0 = __builtin_bit_cast(half8, L[q * kQStride + j]);
        const half8 xl0 = __builtin_bit_cast(half8, L[kPart + q * kQStride + j]);
        const half8 xh1 = __builtin_bit_cast(half8, L[(q + 4) * kQStride + j]);
        const half8 xl1 = __builtin_bit_cast(half8, L[kPart + (q + 4) * kQStride + j]);
        const uint32_t w0a = kk ? w0c.c[g].z : w0c.c[g].x, w0b = kk ? w0c.c[g].w : w0c.c[g].y;
        half8 blo, bhi;
        q4_unpack2(w0a, w0b, sl0, nl0, sh0, nh0, blo, bhi);
        if constexpr (GATEUP) {
          cqa = mfma32(xh0, blo, cqa);
          cqa = mfma32(xl0, blo, cqa);
          cqa = mfma32(xh1, bhi, cqa);
          cqa = mfma32(xl1, bhi, cqa);
          const uint32_t w1a = kk ? w1c.c[g].z : w1c.c[g].x, w1b = kk ? w1c.c[g].w : w1c.c[g].y;
          half8 ulo, uhi;
          q4_unpack2(w1a, w1b, sl1, nl1, sh1, nh1, ulo, uhi);
          cqb = mfma32(xh0, ulo, cqb);
          cqb = mfma32(xl0, ulo, cqb);
          cqb = mfma32(xh1, uhi, cqb);
          cqb = mfma32(xl1, uhi, cqb);
        } else {
          // one matrix: two accumulation chains (low and high nibble sub-blocks)
          cqa = mfma32(xh0, blo, cqa);
          cqb = mfma32(xh1, bhi, cqb);
          cqa = mfma32(xl0, blo, cqa);
          cqb = mfma32(xl1, bhi, cqb);
        }
      }
    }
    const float d0 = h2f(w0c.h.x), m0 = h2f(w0c.h.x >> 16);
    if constexpr (GATEUP) {
      const float d1 = h2f(w1c.h.x), m1 = h2f(w1c.h.x >> 16);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc0[r] = __builtin_fmaf(d0, cqa[r], __builtin_fmaf(-m0, cm0[r], acc0[r]));
        acc1[r] = __builtin_fmaf(d1, cqb[r], __builtin_fmaf(-m1, cm1[r], acc1[r]));
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc0[r] += d0 * (cqa[r] + cqb[r]) - m0 * cm0[r];
    }
    // the staging done (at most the weight loads issued after it
    // outstanding) before the barrier that hands the buffer over
    if (load_next)
      KNJ_BARRIER_VM(WN);
    else
      KNJ_BARRIER_VM(0);
  };
  if constexpr (NSBT > 0) {
#pragma unroll
    for (int i = 0; i < NSBT; ++i) step(i, i % 3, (i + 2) % 3);
  } else {
    // two register sets in turn, so no set is copied (a copy waits for
    // its loads)
    int i = 0;
    for (; i + 2 <= n_it; i += 2) {
      step(i, 0, 1);
      step(i + 1, 1, 0);
    }
    if (i < n_it) step(i, 0, 1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (GATEUP) {
    if (a.oh) {
      // SwiGLU written straight as the down product's operand, the same
      // values, order and roundings as k_split_tile over the f32 rows: the
      // wave's 32 x 32 tile goes through its own LDS range (free after the
      // last barrier) as [pair][row]; lane (pair, 8-group g of the wave's 32
      // rows) then forms the perm8 high parts and remainders and the
      // group's sequential sum, four consecutive lanes the 32-row sum
      if (!rows_ok) return;
      float* vs = reinterpret_cast<float*>(lds) + wave * 32 * 33;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tj = 8 * (i / 4) + 4 * kh + (i % 4);
        const float g = acc0[i];
        vs[tj * 33 + j] = (g / (1.0f + expf(-g))) * acc1[i];
      }
      const int b = rbase >> 5;  // the 32-row sub-block of the wave
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int pr = 16 * r + (lane >> 2), g = lane & 3;
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = vs[pr * 33 + 8 * g + q];
        half8 h, l;
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float x = v[perm8(q)];
          h[q] = (_Float16)x;
          l[q] = (_Float16)(x - (float)h[q]);
          sum += v[q];
        }
        sum = group_sum<4>(sum);
        if (pr < cnt) {
          const uint64_t o = ((uint64_t)((rbase >> 3) + g) * P + p0 + pr) * 8;
          *reinterpret_cast<half8*>(a.oh + o) = h;
          *reinterpret_cast<half8*>(a.ol + o) = l;
          if (g == 0) {
            const _Float16 sv = (_Float16)sum;
            const uint64_t so = ((uint64_t)(b >> 3) * P + p0 + pr) * 8 + (b & 7);
            a.osh[so] = sv;
            a.osl[so] = (_Float16)(sum - (float)sv);
          }
        }
      }
      return;
    }
  }
  if (!rows_ok || rbase + (lane & 31) >= a.n_out) return;
  // acc[i] = C[token 8*(i/4) + 4*kh + i%4][row]
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tj = 8 * (i / 4) + 4 * kh + (i % 4);
    if (tj < cnt) {
      float v = acc0[i];
      if constexpr (GATEUP) v = (v / (1.0f + expf(-v))) * acc1[i];
      const uint64_t o = (uint64_t)(p0 + tj) * a.n_out + row;
      if (!GATEUP && a.ksplit > 1)
        a.partial[(uint64_t)kz * P * a.n_out + o] = v;
      else
        a.out[o] = a.resid ? a.resid[o] + v : v;
    }
  }
}

// Grouped Q4_K product for lists whose experts hold few pairs (decode
// batches: at 32 sequences x 8 slots over 128 experts about 2 pairs each),
// where 32-pair tiles would be mostly padding.  Work item = up to kFew = 8
// pairs of one expert.  One 16x16x32 f16 matrix-core step: the 16 A rows are
// the 8 pairs x {high part, remainder} (A row 2 p + part), the 16 B columns
// are 16 weight rows, so lane l's four results are pairs 2 (l/16) and
// 2 (l/16) + 1 (high and remainder each) of weight row l % 16, and the two
// parts are added in the lane at the end.  Lane group kq = l/16 owns code
// group kq (32 bytes: sub-blocks 2 kq and 2 kq + 1) of its row's
// super-block: step u takes bytes 8 (u/2) .. +7 of the group, nibble u % 2,
// i.e. the 8-group 8 kq + 4 (u % 2) + u/2 of the super-block; the K order of
// a step differs by lane group, and A is read to match.  The scales ride in B
// (sc q is exact in f16); the min term is a ninth step per super-block whose
// K slots 8 kq, 8 kq + 1 carry the sub-block sums (A) and mins (B) of
// sub-blocks 2 kq, 2 kq + 1 and zeros elsewhere.  Per super-block:
// acc += d cq - dmin cm.  A comes straight from global memory (the pairs'
// rows are shared by every workgroup of the expert and stay in L2).
constexpr int kFew = 8;
// the few kernels when pairs < kFewBelow * experts (measured crossover with
// the 32-pair kernels: between 8 and 12 pairs per expert)
constexpr int kFewBelow = 10;

__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}


struct FewBlock {
  uint4 h, c0, c1;  // header (d, dmin, scales), the lane's 32 code bytes
};


// Lane constants of the few-pair kernels: bit positions of the scale and min
// of sub-blocks 2 kq and 2 kq + 1 in the 12 scale bytes (words 1..3 of a
// Q4_K header): 6 bits at byte s of words 1 (scale) and 2 (min) for s < 4;
// else the low (scale) / high (min) nibble of byte s - 4 of word 3 and the top
// two bits of byte s - 4 of words 1 and 2.
struct FewLane {
  bool klo;
  int oa, ob, oc;
  __device__ explicit FewLane(int kq)
      : klo(kq < 2),
        oa(kq < 2 ? 16 * kq : 16 * kq - 32),
        ob(kq < 2 ? 16 * kq + 4 : 16 * kq - 26),
        oc(kq < 2 ? 16 * kq : 16 * kq - 28) {}
};

// One super-block of one (matrix, 16-row tile): the eight code steps and the
// min-term step, acc += d cq - dmin cm.
__device__ __forceinline__ void few_superblock(const FewBlock& b, const half8 (&x)[8], half8 xm,
                                               const FewLane& L, f32x4& acc) {
  const uint32_t X = L.klo ? b.h.y : b.h.w, Y = L.klo ? b.h.z : b.h.w;
  const uint32_t sc0 = __builtin_amdgcn_ubfe(X, L.oa, 4) | (__builtin_amdgcn_ubfe(b.h.y, L.ob, 2) << 4);
  const uint32_t sc1 = __builtin_amdgcn_ubfe(X, L.oa + 8, 4) | (__builtin_amdgcn_ubfe(b.h.y, L.ob + 8, 2) << 4);
  const uint32_t mn0 = __builtin_amdgcn_ubfe(Y, L.oc, 4) | (__builtin_amdgcn_ubfe(b.h.z, L.ob, 2) << 4);
  const uint32_t mn1 = __builtin_amdgcn_ubfe(Y, L.oc + 8, 4) | (__builtin_amdgcn_ubfe(b.h.z, L.ob + 8, 2) << 4);
  const float fs0 = (float)sc0, fs1 = (float)sc1;
  // low nibbles: (1024 + q) sc - 1024 sc; high nibbles, unshifted:
  // (1024 + 16 q) sc / 16 - 64 sc (every value exact in f16)
  const half2v s0 = cvt_h2(fs0), n0 = cvt_h2(-1024.0f * fs0);
  const half2v s1 = cvt_h2(0.0625f * fs1), n1 = cvt_h2(-64.0f * fs1);
  half8 bm = {};
  bm[0] = (_Float16)(float)mn0;
  bm[1] = (_Float16)(float)mn1;
  const f32x4 cm = mfma16(xm, bm, f32x4{0.f, 0.f, 0.f, 0.f});
  f32x4 cq = {0.f, 0.f, 0.f, 0.f};
  const uint32_t wd[8] = {b.c0.x, b.c0.y, b.c0.z, b.c0.w, b.c1.x, b.c1.y, b.c1.z, b.c1.w};
  const uint32_t mlo = kNib, mhi = kNib << 4;
  auto cv = [&](uint32_t w, uint32_t m, half2v sc, half2v nc) {
    return __builtin_elementwise_fma(as_h2(and_or(w, m, kF16Base)), sc, nc);
  };
#pragma unroll
  for (int hw = 0; hw < 4; ++hw) {
    // bytes 8 hw .. 8 hw + 7 of the lane's code group: bytes (0, 2), (1, 3),
    // (4, 6), (5, 7) per half2, low nibbles then high nibbles
    const uint32_t wa = wd[2 * hw], wb = wd[2 * hw + 1], sa = wa >> 8, sb = wb >> 8;
    const half2v l0 = cv(wa, mlo, s0, n0), l1 = cv(sa, mlo, s0, n0);
    const half2v l2 = cv(wb, mlo, s0, n0), l3 = cv(sb, mlo, s0, n0);
    const half2v h0 = cv(wa, mhi, s1, n1), h1 = cv(sa, mhi, s1, n1);
    const half2v h2 = cv(wb, mhi, s1, n1), h3 = cv(sb, mhi, s1, n1);
    cq = mfma16(x[2 * hw], half8{l0.x, l0.y, l1.x, l1.y, l2.x, l2.y, l3.x, l3.y}, cq);
    cq = mfma16(x[2 * hw + 1], half8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y}, cq);
  }
  const float d = h2f(b.h.x), dmin = h2f(b.h.x >> 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] += d * cq[i] - dmin * cm[i];
}

// The few-pair grouped product with the reduction split over the waves of a
// workgroup: workgroup = (FT 16-row tiles of every matrix) x (up to 8 pairs of
// one expert); wave w takes super-blocks w, w + KS, ... (KS = waves, NSBW per
// wave) and issues every load of them before any arithmetic, so a workgroup
// asks for whole rows (all super-blocks) of its tiles at once.  The waves'
// partial tiles meet in LDS and are added in wave order.
template <bool GATEUP, int FT, int NSBW, bool SPLIT = false>
__global__ __launch_bounds__(256) void k_group_fewk(GroupArgs a) {
  static_assert(!SPLIT || (GATEUP && FT == 2), "split output: gate/up over 32 rows");
  constexpr int NM = GATEUP ? 2 : 1;
  __shared__ f32x4 part[4][NM * FT][64];
  __shared__ float vs[SPLIT ? 32 : 1][kFew];  // the workgroup's outputs (split form)
  // (the plain order: the XCD-aware mapping of the 32-pair kernels measured
  // slower here, where an expert rarely has more than one item)
  const int item = blockIdx.y, rblock = blockIdx.x;
  if (item >= *a.n_items) return;  // uniform over the workgroup
  const int2 it = a.items[item];
  const int e = it.x, p0 = a.offsets[e] + it.y;
  const int cnt = min(kFew, a.offsets[e + 1] - p0);
  const int KS = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, kq = lane >> 4;
  const int rbase = rblock * 16 * FT;
  const int nsb = a.n_in >> 8;
  const uint64_t P = (uint64_t)a.P;
  const uint64_t rb = (uint64_t)nsb * KNJ_Q4K_BLOCK;
  const uint64_t slab = rb * (uint64_t)a.n_out;
  // A row of this lane: pair ap (clamped into the item), part apart
  const int ap = p0 + min(col >> 1, cnt - 1), apart = col & 1;
  const _Float16* abase = (apart ? a.al : a.ah) + (uint64_t)ap * 8;
  const _Float16* sbase = (apart ? a.sl : a.sh) + (uint64_t)ap * 8 + 2 * kq;
  const FewLane L(kq);
  struct Buf {
    FewBlock w[NM][FT];
    half8 x[8];
    uint32_t s2;
  };
  Buf B[NSBW];
#pragma unroll
  for (int i = 0; i < NSBW; ++i) {
    const int sb = wave + KS * i;
    if (sb < nsb) {  // uniform over the wave
#pragma unroll
      for (int mtx = 0; mtx < NM; ++mtx)
#pragma unroll
        for (int f = 0; f < FT; ++f) {
          const int row = min(rbase + 16 * f + col, a.n_out - 1);
          const uint8_t* p = (mtx ? a.w1 : a.w0) + (uint64_t)e * slab + (uint64_t)row * rb +
                             (uint64_t)sb * KNJ_Q4K_BLOCK;
          B[i].w[mtx][f].h = *reinterpret_cast<const uint4*>(p);
          B[i].w[mtx][f].c0 = *reinterpret_cast<const uint4*>(p + KNJ_Q4K_QS + 32 * kq);
          B[i].w[mtx][f].c1 = *reinterpret_cast<const uint4*>(p + KNJ_Q4K_QS + 32 * kq + 16);
        }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        B[i].x[u] = ld_h8(abase + (uint64_t)(32 * sb + 8 * kq + 4 * (u & 1) + (u >> 1)) * P * 8);
      B[i].s2 = *reinterpret_cast<const uint32_t*>(sbase + (uint64_t)sb * P * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc[NM][FT];
#pragma unroll
  for (int mtx = 0; mtx < NM; ++mtx)
#pragma unroll
    for (int f = 0; f < FT; ++f) acc[mtx][f] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NSBW; ++i) {
    if (wave + KS * i < nsb) {
      half8 xm = {};
      xm[0] = as_h2(B[i].s2).x;
      xm[1] = as_h2(B[i].s2).y;
#pragma unroll
      for (int mtx = 0; mtx < NM; ++mtx)
#pragma unroll
        for (int f = 0; f < FT; ++f) few_superblock(B[i].w[mtx][f], B[i].x, xm, L, acc[mtx][f]);
    }
  }
#pragma unroll
  for (int mtx = 0; mtx < NM; ++mtx)
#pragma unroll
    for (int f = 0; f < FT; ++f) part[wave][mtx * FT + f][lane] = acc[mtx][f];
  __syncthreads();
  // wave w finishes tiles w, w + KS, ... of every matrix, the ranges added in
  // wave order; lane's four values: pair 2 kq + i / 2, part i % 2, weight row
  // 16 f + col
  for (int f = wave; f < FT; f += KS) {
    const int row = rbase + 16 * f + col;
    if (row >= a.n_out) continue;
    f32x4 s[NM];
#pragma unroll
    for (int mtx = 0; mtx < NM; ++mtx) {
      s[mtx] = part[0][mtx * FT + f][lane];
      for (int w = 1; w < KS; ++w) s[mtx] += part[w][mtx * FT + f][lane];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int pj = 2 * kq + h;
      if (pj >= cnt) continue;
      float v = s[0][2 * h] + s[0][2 * h + 1];
      if constexpr (GATEUP) {
        const float u = s[NM - 1][2 * h] + s[NM - 1][2 * h + 1];
        v = (v / (1.0f + expf(-v))) * u;
      }
      if (SPLIT) {
        vs[16 * f + col][pj] = v;
      } else {
        const uint64_t o = (uint64_t)(p0 + pj) * a.n_out + row;
        a.out[o] = a.resid ? a.resid[o] + v : v;
      }
    }
  }
  if constexpr (SPLIT) {
    // the 32 rows [rbase, rbase + 32) of every pair in k_split_tile's layout:
    // thread (pair p, 8-group g) the group's high parts and remainders in
    // perm8 order; the 32-row sum, split the same way, per pair
    __syncthreads();
    const int P = a.P, t = threadIdx.x;
    if (t < 32) {
      const int pp = t & 7, g = t >> 3;
      if (pp < cnt) {
        half8 h, l;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const float x = vs[8 * g + perm8(jj)][pp];
          h[jj] = (_Float16)x;
          l[jj] = (_Float16)(x - (float)h[jj]);
        }
        const uint64_t o = ((uint64_t)(rbase / 8 + g) * P + p0 + pp) * 8;
        *reinterpret_cast<half8*>(a.oh + o) = h;
        *reinterpret_cast<half8*>(a.ol + o) = l;
      }
    } else if (t < 40) {
      const int pp = t - 32;
      if (pp < cnt) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 32; ++r) sum += vs[r][pp];
        const _Float16 sh = (_Float16)sum;
        const int b = rbase / 32;
        const uint64_t o = ((uint64_t)(b / 8) * P + p0 + pp) * 8 + b % 8;
        a.osh[o] = sh;
        a.osl[o] = (_Float16)(sum - (float)sh);
      }
    }
  }
}

// Q6_K down projection of the grouped MoE (d * sc * (q - 32) per weight,
// sc per 16 weights): the same workgroup tiling and A staging as
// k_group_q4k, but one matrix-core step covers exactly one 16-weight scale
// group G of a super-block: lane half kh supplies weights 16 G + 8 kh + (0..7)
// of its row (in the staging's perm8 order) as exact f16 values q - 32, and
// reads the activations of 8-group 2 G + kh.  A step's two products (high
// parts, remainders) start from zero and are added to the accumulator scaled
// by d * sc_G.  Q6_K blocks are 210 bytes, so the lane's byte runs are read
// as aligned words and shifted into place (ld8_u2).  ksplit 1, no residual.
// With null offsets the P rows are one expert (a dense product, e.g. a Q6_K
// LM head over a batch of rows).
struct Q6WBlock {
  uint32_t la[2][2][2], lb[2][2][2], qh[2][2][2];  // [half n][16-run lh][word]: ql +0, ql +32, qh
  uint32_t sc[4];                                   // the 16 int8 scales
  uint32_t d;                                       // f16 bits
};

__global__ __launch_bounds__(kBlock) void k_group_q6k(GroupArgs a) {
  extern __shared__ uint4 lds[];
  // grouped: work item blockIdx.y; dense (no offsets): tile blockIdx.y of the
  // P rows seen as one expert
  int e = 0, p0 = blockIdx.y * kTok, cnt = min(kTok, a.P - p0), rblock = blockIdx.x;
  if (a.offsets) {
    int item;
    if (!xcd_item(gridDim.x, *a.n_items, rblock, item)) return;  // uniform over the workgroup
    const int2 it = a.items[item];
    e = it.x;
    p0 = a.offsets[e] + it.y;
    cnt = min(a.tile, a.offsets[e + 1] - p0);
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int rbase = rblock * kRowsWG + wave * 32;
  const bool rows_ok = rbase < a.n_out;
  const int row = min(rbase + (lane & 31), a.n_out - 1), kh = lane >> 5;
  const int j = lane & 31;
  const int nsb = a.n_in >> 8;
  const uint64_t P = (uint64_t)a.P;
  const uint64_t rb = (uint64_t)nsb * KNJ_Q6K_BLOCK;
  const uint8_t* wr = a.w0 + (uint64_t)e * rb * (uint64_t)a.n_out + (uint64_t)row * rb;
  // staging by LDS DMA, as in k_group_q4k (no sums: no min term here)
  auto stage = [&](int sb, int buf) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e0 = (8 * wave + u) * 64, ee = e0 + lane;
      const int part = ee >> 10, r = ee & 1023, q = r >> 5, jj = r & 31;
      const _Float16* src = (part ? a.al : a.ah) + ((uint64_t)(32 * sb + q) * P + p0 + min(jj, cnt - 1)) * 8;
      __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(lds + buf * kBuf + e0), 16, 0, 0);
    }
  };
  auto w_load = [&](int sb, Q6WBlock& w) {
    const uint8_t* b = wr + (uint64_t)sb * KNJ_Q6K_BLOCK;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int lh = 0; lh < 2; ++lh) {
        const int l = 16 * lh + 8 * kh;
        ld8_u2(b + KNJ_Q6K_QL + 64 * n + l, w.la[n][lh][0], w.la[n][lh][1]);
        ld8_u2(b + KNJ_Q6K_QL + 64 * n + 32 + l, w.lb[n][lh][0], w.lb[n][lh][1]);
        ld8_u2(b + KNJ_Q6K_QH + 32 * n + l, w.qh[n][lh][0], w.qh[n][lh][1]);
      }
    ld8_u2(b + KNJ_Q6K_SC, w.sc[0], w.sc[1]);
    ld8_u2(b + KNJ_Q6K_SC + 8, w.sc[2], w.sc[3]);
    w.d = *reinterpret_cast<const uint16_t*>(b + KNJ_Q6K_D);
  };
  Q6WBlock wc, wn;
  stage(0, 0);
  w_load(0, wc);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  f32x16 acc = {};
  const half2v bias = half2v{(_Float16)1056.0f, (_Float16)1056.0f};  // 1024 + 32
  auto cv = [&](uint32_t w) { return as_h2((w & 0x00FF00FFu) | 0x64006400u) - bias; };
  for (int sb = 0; sb < nsb; ++sb) {
    const int buf = sb & 1;
    const int nx = min(sb + 1, nsb - 1);  // the last iteration reloads its own block, unused
    // the staging first, then the weights, all before this block's arithmetic
    if (sb + 1 < nsb) stage(nx, buf ^ 1);
    w_load(nx, wn);
    __builtin_amdgcn_sched_barrier(0);
    const uint4* L = lds + buf * kBuf;
    const float d = h2f(wc.d);
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int lh = 0; lh < 2; ++lh)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const int G = 8 * n + 2 * s4 + lh;  // weights 16 G .. 16 G + 15
          const uint32_t* ql = (s4 & 1) ? wc.lb[n][lh] : wc.la[n][lh];
          const int nsh = 4 * (s4 >> 1), hsh = 2 * s4;
          const uint32_t q0 = ((ql[0] >> nsh) & 0x0F0F0F0Fu) | (((wc.qh[n][lh][0] >> hsh) & 0x03030303u) << 4);
          const uint32_t q1 = ((ql[1] >> nsh) & 0x0F0F0F0Fu) | (((wc.qh[n][lh][1] >> hsh) & 0x03030303u) << 4);
          const half2v b0 = cv(q0), b1 = cv(q0 >> 8), b2 = cv(q1), b3 = cv(q1 >> 8);
          const half8 bw = half8{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
          const half8 xh = __builtin_bit_cast(half8, L[(2 * G + kh) * kQStride + j]);
          const half8 xl = __builtin_bit_cast(half8, L[kPart + (2 * G + kh) * kQStride + j]);
          f32x16 c = mfma32(xh, bw, f32x16{});
          c = mfma32(xl, bw, c);
          const float sg = d * (float)(int8_t)((wc.sc[G >> 2] >> (8 * (G & 3))) & 0xFFu);
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[i] += sg * c[i];
        }
    wc = wn;
    __builtin_amdgcn_s_waitcnt(0);  // the staging landed before the barrier hands it over
    __syncthreads();
  }
  if (!rows_ok || rbase + (lane & 31) >= a.n_out) return;
  // acc[i] = C[token 8*(i/4) + 4*kh + i%4][row]
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tj = 8 * (i / 4) + 4 * kh + (i % 4);
    if (tj < cnt) a.out[(uint64_t)(p0 + tj) * a.n_out + row] = acc[i];
  }
}

// out[i] = resid[i] + sum_z partial[z][i], the ranges added in order (resid
// may alias out).
__global__ __launch_bounds__(kBlock) void k_ksum(const float* __restrict__ partial, int ksplit,
                                                 uint64_t n, const float* resid, float* out) {
  const uint64_t i4 = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) * 4;
  if (i4 >= n) return;  // n is a multiple of 4
  float4 v[16];
#pragma unroll
  for (int z = 0; z < 16; ++z)
    if (z < ksplit) v[z] = *reinterpret_cast<const float4*>(partial + (uint64_t)z * n + i4);
  float4 r = resid ? *reinterpret_cast<const float4*>(resid + i4) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int z = 0; z < 16; ++z)
    if (z < ksplit) {
      r.x += v[z].x;
      r.y += v[z].y;
      r.z += v[z].z;
      r.w += v[z].w;
    }
  *reinterpret_cast<float4*>(out + i4) = r;
}

// k_ksum and k_norm_rows in one launch, one workgroup per row (n <= 4096,
// n % 256 == 0): out = resid + the ranges in order (k_ksum's additions), then
// norm_out = out * scale * w with k_norm_rows's thread mapping and block sum,
// so both are the bits the two launches give.
__global__ __launch_bounds__(kBlock) void k_ksum_norm(const float* __restrict__ partial, int ksplit,
                                                      uint64_t total, int n, const float* resid,
                                                      float* out, const float* __restrict__ nw,
                                                      float eps, float* __restrict__ norm_out) {
  __shared__ float red[8];
  const uint64_t row = blockIdx.x;
  float4 r[4];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * threadIdx.x + 4 * kBlock * u;
    if (i < n) {
      const uint64_t e = row * n + i;
      float4 v[16];
#pragma unroll
      for (int z = 0; z < 16; ++z)
        if (z < ksplit) v[z] = *reinterpret_cast<const float4*>(partial + (uint64_t)z * total + e);
      float4 a = resid ? *reinterpret_cast<const float4*>(resid + e) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int z = 0; z < 16; ++z)
        if (z < ksplit) {
          a.x += v[z].x;
          a.y += v[z].y;
          a.z += v[z].z;
          a.w += v[z].w;
        }
      *reinterpret_cast<float4*>(out + e) = a;
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      r[u] = a;
    }
  }
  ss = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * threadIdx.x + 4 * kBlock * u;
    if (i < n) {
      const float4 w = *reinterpret_cast<const float4*>(nw + i);
      *reinterpret_cast<float4*>(norm_out + row * n + i) =
          make_float4(r[u].x * scale * w.x, r[u].y * scale * w.y, r[u].z * scale * w.z, r[u].w * scale * w.w);
    }
  }
}

// ------------------------------------------------------------------ bf16 weights (LM head)
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Row p of src (n floats) as three bf16 parts x = hi + mid + lo (24
// significant bits), natural order, pairs interleaved: part[(q * P + p) * 8 + j].
__global__ __launch_bounds__(kBlock) void k_split_bf16x3(const float* __restrict__ src, int n,
                                                         int P, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ mid,
                                                         uint16_t* __restrict__ lo) {
  const int p = blockIdx.x;
  const float* s = src + (uint64_t)p * n;
  for (int g = threadIdx.x; 8 * g < n; g += kBlock) {
    uint16_t h[8], md[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = s[8 * g + j];
      h[j] = knj_f32_to_bf16(x);
      const float r1 = x - knj_bf16_to_f32(h[j]);
      md[j] = knj_f32_to_bf16(r1);
      l[j] = knj_f32_to_bf16(r1 - knj_bf16_to_f32(md[j]));
    }
    const uint64_t o = ((uint64_t)g * P + p) * 8;
    *reinterpret_cast<uint4*>(hi + o) = *reinterpret_cast<const uint4*>(h);
    *reinterpret_cast<uint4*>(mid + o) = *reinterpret_cast<const uint4*>(md);
    *reinterpret_cast<uint4*>(lo + o) = *reinterpret_cast<const uint4*>(l);
  }
}

__device__ __forceinline__ bf16x8 ld_b8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// out[p][row] = W[row] . x_p for bf16 W [n_out][n_in] and tiles of 32 pairs
// (blockIdx.y = tile): workgroup = 128 rows, wave = 32, lane l owns row l % 32;
// three 32x32x16 bf16 matrix-core steps per 16 weights (x hi, mid, lo).
__global__ __launch_bounds__(kBlock) void k_dense_bf16(const uint16_t* __restrict__ w, int n_in,
                                                       int n_out, int P,
                                                       const uint16_t* __restrict__ xh,
                                                       const uint16_t* __restrict__ xm,
                                                       const uint16_t* __restrict__ xl,
                                                       float* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rbase = blockIdx.x * kRowsWG + wave * 32;
  if (rbase >= n_out) return;
  const int row = min(rbase + (lane & 31), n_out - 1), kh = lane >> 5;
  const int p0 = blockIdx.y * kTok, cnt = min(kTok, P - p0);
  const int pj = p0 + min(lane & 31, cnt - 1);
  const uint64_t qs = (uint64_t)P * 8;
  const uint16_t* wr = w + (uint64_t)row * n_in + 8 * kh;
  const uint64_t xo = (uint64_t)pj * 8 + kh * qs;
  f32x16 acc = {};
  for (int k0 = 0; k0 < n_in; k0 += 64) {
    bf16x8 b[4], ah[4], am[4], al[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      b[u] = ld_b8(wr + k0 + 16 * u);
      const uint64_t q = (uint64_t)((k0 + 16 * u) / 8) * qs + xo;
      ah[u] = ld_b8(xh + q);
      am[u] = ld_b8(xm + q);
      al[u] = ld_b8(xl + q);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[u], b[u], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[u], b[u], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[u], b[u], acc, 0, 0, 0);
    }
  }
  if (rbase + (lane & 31) >= n_out) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tj = 8 * (i / 4) + 4 * kh + (i % 4);
    if (tj < cnt) out[(uint64_t)(p0 + tj) * n_out + row] = acc[i];
  }
}

// Greedy token of each row of logits [m][n] (first maximum wins), in two
// passes: workgroup (c, r) reduces chunk c of 8192 entries of row r to one
// packed (value, index) key; then one workgroup per row reduces its keys.
constexpr int kArgChunk = 8192;

__global__ __launch_bounds__(kBlock) void k_argmax_part(const float* __restrict__ logits, int n,
                                                        unsigned long long* __restrict__ keys) {
  const int r = blockIdx.y, c = blockIdx.x;
  const float* row = logits + (uint64_t)r * n;
  const int i0 = c * kArgChunk, i1 = min(n, i0 + kArgChunk);
  unsigned long long best = 0;
  for (int i = i0 + threadIdx.x; i < i1; i += kBlock) {
    const unsigned long long k = argmax_key(row[i], i);
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  __shared__ unsigned long long wb[kBlock / 64];
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kBlock / 64; ++q) best = wb[q] > best ? wb[q] : best;
    best = wb[0] > best ? wb[0] : best;
    keys[(uint64_t)r * gridDim.x + c] = best;
  }
}

__global__ void k_argmax_final(const unsigned long long* __restrict__ keys, int nk,
                               int32_t* __restrict__ tok) {
  const int r = blockIdx.x;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < nk; i += 64) {
    const unsigned long long k = keys[(uint64_t)r * nk + i];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if (threadIdx.x == 0) tok[r] = argmax_index(best);
}

// ------------------------------------------------------------------ combine
// out[t] = resid[t] + sum over token t's k slots, in ascending expert order,
// of w * y[pair] (the scatter order of model.cpp:499-507).
__global__ __launch_bounds__(64) void k_combine(const float* __restrict__ y,
                                                const int* __restrict__ pair_of,
                                                const int32_t* __restrict__ topk_idx,
                                                const float* __restrict__ topk_w, int k, int n,
                                                const float* __restrict__ resid,
                                                float* __restrict__ out,
                                                float* __restrict__ out2) {
  // one wave: lane s < k reads slot s, finds its rank among the token's
  // experts (distinct ids) and files its pair and weight under that rank
  __shared__ int ps[16];
  __shared__ float ws[16];
  const int t = blockIdx.x, lane = threadIdx.x;
  const bool in = lane < k;
  const int id = in ? topk_idx[(uint64_t)t * k + lane] : 0x7FFFFFFF;
  const float wt = in ? topk_w[(uint64_t)t * k + lane] : 0.0f;
  const int pr = in ? pair_of[(uint64_t)t * k + lane] : 0;
  int rank = 0;
  for (int q = 0; q < k; ++q) rank += __shfl(id, q, 64) < id ? 1 : 0;
  if (in) {
    ps[rank] = pr;
    ws[rank] = wt;
  }
  __syncthreads();
  // one float4 of columns per lane (blockIdx.y picks the 256-column range):
  // every slot's load is issued before the first use
  const int i = 4 * (blockIdx.y * 64 + lane);
  if (i >= n) return;
  float4 v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (r < k) v[r] = *reinterpret_cast<const float4*>(y + (uint64_t)ps[r] * n + i);
  const float4 rs = resid ? *reinterpret_cast<const float4*>(resid + (uint64_t)t * n + i)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (r < k) {
      const float w = ws[r];
      o.x = __fadd_rn(o.x, __fmul_rn(w, v[r].x));
      o.y = __fadd_rn(o.y, __fmul_rn(w, v[r].y));
      o.z = __fadd_rn(o.z, __fmul_rn(w, v[r].z));
      o.w = __fadd_rn(o.w, __fmul_rn(w, v[r].w));
    }
  if (resid) {
    o.x = __fadd_rn(rs.x, o.x);
    o.y = __fadd_rn(rs.y, o.y);
    o.z = __fadd_rn(rs.z, o.z);
    o.w = __fadd_rn(rs.w, o.w);
  }
  *reinterpret_cast<float4*>(out + (uint64_t)t * n + i) = o;
  if (out2) *reinterpret_cast<float4*>(out2 + (uint64_t)t * n + i) = o;
}

// k_combine over whole rows, then the next step's input from them: one
// workgroup per token, thread t on the float4 at 4 t + 1024 u (k_norm_rows's
// mapping).  The weighted sum is k_combine's (ascending expert, the same
// roundings); with nw, the row's RMS norm as k_norm_rows computes it into hx
// and/or the split operand as k_split_tile computes it (8-groups in perm8
// order through LDS, sequential sums per 8-group, pairwise per 32).  k = 0:
// out = resid (the norm and split of a row alone).
__global__ __launch_bounds__(kBlock) void k_combine_norm(
    const float* __restrict__ y, const int* __restrict__ pair_of, const int32_t* __restrict__ topk_idx,
    const float* __restrict__ topk_w, int k, int n, int P, const float* resid, float* out,
    float* __restrict__ out2, const float* __restrict__ nw, float eps, float* __restrict__ hx,
    _Float16* __restrict__ shi, _Float16* __restrict__ slo, _Float16* __restrict__ sshi,
    _Float16* __restrict__ sslo) {
  __shared__ int ps[16];
  __shared__ float ws[16];
  __shared__ float red[8];
  __shared__ float row[4096];
  const int t = blockIdx.x, tid = threadIdx.x;
  if (tid < 64) {
    const bool in = tid < k;
    const int id = in ? topk_idx[(uint64_t)t * k + tid] : 0x7FFFFFFF;
    const float wt = in ? topk_w[(uint64_t)t * k + tid] : 0.0f;
    const int pr = in ? pair_of[(uint64_t)t * k + tid] : 0;
    int rank = 0;
    for (int q = 0; q < k; ++q) rank += __shfl(id, q, 64) < id ? 1 : 0;
    if (in) {
      ps[rank] = pr;
      ws[rank] = wt;
    }
  }
  __syncthreads();
  float4 o4[4];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * tid + 4 * kBlock * u;
    if (i < n) {
      float4 v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (r < k) v[r] = *reinterpret_cast<const float4*>(y + (uint64_t)ps[r] * n + i);
      const float4 rs = resid ? *reinterpret_cast<const float4*>(resid + (uint64_t)t * n + i)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (r < k) {
          const float w = ws[r];
          o.x = __fadd_rn(o.x, __fmul_rn(w, v[r].x));
          o.y = __fadd_rn(o.y, __fmul_rn(w, v[r].y));
          o.z = __fadd_rn(o.z, __fmul_rn(w, v[r].z));
          o.w = __fadd_rn(o.w, __fmul_rn(w, v[r].w));
        }
      if (resid) {
        o.x = __fadd_rn(rs.x, o.x);
        o.y = __fadd_rn(rs.y, o.y);
        o.z = __fadd_rn(rs.z, o.z);
        o.w = __fadd_rn(rs.w, o.w);
      }
      *reinterpret_cast<float4*>(out + (uint64_t)t * n + i) = o;
      if (out2) *reinterpret_cast<float4*>(out2 + (uint64_t)t * n + i) = o;
      ss += o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
      o4[u] = o;
    }
  }
  if (!nw) return;  // uniform
  ss = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * tid + 4 * kBlock * u;
    if (i < n) {
      const float4 w = *reinterpret_cast<const float4*>(nw + i);
      const float4 h = make_float4(o4[u].x * scale * w.x, o4[u].y * scale * w.y,
                                   o4[u].z * scale * w.z, o4[u].w * scale * w.w);
      if (hx) *reinterpret_cast<float4*>(hx + (uint64_t)t * n + i) = h;
      *reinterpret_cast<float4*>(row + i) = h;
    }
  }
  if (!shi) return;  // uniform
  __syncthreads();
  for (int g = tid; 8 * g < n; g += kBlock) {  // 8-group g of the row
    half8 hv, lv;
    float s8 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = row[8 * g + perm8(j)];
      hv[j] = (_Float16)x;
      lv[j] = (_Float16)(x - (float)hv[j]);
      s8 += row[8 * g + j];
    }
    const uint64_t o = ((uint64_t)g * P + t) * 8;
    *reinterpret_cast<half8*>(shi + o) = hv;
    *reinterpret_cast<half8*>(slo + o) = lv;
    const float sum = group_sum<4>(s8);  // the four 8-groups of 32-sub-block g / 4
    if ((g & 3) == 0) {
      const int b = g >> 2;
      const _Float16 sv = (_Float16)sum;
      const uint64_t so = ((uint64_t)(b >> 3) * P + t) * 8 + (b & 7);
      sshi[so] = sv;
      sslo[so] = (_Float16)(sum - (float)sv);
    }
  }
}

}  // namespace

uint64_t moe_batch_scratch_bytes(int m, int n_embd, int n_ff, int n_expert, int k) {
  const uint64_t P = (uint64_t)m * k, H = n_embd, F = n_ff;
  const uint64_t items = (uint64_t)n_expert + (P + kFew - 1) / kFew;  // the smaller tile bounds both lists
  uint64_t b = 0;
  auto add = [&](uint64_t bytes) { b += (bytes + 255) & ~255ull; };
  add(m * H * 4);                       // hx
  add(P * H * 2); add(P * H * 2);       // x hi/lo per pair
  add(P * H / 16); add(P * H / 16);     // x sums hi/lo
  add((n_expert + 1) * 4);              // offsets
  add(P * 4); add(P * 4);               // pair_tok, pair_of
  add(items * 8); add(256);             // items, n_items
  add(P * F * 4);                       // act
  add(P * F * 2); add(P * F * 2);       // act hi/lo
  add(P * F / 16); add(P * F / 16);     // act sums hi/lo
  add(P * H * 4);                       // y
  const int kz = router_groups(m, n_expert);
  if (kz > 1) add((uint64_t)kz * m * n_expert * 4);  // router slice-group sums
  return b;
}

// The grouped kernels use more than the default 64 KB of dynamic LDS.
hipError_t group_lds_attr() {
  static hipError_t e = [] {
    hipError_t r = hipFuncSetAttribute((const void*)k_group_q4k<true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGroupLds);
    if (r == hipSuccess)
      r = hipFuncSetAttribute((const void*)k_group_q4k<false>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGroupLds);
    if (r == hipSuccess)
      r = hipFuncSetAttribute((const void*)k_group_q4k<false, 3>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGroupLds);
    if (r == hipSuccess)
      r = hipFuncSetAttribute((const void*)k_group_q6k,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGroupLds);
    return r;
  }();
  return e;
}

// The few-pair product over n_in: KS = min(4, super-blocks) waves per
// workgroup, each with NSBW super-blocks; ft 16-row tiles per workgroup.
template <bool GATEUP>
hipError_t launch_fewk(const GroupArgs& g, int max_items, int ft, hipStream_t s) {
  const int nsb = g.n_in >> 8, ks = std::min(4, nsb), nw = (nsb + ks - 1) / ks;
  const dim3 grid((g.n_out + 16 * ft - 1) / (16 * ft), max_items), block(64 * ks);
#define KNJ_FEWK(FT, NW) \
  if (ft == FT && nw <= NW) { KNJ_LAUNCH((k_group_fewk<GATEUP, FT, NW>), grid, block, 0, s, g); return hipGetLastError(); }
  if constexpr (GATEUP) {
    if (g.oh) {  // the split output (32 rows per workgroup)
      if (ft != 2 || g.n_out % 32) return hipErrorInvalidValue;
      if (nw <= 1) { KNJ_LAUNCH((k_group_fewk<GATEUP, 2, 1, true>), grid, block, 0, s, g); return hipGetLastError(); }
      if (nw <= 2) { KNJ_LAUNCH((k_group_fewk<GATEUP, 2, 2, true>), grid, block, 0, s, g); return hipGetLastError(); }
      if (nw <= 4) { KNJ_LAUNCH((k_group_fewk<GATEUP, 2, 4, true>), grid, block, 0, s, g); return hipGetLastError(); }
      return hipErrorInvalidValue;
    }
  }
  KNJ_FEWK(2, 1) KNJ_FEWK(2, 2) KNJ_FEWK(2, 4) KNJ_FEWK(4, 1)
#undef KNJ_FEWK
  return hipErrorInvalidValue;
}

hipError_t launch_moe_batch(const MoeBatchArgs& a, void* scratch, hipStream_t s) {
  if (hipError_t e = group_lds_attr()) return e;
  const int m = a.m, H = a.n_embd, F = a.n_ff, E = a.n_expert, K = a.k;
  if (H % 256 || F % 256 || H > 4096 || F > 4096 || E > 256 || K > 16 || m <= 0 ||
      (a.type_down != KNJ_TYPE_Q4_K && a.type_down != KNJ_TYPE_Q6_K))
    return hipErrorInvalidValue;
  const uint64_t P = (uint64_t)m * K;
  // few pairs per expert on average (decode batches): 8-pair items on the
  // 16x16x32 kernels; else 32-pair items on the 32x32x16 kernels
  const bool few = P < (uint64_t)kFewBelow * E;
  const int tile = few ? kFew : kTok;
  const int max_items = E + (int)((P + tile - 1) / tile);
  uint8_t* p = (uint8_t*)scratch;
  auto take = [&](uint64_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) & ~255ull;
    return q;
  };
  float* hx = (float*)take((uint64_t)m * H * 4);
  _Float16* xh = (_Float16*)take(P * H * 2);
  _Float16* xl = (_Float16*)take(P * H * 2);
  _Float16* sxh = (_Float16*)take(P * H / 16);
  _Float16* sxl = (_Float16*)take(P * H / 16);
  int* offsets = (int*)take((uint64_t)(E + 1) * 4);
  int* pair_tok = (int*)take(P * 4);
  int* pair_of = (int*)take(P * 4);
  int2* items = (int2*)take((uint64_t)max_items * 8);
  int* n_items = (int*)take(256);
  float* act = (float*)take(P * F * 4);
  _Float16* ah = (_Float16*)take(P * F * 2);
  _Float16* al = (_Float16*)take(P * F * 2);
  _Float16* sah = (_Float16*)take(P * F / 16);
  _Float16* sal = (_Float16*)take(P * F / 16);
  float* y = (float*)take(P * H * 4);
  const int kz = router_groups(m, E);
  float* rpart = kz > 1 ? (float*)take((uint64_t)kz * m * E * 4) : a.logits;

  const float* xin = a.x;
  if (a.norm_w) {
    KNJ_LAUNCH(k_norm_rows, dim3(m), dim3(kBlock), 0, s, a.x, a.norm_w, a.eps, H, hx);
    xin = hx;
  }
  KNJ_LAUNCH(k_router_batch, dim3((m + 15) / 16, (E + 15) / 16, kz), dim3(64 * kRouterSlices / kz), 0,
             s, xin, a.router_w, m, H, E, rpart);
  KNJ_LAUNCH(k_route_batch, dim3((m + 3) / 4), dim3(kBlock), 0, s, rpart, kz, m, E, K, a.logits,
             a.topk_idx, a.topk_w);
  KNJ_LAUNCH(k_bucket, dim3(1), dim3(kBucketThreads), 0, s, a.topk_idx, m, K, E, offsets, pair_tok,
                     pair_of, items, n_items, tile);
  KNJ_LAUNCH(k_split_tile, dim3((unsigned)((P + 31) / 32), H / 64), dim3(kBlock), 0, s, xin,
             pair_tok, H, (int)P, xh, xl, sxh, sxl);
  GroupArgs gu{a.gate, a.up, H, F, xh, xl, sxh, sxl, (int)P, offsets, items, n_items, act};
  gu.tile = tile;
  // (measured at 32 sequences: 32 rows per workgroup for gate/up, whose
  // super-blocks fill two per wave; 64 for down, one per wave)
  if (few) {
    // SwiGLU written straight in the down product's operand layout
    gu.oh = ah;
    gu.ol = al;
    gu.osh = sah;
    gu.osl = sal;
    if (hipError_t e = launch_fewk<true>(gu, max_items, 2, s)) return e;
  } else {
    // SwiGLU written straight in the down product's operand layout
    gu.oh = ah;
    gu.ol = al;
    gu.osh = sah;
    gu.osl = sal;
    KNJ_LAUNCH(k_group_q4k<true>, dim3((F + kRowsWG - 1) / kRowsWG, max_items + 8), dim3(kBlock),
               kGroupLds, s, gu);
  }
  GroupArgs dn{a.down, nullptr, F, H, ah, al, sah, sal, (int)P, offsets, items, n_items, y};
  dn.tile = tile;
  if (few && a.type_down == KNJ_TYPE_Q4_K) {
    if (hipError_t e = launch_fewk<false>(dn, max_items, (F >> 8) <= 4 ? 4 : 2, s)) return e;
  } else if (a.type_down == KNJ_TYPE_Q6_K)
    KNJ_LAUNCH(k_group_q6k, dim3((H + kRowsWG - 1) / kRowsWG, max_items + 8), dim3(kBlock), kGroupLds,
               s, dn);
  else if (F == 3 * 256)  // the model's 768-wide expert rows: the unrolled form
    KNJ_LAUNCH((k_group_q4k<false, 3>), dim3((H + kRowsWG - 1) / kRowsWG, max_items + 8), dim3(kBlock),
               kGroupLds, s, dn);
  else
    KNJ_LAUNCH(k_group_q4k<false>, dim3((H + kRowsWG - 1) / kRowsWG, max_items + 8), dim3(kBlock),
               kGroupLds, s, dn);
  if (a.next_norm_w) {
    _Float16* const* sp = a.next_split;
    KNJ_LAUNCH(k_combine_norm, dim3(m), dim3(kBlock), 0, s, y, pair_of, a.topk_idx, a.topk_w, K, H, m,
               a.resid, a.out, a.hidden_copy, a.next_norm_w, a.next_eps, a.next_hx,
               sp ? sp[0] : nullptr, sp ? sp[1] : nullptr, sp ? sp[2] : nullptr, sp ? sp[3] : nullptr);
  } else {
    // one wave per 256 columns of a token: enough workgroups for the chip at
    // decode batch sizes
    KNJ_LAUNCH(k_combine, dim3(m, (H + 255) / 256), dim3(64), 0, s, y, pair_of, a.topk_idx,
               a.topk_w, K, H, a.resid, a.out, a.hidden_copy);
  }
  return hipGetLastError();
}

// ---- dense batched GEMMs of the batched decode step
// Ranges of the reduction a dense Q4_K product is split into: enough
// workgroups for the chip, about 512 (at most 16 ranges, at most one per
// super-block).
int dense_ksplit(int m, int n_in, int n_out) {
  if (m <= 0 || n_out <= 0) return 1;
  const int tiles = (m + kTok - 1) / kTok, rows = (n_out + kRowsWG - 1) / kRowsWG;
  // about two workgroups per CU (measured: 512 beats 256 and 1024)
  constexpr int target = 512;
  const int want = (target + tiles * rows - 1) / (tiles * rows);
  return std::max(1, std::min({want, n_in >> 8, 16}));
}

uint64_t dense_scratch_bytes(int m, int n_in, int n_out) {
  const uint64_t P = (uint64_t)m;
  const int ks = dense_ksplit(m, n_in, n_out);
  const uint64_t part = ks > 1 ? (uint64_t)ks * P * n_out * 4 : 0;
  return 4 * ((P * n_in * 2 + 255) & ~255ull) + 2 * ((P * n_in / 16 + 255) & ~255ull) +
         ((part + 255) & ~255ull);
}

hipError_t launch_norm_split(const float* x, const float* nw, float eps, int m, int n, float* hx,
                             _Float16* const* split, hipStream_t s) {
  if (n > 4096 || n % 256) return hipErrorInvalidValue;
  KNJ_LAUNCH(k_combine_norm, dim3(m), dim3(kBlock), 0, s, nullptr, nullptr, nullptr, nullptr, 0, n,
             m, x, const_cast<float*>(x), nullptr, nw, eps, hx, split ? split[0] : nullptr,
             split ? split[1] : nullptr, split ? split[2] : nullptr, split ? split[3] : nullptr);
  return hipGetLastError();
}

hipError_t launch_norm_rows(const float* x, const float* nw, float eps, int m, int n, float* out,
                            hipStream_t s) {
  if (n > 4096 || n % 256) return hipErrorInvalidValue;
  KNJ_LAUNCH(k_norm_rows, dim3(m), dim3(kBlock), 0, s, x, nw, eps, n, out);
  return hipGetLastError();
}

uint64_t split_operand_bytes(int m, int n) {
  const uint64_t P = (uint64_t)m;
  return 2 * ((P * n * 2 + 255) & ~255ull) + 2 * ((P * n / 16 + 255) & ~255ull);
}

hipError_t launch_dense_q4k(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                            const float* resid, float* out, void* scratch, hipStream_t s) {
  return launch_dense_q4k_ex(w, n_in, n_out, m, x, resid, out, scratch, DenseQ4Extra{}, s);
}

hipError_t launch_dense_q4k_ex(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                               const float* resid, float* out, void* scratch,
                               const DenseQ4Extra& ex, hipStream_t s) {
  if (hipError_t e = group_lds_attr()) return e;
  if (n_in > 4096 || n_in % 256 || n_out % 32 || m > 1024) return hipErrorInvalidValue;
  const uint64_t P = (uint64_t)m;
  uint8_t* p = (uint8_t*)scratch;
  auto take = [&](uint64_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) & ~255ull;
    return q;
  };
  const _Float16* xh = (_Float16*)take(P * n_in * 2);
  const _Float16* xl = (_Float16*)take(P * n_in * 2);
  const _Float16* sh = (_Float16*)take(P * n_in / 16);
  const _Float16* sl = (_Float16*)take(P * n_in / 16);
  const int ks = dense_ksplit(m, n_in, n_out);
  float* part = ks > 1 ? (float*)take((uint64_t)ks * P * n_out * 4) : nullptr;
  if (ex.pre) {
    xh = ex.pre[0];
    xl = ex.pre[1];
    sh = ex.pre[2];
    sl = ex.pre[3];
  } else {
    KNJ_LAUNCH(k_split_tile, dim3((m + 31) / 32, n_in / 64), dim3(kBlock), 0, s, x, nullptr,
               n_in, m, const_cast<_Float16*>(xh), const_cast<_Float16*>(xl),
               const_cast<_Float16*>(sh), const_cast<_Float16*>(sl));
  }
  GroupArgs g{w, nullptr, n_in, n_out, xh, xl, sh, sl, m, nullptr, nullptr, nullptr, out, resid};
  g.ksplit = ks;
  g.partial = part;
  const int tiles = (m + kTok - 1) / kTok;
  KNJ_LAUNCH(k_group_q4k<false>, dim3((n_out + kRowsWG - 1) / kRowsWG, tiles, ks),
                     dim3(kBlock), kGroupLds, s, g);
  const bool fuse = ex.norm_w && ks > 1 && n_out <= 4096 && n_out % 256 == 0;
  if (fuse) {
    KNJ_LAUNCH(k_ksum_norm, dim3(m), dim3(kBlock), 0, s, part, ks, P * n_out, n_out, resid, out,
               ex.norm_w, ex.eps, ex.norm_out);
  } else if (ks > 1) {
    const uint64_t n = P * n_out;
    KNJ_LAUNCH(k_ksum, dim3((unsigned)((n / 4 + kBlock - 1) / kBlock)), dim3(kBlock), 0, s, part, ks,
               n, resid, out);
  }
  if (ex.norm_w && !fuse)
    KNJ_LAUNCH(k_norm_rows, dim3(m), dim3(kBlock), 0, s, out, ex.norm_w, ex.eps, n_out, ex.norm_out);
  return hipGetLastError();
}

hipError_t launch_dense_bf16(const uint16_t* w, int n_in, int n_out, int m, const float* x,
                             float* out, void* scratch, hipStream_t s) {
  if (n_in % 64) return hipErrorInvalidValue;
  const uint64_t P = (uint64_t)m;
  uint8_t* p = (uint8_t*)scratch;
  auto take = [&](uint64_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) & ~255ull;
    return q;
  };
  uint16_t* xh = (uint16_t*)take(P * n_in * 2);
  uint16_t* xm = (uint16_t*)take(P * n_in * 2);
  uint16_t* xl = (uint16_t*)take(P * n_in * 2);
  KNJ_LAUNCH(k_split_bf16x3, dim3(m), dim3(kBlock), 0, s, x, n_in, m, xh, xm, xl);
  KNJ_LAUNCH(k_dense_bf16, dim3((n_out + kRowsWG - 1) / kRowsWG, (m + kTok - 1) / kTok),
                     dim3(kBlock), 0, s, w, n_in, n_out, m, xh, xm, xl, out);
  return hipGetLastError();
}

hipError_t launch_dense_q6k(const uint8_t* w, int n_in, int n_out, int m, const float* x,
                            float* out, void* scratch, hipStream_t s) {
  if (hipError_t e = group_lds_attr()) return e;
  if (n_in > 4096 || n_in % 256 || n_out % 32 || m > 1024 || m <= 0) return hipErrorInvalidValue;
  const uint64_t P = (uint64_t)m;
  uint8_t* p = (uint8_t*)scratch;
  auto take = [&](uint64_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) & ~255ull;
    return q;
  };
  _Float16* xh = (_Float16*)take(P * n_in * 2);
  _Float16* xl = (_Float16*)take(P * n_in * 2);
  _Float16* sh = (_Float16*)take(P * n_in / 16);
  _Float16* sl = (_Float16*)take(P * n_in / 16);
  KNJ_LAUNCH(k_split_tile, dim3((m + 31) / 32, n_in / 64), dim3(kBlock), 0, s, x, nullptr,
             n_in, m, xh, xl, sh, sl);
  GroupArgs g{w, nullptr, n_in, n_out, xh, xl, sh, sl, m, nullptr, nullptr, nullptr, out, nullptr};
  KNJ_LAUNCH(k_group_q6k, dim3((n_out + kRowsWG - 1) / kRowsWG, (m + kTok - 1) / kTok),
             dim3(kBlock), kGroupLds, s, g);
  return hipGetLastError();
}

int argmax_key_count(int n) { return (n + kArgChunk - 1) / kArgChunk; }

hipError_t launch_argmax_rows(const float* logits, int m, int n, unsigned long long* keys,
                              int32_t* tok, hipStream_t s) {
  const int nk = argmax_key_count(n);
  KNJ_LAUNCH(k_argmax_part, dim3(nk, m), dim3(kBlock), 0, s, logits, n, keys);
  KNJ_LAUNCH(k_argmax_final, dim3(m), dim3(64), 0, s, keys, nk, tok);
  return hipGetLastError();
}

}  // namespace knj
