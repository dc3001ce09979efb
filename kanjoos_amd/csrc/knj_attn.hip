// kanjoos_amd/csrc/knj_attn.hip -- decode attention of one token over the f16 KV cache.
//
// Device side of the attention block of Model::forward
// (/root/reference/src/model/model.cpp:560-617): per-head RMSNorm of q and k
// (q_norm / k_norm), NEOX RoPE, append of k and v to the cache, then for every
// query head h (kv head h / group) scores q.k * 1/sqrt(D) over positions
// 0..pos, softmax, and sum a*v.
//
// Split-KV in two launches.  Workgroup (kv head, split) owns 64 cache slots:
// it normalises and rotates the `group` query heads itself, stages its K and V
// slots in LDS (the slot being written this step comes from registers, and
// only the workgroup that owns it writes it to the cache), and emits a partial
// record {max, sum, sum a*v} per query head.  A second launch merges each
// head's partials.
#include "knj_common.h"
#include "knj_dev.h"

namespace knj {
namespace {

using namespace dev;

constexpr int kChunk = 64;


// q/k normalisation + rotation of one head held as 4 floats per thread in a
// group of D/4 threads: returns the thread's 4 outputs (elements 4c..4c+3).
template <int D>
__device__ __forceinline__ float4 norm_rope4(float4 v, int c, float4 w, float eps, float4 cs,
                                             float4 sn) {
  constexpr int T = D / 4;  // threads per head
  float ss = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  ss = group_sum<T>(ss);
  const float scale = 1.0f / sqrtf(ss / (float)D + eps);
  float4 n;
  n.x = v.x * scale * w.x;
  n.y = v.y * scale * w.y;
  n.z = v.z * scale * w.z;
  n.w = v.w * scale * w.w;
  // partner: elements 4c +- D/2 live in thread c +- T/2
  static_assert(T == 16 || T == 32, "head_dim 64 or 128");
  auto partner = [](float x) {
    if constexpr (T == 32) return xor16_f(x);
    else return dev::dpp_f<dev::kDppRor8>(x);
  };
  float4 p;
  p.x = partner(n.x);
  p.y = partner(n.y);
  p.z = partner(n.z);
  p.w = partner(n.w);
  const bool lo = c < T / 2;
  // (x0, x1) -> (x0*c - x1*s, x0*s + x1*c) with x0 the low-half element
  float4 out;
  out.x = lo ? (n.x * cs.x - p.x * sn.x) : (p.x * sn.x + n.x * cs.x);
  out.y = lo ? (n.y * cs.y - p.y * sn.y) : (p.y * sn.y + n.y * cs.y);
  out.z = lo ? (n.z * cs.z - p.z * sn.z) : (p.z * sn.z + n.z * cs.z);
  out.w = lo ? (n.w * cs.w - p.w * sn.w) : (p.w * sn.w + n.w * cs.w);
  return out;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

// The 8-weight order of the grouped GEMMs' operands (knj_moe_batch.hip):
// position j of an 8-group holds element perm8_a(j) (bits 0 and 1 swapped).
__host__ __device__ constexpr int perm8_a(int j) { return (j & 4) | ((j & 1) << 1) | ((j & 2) >> 1); }

// One 16x16x32 f16 matrix-core step: acc[i] += sum_k A[4*(l/16)+i][k] B[k][l%16]
// where lane l supplies A[l%16][8*(l/16) + j] and B[8*(l/16) + j][l%16], j < 8.
__device__ __forceinline__ f32x4 mfma16(h16x8 a, h16x8 b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}

// f32 values as f16 high parts and f16 remainders (x = hi + lo to ~22 bits):
// against f16 cache values the two products are exact and summed in f32.
__device__ __forceinline__ void split_h8(const float4& p, const float4& q, h16x8& hi, h16x8& lo) {
  const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    hi[j] = (_Float16)v[j];
    lo[j] = (_Float16)(v[j] - (float)hi[j]);
  }
}


typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// 32-bit LDS address of a pointer into shared memory
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Four f16 of a transposed LDS read (ds_read_b64_tr_b16).  Within each group
// of 16 lanes, lane 4q + e receives element e of the 8-byte pieces addressed
// by lanes q, 4 + q, 8 + q and 12 + q, in that order: a 4 x 16 block of a
// row-major matrix read one piece per lane arrives as its columns.  Issued as
// asm: the compiler's wait placement treats the builtin as aliasing every
// LDS DMA in flight and would wait for the next chunk's DMA before it; the
// caller waits for the reads itself (lds_wait8) before using the values.
template <int OFF>
__device__ __forceinline__ u32x2 lds_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
// every LDS access of this wave complete; the eight values are tied to the
// wait so that no use moves above it
__device__ __forceinline__ void lds_wait8(u32x2* v) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
}
// LDS DMA of 16 bytes per lane (global_load_lds_dwordx4) by asm: lane l's
// 16 bytes from g land at LDS address base + 16 l (base wave-uniform).  The
// compiler's wait placement treats every LDS access after a DMA it knows of
// as aliasing it and waits for all of them; a kernel using this form waits
// for its DMA itself (vmcnt; in-order) before the barriers that hand the
// rows over, and the compiler's own counts only grow stricter by it.  M0 is
// reserved to the compiler, which sets it right before each of its own uses
// and keeps no value in it across this asm.
// A 16-byte global load by asm (for loads that precede an asm DMA: the
// caller waits for them with an explicit count, which the compiler's own
// count, blind to the DMA, would set too deep), and that wait.
__device__ __forceinline__ f32x4 ld16_asm(const void* g) {
  f32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(g) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void vm_wait7(f32x4& a, f32x4& b, f32x4& c, f32x4& d, f32x4& e, f32x4& f, f32x4& g) {
  asm volatile("s_waitcnt vmcnt(%7)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g) : "i"(N));
}
__device__ __forceinline__ float4 as_f4(f32x4 v) { return make_float4(v[0], v[1], v[2], v[3]); }

__device__ __forceinline__ void dma16(const void* g, uint32_t base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(base) : "memory");
}

__device__ __forceinline__ void lds_tie8(u32x2* v) {
  asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
}

// s_waitcnt immediates (gfx9 encoding): at most n vector memory operations
// of this wave outstanding and every LDS access complete; LDS only
constexpr int vm_lds_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }
constexpr int kLdsOnly = vm_lds_imm(63);
// Workgroup barrier after the wait `imm`.  __syncthreads() is a release fence
// plus the barrier and the fence waits for every LDS DMA in flight, which
// would drain the next chunk's fetch at every barrier of a chunk; the asm's
// memory clobber keeps the compiler from moving memory accesses across it.
#define KNJ_ATTN_BARRIER(imm)                 \
  do {                                        \
    __builtin_amdgcn_s_waitcnt(imm);          \
    __builtin_amdgcn_sched_barrier(0);        \
    asm volatile("s_barrier" ::: "memory");   \
    __builtin_amdgcn_sched_barrier(0);        \
  } while (0)

// Decode attention of one new token per sequence: workgroup (kv head, split
// of the KV range, sequence).  The G query heads of the kv head are
// normalised and rotated in LDS; per 64-slot chunk, the scores on the matrix
// cores (wave w: slots 16w .. 16w+15 against the heads), an online softmax
// per head (wave w: heads 2w, 2w+1, lane = slot), and the values on the
// matrix cores (wave w: dims 32w .. 32w+31).  K/V chunks reach LDS by DMA
// (dma16; 39 KB of LDS: four workgroups per CU), row-major with the 16-byte
// slots of a row XOR-permuted by the row index as in the prompt kernel; one
// stage, the next chunk's K fetched once the scores are written and its V
// once the value products are done; each barrier waits only for the rows it
// hands over (K at the chunk's start, V before the value products).  The
// step's key/value row is written to the cache after the loop (no fetch of
// this launch reads it); the workgroup holding it writes it into the staged
// chunk and zeroes the V rows past it (slots past the valid length under a
// weight of 0).  The query/key/value, norm and RoPE loads are issued before
// the first chunk's DMA (measured 1-3% faster per step than the chunk first).
template <int D>
__global__ __launch_bounds__(kBlock, 4) void k_attention(AttnArgs a, int cpw) {  // 4 waves per SIMD: 128 VGPRs
  constexpr int ROWH = D + 8;            // f16 elements per query LDS row (16-byte pad)
  constexpr int EROW = kChunk + 4;       // floats per score row
  constexpr int T = D / 4;               // threads per head for the q pass
  constexpr int RB = 2 * D, RPB = 256 / RB, NSLOT = RB / 16, NPAIR = RB / 32;
  constexpr int CB = kChunk * RB;        // bytes of one matrix's chunk
  constexpr int NI = CB / 1024 / (kBlock / 64);  // 1 KB DMA instructions per wave per matrix
  static_assert(NI >= 1 && CB % (1024 * (kBlock / 64)) == 0, "head_dim 64 or 128");
  auto kslot = [](int p, int sl) { return sl ^ ((p / RPB) & (NSLOT - 1)); };
  auto vslot = [](int p, int sl) { return sl ^ (((p / RPB) & (NPAIR - 1)) << 1); };
  __shared__ __align__(16) _Float16 qh[8 * ROWH];  // normalised, rotated queries: f16 high parts
  __shared__ __align__(16) _Float16 ql[8 * ROWH];  // and remainders
  __shared__ __align__(16) float es[8 * EROW];     // scores, then exp(score - running max), per head
  __shared__ float alpha[16];                      // per head: rescale of the running sums this chunk
  __shared__ __align__(16) uint8_t ks[CB];          // the chunk's K rows
  __shared__ __align__(16) uint8_t vs[CB];          // and V rows
  const int kvh = blockIdx.x, split = blockIdx.y, n_split = gridDim.y;
  const int G = a.n_head / a.n_head_kv;
  KNJ_STAMP(0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = split * cpw;            // first chunk of this workgroup
  const int z = blockIdx.z;  // sequence
  uint16_t* kc = a.k_cache + z * a.kv_stride + (uint64_t)kvh * a.n_ctx * D;
  uint16_t* vc = a.v_cache + z * a.kv_stride + (uint64_t)kvh * a.n_ctx * D;
  float* part = a.partial + (uint64_t)z * a.n_head * n_split * (D + 2) +
                ((uint64_t)(kvh * G) * n_split + split) * (D + 2);
  const float* qz = a.q + z * a.qkv_stride;
  const float* kz = a.k + z * a.qkv_stride;
  const float* vz = a.v + z * a.qkv_stride;
  const float* rc = a.rope_cos + (uint64_t)z * a.rope_stride;
  const float* rs = a.rope_sin + (uint64_t)z * a.rope_stride;
  const uint64_t hstride = (uint64_t)n_split * (D + 2);
  // wave w's DMA instruction i fills bytes (w NI + i) KB .. +1 KB of the
  // chunk's K and V (rows past the cache clamp to its last row)
  const uint8_t* kcb = reinterpret_cast<const uint8_t*>(kc);
  const uint8_t* vcb = reinterpret_cast<const uint8_t*>(vc);
  auto dma = [&](int p0, bool k, bool v) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int o0 = (wave * NI + i) * 1024, o = o0 + 16 * lane;
      const int p = o / RB, sl = (o % RB) / 16;
      const uint64_t row = (uint64_t)min(p0 + p, a.n_ctx - 1) * RB;
      if (k) dma16(kcb + row + 16 * kslot(p, sl), __builtin_amdgcn_readfirstlane(lds_addr(ks + o0)));
      if (v) dma16(vcb + row + 16 * vslot(p, sl), __builtin_amdgcn_readfirstlane(lds_addr(vs + o0)));
    }
  };
  // 1) every load that does not depend on the position first: the raw
  // query/key/value, the norm weights and the RoPE row, then the first
  // chunk's DMA
  // (asm loads: the wait below leaves the chunk's 2 NI DMA instructions,
  // issued after them, in flight while the queries are prepared)
  const int qhd = min(tid / T, G - 1), qc = tid % T;
  const int ri = (qc < T / 2) ? 4 * qc : 4 * qc - D / 2;  // rotation index of element 4qc
  f32x4 l_q = ld16_asm(qz + (uint64_t)(kvh * G + qhd) * D + 4 * qc);
  f32x4 l_qn = ld16_asm(a.q_norm + 4 * qc);
  f32x4 l_k = ld16_asm(kz + (uint64_t)kvh * D + 4 * qc);
  f32x4 l_v = ld16_asm(vz + (uint64_t)kvh * D + 4 * qc);
  f32x4 l_kn = ld16_asm(a.k_norm + 4 * qc);
  f32x4 l_cs = ld16_asm(rc + ri);
  f32x4 l_sn = ld16_asm(rs + ri);
  dma(c0 * kChunk, true, false);  // all of K, then all of V: the counter is in order
  dma(c0 * kChunk, false, true);
  // the position by a scalar load (asm: as a vector load, the compiler's wait
  // for it would also wait for the DMA issued before it)
  int pos;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(pos) : "s"(a.pos + z) : "memory");
  vm_wait7<2 * NI>(l_q, l_qn, l_k, l_v, l_kn, l_cs, l_sn);
  const float4 qraw = as_f4(l_q), qnw = as_f4(l_qn), kraw = as_f4(l_k), vraw = as_f4(l_v);
  const float4 knw = as_f4(l_kn), cs = as_f4(l_cs), sn = as_f4(l_sn);
  const int n_kv = pos + 1;
  const int nch = min(cpw, (n_kv - c0 * kChunk + kChunk - 1) / kChunk);  // chunks holding slots
  KNJ_STAMP(1);

  if (nch <= 0) {
    for (int i = tid; i < G * (D + 2); i += kBlock) {
      const int g = i / (D + 2), j = i % (D + 2);
      *(part + g * hstride + j) = (j == 0) ? -INFINITY : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the fetch lands before the workgroup ends
    return;
  }
  // 2) queries of this kv head: 4 floats per thread, T threads per head
  if (tid < G * T) {
    const float4 r = norm_rope4<D>(qraw, qc, qnw, a.eps, cs, sn);
    const float rv[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const _Float16 h = (_Float16)rv[i];
      qh[qhd * ROWH + 4 * qc + i] = h;
      ql[qhd * ROWH + 4 * qc + i] = (_Float16)(rv[i] - (float)h);
    }
  }
  // the key/value of this step as f16 (cache and staged chunk)
  uint2 kh2 = make_uint2(0u, 0u), vh2 = make_uint2(0u, 0u);
  if (tid < T) {
    const float4 r = norm_rope4<D>(kraw, tid, knw, a.eps, cs, sn);
    kh2 = make_uint2((uint32_t)f2h(r.x) | ((uint32_t)f2h(r.y) << 16), (uint32_t)f2h(r.z) | ((uint32_t)f2h(r.w) << 16));
    vh2 = make_uint2((uint32_t)f2h(vraw.x) | ((uint32_t)f2h(vraw.y) << 16),
                     (uint32_t)f2h(vraw.z) | ((uint32_t)f2h(vraw.w) << 16));
  }
  const int r = lane & 15, kq = lane >> 4;
  const bool hv = r < G;
  const int h0 = 2 * wave, h1 = 2 * wave + 1;
  // softmax in base 2: scores carry log2(e), so e^(s - m) = 2^(s log2 e - m log2 e);
  // the partial records' maxima are in these units (the merges use exp2)
  const float scale2 = a.scale * 1.4426950408889634f;
  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;  // running max / sum (softmax waves)
  f32x4 oe = {0.0f, 0.0f, 0.0f, 0.0f}, oo = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j = 0; j < nch; ++j) {
    const int p0 = (c0 + j) * kChunk;
    const int cnt = min(kChunk, n_kv - p0);
    // 3) chunk j's K has landed (its V, fetched after it, may still be in
    // flight); the barrier also hands the query rows over on the first pass
    KNJ_ATTN_BARRIER(vm_lds_imm(NI));
    KNJ_STAMP(2);
    const bool here = pos >= p0 && pos < p0 + kChunk;  // uniform
    const int lp = pos - p0;
    if (here) {
      // the step's key replaces the fetched row (fetched before this step's write)
      if (tid < T) *reinterpret_cast<uint2*>(ks + lp * RB + 16 * kslot(lp, tid >> 1) + 8 * (tid & 1)) = kh2;
      KNJ_ATTN_BARRIER(kLdsOnly);
    }
    KNJ_STAMP(3);
    // 4) scores on the matrix cores: wave w computes S[p][h] for the 16 slots
    // 16w..16w+15 (rows) and the query heads (columns, zero past G).  Lane
    // (r = l%16, kq = l/16) contributes dims 8kq .. 8kq+7 of each 32.
    {
      // A = K (16 slots x 32 dims per step), B = the queries (hi, then lo)
      const int p = 16 * wave + r;
      const uint8_t* krow = ks + p * RB;
      // (columns past G take head G - 1's queries: their scores, in
      // columns of their own, are never stored)
      const int hq = min(r, G - 1);
      f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        const h16x8 ka = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(krow + 16 * kslot(p, 4 * c + kq)));
        const h16x8 bh = *reinterpret_cast<const h16x8*>(qh + hq * ROWH + 32 * c + 8 * kq);
        const h16x8 bl = *reinterpret_cast<const h16x8*>(ql + hq * ROWH + 32 * c + 8 * kq);
        sa = mfma16(ka, bh, sa);
        sa = mfma16(ka, bl, sa);
      }
      if (hv) {
#pragma unroll
        for (int i = 0; i < 4; ++i) es[r * EROW + 16 * wave + 4 * kq + i] = sa[i] * scale2;
      }
    }
    KNJ_ATTN_BARRIER(kLdsOnly);
    // every wave's K reads are done: the next chunk's K
    if (j + 1 < nch) dma(p0 + kChunk, true, false);
    // 5) online softmax of the chunk: wave w owns heads 2w, 2w+1; lane = slot
    if (h0 < G) {
      const float s0 = lane < cnt ? es[h0 * EROW + lane] : -INFINITY;
      const float s1 = (lane < cnt && h1 < G) ? es[h1 * EROW + lane] : -INFINITY;
      const float n0 = fmaxf(m0, group_max<64>(s0)), n1 = fmaxf(m1, group_max<64>(s1));
      const float a0 = exp2f(m0 - n0), a1 = h1 < G ? exp2f(m1 - n1) : 0.0f;  // 2^-inf = 0 first
      const float e0 = lane < cnt ? exp2f(s0 - n0) : 0.0f;
      const float e1 = (lane < cnt && h1 < G) ? exp2f(s1 - n1) : 0.0f;
      l0 = l0 * a0 + group_sum<64>(e0);
      l1 = l1 * a1 + group_sum<64>(e1);
      m0 = n0;
      m1 = n1;
      // the weights replace the scores in the head's row (this wave's reads
      // of the row are done: one wave's LDS accesses complete in order) as
      // f16 high parts (halves 0..63) and remainders (64..127), slot
      // 32 c + 16 u + 4 q + i at half 32 c + 8 q + 4 u + i, so that the
      // value product's lane (q, row) reads its eight weights of step c
      // (slots 32 c + 4 q + i and 32 c + 16 + 4 q + i) as one 16-byte piece
      const int ps = (lane & 32) | ((lane & 12) << 1) | ((lane & 16) >> 2) | (lane & 3);
      _Float16* w0 = reinterpret_cast<_Float16*>(es + h0 * EROW);
      const _Float16 e0h = (_Float16)e0;
      w0[ps] = e0h;
      w0[64 + ps] = (_Float16)(e0 - (float)e0h);
      if (h1 < G) {
        _Float16* w1 = reinterpret_cast<_Float16*>(es + h1 * EROW);
        const _Float16 e1h = (_Float16)e1;
        w1[ps] = e1h;
        w1[64 + ps] = (_Float16)(e1 - (float)e1h);
      }
      if (lane == 0) {
        alpha[h0] = a0;
        if (h1 < G) alpha[h1] = a1;
      }
    }
    // chunk j's V has landed (the next chunk's K may stay in flight)
    if (j + 1 < nch) KNJ_ATTN_BARRIER(vm_lds_imm(NI));
    else KNJ_ATTN_BARRIER(vm_lds_imm(0));
    if (here) {
      // the step's value replaces the fetched row, and the rows past it
      // become zeros (finite under their weight of 0)
      if (tid < T) *reinterpret_cast<uint2*>(vs + lp * RB + 16 * vslot(lp, tid >> 1) + 8 * (tid & 1)) = vh2;
      for (int o = (lp + 1) * RB + 16 * tid; o < CB; o += 16 * kBlock)
        *reinterpret_cast<uint4*>(vs + o) = make_uint4(0u, 0u, 0u, 0u);
      KNJ_ATTN_BARRIER(kLdsOnly);
    }
    KNJ_STAMP(4);
    // 6) sum e*v on the matrix cores: O[h][d] over the 64 slots.  Wave w owns
    // dims 32w .. 32w+31 as two 16-column tiles; step c's 32 reduction
    // indices of lane (r, kq) are slots 32c + 4kq + i and 32c + 16 + 4kq + i
    // (i < 4): A = e (heads x slots, hi then lo), B = V (slots x 16 dims) by
    // transposed reads of rows 32c (+16) + 4kq + r/4, dims 4(r%4) .. +3 of
    // the tile, which deliver dim r of the four rows
    if (32 * wave < D) {
      // (rows past G read head G - 1's weights: their outputs, in rows of
      // their own, are never stored)
      const _Float16* erow = reinterpret_cast<const _Float16*>(es + min(r, G - 1) * EROW) + 8 * kq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * kq + i;
        const float al = h < G ? alpha[h] : 0.0f;
        oe[i] *= al;
        oo[i] *= al;
      }
      const int pa = 4 * kq + (r >> 2), sub = 8 * (r & 3);
      // rows pa + 32c and pa + 32c + 16 share the swizzle of row pa
      const uint32_t vrow = lds_addr(vs) + pa * RB + (sub & 15);
      const uint32_t ad0 = vrow + 16 * vslot(pa, (64 * wave + sub) >> 4);
      const uint32_t ad1 = vrow + 16 * vslot(pa, (64 * wave + 32 + sub) >> 4);
      u32x2 vv[8];
      vv[0] = lds_tr16<0>(ad0);
      vv[1] = lds_tr16<16 * RB>(ad0);
      vv[2] = lds_tr16<0>(ad1);
      vv[3] = lds_tr16<16 * RB>(ad1);
      vv[4] = lds_tr16<32 * RB>(ad0);
      vv[5] = lds_tr16<48 * RB>(ad0);
      vv[6] = lds_tr16<32 * RB>(ad1);
      vv[7] = lds_tr16<48 * RB>(ad1);
      lds_wait8(vv);
#pragma unroll
      for (int c = 0; c < kChunk / 32; ++c) {
        const h16x8 eh = *reinterpret_cast<const h16x8*>(erow + 32 * c);
        const h16x8 el = *reinterpret_cast<const h16x8*>(erow + 64 + 32 * c);
        const h16x8 v0 = __builtin_bit_cast(h16x8, make_uint4(vv[4 * c].x, vv[4 * c].y, vv[4 * c + 1].x, vv[4 * c + 1].y));
        const h16x8 v1 = __builtin_bit_cast(h16x8, make_uint4(vv[4 * c + 2].x, vv[4 * c + 2].y, vv[4 * c + 3].x, vv[4 * c + 3].y));
        oe = mfma16(eh, v0, oe);
        oe = mfma16(el, v0, oe);
        oo = mfma16(eh, v1, oo);
        oo = mfma16(el, v1, oo);
      }
    }
    // every wave is done with V and es: the next chunk's V
    KNJ_ATTN_BARRIER(kLdsOnly);
    if (j + 1 < nch) dma(p0 + kChunk, false, true);
  }
  // 7) the step's row to the cache, by the workgroup that holds it
  if (pos >= c0 * kChunk && pos < (c0 + nch) * kChunk && tid < T) {
    *reinterpret_cast<uint2*>(kc + (uint64_t)pos * D + 4 * tid) = kh2;
    *reinterpret_cast<uint2*>(vc + (uint64_t)pos * D + 4 * tid) = vh2;
  }
  // 8) the partial record {max, sum, sum e*v} of each head
  if (h0 < G && lane == 0) {
    *(part + h0 * hstride + 0) = m0;
    *(part + h0 * hstride + 1) = l0;
    if (h1 < G) {
      *(part + h1 * hstride + 0) = m1;
      *(part + h1 * hstride + 1) = l1;
    }
  }
  if (32 * wave < D) {
    const int d = 32 * wave + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kq + i;
      if (h < G) {
        part[h * hstride + 2 + d] = oe[i];
        part[h * hstride + 2 + d + 16] = oo[i];
      }
    }
  }
  KNJ_STAMP(5);
}

// Merge of the split partials of one query head over DW of its dims (one
// workgroup per (head, DW dims)): M = max m_s, f_s = exp(m_s - M),
// out = sum_s acc_s f_s / sum_s l_s f_s.  Every split's record is written on
// every call (splits past the position hold m = -inf, l = 0, acc = 0), so no
// load waits on the position.  Thread (dim j, part p) folds the splits of part
// p (kBlock / DW contiguous ranges, in order); every load of a thread is
// issued before the first use ({m, l} as one 8-byte load), and the parts are
// added in order.
template <int D, int PMAX, int DW>  // PMAX splits per part: n_split <= (kBlock / DW) PMAX
__global__ __launch_bounds__(kBlock) void k_attn_merge(AttnArgs a, int n_split) {
  constexpr int NP = kBlock / DW;  // parts
  __shared__ float pm[NP], pl[NP];
  __shared__ float pacc[NP][DW];
  // head = linear index mod n_head: workgroups are dispatched to the eight
  // XCDs in turn by linear index, so the D / DW workgroups of a head share
  // one XCD and its L2 fetches the head's split records once (head-major
  // order spread them over all eight: 4.5 MB fetched per launch for 1.1 MB of
  // records at 65 splits)
  const int h = blockIdx.x % a.n_head, d0 = DW * (blockIdx.x / a.n_head);
  const int z = blockIdx.y, tid = threadIdx.x, j = tid % DW, part = tid / DW;
  const float* ph = a.partial + ((uint64_t)z * a.n_head + h) * n_split * (D + 2);
  const int per = (n_split + NP - 1) / NP;
  const int s0 = part * per, s1 = min(n_split, s0 + per);
  float m[PMAX], l[PMAX], v[PMAX];
#pragma unroll
  for (int i = 0; i < PMAX; ++i) {
    const bool ok = s0 + i < s1;
    const float* rec = ph + (uint64_t)(ok ? s0 + i : 0) * (D + 2);
    const float2 ml = *reinterpret_cast<const float2*>(rec);  // records are 8-byte aligned
    m[i] = ok ? ml.x : -INFINITY;
    l[i] = ok ? ml.y : 0.0f;
    v[i] = ok ? rec[2 + d0 + j] : 0.0f;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PMAX; ++i) mx = fmaxf(mx, m[i]);
  if (j == 0) pm[part] = mx;
  __syncthreads();
  float M = pm[0];
#pragma unroll
  for (int q = 1; q < NP; ++q) M = fmaxf(M, pm[q]);
  float ls = 0.0f, acc = 0.0f;
#pragma unroll
  for (int i = 0; i < PMAX; ++i) {
    const float f = m[i] == -INFINITY ? 0.0f : exp2f(m[i] - M);
    ls += l[i] * f;
    acc += v[i] * f;
  }
  if (j == 0) pl[part] = ls;
  pacc[part][j] = acc;
  __syncthreads();
  if (tid < DW) {
    float L = pl[0], o = pacc[0][tid];
#pragma unroll
    for (int q = 1; q < NP; ++q) {
      L += pl[q];
      o += pacc[q][tid];
    }
    a.out[z * a.out_stride + (uint64_t)h * D + d0 + tid] = o / L;
  }
}

// Merge of the split partials of one query head (one workgroup per head),
// used for several sequences at once, where a workgroup per 32 dims would
// launch four times the workgroups for the same bytes:
// M = max m_s, f_s = exp(m_s - M), out = sum_s acc_s f_s / sum_s l_s f_s.
// Every split's record is written on every call (splits past the position
// hold m = -inf, l = 0, acc = 0), so no load here waits on the position.
// Threads [0, D), [D, 2D) .. each fold a contiguous range of splits in order
// (the first CH accumulator loads are issued before the max/sum pass); the
// ranges are added in split order.
template <int D>
__global__ __launch_bounds__(kBlock) void k_attn_merge_head(AttnArgs a, int n_split) {
  constexpr int NP = kBlock / D;  // 2 for D = 128, 4 for D = 64
  constexpr int CH = 16;
  __shared__ float fs[1024];
  __shared__ float red[8];
  __shared__ float parts[kBlock];
  const int h = blockIdx.x, tid = threadIdx.x, z = blockIdx.y;
  const float* ph = a.partial + ((uint64_t)z * a.n_head + h) * n_split * (D + 2);
  const int d = tid % D, pt = tid / D;
  const int per = (n_split + NP - 1) / NP;
  const int s0 = pt * per, s1 = min(n_split, s0 + per);
  float r[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) r[j] = s0 + j < s1 ? ph[(uint64_t)(s0 + j) * (D + 2) + 2 + d] : 0.0f;
  float m_own[4], l_own[4];
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s2 = tid + kBlock * j;
    m_own[j] = s2 < n_split ? ph[(uint64_t)s2 * (D + 2)] : -INFINITY;
    l_own[j] = s2 < n_split ? ph[(uint64_t)s2 * (D + 2) + 1] : 0.0f;
    M = fmaxf(M, m_own[j]);
  }
  M = group_max<64>(M);
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float lsum = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s2 = tid + kBlock * j;
    if (s2 < n_split) {
      const float f = m_own[j] == -INFINITY ? 0.0f : exp2f(m_own[j] - M);
      fs[s2] = f;
      lsum += l_own[j] * f;
    }
  }
  const float L = block_sum(lsum, red);  // includes the barrier that publishes fs
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < CH; ++j)
    if (s0 + j < s1) acc += r[j] * fs[s0 + j];
  for (int b = s0 + CH; b < s1; b += CH) {
#pragma unroll
    for (int j = 0; j < CH; ++j) r[j] = b + j < s1 ? ph[(uint64_t)(b + j) * (D + 2) + 2 + d] : 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j)
      if (b + j < s1) acc += r[j] * fs[b + j];
  }
  // fold the ranges in order: part 0 + part 1 (+ 2 + 3)
  parts[tid] = acc;
  __syncthreads();
  float res = 0.0f;
  if (tid < D) {
    float o = parts[tid];
    for (int q = 1; q < NP; ++q) o += parts[tid + q * D];
    res = o / L;
    a.out[z * a.out_stride + (uint64_t)h * D + tid] = res;
  }
  if (!a.split_hi) return;  // uniform
  // the row's D columns h D .. h D + D - 1 in k_split_tile's layout, with its
  // arithmetic: f16 high part and remainder, each 8-group in perm8 order; each
  // 32-column sum as eight sequential additions per 8-group, the four groups
  // added pairwise
  __syncthreads();  // parts[] is read above
  if (tid < D) fs[tid] = res;
  __syncthreads();
  const int P = a.n_seq, c0 = h * D;
  if (tid < D / 8) {
    const int g = tid, q = (c0 >> 3) + g;
    _Float16 hv[8], lv[8];
    float s8 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = fs[8 * g + perm8_a(j)];
      hv[j] = (_Float16)x;
      lv[j] = (_Float16)(x - (float)hv[j]);
      s8 += fs[8 * g + j];
    }
    const uint64_t o = ((uint64_t)q * P + z) * 8;
    *reinterpret_cast<uint4*>(a.split_hi + o) = *reinterpret_cast<const uint4*>(hv);
    *reinterpret_cast<uint4*>(a.split_lo + o) = *reinterpret_cast<const uint4*>(lv);
    parts[g] = s8;
  }
  __syncthreads();
  if (tid < D / 32) {
    const int b = (c0 >> 5) + tid;
    const float sum = (parts[4 * tid] + parts[4 * tid + 1]) + (parts[4 * tid + 2] + parts[4 * tid + 3]);
    const _Float16 sh = (_Float16)sum;
    const uint64_t o = ((uint64_t)(b >> 3) * P + z) * 8 + (b & 7);
    a.split_shi[o] = sh;
    a.split_slo[o] = (_Float16)(sum - (float)sh);
  }
}

// Prefill, step 1: row t = blockIdx.x at position pos0 + t.  Each group of
// D/4 threads holds one head (queries first, then keys): the query is
// normalised and rotated in place, the key normalised, rotated and written to
// the cache as f16, the value written as f16.  Same arithmetic as the decode
// kernel's (norm_rope4).
template <int D>
__global__ __launch_bounds__(kBlock) void k_prefill_rope_append(PrefillAttnArgs a) {
  constexpr int T = D / 4, HPB = kBlock / T;  // threads per head, heads per workgroup
  const int t = blockIdx.x, p = a.pos0 + t;
  const int nh = a.n_head + a.n_head_kv;
  const int hh = blockIdx.y * HPB + threadIdx.x / T, c = threadIdx.x % T;
  const int hc = min(hh, nh - 1);  // every lane computes; lanes past the heads store nothing
  const bool is_q = hc < a.n_head;
  float* row = a.qkv + (uint64_t)t * a.qkv_stride;
  float* src = row + (uint64_t)hc * D + 4 * c;  // q heads, then k heads, are contiguous
  const float4 raw = *reinterpret_cast<const float4*>(src);
  const float4 w = *reinterpret_cast<const float4*>((is_q ? a.q_norm : a.k_norm) + 4 * c);
  const int ri = (c < T / 2) ? 4 * c : 4 * c - D / 2;
  const float4 cs = *reinterpret_cast<const float4*>(a.rope_cos + (uint64_t)p * (D / 2) + ri);
  const float4 sn = *reinterpret_cast<const float4*>(a.rope_sin + (uint64_t)p * (D / 2) + ri);
  const float4 r = norm_rope4<D>(raw, c, w, a.eps, cs, sn);
  if (hh >= nh) return;
  if (is_q) {
    *reinterpret_cast<float4*>(src) = r;
    return;
  }
  const int kvh = hc - a.n_head;
  const uint64_t slot = ((uint64_t)kvh * a.n_ctx + p) * D + 4 * c;
  const float4 v = *reinterpret_cast<const float4*>(row + (uint64_t)(a.n_head + a.n_head_kv) * D +
                                                      (uint64_t)kvh * D + 4 * c);
  uint2 kk, vv;
  kk.x = (uint32_t)f2h(r.x) | ((uint32_t)f2h(r.y) << 16);
  kk.y = (uint32_t)f2h(r.z) | ((uint32_t)f2h(r.w) << 16);
  vv.x = (uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16);
  vv.y = (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16);
  *reinterpret_cast<uint2*>(a.k_cache + slot) = kk;
  *reinterpret_cast<uint2*>(a.v_cache + slot) = vv;
}

// Prefill, step 2: causal attention of a tile of prompt rows.  Workgroup
// (kv head, tile) takes 64 query columns, column = (row t0 + c / G, head
// kvh*G + c % G), so every K/V chunk staged in LDS serves 64 queries.  Wave w
// owns columns 16w .. 16w+15 for the whole pass, with its queries held in
// registers (f16 high parts and remainders) as the B operand:
//   scores   S[slot][col] = K (16 slots x 32 dims) x Q (32 dims x 16 cols),
//            lane (r = l%16, kq = l/16) ends with column r's scores of slots
//            16*st + 4*kq + i (st = slot tile, i < 4);
//   softmax  per column in registers: the column's 16 scores of the lane,
//            then the xor-16 and xor-32 partners (the other kq);
//   values   O^T[d][col] = V^T (16 dims x 32 slots) x E (32 slots x 16 cols).
//            A step's 32 reduction indices are the slots the lane already
//            holds (32c + 4kq + i and 32c + 16 + 4kq + i), so the softmax
//            weights feed the matrix cores without leaving the lane; the V^T
//            operand comes from V's row-major rows by transposed LDS reads.
// K/V chunks of 64 slots reach LDS by DMA (no registers, no staging
// arithmetic), row-major with the 16-byte slots of a row permuted by an XOR
// of the row index, so the operand reads of 16 (K) or 8 (V) rows fall on
// distinct banks; two stages, the next chunk's DMA in flight while the
// current one is computed, one barrier per chunk.  Slots past the tile's last
// position are fetched from that last position (finite values under a weight
// of 0).  Online softmax over the chunks as in the decode kernel, in base 2
// (the scores scaled by log2 e, the exponentials 2^x on the hardware's exp2);
// slot s counts for the row at position qp when s <= qp.  Grid z splits the KV
// range: split z walks chunks [z cps, (z + 1) cps) and, when there are
// several, leaves a partial record per column for k_prefill_merge.
template <int D>
__global__ __launch_bounds__(kBlock) void k_prefill_attn(PrefillAttnArgs a, int cps) {
  constexpr int NT = kBlock, NC = 64;  // query columns: 16 per wave
  constexpr int RB = 2 * D;            // bytes of one K or V row
  constexpr int RPB = 256 / RB;        // rows per 256 bytes (the 64 banks)
  constexpr int NSLOT = RB / 16, NPAIR = RB / 32;
  constexpr int CB = kChunk * RB;      // bytes of one matrix's chunk
  constexpr int NI = CB / 1024 / (NT / 64);  // 1 KB DMA instructions per wave per matrix
  static_assert(NI >= 1 && CB % (1024 * (NT / 64)) == 0, "head_dim 64 or 128");
  // K: 16-byte slot s of row p at s ^ (p / RPB mod NSLOT); V: 32-byte pair at
  // pair ^ (p / RPB mod NPAIR).  Both are involutions.
  auto kslot = [](int p, int sl) { return sl ^ ((p / RPB) & (NSLOT - 1)); };
  auto vslot = [](int p, int sl) { return sl ^ (((p / RPB) & (NPAIR - 1)) << 1); };
  __shared__ __align__(16) uint8_t kvs[2][2][CB];  // [stage][K, V][chunk]
  const int kvh = blockIdx.x;
  const int G = a.n_head / a.n_head_kv, QT = NC / G;
  const int t0 = blockIdx.y * QT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int col = 16 * wave + r, g = col % G;
  const bool live = t0 + col / G < a.n_rows;
  const int t = min(t0 + col / G, a.n_rows - 1);
  const int qp = a.pos0 + t;
  const int n_kv = a.pos0 + min(t0 + QT, a.n_rows);  // slots any row of the tile sees
  // split z of gridDim.z walks chunks [c0, c1) of the tile's range
  const int c0 = blockIdx.z * cps;
  const int c1 = min((n_kv + kChunk - 1) / kChunk, c0 + cps);
  const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.k_cache + (uint64_t)kvh * a.n_ctx * D);
  const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.v_cache + (uint64_t)kvh * a.n_ctx * D);
  // wave w's DMA instruction i fills bytes (w NI + i) KB .. +1 KB of the
  // chunk's K and V, lane l the 16 bytes at 16 l: slot sl of row p there
  // holds the row's logical slot kslot(p, sl) (K) or vslot(p, sl) (V)
  auto dma = [&](int p0, int st) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int o0 = (wave * NI + i) * 1024, o = o0 + 16 * lane;
      const int p = o / RB, sl = (o % RB) / 16;
      const uint64_t row = (uint64_t)min(p0 + p, n_kv - 1) * RB;
      __builtin_amdgcn_global_load_lds((glb_void*)(kc + row + 16 * kslot(p, sl)), (lds_void*)(&kvs[st][0][o0]), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((glb_void*)(vc + row + 16 * vslot(p, sl)), (lds_void*)(&kvs[st][1][o0]), 16, 0, 0);
    }
  };
  if (c0 < c1) dma(c0 * kChunk, 0);
  // this lane's query column: dims 32c + 8kq .. +7 of every 32-dim step
  h16x8 qhi[D / 32], qlo[D / 32];
  const float* qrow = a.qkv + (uint64_t)t * a.qkv_stride + (uint64_t)(kvh * G + g) * D;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    const float4 x0 = *reinterpret_cast<const float4*>(qrow + 32 * c + 8 * kq);
    const float4 x1 = *reinterpret_cast<const float4*>(qrow + 32 * c + 8 * kq + 4);
    split_h8(x0, x1, qhi[c], qlo[c]);
  }
  // softmax in base 2: scores carry log2(e), e^(s - m) = 2^(s log2 e - m log2 e)
  const float scale2 = a.scale * 1.4426950408889634f;
  float mrun = -INFINITY, lrun = 0.0f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int j = c0; j < c1; ++j) {
    const int p0 = j * kChunk, st = (j - c0) & 1;
    // this wave's DMA of chunk j has landed (the only loads outstanding);
    // the barrier hands every wave's part over and also ends every wave's
    // reads of the other stage, which the next chunk's DMA then refills
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (j + 1 < c1) dma(p0 + kChunk, st ^ 1);
    const uint8_t* ks = kvs[st][0];
    const uint8_t* vs = kvs[st][1];
    // scores of this lane's column over the chunk's 64 slots
    f32x4 sc[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f};
      const int p = 16 * s4 + r;
      const uint8_t* krow = ks + p * RB;
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        const h16x8 ka = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(krow + 16 * kslot(p, 4 * c + kq)));
        sa = mfma16(ka, qhi[c], sa);
        sa = mfma16(ka, qlo[c], sa);
      }
      sc[s4] = sa;
    }
    // the causal mask only where the chunk reaches past the tile's first row
    // (uniform); the exponentials on the hardware's exp2 (results below
    // 2^-126, which the library routine would keep as denormals, weigh
    // nothing against a running sum of at least 1)
    float cmax = -INFINITY;
    const bool masked = p0 + kChunk - 1 > a.pos0 + t0;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ps = p0 + 16 * s4 + 4 * kq + i;
        const float v = (!masked || ps <= qp) ? sc[s4][i] * scale2 : -INFINITY;
        sc[s4][i] = v;
        cmax = fmaxf(cmax, v);
      }
    }
    cmax = fmaxf(cmax, xor16_f(cmax));
    cmax = fmaxf(cmax, xor32_f(cmax));
    // -inf while every slot so far is past the row's position (a split that
    // starts after it); the exponents then use 0 so that no -inf - -inf occurs
    const float mnew = fmaxf(mrun, cmax);
    const float mref = mnew == -INFINITY ? 0.0f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(mrun - mref);
    float esum = 0.0f;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(sc[s4][i] - mref);  // 2^-inf = 0 past the row's position
        sc[s4][i] = e;
        esum += e;
      }
    }
    esum += xor16_f(esum);
    esum += xor32_f(esum);
    lrun = lrun * alpha + esum;
    mrun = mnew;
    // the rescale multiplies by exactly 1 when no column of the wave found a
    // larger score: skipped then
    if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[dt][i] *= alpha;
      }
    }
    // values: step c covers slots 32c + 4kq + i (i < 4) and 32c + 16 + 4kq + i;
    // lane r's transposed read takes row 32c (+16) + 4kq + r/4, dims
    // 16dt + 4(r%4) .. +3, and receives dim 16dt + r of the four rows
    const int pa = 4 * kq + (r >> 2), sub = 8 * (r & 3);  // row in the 16-slot step, byte in 32-dim block
    // rows pa + 32c and pa + 32c + 16 share the swizzle of row pa
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float4 ea = make_float4(sc[2 * c][0], sc[2 * c][1], sc[2 * c][2], sc[2 * c][3]);
      const float4 eb = make_float4(sc[2 * c + 1][0], sc[2 * c + 1][1], sc[2 * c + 1][2], sc[2 * c + 1][3]);
      h16x8 eh, el;
      split_h8(ea, eb, eh, el);
      const uint32_t vrow = lds_addr(vs) + (32 * c + pa) * RB + (sub & 15);
      u32x2 va[8], vb[8];
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const uint32_t ad = vrow + 16 * vslot(pa, (32 * dt + sub) >> 4);
        va[dt] = lds_tr16<0>(ad);
        vb[dt] = lds_tr16<16 * RB>(ad);
      }
      lds_wait8(va);
      lds_tie8(vb);
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const h16x8 vv = __builtin_bit_cast(h16x8, make_uint4(va[dt].x, va[dt].y, vb[dt].x, vb[dt].y));
        acc[dt] = mfma16(vv, eh, acc[dt]);
        acc[dt] = mfma16(vv, el, acc[dt]);
      }
    }
  }
  if (gridDim.z > 1) {
    // partial record {max, sum, sum e*v} of this column for the merge (a
    // split past the tile's range leaves max = -inf, sum = 0, acc = 0)
    float* rec = a.partial + ((((uint64_t)blockIdx.y * gridDim.x + kvh) * gridDim.z + blockIdx.z) * NC + col) * (D + 2);
    if (kq == 0) {
      rec[0] = mrun;
      rec[1] = lrun;
    }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      *reinterpret_cast<float4*>(rec + 2 + 16 * dt + 4 * kq) = make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
    return;
  }
  if (!live) return;
  const float inv = 1.0f / lrun;
  float* orow = a.out + (uint64_t)t * a.n_head * D + (uint64_t)(kvh * G + g) * D;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    *reinterpret_cast<float4*>(orow + 16 * dt + 4 * kq) =
        make_float4(acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv);
  }
}

// Merge of the split partials: thread = one (row, head, dim) output,
// M = max_s m_s, out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), the
// splits folded in order in one pass (running maximum, rescaled sums).  The
// maxima are in the base-2 units of k_prefill_attn.
template <int D>
__global__ __launch_bounds__(kBlock) void k_prefill_merge(PrefillAttnArgs a, int n_split) {
  constexpr int NC = 64;
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const int HD = a.n_head * D;
  if (i >= (uint64_t)a.n_rows * HD) return;
  const int t = (int)(i / HD), hd = (int)(i - (uint64_t)t * HD);
  const int h = hd / D, d = hd - h * D;
  const int G = a.n_head / a.n_head_kv, QT = NC / G;
  const int tile = t / QT, kvh = h / G, col = (t - tile * QT) * G + h % G;
  const uint64_t stride = (uint64_t)NC * (D + 2);
  const float* rec = a.partial + (((uint64_t)tile * a.n_head_kv + kvh) * n_split * NC + col) * (D + 2);
  float M = -INFINITY, L = 0.0f, o = 0.0f;
  for (int sp = 0; sp < n_split; ++sp) {
    const float m = rec[sp * stride], l = rec[sp * stride + 1], v = rec[sp * stride + 2 + d];
    const float Mn = fmaxf(M, m);
    const float ref = Mn == -INFINITY ? 0.0f : Mn;
    const float fo = exp2f(M - ref), fn = exp2f(m - ref);
    L = L * fo + l * fn;
    o = o * fo + v * fn;
    M = Mn;
  }
  a.out[i] = o / L;
}

}  // namespace

int attn_splits(int n_ctx) { return (n_ctx + kChunk - 1) / kChunk; }

// splits of one head: one 64-slot chunk per workgroup up to kMaxSplit1
// chunks at one sequence, several chunks per workgroup beyond (measured at
// 32,770 slots, 513 chunks: 103 splits of 5 chunks 2.47 ms/token, 129 of 4
// and 171 of 3 2.48, 86 of 6 and 73 of 7-8 2.52, 257 of 2 and an even 256-way
// partition 2.55), up to kMaxSplit with several sequences (the per-head merge)
constexpr int kMaxSplit = 256, kMaxSplit1 = 103;

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
  // one 64-slot chunk per workgroup up to kMaxSplit chunks; beyond, several
  // chunks per workgroup so the merge sees at most kMaxSplit partials per head
  const int chunks = attn_splits(a.n_ctx);
  // several sequences fill the chip with their own splits: at least three
  // chunks per workgroup there (measured at 32 sequences x 2048 slots: 8.55
  // ms/step with two, 8.42 with three, 8.59 with four; one chunk is faster at
  // batch 1)
  const int max_split = a.n_seq > 1 ? kMaxSplit : kMaxSplit1;
  const int cpw = std::max((chunks + max_split - 1) / max_split, a.n_seq > 1 ? 3 : 1);
  const int n_split = (chunks + cpw - 1) / cpw;
  if (n_split > max_split) return hipErrorInvalidValue;
  const int z = std::max(1, a.n_seq);
  if (a.head_dim == 128) {
    KNJ_LAUNCH(k_attention<128>, dim3(a.n_head_kv, n_split, z), dim3(kBlock), 0, s, a, cpw);
    // up to 128 splits: 16 dims per workgroup, 16 parts of at most 8 splits
    // (the loads a part holds cost at short contexts)
    if (z == 1 && !a.split_hi && n_split <= 128)
      KNJ_LAUNCH((k_attn_merge<128, 8, 16>), dim3(a.n_head * 8, z), dim3(kBlock), 0, s, a, n_split);
    else if (z == 1 && !a.split_hi && n_split <= 256)
      KNJ_LAUNCH((k_attn_merge<128, 32, 32>), dim3(a.n_head * 4, z), dim3(kBlock), 0, s, a, n_split);
    else
      KNJ_LAUNCH(k_attn_merge_head<128>, dim3(a.n_head, z), dim3(kBlock), 0, s, a, n_split);
  } else if (a.head_dim == 64) {
    KNJ_LAUNCH(k_attention<64>, dim3(a.n_head_kv, n_split, z), dim3(kBlock), 0, s, a, cpw);
    if (z == 1 && !a.split_hi && n_split <= 128)
      KNJ_LAUNCH((k_attn_merge<64, 16, 32>), dim3(a.n_head * 2, z), dim3(kBlock), 0, s, a, n_split);
    else if (z == 1 && !a.split_hi && n_split <= 256)
      KNJ_LAUNCH((k_attn_merge<64, 32, 32>), dim3(a.n_head * 2, z), dim3(kBlock), 0, s, a, n_split);
    else
      KNJ_LAUNCH(k_attn_merge_head<64>, dim3(a.n_head, z), dim3(kBlock), 0, s, a, n_split);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

constexpr int kPrefillWGs = 1024;  // split-KV target for the prompt-pass attention

bool prefill_attention_ok(int n_head, int n_head_kv, int head_dim) {
  if (n_head_kv <= 0 || n_head % n_head_kv) return false;
  const int G = n_head / n_head_kv;
  return (head_dim == 128 || head_dim == 64) && G <= 64 && 64 % G == 0;
}

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t s) {
  if (!prefill_attention_ok(a.n_head, a.n_head_kv, a.head_dim) || a.n_rows <= 0 || a.pos0 < 0 ||
      a.pos0 + a.n_rows > a.n_ctx)
    return hipErrorInvalidValue;
  const int G = a.n_head / a.n_head_kv;
  const int nh = a.n_head + a.n_head_kv;
  const int QT = 64 / G;
  const int n_tiles = (a.n_rows + QT - 1) / QT;
  // split the KV range when the tiles alone leave the chip short of work and
  // the range is long: at most kPrefillWGs workgroups, at least 8 chunks each
  const int nch = (a.pos0 + a.n_rows + kChunk - 1) / kChunk;
  const int base = a.n_head_kv * n_tiles;
  int n_split = 1;
  if (nch >= 16 && base < kPrefillWGs) n_split = std::min(nch / 8, kPrefillWGs / base);
  if (n_split > 1 &&
      (!a.partial ||
       (uint64_t)base * n_split * 64 * (a.head_dim + 2) * sizeof(float) > a.partial_bytes))
    return hipErrorInvalidValue;
  const int cps = (nch + n_split - 1) / n_split;
  n_split = (nch + cps - 1) / cps;
  const dim3 grid(a.n_head_kv, n_tiles, n_split);
  const dim3 mgrid((unsigned)(((uint64_t)a.n_rows * a.n_head * a.head_dim + kBlock - 1) / kBlock));
#define KNJ_PREFILL(DD, HPB)                                                                      \
  KNJ_LAUNCH(k_prefill_rope_append<DD>, dim3(a.n_rows, (nh + (HPB) - 1) / (HPB)), dim3(kBlock), 0, s, a); \
  KNJ_LAUNCH(k_prefill_attn<DD>, grid, dim3(kBlock), 0, s, a, cps);                                \
  if (n_split > 1) KNJ_LAUNCH(k_prefill_merge<DD>, mgrid, dim3(kBlock), 0, s, a, n_split);
  if (a.head_dim == 128) {
    KNJ_PREFILL(128, kBlock / 32)
  } else {
    KNJ_PREFILL(64, kBlock / 16)
  }
#undef KNJ_PREFILL
  return hipGetLastError();
}

uint64_t prefill_partial_bytes(int n_head, int n_head_kv, int head_dim, int max_rows) {
  if (!prefill_attention_ok(n_head, n_head_kv, head_dim)) return 0;
  // n_split <= kPrefillWGs / tiles when it is above 1
  const int QT = 64 / (n_head / n_head_kv);
  const uint64_t base = (uint64_t)n_head_kv * ((max_rows + QT - 1) / QT);
  const uint64_t wgs = std::max<uint64_t>(base, kPrefillWGs);
  return wgs * 64 * (head_dim + 2) * 4;
}

}  // namespace knj
