// kanjoos_amd/csrc/knj_dev.h -- device-side helpers shared by the gfx950 kernels.
//
// Conventions: workgroups of 256 threads (4 wave64s); weights are read with
// 16-byte loads issued before anything that waits on activations, so their HBM
// latency overlaps the activation staging; activations that every lane of a
// row needs are kept in registers ("x slice") and reused across the rows a
// wave processes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/knj_format.h"

// Phase timestamps of workgroup 0 (thread 0) for timing builds that define
// KNJ_STAMPS; compiled out otherwise.
#ifdef KNJ_STAMPS
__device__ unsigned long long g_knj_stamps[64];
#define KNJ_STAMP(i)                                                                 \
  do {                                                                               \
    if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0)                      \
      g_knj_stamps[i] = __builtin_amdgcn_s_memrealtime();                            \
  } while (0)
// per-workgroup start/end times (slot 0/1) of up to 4096 workgroups
__device__ unsigned long long g_knj_wg[2][4096];
#define KNJ_WG_STAMP(slot)                                                           \
  do {                                                                               \
    if (threadIdx.x == 0 && blockIdx.x < 4096)                                       \
      g_knj_wg[slot][blockIdx.x] = __builtin_amdgcn_s_memrealtime();                 \
  } while (0)
#else
#define KNJ_STAMP(i) \
  do {               \
  } while (0)
#define KNJ_WG_STAMP(slot) \
  do {                     \
  } while (0)
#endif

namespace knj {
namespace dev {

constexpr int kBlock = 256;

// s_waitcnt immediate that waits for this wave's LDS accesses only (gfx9
// encoding: vmcnt 63, expcnt 7, lgkmcnt 0): a barrier after it hands over LDS
// writes while vector memory loads stay in flight.
constexpr int kWaitLdsOnly = 0xC07F;

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits16 & 0xFFFFu));
}

__device__ __forceinline__ uint16_t f2h(float v) {
  // v_cvt_f16_f32, round-to-nearest-even (knj_f32_to_f16 semantics)
  return __builtin_bit_cast(unsigned short, (_Float16)v);
}

// ---- cross-lane moves without the LDS crossbar.  Rows of 16 lanes exchange
// through DPP (quad permutes, the 8- and 16-lane mirrors, row rotation); rows
// and half-waves through the gfx950 permlane swaps.  Every lane of the group
// taking part must be active.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <- 15 - i within 16
constexpr int kDppRor8 = 0x128;       // lane i <- (i + 8) % 16 within 16, i.e. i ^ 8

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}

// the value of lane l ^ 16
__device__ __forceinline__ uint32_t xor16_u32(uint32_t v) {
  // odd rows of the first result hold the even rows of v, even rows of the
  // second result the odd rows
  const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (__lane_id() & 16) ? p[0] : p[1];
}

// the value of lane l ^ 32
__device__ __forceinline__ uint32_t xor32_u32(uint32_t v) {
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (__lane_id() & 32) ? p[0] : p[1];
}

__device__ __forceinline__ float xor16_f(float v) { return __uint_as_float(xor16_u32(__float_as_uint(v))); }
__device__ __forceinline__ float xor32_f(float v) { return __uint_as_float(xor32_u32(__float_as_uint(v))); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v))); }

// Reduction over aligned groups of W lanes (W a power of two <= 64) as a
// butterfly: partners are combined in both orders only by commutative ops, so
// every lane of a group returns the same bits.
template <int W, class Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group of 1..64 lanes");
  if constexpr (W >= 2) v = op(v, dpp_f<kDppXor1>(v));
  if constexpr (W >= 4) v = op(v, dpp_f<kDppXor2>(v));
  if constexpr (W >= 8) v = op(v, dpp_f<kDppHalfMirror>(v));
  if constexpr (W >= 16) v = op(v, dpp_f<kDppMirror>(v));
  if constexpr (W >= 32) v = op(v, xor16_f(v));
  if constexpr (W >= 64) v = op(v, xor32_f(v));
  return v;
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
  return group_reduce<W>(v, [](float a, float b) { return a + b; });
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
  return group_reduce<W>(v, [](float a, float b) { return fmaxf(a, b); });
}

// Maximum of an unsigned 32-bit value over the wave; every lane returns it.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppMirror>(v));
  v = max(v, xor16_u32(v));
  v = max(v, xor32_u32(v));
  return v;
}

// Maximum of a 64-bit key over the wave; every lane returns it.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  auto step = [&](uint32_t lo, uint32_t hi) {
    const unsigned long long t = ((unsigned long long)hi << 32) | lo;
    v = t > v ? t : v;
  };
  step(dpp_u32<kDppXor1>((uint32_t)v), dpp_u32<kDppXor1>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppXor2>((uint32_t)v), dpp_u32<kDppXor2>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppHalfMirror>((uint32_t)v), dpp_u32<kDppHalfMirror>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppMirror>((uint32_t)v), dpp_u32<kDppMirror>((uint32_t)(v >> 32)));
  step(xor16_u32((uint32_t)v), xor16_u32((uint32_t)(v >> 32)));
  step(xor32_u32((uint32_t)v), xor32_u32((uint32_t)(v >> 32)));
  return v;
}

// The value of lane `src` (the same for the whole wave) in every lane.
__device__ __forceinline__ float lane_bcast(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ int lane_bcast(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// Sum over a workgroup of kBlock threads: wave trees, then the waves in order.
// Every thread returns the same value.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = group_sum<64>(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock / 64; ++i) t += red[i];
  __syncthreads();
  return t;
}

__device__ __forceinline__ float ld_acquire_f(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-workgroup hand-off inside one launch without a device-wide fence.
// A device-scope fence writes back the whole L2 and serialises across the
// chip (measured ~60 ns per workgroup on gfx950), so producers instead store
// the values other workgroups will read with agent-scope atomic stores (they
// bypass the non-coherent L2 of the producer's XCD), wait for their own
// stores to complete, and take a ticket; the last workgroup reads the values
// with agent-scope atomic loads.
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exactly one workgroup (the last to arrive) gets true; it then sees every
// other workgroup's published values.  The counter is returned to zero.
__device__ __forceinline__ bool last_block_done(unsigned int* counter, unsigned int nblocks,
                                                unsigned int* flag_lds) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's published stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int t = atomicAdd(counter, 1u);
    const bool last = (t == nblocks - 1);
    if (last) atomicExch(counter, 0u);
    *flag_lds = last ? 1u : 0u;
  }
  __syncthreads();
  return *flag_lds != 0u;
}

// Padded LDS layout of an activation vector: 16 bytes of padding after every 64
// floats, so the 64-float slices that consecutive lanes read with ds_read_b128
// start on different banks.
__device__ __forceinline__ int xpad(int i) { return i + ((i >> 6) << 2); }
constexpr int xpad_size(int n) { return n + (n >> 6) * 4; }

// Stage x (n <= 4096 floats) into padded LDS, optionally RMS-normalised:
// xs = x * (1/sqrt(sum(x^2)/n + eps)) * w.  All threads take part.  Split in
// two so a kernel can issue the loads (x and the norm weight together) early
// and do the reduction and LDS stores later.
struct XRegs {
  float4 v[4], w[4];
};

__device__ __forceinline__ void stage_x_load(const float* __restrict__ x,
                                             const float* __restrict__ nw, int n, XRegs& r) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * threadIdx.x + 1024 * j;
    if (i < n) {
      r.v[j] = *reinterpret_cast<const float4*>(x + i);
      if (nw) r.w[j] = *reinterpret_cast<const float4*>(nw + i);
    }
  }
}

__device__ __forceinline__ void stage_x_store(const XRegs& r, bool norm, float eps, int n,
                                              float* xs, float* red, float* xsum = nullptr) {
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * threadIdx.x + 1024 * j;
    if (i < n) ss += r.v[j].x * r.v[j].x + r.v[j].y * r.v[j].y + r.v[j].z * r.v[j].z + r.v[j].w * r.v[j].w;
  }
  float scale = 1.0f;
  if (norm) {
    ss = block_sum(ss, red);
    scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * threadIdx.x + 1024 * j;
    if (i < n) {
      float4 o = r.v[j];
      if (norm) {
        o.x = r.v[j].x * scale * r.w[j].x;
        o.y = r.v[j].y * scale * r.w[j].y;
        o.z = r.v[j].z * scale * r.w[j].z;
        o.w = r.v[j].w * scale * r.w[j].w;
      }
      *reinterpret_cast<float4*>(xs + xpad(i)) = o;
      if (xsum) {  // sums of the 32-element sub-blocks: eight consecutive threads hold one
        const float t = group_sum<8>((o.x + o.y) + (o.z + o.w));
        if ((threadIdx.x & 7) == 0) xsum[i >> 5] = t;
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void stage_x(const float* __restrict__ x,
                                        const float* __restrict__ nw, float eps, int n, float* xs,
                                        float* red) {
  XRegs r;
  stage_x_load(x, nw, n, r);
  stage_x_store(r, nw != nullptr, eps, n, xs, red);
}

// ---------------------------------------------------------------- Q4_K slices
// A slice is one 32-byte code group g of a super-block: sub-blocks 2g (low
// nibbles) and 2g+1 (high nibbles), 64 weights, plus the block header.
struct Q4Slice {
  uint4 h, a, b;
};

__device__ __forceinline__ Q4Slice q4k_load(const uint8_t* __restrict__ blk, int g) {
  Q4Slice s;
  s.h = *reinterpret_cast<const uint4*>(blk);
  s.a = *reinterpret_cast<const uint4*>(blk + KNJ_Q4K_QS + 32 * g);
  s.b = *reinterpret_cast<const uint4*>(blk + KNJ_Q4K_QS + 32 * g + 16);
  return s;
}

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

// All eight 6-bit scales and mins of a Q4_K super-block at once, one byte
// each: s[0] = sc0..3, s[1] = sc4..7, m[0] = m0..3, m[1] = m4..7 (the same
// values as q4k_scale_min for s = 0..7, byte-parallel).
struct Q4Scales8 {
  uint32_t s[2], m[2];
};
__device__ __forceinline__ Q4Scales8 q4k_scales8(uint32_t w1, uint32_t w2, uint32_t w3) {
  Q4Scales8 r;
  r.s[0] = w1 & 0x3F3F3F3Fu;
  r.m[0] = w2 & 0x3F3F3F3Fu;
  r.s[1] = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
  r.m[1] = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
  return r;
}

// The 64 activations of a slice, in registers, with the two sub-block sums.
struct XSlice {
  float v[64];
  float s0, s1;
};

__device__ __forceinline__ void xslice_load(const float* xs_pad, int slice, XSlice& x) {
  const float* p = xs_pad + 68 * slice;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(p + 4 * k);
    x.v[4 * k] = t.x;
    x.v[4 * k + 1] = t.y;
    x.v[4 * k + 2] = t.z;
    x.v[4 * k + 3] = t.w;
  }
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    a += x.v[l];
    b += x.v[32 + l];
  }
  x.s0 = a;
  x.s1 = b;
}

// The same with the two sub-block sums already known.
__device__ __forceinline__ void xslice_load_sums(const float* xs_pad, int slice, float s0, float s1,
                                                 XSlice& x) {
  const float* p = xs_pad + 68 * slice;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(p + 4 * k);
    x.v[4 * k] = t.x;
    x.v[4 * k + 1] = t.y;
    x.v[4 * k + 2] = t.z;
    x.v[4 * k + 3] = t.w;
  }
  x.s0 = s0;
  x.s1 = s1;
}

// Byte n of a word as f32: one v_cvt_f32_ubyteN each (the compiler otherwise
// extracts each nibble with a bit-field extract first).
__device__ __forceinline__ float ub0(uint32_t v) { float r; asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ub1(uint32_t v) { float r; asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ub2(uint32_t v) { float r; asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ub3(uint32_t v) { float r; asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v)); return r; }
// byte n (a constant) of a word as f32
__device__ __forceinline__ float ubn(uint32_t v, int n) {
  return n == 0 ? ub0(v) : n == 1 ? ub1(v) : n == 2 ? ub2(v) : ub3(v);
}

// 16 code bytes: low nibbles against xlo (sub-block 2g), high nibbles against
// xhi (sub-block 2g+1), each summed in element order.
__device__ __forceinline__ void q4k_codes16(uint4 q, const float* xlo, const float* xhi, float& slo,
                                            float& shi) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = w[k] & 0x0F0F0F0Fu;
    const uint32_t hi = (w[k] >> 4) & 0x0F0F0F0Fu;
    slo += ub0(lo) * xlo[4 * k];
    slo += ub1(lo) * xlo[4 * k + 1];
    slo += ub2(lo) * xlo[4 * k + 2];
    slo += ub3(lo) * xlo[4 * k + 3];
    shi += ub0(hi) * xhi[4 * k];
    shi += ub1(hi) * xhi[4 * k + 1];
    shi += ub2(hi) * xhi[4 * k + 2];
    shi += ub3(hi) * xhi[4 * k + 3];
  }
}

// sum over the slice's 64 weights of w*x, in the factored form
// d1*sum(q*x) - m1*sum(x) per sub-block (dot_q4_k, dequant.cpp:954-984)
__device__ __forceinline__ float q4k_dot(const Q4Slice& w, int g, const XSlice& x) {
  float s0 = 0.0f, s1 = 0.0f;
  q4k_codes16(w.a, x.v, x.v + 32, s0, s1);
  q4k_codes16(w.b, x.v + 16, x.v + 48, s0, s1);
  const float d = h2f(w.h.x), dmin = h2f(w.h.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(w.h.y, w.h.z, w.h.w, 2 * g, sc0, m0);
  q4k_scale_min(w.h.y, w.h.z, w.h.w, 2 * g + 1, sc1, m1);
  const float d0 = d * (float)sc0, dm0 = dmin * (float)m0;
  const float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
  return (d0 * s0 - dm0 * x.s0) + (d1 * s1 - dm1 * x.s1);
}

// ---------------------------------------------------------------- Q6_K slices
// Quarter t (0..3) of half hf (0..1) of one Q6_K block: 32 weights, two
// 16-weight scale groups.  Q6_K blocks are 210 bytes (2-byte aligned only), so
// the codes are read as bytes.
__device__ __forceinline__ float q6k_quarter(const uint8_t* __restrict__ blk, int hf, int t,
                                             const float* xq) {
  const float d = h2f((uint32_t)blk[KNJ_Q6K_D] | ((uint32_t)blk[KNJ_Q6K_D + 1] << 8));
  const uint8_t* ql = blk + KNJ_Q6K_QL + 64 * hf + 32 * (t & 1);
  const uint8_t* qh = blk + KNJ_Q6K_QH + 32 * hf;
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

// A Q6_K "unit": quarter-octet o (0..3) of half hf of one block -- weights
// 128 hf + 32 t + 8 o + i (t, i < 4, 8): ql bytes 64 hf + 8 o (quarters 0, 2)
// and 64 hf + 32 + 8 o (quarters 1, 3), qh bytes 32 hf + 8 o, the scales of
// sub-group o/2 of each quarter and d (dequant_q6_k, dequant.cpp:164-191).
// Q6_K blocks are 210 bytes, so these runs are only 2-byte aligned: each is
// read as three aligned words and shifted into place.
struct Q6Unit {
  uint32_t l0a, l0b, l1a, l1b, ha, hb;  // ql run 0, ql run 1, qh run (8 bytes each)
  int32_t sc[4];                        // the quarters' scales
  uint32_t d;                           // f16 bits of d
};

__device__ __forceinline__ void ld8_u2(const uint8_t* p, uint32_t& a, uint32_t& b) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(addr & ~(uintptr_t)3);
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
  const uint32_t sh = (uint32_t)(addr & 3) * 8;
  a = sh ? __builtin_amdgcn_alignbit(w1, w0, sh) : w0;
  b = sh ? __builtin_amdgcn_alignbit(w2, w1, sh) : w1;
}

__device__ __forceinline__ Q6Unit q6_unit_load(const uint8_t* __restrict__ blk, int hf, int o) {
  Q6Unit u;
  ld8_u2(blk + KNJ_Q6K_QL + 64 * hf + 8 * o, u.l0a, u.l0b);
  ld8_u2(blk + KNJ_Q6K_QL + 64 * hf + 32 + 8 * o, u.l1a, u.l1b);
  ld8_u2(blk + KNJ_Q6K_QH + 32 * hf + 8 * o, u.ha, u.hb);
  // (scales and d by narrow loads, which stay inside the block)
  const int8_t* sp = reinterpret_cast<const int8_t*>(blk + KNJ_Q6K_SC + 8 * hf + (o >> 1));
#pragma unroll
  for (int t = 0; t < 4; ++t) u.sc[t] = sp[2 * t];
  u.d = *reinterpret_cast<const uint16_t*>(blk + KNJ_Q6K_D);
  return u;
}

// sum over the unit's 32 weights of w*x = d * sum_t sc_t * (sum_i q x - 32 sum_i x),
// with x8[t] the unit's 8 x of quarter t and sx[t] their sum.
__device__ __forceinline__ float q6_unit_dot(const Q6Unit& u, const float4 (&x8)[4][2],
                                             const float (&sx)[4]) {
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t la = (t & 1) ? u.l1a : u.l0a, lb = (t & 1) ? u.l1b : u.l0b;
    const int ns = (t >> 1) * 4;
    const uint32_t qa = ((la >> ns) & 0x0F0F0F0Fu) | (((u.ha >> (2 * t)) & 0x03030303u) << 4);
    const uint32_t qb = ((lb >> ns) & 0x0F0F0F0Fu) | (((u.hb >> (2 * t)) & 0x03030303u) << 4);
    float acc = 0.0f;
    acc += (float)((qa >> 0) & 0xFFu) * x8[t][0].x;
    acc += (float)((qa >> 8) & 0xFFu) * x8[t][0].y;
    acc += (float)((qa >> 16) & 0xFFu) * x8[t][0].z;
    acc += (float)(qa >> 24) * x8[t][0].w;
    acc += (float)((qb >> 0) & 0xFFu) * x8[t][1].x;
    acc += (float)((qb >> 8) & 0xFFu) * x8[t][1].y;
    acc += (float)((qb >> 16) & 0xFFu) * x8[t][1].z;
    acc += (float)(qb >> 24) * x8[t][1].w;
    r += (float)u.sc[t] * (acc - 32.0f * sx[t]);
  }
  return h2f(u.d) * r;
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// Workgroup maximum of a packed key, stored (plain store) to keys[blockIdx.x].
__device__ __forceinline__ void block_argmax_store(unsigned long long best,
                                                   unsigned long long* keys) {
  __shared__ unsigned long long wbest[4];
  best = wave_max_u64(best);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) wbest[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = wbest[w] > b ? wbest[w] : b;
    keys[blockIdx.x] = b;
  }
}

__device__ __forceinline__ int argmax_index(unsigned long long key) {
  return (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

// Softmax + top-k routing of one token by one wave, with no LDS and no
// barrier (Model::moe, /root/reference/src/model/model.cpp:420-460): each lane holds
// experts lane, lane+64, ..  Probabilities are non-negative, so their bit
// patterns order like the values; a key is those bits + 1 (0 marks an expert
// already taken).  Each of the k rounds takes the wave maximum of the keys and,
// among the experts holding it, the lowest index (the strict-'>' argmax with
// ties to the lower index, model.cpp:442-451).  Lane q < k returns selection
// q: its expert and its weight p / sum of the kept p, the sum taken in
// selection order (model.cpp:452-458).  n_expert <= 256.
// The same from logits already in registers: lane holds experts lane + 64 j
// (-inf past n_expert).
__device__ __forceinline__ void wave_route_lg(const float (&lg)[4], int n_expert, int k, int& my_idx,
                                              float& my_w);

__device__ __forceinline__ void wave_route(const float* __restrict__ logits, int n_expert, int k,
                                           int& my_idx, float& my_w) {
  const int lane = threadIdx.x & 63;
  float lg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) lg[j] = lane + 64 * j < n_expert ? logits[lane + 64 * j] : -INFINITY;
  wave_route_lg(lg, n_expert, k, my_idx, my_w);
}

__device__ __forceinline__ void wave_route_lg(const float (&lg)[4], int n_expert, int k, int& my_idx,
                                              float& my_w) {
  const int lane = threadIdx.x & 63;
  float mx = fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3]));
  mx = group_max<64>(mx);
  float ex[4], s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ex[j] = lane + 64 * j < n_expert ? expf(lg[j] - mx) : 0.0f;
    s += ex[j];
  }
  const float sum = group_sum<64>(s);
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    key[j] = lane + 64 * j < n_expert ? __float_as_uint(ex[j] / sum) + 1u : 0u;
  my_idx = 0;
  float my_p = 0.0f, keep = 0.0f;
  for (int q = 0; q < k; ++q) {
    uint32_t b = max(max(key[0], key[1]), max(key[2], key[3]));
    b = wave_max_u32(b);
    const unsigned long long m0 = __ballot(key[0] == b), m1 = __ballot(key[1] == b);
    const unsigned long long m2 = __ballot(key[2] == b), m3 = __ballot(key[3] == b);
    const int e = m0 ? __builtin_ctzll(m0)
                     : m1 ? 64 + __builtin_ctzll(m1)
                          : m2 ? 128 + __builtin_ctzll(m2) : 192 + __builtin_ctzll(m3);
    const float p = __uint_as_float(b - 1u);
    keep += p;
    if (lane == q) {
      my_idx = e;
      my_p = p;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) key[j] = (lane == (e & 63) && j == (e >> 6)) ? 0u : key[j];
  }
  const float inv = keep > 0.0f ? 1.0f / keep : 0.0f;
  my_w = my_p * inv;
}

}  // namespace dev
}  // namespace knj
