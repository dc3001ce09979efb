/* include/knj_synth.h -- seeded synthetic weights, bit-identical on host and GPU.
 *
 * The benchmark configurations call for random-init weights drawn ~N(0, std) and
 * then quantised to Q4_K / Q6_K (or rounded to bf16).  No checkpoint exists, so
 * the weights are a pure function of (seed, tensor, element index):
 *
 *   h  = splitmix64 output for counter (tensor_key + index * golden-gamma)
 *   u1 = (2*(h >> 41) + 1) * 2^-24      in (0, 1), exact in f32
 *   u2 = (h & 0xFFFFFF) * 2^-24         in [0, 1), exact in f32
 *   z  = sqrt(-2 ln u1) * cos(2 pi u2)  (Box-Muller, one normal per draw)
 *
 * ln and cos are evaluated here from their series with explicit fused
 * multiply-adds, and the only other operations are IEEE-exact ones (+ - * /,
 * sqrt, floor), so the host build and the gfx950 build produce the same bits.
 * Contraction of a*b+c into an FMA is switched off for every function in this
 * file; a fused step is always written as knj_fmaf.
 *
 * The quantisers are this build's own (the reference has none): per 32-weight
 * sub-block min/max for Q4_K, per 16-weight absmax for Q6_K, 6-/8-bit scales
 * relative to an f16 super-block scale, round-half-up codes.  Only their output
 * bytes matter to the decode path, which reads them through knj_format.h.
 */
#ifndef KNJ_SYNTH_H
#define KNJ_SYNTH_H

#include "knj_format.h"

#if defined(__clang__)
#define KNJ_NOCONTRACT _Pragma("clang fp contract(off)")
#else
#define KNJ_NOCONTRACT
#endif

KNJ_HD float knj_fmaf(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

/* splitmix64 finaliser (Steele, Lea, Flood 2014). */
KNJ_HD uint64_t knj_mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Tensor kinds, part of the key so every tensor has its own stream. */
enum {
  KNJ_T_EMBD = 1,
  KNJ_T_HEAD = 2,
  KNJ_T_Q = 3,
  KNJ_T_K = 4,
  KNJ_T_V = 5,
  KNJ_T_O = 6,
  KNJ_T_ROUTER = 7,
  KNJ_T_GATE = 8,
  KNJ_T_UP = 9,
  KNJ_T_DOWN = 10,
  KNJ_T_INPUT = 11 /* synthetic activations (e.g. the x of a layer test) */
};

KNJ_HD uint64_t knj_tensor_key(uint64_t seed, int layer, int kind, int expert) {
  const uint64_t t = ((uint64_t)(uint32_t)(layer + 1) << 40) ^ ((uint64_t)(uint32_t)kind << 24) ^
                     (uint64_t)(uint32_t)(expert + 1);
  return knj_mix64(seed ^ knj_mix64(t));
}

/* ln(u) for u > 0 (finite, normal).  u = m * 2^e with m in [sqrt(1/2), sqrt(2));
 * ln m = 2 atanh(s), s = (m-1)/(m+1), |s| <= 0.1716, series through s^11. */
KNJ_HD float knj_logf(float u) {
  KNJ_NOCONTRACT
  const uint32_t b = knj_f32_bits(u);
  int e = (int)((b >> 23) & 0xFFu) - 127;
  float m = knj_bits_f32((b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = knj_fmaf(z, 1.0f / 11.0f, 1.0f / 9.0f);
  p = knj_fmaf(z, p, 1.0f / 7.0f);
  p = knj_fmaf(z, p, 1.0f / 5.0f);
  p = knj_fmaf(z, p, 1.0f / 3.0f);
  const float s2 = s + s;
  const float lnm = knj_fmaf(s2 * z, p, s2);
  return knj_fmaf((float)e, 0.693147180559945309f, lnm);
}

/* cos(2 pi t) for t in [0, 1): fold to [0, 1/8] with exact reflections, then a
 * Taylor series of cos or sin on [0, pi/4]. */
KNJ_HD float knj_cos2pi(float t) {
  KNJ_NOCONTRACT
  float a = t;
  if (a >= 0.5f) a = 1.0f - a;
  float sign = 1.0f;
  if (a > 0.25f) {
    a = 0.5f - a;
    sign = -1.0f;
  }
  const bool use_sin = a > 0.125f;
  if (use_sin) a = 0.25f - a;
  const float x = a * 6.28318530717958648f;
  const float x2 = x * x;
  float r;
  if (use_sin) {
    float p = knj_fmaf(x2, 1.0f / 362880.0f, -1.0f / 5040.0f);
    p = knj_fmaf(x2, p, 1.0f / 120.0f);
    p = knj_fmaf(x2, p, -1.0f / 6.0f);
    r = knj_fmaf(x * x2, p, x);
  } else {
    float p = knj_fmaf(x2, 1.0f / 3628800.0f * -1.0f, 1.0f / 40320.0f);
    p = knj_fmaf(x2, p, -1.0f / 720.0f);
    p = knj_fmaf(x2, p, 1.0f / 24.0f);
    p = knj_fmaf(x2, p, -0.5f);
    r = knj_fmaf(x2, p, 1.0f);
  }
  return sign * r;
}

/* One standard normal for (key, index). */
KNJ_HD float knj_normal(uint64_t key, uint64_t index) {
  KNJ_NOCONTRACT
  const uint64_t h = knj_mix64(key + index * 0x9E3779B97F4A7C15ull);
  const float u1 = (float)(2u * (uint32_t)(h >> 41) + 1u) * (1.0f / 16777216.0f);
  const float u2 = (float)(uint32_t)(h & 0xFFFFFFu) * (1.0f / 16777216.0f);
  const float r = __builtin_sqrtf(-2.0f * knj_logf(u1));
  return r * knj_cos2pi(u2);
}

/* N(0, std) value of element `index` of a tensor. */
KNJ_HD float knj_synth_value(uint64_t key, uint64_t index, float stddev) {
  KNJ_NOCONTRACT
  return knj_normal(key, index) * stddev;
}

KNJ_HD float knj_round_half_up(float v) { return __builtin_floorf(v + 0.5f); }

/* Quantise 256 floats into one Q4_K block (144 bytes). */
KNJ_HD void knj_quantize_q4k_block(const float* x, uint8_t* blk) {
  KNJ_NOCONTRACT
  float scale[8], negmin[8];
  float max_scale = 0.0f, max_min = 0.0f;
  for (int s = 0; s < 8; ++s) {
    float lo = x[32 * s], hi = x[32 * s];
    for (int l = 1; l < 32; ++l) {
      const float v = x[32 * s + l];
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
    if (lo > 0.0f) lo = 0.0f;
    scale[s] = (hi - lo) / 15.0f;
    negmin[s] = -lo;
    max_scale = scale[s] > max_scale ? scale[s] : max_scale;
    max_min = negmin[s] > max_min ? negmin[s] : max_min;
  }
  const uint16_t dh = knj_f32_to_f16(max_scale / 63.0f);
  const uint16_t mh = knj_f32_to_f16(max_min / 63.0f);
  const float dq = knj_f16_to_f32(dh), mq = knj_f16_to_f32(mh);
  uint8_t sc[8], mn[8];
  for (int s = 0; s < 8; ++s) {
    float a = dq > 0.0f ? knj_round_half_up(scale[s] / dq) : 0.0f;
    float b = mq > 0.0f ? knj_round_half_up(negmin[s] / mq) : 0.0f;
    a = a < 0.0f ? 0.0f : (a > 63.0f ? 63.0f : a);
    b = b < 0.0f ? 0.0f : (b > 63.0f ? 63.0f : b);
    sc[s] = (uint8_t)a;
    mn[s] = (uint8_t)b;
  }
  blk[KNJ_Q4K_D] = (uint8_t)(dh & 0xFF);
  blk[KNJ_Q4K_D + 1] = (uint8_t)(dh >> 8);
  blk[KNJ_Q4K_DMIN] = (uint8_t)(mh & 0xFF);
  blk[KNJ_Q4K_DMIN + 1] = (uint8_t)(mh >> 8);
  knj_q4k_pack_scales(sc, mn, blk + KNJ_Q4K_SCALES);
  for (int i = 0; i < 128; ++i) blk[KNJ_Q4K_QS + i] = 0;
  for (int s = 0; s < 8; ++s) {
    const float d1 = dq * (float)sc[s];
    const float m1 = mq * (float)mn[s];
    for (int l = 0; l < 32; ++l) {
      float q = d1 > 0.0f ? knj_round_half_up((x[32 * s + l] + m1) / d1) : 0.0f;
      q = q < 0.0f ? 0.0f : (q > 15.0f ? 15.0f : q);
      const uint32_t qi = (uint32_t)q;
      uint8_t* byte = blk + KNJ_Q4K_QS + (s >> 1) * 32 + l;
      *byte = (uint8_t)(*byte | ((s & 1) ? (qi << 4) : qi));
    }
  }
}

/* Quantise 256 floats into one Q6_K block (210 bytes). */
KNJ_HD void knj_quantize_q6k_block(const float* x, uint8_t* blk) {
  KNJ_NOCONTRACT
  float scale[16];
  float max_scale = 0.0f;
  for (int g = 0; g < 16; ++g) {
    float amax = 0.0f;
    for (int l = 0; l < 16; ++l) {
      const float v = x[16 * g + l];
      const float a = v < 0.0f ? -v : v;
      amax = a > amax ? a : amax;
    }
    scale[g] = amax / 31.0f;
    max_scale = scale[g] > max_scale ? scale[g] : max_scale;
  }
  const uint16_t dh = knj_f32_to_f16(max_scale / 127.0f);
  const float dq = knj_f16_to_f32(dh);
  for (int i = 0; i < KNJ_Q6K_BLOCK; ++i) blk[i] = 0;
  int8_t sc[16];
  for (int g = 0; g < 16; ++g) {
    float a = dq > 0.0f ? knj_round_half_up(scale[g] / dq) : 0.0f;
    a = a > 127.0f ? 127.0f : a;
    sc[g] = (int8_t)(int)a;
  }
  /* weight r lives at half h, quarter t, position l; its scale group is
   * 8h + 2t + (l >= 16), which is r / 16 */
  for (int r = 0; r < 256; ++r) {
    const int h = r >> 7, t = (r >> 5) & 3, l = r & 31;
    const int g = r >> 4;
    const float step = dq * (float)sc[g];
    float q = step > 0.0f ? knj_round_half_up(x[r] / step) : 0.0f;
    q = q < -32.0f ? -32.0f : (q > 31.0f ? 31.0f : q);
    const uint32_t u = (uint32_t)((int)q + 32);
    uint8_t* lowbyte = blk + KNJ_Q6K_QL + 64 * h + l + 32 * (t & 1);
    *lowbyte = (uint8_t)(*lowbyte | ((t < 2) ? (u & 0x0Fu) : ((u & 0x0Fu) << 4)));
    uint8_t* hb = blk + KNJ_Q6K_QH + 32 * h + l;
    *hb = (uint8_t)(*hb | (((u >> 4) & 3u) << (2 * t)));
  }
  for (int g = 0; g < 16; ++g) blk[KNJ_Q6K_SC + g] = (uint8_t)sc[g];
  blk[KNJ_Q6K_D] = (uint8_t)(dh & 0xFF);
  blk[KNJ_Q6K_D + 1] = (uint8_t)(dh >> 8);
}

/* Block `b` (0-based, row-major over [n_rows][n_in/256]) of a synthetic
 * quantised tensor: 256 values N(0, std) for elements row*n_in + 256*(b%nb) ...
 * then quantised.  `tmp` holds 256 floats. */
KNJ_HD void knj_synth_quant_block(uint64_t key, int type, uint64_t n_in, uint64_t b, float stddev,
                                  float* tmp, uint8_t* out) {
  const uint64_t nb = n_in / KNJ_QK;
  const uint64_t row = b / nb, col0 = (b % nb) * KNJ_QK;
  const uint64_t base = row * n_in + col0;
  for (int i = 0; i < KNJ_QK; ++i) tmp[i] = knj_synth_value(key, base + (uint64_t)i, stddev);
  if (type == KNJ_TYPE_Q4_K) knj_quantize_q4k_block(tmp, out);
  else knj_quantize_q6k_block(tmp, out);
}

#endif /* KNJ_SYNTH_H */
