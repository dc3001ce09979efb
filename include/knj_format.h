/* include/knj_format.h -- byte semantics of the weight formats on the decode path.
 *
 * One definition of every format the decode loop touches, callable from host C/C++
 * and from HIP device code alike (no HIP header is included; under hipcc the
 * functions gain __host__ __device__).  The CPU oracle, the synthetic-weight
 * generator and the gfx950 kernels all decode bytes through this file, so a byte
 * that means one thing on the host cannot mean another on the device.
 *
 * Formats (ggml block layouts, ggml type ids kept so GGUF tensors drop in):
 *
 *   Q4_K  256 weights / 144 bytes
 *           [0..2)   f16 d      scale applied to the 6-bit sub-block scales
 *           [2..4)   f16 dmin   scale applied to the 6-bit sub-block minima
 *           [4..16)  12 bytes   eight 6-bit scales + eight 6-bit minima, packed
 *           [16..144) 128 bytes codes: four 32-byte groups; group g holds
 *                     sub-block 2g in its low nibbles and 2g+1 in its high
 *                     nibbles, position l of the sub-block in byte l
 *         weight = (d*sc_s) * q - (dmin*m_s)          q in [0,15]
 *   Q6_K  256 weights / 210 bytes
 *           [0..128)   ql  low 4 bits      [128..192) qh  high 2 bits
 *           [192..208) 16 x int8 scales    [208..210) f16 d
 *         two 128-weight halves; in half h, quarter t (32 weights, t = 0..3)
 *         position l: low nibble of ql[64h + l + 32*(t&1)] (t<2) or its high
 *         nibble (t>=2), high bits (qh[32h + l] >> 2t) & 3, code biased by -32,
 *         scale index 8h + 2t + (l >= 16)
 *         weight = (d*sc) * q                           q in [-32,31]
 *   BF16  upper 16 bits of an IEEE f32
 *   F16   IEEE binary16
 *
 * Follows (semantics, not code) /root/reference/src/loader/dequant.cpp:64-72
 * (scale/min unpack), :102-125 (Q4_K), :164-191 (Q6_K), :1032-1073 (f16/bf16) and
 * /root/reference/kernels/knj_q4k.h:63-77 (offsets).
 */
#ifndef KNJ_FORMAT_H
#define KNJ_FORMAT_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KNJ_HD __host__ __device__ static inline
#else
#define KNJ_HD static inline
#endif

/* ggml type ids (gguf.h GgmlType) for the formats this build decodes. */
enum {
  KNJ_TYPE_F32 = 0,
  KNJ_TYPE_F16 = 1,
  KNJ_TYPE_Q4_K = 12,
  KNJ_TYPE_Q6_K = 14,
  KNJ_TYPE_BF16 = 30
};

#define KNJ_QK 256            /* weights per K-quant super-block */
#define KNJ_Q4K_BLOCK 144     /* bytes per Q4_K super-block */
#define KNJ_Q6K_BLOCK 210     /* bytes per Q6_K super-block */

#define KNJ_Q4K_D 0
#define KNJ_Q4K_DMIN 2
#define KNJ_Q4K_SCALES 4
#define KNJ_Q4K_QS 16

#define KNJ_Q6K_QL 0
#define KNJ_Q6K_QH 128
#define KNJ_Q6K_SC 192
#define KNJ_Q6K_D 208

KNJ_HD uint32_t knj_f32_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}

KNJ_HD float knj_bits_f32(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

/* Bytes for one row of `n` weights of `type` (n a whole number of blocks). */
KNJ_HD uint64_t knj_row_bytes(int type, uint64_t n) {
  switch (type) {
    case KNJ_TYPE_F32: return n * 4u;
    case KNJ_TYPE_F16:
    case KNJ_TYPE_BF16: return n * 2u;
    case KNJ_TYPE_Q4_K: return n / KNJ_QK * KNJ_Q4K_BLOCK;
    case KNJ_TYPE_Q6_K: return n / KNJ_QK * KNJ_Q6K_BLOCK;
    default: return 0;
  }
}

/* Weights per block (1 for the plain float types). */
KNJ_HD uint32_t knj_block_weights(int type) {
  return (type == KNJ_TYPE_Q4_K || type == KNJ_TYPE_Q6_K) ? KNJ_QK : 1u;
}

/* binary16 -> binary32, exact for every pattern: normals, subnormals (rescaled
 * into the f32 normal range), signed zeros, infinities and NaN payloads. */
KNJ_HD float knj_f16_to_f32(uint16_t h) {
  const uint32_t sgn = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t mant = (uint32_t)h & 0x3FFu;
  if (ex == 0x1Fu) return knj_bits_f32(sgn | 0x7F800000u | (mant << 13));
  if (ex != 0u) return knj_bits_f32(sgn | ((ex + 112u) << 23) | (mant << 13));
  if (mant == 0u) return knj_bits_f32(sgn);
  /* subnormal: value = mant * 2^-24; shift the leading one up to bit 10 */
  uint32_t e32 = 113u; /* exponent field for 2^-14 */
  while ((mant & 0x400u) == 0u) {
    mant <<= 1;
    e32 -= 1u;
  }
  return knj_bits_f32(sgn | (e32 << 23) | ((mant & 0x3FFu) << 13));
}

/* binary32 -> binary16 with IEEE round-to-nearest-even, gradual underflow to
 * f16 subnormals, overflow to infinity, NaN kept quiet.  The KV cache and the
 * quantiser's d/dmin use this; the GPU's v_cvt_f16_f32 in its default rounding
 * mode produces the same bits. */
KNJ_HD uint16_t knj_f32_to_f16(float f) {
  const uint32_t x = knj_f32_bits(f);
  const uint16_t sgn = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf or nan */
    return (uint16_t)(sgn | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sgn | 0x7C00u); /* rounds to >= 65520 */
  if (ax < 0x38800000u) {
    /* result is an f16 subnormal (or zero): value / 2^-24 rounded to integer */
    if (ax < 0x33000000u) return sgn; /* below half of the smallest subnormal */
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e; /* 14..24 */
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) r += 1u;
    return (uint16_t)(sgn | r);
  }
  /* normal range: drop 13 mantissa bits with round-to-nearest-even; a carry
   * out of the mantissa correctly bumps the exponent */
  uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 (<<23 domain) */
  const uint32_t rem = r & 0x1FFFu;
  r >>= 13;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u;
  return (uint16_t)(sgn | r);
}

KNJ_HD float knj_bf16_to_f32(uint16_t b) { return knj_bits_f32((uint32_t)b << 16); }

/* binary32 -> bfloat16, round-to-nearest-even, NaN kept quiet. */
KNJ_HD uint16_t knj_f32_to_bf16(float f) {
  const uint32_t x = knj_f32_bits(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  const uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7FFFu + lsb) >> 16);
}

KNJ_HD uint16_t knj_rd_u16(const uint8_t* p) {
  return (uint16_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

/* Q4_K: 6-bit scale and min of sub-block s (0..7) from the 12 packed bytes.
 * Sub-blocks 0..3 keep theirs in the low six bits of bytes s (scale) and s+4
 * (min).  Sub-blocks 4..7 keep their low four bits in the nibbles of byte s+4
 * (scale low, min high) and their top two bits in the top two bits of bytes
 * s-4 (scale) and s (min). */
KNJ_HD void knj_q4k_sub_scale(const uint8_t* sc12, int s, uint32_t* scale, uint32_t* mn) {
  if (s < 4) {
    *scale = (uint32_t)sc12[s] & 0x3Fu;
    *mn = (uint32_t)sc12[s + 4] & 0x3Fu;
  } else {
    const uint32_t lo = sc12[s + 4];
    *scale = (lo & 0x0Fu) | (((uint32_t)sc12[s - 4] >> 6) << 4);
    *mn = (lo >> 4) | (((uint32_t)sc12[s] >> 6) << 4);
  }
}

/* Inverse of knj_q4k_sub_scale for all eight sub-blocks (used by the quantiser). */
KNJ_HD void knj_q4k_pack_scales(const uint8_t sc[8], const uint8_t mn[8], uint8_t out[12]) {
  for (int i = 0; i < 12; ++i) out[i] = 0;
  for (int s = 0; s < 4; ++s) {
    out[s] = (uint8_t)((sc[s] & 0x3F) | ((sc[s + 4] >> 4) << 6));
    out[s + 4] = (uint8_t)((mn[s] & 0x3F) | ((mn[s + 4] >> 4) << 6));
    out[s + 8] = (uint8_t)((sc[s + 4] & 0x0F) | ((mn[s + 4] & 0x0F) << 4));
  }
}

/* The 4-bit code of weight r (0..255) inside a Q4_K block. */
KNJ_HD uint32_t knj_q4k_code(const uint8_t* blk, int r) {
  const int s = r >> 5, l = r & 31;
  const uint32_t byte = blk[KNJ_Q4K_QS + (s >> 1) * 32 + l];
  return (s & 1) ? (byte >> 4) : (byte & 0x0Fu);
}

/* Sub-block factors: d1 = d*sc, m1 = dmin*mn.  Both products are exact in f32
 * (an f16 times a 6-bit integer fits in 17 significant bits). */
KNJ_HD void knj_q4k_factors(const uint8_t* blk, int s, float* d1, float* m1) {
  const float d = knj_f16_to_f32(knj_rd_u16(blk + KNJ_Q4K_D));
  const float dmin = knj_f16_to_f32(knj_rd_u16(blk + KNJ_Q4K_DMIN));
  uint32_t sc, mn;
  knj_q4k_sub_scale(blk + KNJ_Q4K_SCALES, s, &sc, &mn);
  *d1 = d * (float)sc;
  *m1 = dmin * (float)mn;
}

/* Weight r of a Q4_K block: d1*q - m1.  d1*q is exact (<= 21 significant bits),
 * so the result is the single rounding of the subtraction whether or not the
 * compiler fuses it into an FMA. */
KNJ_HD float knj_q4k_weight(const uint8_t* blk, int r) {
  float d1, m1;
  knj_q4k_factors(blk, r >> 5, &d1, &m1);
  return d1 * (float)knj_q4k_code(blk, r) - m1;
}

/* The signed 6-bit code (-32..31) of weight r inside a Q6_K block. */
KNJ_HD int knj_q6k_code(const uint8_t* blk, int r) {
  const int h = r >> 7, t = (r >> 5) & 3, l = r & 31;
  const uint32_t lowbyte = blk[KNJ_Q6K_QL + 64 * h + l + 32 * (t & 1)];
  const uint32_t lo4 = (t < 2) ? (lowbyte & 0x0Fu) : (lowbyte >> 4);
  const uint32_t hi2 = ((uint32_t)blk[KNJ_Q6K_QH + 32 * h + l] >> (2 * t)) & 3u;
  return (int)(lo4 | (hi2 << 4)) - 32;
}

/* int8 scale of weight r inside a Q6_K block. */
KNJ_HD int knj_q6k_scale(const uint8_t* blk, int r) {
  const int h = r >> 7, t = (r >> 5) & 3, l = r & 31;
  return (int)(int8_t)blk[KNJ_Q6K_SC + 8 * h + 2 * t + (l >> 4)];
}

/* Weight r of a Q6_K block, associated as (d*sc)*q: d*sc is exact (f16 times an
 * 8-bit integer), the product with q rounds once. */
KNJ_HD float knj_q6k_weight(const uint8_t* blk, int r) {
  const float d = knj_f16_to_f32(knj_rd_u16(blk + KNJ_Q6K_D));
  return d * (float)knj_q6k_scale(blk, r) * (float)knj_q6k_code(blk, r);
}

#endif /* KNJ_FORMAT_H */
