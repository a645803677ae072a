/*
 * sta_oracle_common.h -- helpers shared by the oracle's translation units (TEST INFRASTRUCTURE
 * ONLY): dtype conversions, the half-split RoPE row rotation and the fp32 score of two rotated
 * rows, with the fp32 rounding points of the reference's kernels.
 */
#ifndef STA_ORACLE_COMMON_H_
#define STA_ORACLE_COMMON_H_
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

/* ------------------------------------------------------------------------------------------- */
/* scalar conversions                                                                          */
/* ------------------------------------------------------------------------------------------- */
static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float f = (float)man * 5.9604644775390625e-08f;
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_f16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (a < 0x38800000u) {                                   /* subnormal / zero in fp16 */
    float af;
    memcpy(&af, &a, 4);
    float q = af * 16777216.0f; /* exact: scale by 2^24, then round to integer (RNE) */
    uint32_t m = (uint32_t)nearbyintf(q);
    return (uint16_t)(sign | m);
  }
  uint32_t exp = ((a >> 23) - 112u) << 10;
  uint32_t man = (a >> 13) & 0x3ffu;
  uint32_t rest = a & 0x1fffu;
  uint32_t h = exp | man;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static inline float load_elem(const void* base, int dtype, size_t i) {
  if (dtype == 0) return ((const float*)base)[i];
  if (dtype == 1) return bf16_to_f32(((const uint16_t*)base)[i]);
  return f16_to_f32(((const uint16_t*)base)[i]);
}

/* value after a cast to the input dtype (p.to(vv.dtype), exact_2.py:220) */
static inline float round_to_dtype(float x, int dtype) {
  if (dtype == 0) return x;
  if (dtype == 1) return bf16_to_f32(f32_to_bf16_rne(x));
  return f16_to_f32(f32_to_f16_rne(x));
}

static inline void oracle_round_to_dtype_impl(const float* in, void* out, size_t n, int dtype) {
  for (size_t i = 0; i < n; ++i) {
    if (dtype == 0) ((float*)out)[i] = in[i];
    else if (dtype == 1) ((uint16_t*)out)[i] = f32_to_bf16_rne(in[i]);
    else ((uint16_t*)out)[i] = f32_to_f16_rne(in[i]);
  }
}

static inline void oracle_to_f32_impl(const void* in, float* out, size_t n, int dtype) {
  for (size_t i = 0; i < n; ++i) out[i] = load_elem(in, dtype, i);
}

/* ------------------------------------------------------------------------------------------- */
/* RoPE, half-split (Llama) form                                                               */
/* ------------------------------------------------------------------------------------------- */
/* Rotate row x (D values, dtype) at an fp32 angle base `posf` (already pos*pos_scale, or newpos).
 * exact_2.py:74-83 (Kernel A), 174-185 / 199-207 (Kernel C), torch twin _rope_rotate 495-502. */
static inline void rope_row(const void* x, int dtype, size_t off, int D, float posf, const float* inv_freq,
                     float rope_scale, float* out) {
  const int half = D / 2;
  for (int i = 0; i < half; ++i) {
    volatile float ang = posf * inv_freq[i];
    volatile float c = cosf(ang) * rope_scale;
    volatile float s = sinf(ang) * rope_scale;
    float x1 = load_elem(x, dtype, off + i);
    float x2 = load_elem(x, dtype, off + half + i);
    volatile float a = x1 * c;
    volatile float b = x2 * s;
    volatile float e = x2 * c;
    volatile float f = x1 * s;
    out[i] = a - b;
    out[half + i] = e + f;
  }
}


/* fl(fl(dot(a[:h], b[:h]) + dot(a[h:], b[h:])) * sm_scale) with each half dot accumulated in double */
static inline float score_of(const float* a, const float* b, int D, float sm_scale) {
  const int half = D / 2;
  double d1 = 0.0, d2 = 0.0;
  for (int i = 0; i < half; ++i) d1 += (double)a[i] * (double)b[i];
  for (int i = half; i < D; ++i) d2 += (double)a[i] * (double)b[i];
  volatile float f1 = (float)d1;
  volatile float f2 = (float)d2;
  volatile float sum = f1 + f2;
  return sum * sm_scale;
}

#endif /* STA_ORACLE_COMMON_H_ */
