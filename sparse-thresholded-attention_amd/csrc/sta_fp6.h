// sta_fp6.h -- block-scaled e2m3 (OCP MX fp6) operands of the pass-2 correction product.
//
// Pass 2 of the shared score passes (shared_selection_triton_exact_2.py:105-140) needs each
// score to well within the 1e-3 selection band.  The three-product score
//   hi(q).hi(k) + hi(q).lo(k) + lo(q).hi(k)          (bf16, error ~1e-6)
// spends two of its three products on the correction terms, which are about 2^-8 of the score.
// The fp6 pass 2 keeps the main product in bf16 and computes the correction
//   Q6(q_hi).Q6(k - k_hi) + Q6(q - q_hi).Q6(k_hi)
// with v_mfma_scale_f32_32x32x64_f8f6f4 on e2m3 operands: Q6 rounds each element to e2m3 (3
// mantissa bits) under one power-of-two (E8M0) scale per 32 elements.  The correction's relative
// error of ~2^-5 on a term of ~2^-8 leaves an error of ~1e-4 on unit-scale scores.  That error is
// statistical (a sum of independent roundings), so every head is guarded: the correction's
// standard deviation for the head's largest-norm rows must stay below a quarter of the band, or
// the head takes the three-product pass 2 (fast6_sigma below).  The rounding itself is the
// hardware's (v_cvt_scalef32_2xpk16_fp6_f32, round to nearest even).  Plain C++.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define STA_HD __host__ __device__
#else
#define STA_HD
#endif

namespace sta {

// the selection band of the set contract (keys within 1e-3 of max - tau may differ) and the
// largest standard deviation of the fp6 correction's error a head may have, on the scaled score
constexpr float FAST6_BAND = 1e-3f;
constexpr float FAST6_SIGMA_LIMIT = 0.25f * FAST6_BAND;

STA_HD inline uint32_t fp6_f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

// E8M0 exponent of a block whose largest magnitude is bm: the smallest e with bm <= 7.5 * 2^e
// (7.5 is e2m3's largest value), clamped to [-126, 127] so that 2^e is a normal fp32 scale (the
// hardware conversion reads the scale's exponent); 0 for a zero (or NaN) block.
// bm = 1.f * 2^(E - 127) fits under 7.5 * 2^(E - 129) exactly when 1.f <= 1.875.
STA_HD inline int e2m3_block_exp(float bm) {
  if (!(bm > 0.0f)) return 0;
  const uint32_t u = fp6_f2u(bm);
  const int E = (int)((u >> 23) & 0xff);
  if (E == 0) return -126;                       // subnormal: the smallest scale fits
  int e = (u & 0x7fffffu) <= 0x700000u ? E - 129 : E - 128;
  if (e > 127) e = 127;
  if (e < -126) e = -126;
  return e;
}

// Standard deviation of the fp6 correction's error on the scaled score for rows with norms
// (||hi||, ||x - hi||) = (qh, ql), (kh, kl) and quantisation-error norms (dqh, dql), (dkh, dkl):
// each error term is a row dotted with an independent rounding vector, of standard deviation
// ||a|| ||b|| / sqrt(D).
STA_HD inline float fast6_sigma(float qh, float ql, float dqh, float dql, float kh, float kl, float dkh,
                                float dkl, float sm, int D) {
  const float t1 = dqh * kl, t2 = qh * dkl, t3 = dql * kh, t4 = ql * dkh;
  return sm * sqrtf((t1 * t1 + t2 * t2 + t3 * t3 + t4 * t4) / (float)D);
}

// Bound (Cauchy-Schwarz) on |fp6 score - fp32 dot of the (hi + lo) operands| of one pair, the lo
// parts being bf16(x - hi): the quantisation terms, lo against x - hi (within 2^-8 relative),
// the dropped lo.lo term and the fp32 accumulation of both values.
STA_HD inline float fast6_delta(float qh, float ql, float dqh, float dql, float kh, float kl, float dkh,
                                float dkl) {
  const float qr = 1.005f * ql, kr = 1.005f * kl;
  const float quant = dqh * kr + qh * dkl + dqh * dkl + dql * kh + qr * dkh + dql * dkh;
  const float resid = 0x1p-8f * (qh * kr + qr * kh) + ql * kl;
  return 1.001f * (quant + resid + 0x1p-15f * (qh + qr) * (kh + kr));
}

}  // namespace sta
