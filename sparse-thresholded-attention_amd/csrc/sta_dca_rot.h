// sta_dca_rot.h -- DCA's table-lookup rotation, shared by the prefill (sta_dca.hip) and the
// decode and key-cache kernels (sta_dca_dec.hip).
//
// dca_kernel.py:166-231, 278-286: a table entry is cos / sin of the fp32 angle fl(t * inv_freq)
// times mscale, cast to the model dtype; the rotation x*cos + rotate_half(x)*sin runs in the
// model dtype, each product and the sum rounded.
#pragma once
#include "sta_device.h"

namespace sta {

template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == DT_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else if constexpr (DT == DT_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return x;
}

// The fp32 value x, opaque to the optimiser.  gfx950 can fold fptrunc(fmul f32) into one
// mixed-precision multiply (v_fma_mixlo_f16) that rounds the exact product once to fp16; the
// reference rounds the fp32 product first and then casts, which differs on double-rounding cases.
// The empty asm keeps the fp32 product as a value of its own.
__device__ __forceinline__ float opaque_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Eight rotated outputs o[e] for dims d0 + e of a row at table position t, given the row's
// elements a[e] = x[i0 + e] and b[e] = x[D/2 + i0 + e] (i0 = d0 mod D/2; first: d0 < D/2).
// One table entry: cos / sin of the fp32 angle fl(t * f), correctly rounded to fp32 (through
// double), times mscale and rounded to the model dtype.  A one-ulp difference between fp32 cosine
// implementations can flip a bf16 entry; the correctly rounded value is the one every
// implementation approximates, and the CPU oracle computes the same.
template <int DT>
__device__ __forceinline__ void dca_table_entry(int t, float f, float mscale, float& cs, float& sn) {
#pragma clang fp contract(off)
  const float ang = (float)t * f;
  double sd, cd;
  sincos((double)ang, &sd, &cd);
  cs = round_dt<DT>(opaque_f32((float)cd * mscale));
  sn = round_dt<DT>(opaque_f32((float)sd * mscale));
}

// The rotation of eight elements with given table values (cs[e], sn[e]) for dims i0 + e.
template <int DT>
__device__ __forceinline__ void dca_rot8_cs(const float* a, const float* b, const float* cs, const float* sn,
                                            bool first, float* o) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (first) {                                                // x1*cos + (-x2)*sin
      const float p = round_dt<DT>(a[e] * cs[e]), q = round_dt<DT>(-b[e] * sn[e]);
      o[e] = round_dt<DT>(p + q);
    } else {                                                    // x2*cos + x1*sin
      const float p = round_dt<DT>(b[e] * cs[e]), q = round_dt<DT>(a[e] * sn[e]);
      o[e] = round_dt<DT>(p + q);
    }
  }
}

template <int DT>
__device__ __forceinline__ void dca_rot8(const float* a, const float* b, int t, int i0, bool first,
                                         const float* __restrict__ inv_freq, float mscale, float* o) {
#pragma clang fp contract(off)
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dca_table_entry<DT>(t, inv_freq[i0 + e], mscale, cs[e], sn[e]);
  dca_rot8_cs<DT>(a, b, cs, sn, first, o);
}

}  // namespace sta
