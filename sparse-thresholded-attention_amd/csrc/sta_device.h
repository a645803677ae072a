// sta_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Operand fragments follow the CDNA4 MFMA lane layouts (checked on an MI355X):
//   v_mfma_f32_32x32x16_bf16: lane l holds A row / B column (l % 32) and the 8 contraction
//     elements 8*(l/32) .. 8*(l/32)+7 of a 16-wide k step; result slot i of lane l is
//     row (i/4)*8 + (l/32)*4 + (i%4), column l % 32.
//   v_mfma_f32_16x16x32_bf16: lane l holds A row / B column (l % 16) and contraction elements
//     8*(l/16) .. +7 of a 32-wide k step; result slot i of lane l is row 4*(l/16)+i, column l%16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sta {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// ------------------------------------------------------------------------------------------
// scalar conversions (bit-exact, round to nearest even)
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)x;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 x = (_Float16)f;  // hardware conversion rounds to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

template <int DT>
__device__ __forceinline__ float load_scalar(const void* p, int64_t i) {
  if constexpr (DT == DT_F32) return ((const float*)p)[i];
  else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else return f16_bits_to_f32(((const uint16_t*)p)[i]);
}

// Load 8 consecutive elements starting at element i (16- or 32-byte aligned) as fp32.
template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float* out) {
  if constexpr (DT == DT_F32) {
    const float4* q = (const float4*)((const float*)p + i);
    float4 a = q[0], b = q[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    u32x4 w = *(const u32x4*)((const uint16_t*)p + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == DT_BF16) {
        out[2 * e] = __uint_as_float(w[e] << 16);
        out[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
      } else {
        out[2 * e] = f16_bits_to_f32(w[e] & 0xffffu);
        out[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
      }
    }
  }
}

// Split 8 fp32 values into bf16 hi = rne(x) and lo = rne(x - hi); both packed as 4 x u32.
// x - hi is exact in fp32 and |x - hi - lo| <= 2^-16 |x|.
__device__ __forceinline__ void split_bf16x8(const float* x, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t h0 = f32_to_bf16_bits(x[2 * e]), h1 = f32_to_bf16_bits(x[2 * e + 1]);
    float r0 = x[2 * e] - bf16_bits_to_f32(h0), r1 = x[2 * e + 1] - bf16_bits_to_f32(h1);
    uint32_t l0 = f32_to_bf16_bits(r0), l1 = f32_to_bf16_bits(r1);
    hi[e] = h0 | (h1 << 16);
    lo[e] = l0 | (l1 << 16);
  }
}

__device__ __forceinline__ u32x4 pack_bf16x8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16_bits(x[2 * e]) | (f32_to_bf16_bits(x[2 * e + 1]) << 16);
  return r;
}

__device__ __forceinline__ u32x4 pack_f16x8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = f32_to_f16_bits(x[2 * e]) | (f32_to_f16_bits(x[2 * e + 1]) << 16);
  return r;
}

// ------------------------------------------------------------------------------------------
// MFMA wrappers on packed operands
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ floatx16 mfma32(const u32x4& a, const u32x4& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 mfma32_f16(const u32x4& a, const u32x4& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma16(const u32x4& a, const u32x4& b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma16_f16(const u32x4& a, const u32x4& b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------
// 8 consecutive elements in their storage format (loaded now, converted later)
template <int DT>
struct Raw8 {
  u32x4 w;
  __device__ __forceinline__ void load(const void* p, int64_t i) { w = *(const u32x4*)((const uint16_t*)p + i); }
  __device__ __forceinline__ void zero() { w = u32x4{0, 0, 0, 0}; }
  __device__ __forceinline__ void to_f32(float* o) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == DT_BF16) {
        o[2 * e] = __uint_as_float(w[e] << 16);
        o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
      } else {
        o[2 * e] = f16_bits_to_f32(w[e] & 0xffffu);
        o[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
      }
    }
  }
};
template <>
struct Raw8<DT_F32> {
  u32x4 a, b;
  __device__ __forceinline__ void load(const void* p, int64_t i) {
    const u32x4* q = (const u32x4*)((const float*)p + i);
    a = q[0];
    b = q[1];
  }
  __device__ __forceinline__ void zero() { a = u32x4{0, 0, 0, 0}; b = a; }
  __device__ __forceinline__ void to_f32(float* o) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) { o[e] = __uint_as_float(a[e]); o[4 + e] = __uint_as_float(b[e]); }
  }
};

// ------------------------------------------------------------------------------------------
// sin/cos of an fp32 angle for the attend-side rotation.
// Two-constant Cody-Waite reduction by 2*pi with fused multiply-adds (the product k*C is exact
// inside the fma), then the hardware sine/cosine, which take their argument in revolutions.
// Absolute error about 5e-7 for |x| < 2^17; the angle itself is the reference's fp32 product.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void fast_sincos(float x, float& s, float& c) {
  const float kInv2Pi = 0.15915494309189535f;
  const float kC1 = 6.28318548202514648f;        // fp32(2*pi)
  const float kC2 = -1.7484555314695172e-07f;    // fp32(2*pi - kC1)
  float k = rintf(x * kInv2Pi);
  float r = fmaf(-k, kC1, x);
  r = fmaf(-k, kC2, r);
  float t = r * kInv2Pi;
  s = __builtin_amdgcn_sinf(t);
  c = __builtin_amdgcn_cosf(t);
}

// xor-butterfly helpers over a 64-lane wavefront
__device__ __forceinline__ float wave_shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ int wave_shfl_xor(int v, int m) { return __shfl_xor(v, m, 64); }

}  // namespace sta
