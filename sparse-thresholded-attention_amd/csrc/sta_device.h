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

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Two fp32 values -> packed bf16 (a in the low half), rounded to nearest even by the hardware
// conversion (v_cvt_pk_bf16_f32; checked against a bitwise RNE on 2^24 inputs including ties).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  const float2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack2_bf16(f, f) & 0xffffu; }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)x;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 x = (_Float16)f;  // hardware conversion rounds to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

// two fp32 values in the 16-bit storage format DT (bf16 or f16)
template <int DT>
__device__ __forceinline__ uint32_t pack2_dt(float a, float b) {
  if constexpr (DT == 2) return pack2_f16(a, b);
  else return pack2_bf16(a, b);
}

// c + a.lo * b.lo + a.hi * b.hi over packed 16-bit pairs of the format DT (bf16 or f16), fp32
// accumulation (v_dot2c_f32_bf16 / v_dot2c_f32_f16)
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ float dot2_dt(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == 2)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Transpose four rows of eight 16-bit elements (u32x4 each) into eight columns of four:
// out[e] = {r0[e] | r1[e] << 16, r2[e] | r3[e] << 16}.  Pure bit moves.
__device__ __forceinline__ void transpose4x8_16(const u32x4& r0, const u32x4& r1, const u32x4& r2,
                                                const u32x4& r3, u32x2* out) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    out[2 * w][0] = __builtin_amdgcn_perm(r1[w], r0[w], 0x05040100u);       // low halves
    out[2 * w][1] = __builtin_amdgcn_perm(r3[w], r2[w], 0x05040100u);
    out[2 * w + 1][0] = __builtin_amdgcn_perm(r1[w], r0[w], 0x07060302u);   // high halves
    out[2 * w + 1][1] = __builtin_amdgcn_perm(r3[w], r2[w], 0x07060302u);
  }
}

// LDS layout of a transposed V tile (D rows = head dims, BN columns = key slots, 16-bit
// elements), read as an MFMA operand 4 slots at a time.  SWZ: the 4-slot column groups are
// XOR-swizzled by row so that both access patterns hit distinct banks: the transposing stores
// (16 lanes on rows 8 apart, one column group) and the operand reads (16 lanes on 16 consecutive
// rows starting at a multiple of 16, one column group).  Without SWZ the rows are padded by 4
// elements: the row stride is then 8 bytes times an odd number, so the operand reads are
// conflict-free with no extra address registers (the stores keep 8-way conflicts).
template <int BN, bool SWZ = true>
struct VtLayout {
  static_assert(BN == 32 || BN == 64, "slots per block");
  static constexpr int STR = !SWZ ? BN + 4 : (BN == 64 ? 64 : 36);   // row stride in elements
  __device__ static __forceinline__ int off(int row, int grp) {
    if constexpr (!SWZ) return row * STR + (grp << 2);
    const int g = BN == 64 ? ((row ^ (row >> 3)) & 15) : ((row >> 4) & 7);
    return row * STR + ((grp ^ g) << 2);
  }
};

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
    const uint32_t h = pack2_bf16(x[2 * e], x[2 * e + 1]);
    const float r0 = x[2 * e] - __uint_as_float(h << 16), r1 = x[2 * e + 1] - __uint_as_float(h & 0xffff0000u);
    hi[e] = h;
    lo[e] = pack2_bf16(r0, r1);
  }
}

__device__ __forceinline__ u32x4 pack_bf16x8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = pack2_bf16(x[2 * e], x[2 * e + 1]);
  return r;
}

__device__ __forceinline__ u32x4 pack_f16x8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = pack2_f16(x[2 * e], x[2 * e + 1]);
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

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane L reads 4 16-bit elements at
// its own address and the group's 64 elements are transposed: lane i receives element i % 4 of
// lanes i/4, 4 + i/4, 8 + i/4 and 12 + i/4 (layout checked on an MI355X).  Addressing slot
// base + L/4, columns c + 4 (L % 4) .. +3 of a row-major tile hands lane L column c + L of
// slots base .. base + 3: a k-contiguous MFMA operand from a k-strided layout.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 tr_read16x4(const uint16_t* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
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
// The argument is reduced straight to revolutions, t = x / (2 pi) - k, with 1 / (2 pi) split
// into two fp32 terms kH + kL: fma(x, kH, -k) is the exact product minus the integer k, rounded
// once, and fma(x, kL, .) adds the low term.  The hardware sine/cosine take t in revolutions.
// Reduction error below 4e-8 revolutions for |x| < 5000 and below 6e-8 up to |x| = 65536, where
// k can round to the neighbouring integer and |t| slightly exceeds 0.5 (a two-constant Cody-Waite
// reduction by 2 pi takes one more instruction and reaches 6e-8 already below 5000); the angle
// itself is the reference's fp32 product.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void fast_sincos(float x, float& s, float& c) {
  const float kH = 0.15915494f;        // fp32(1 / (2 pi)), 0x3e22f983
  const float kL = 6.4206382e-09f;     // fp32(1 / (2 pi) - kH), 0x31dc9c88
  const float k = rintf(x * kH);
  float t = fmaf(x, kH, -k);
  t = fmaf(x, kL, t);
  s = __builtin_amdgcn_sinf(t);
  c = __builtin_amdgcn_cosf(t);
}

// The smallest float x with fl(x * c) >= thr, for c > 0: fl(x * c) is monotone in x, so
// acc >= x0 <=> fl(acc * c) >= thr, the reference's keep test on the scaled score with one
// compare on the raw dot.  Non-finite thresholds pass through.
__device__ __forceinline__ float min_arg_for(float thr, float c) {
#pragma clang fp contract(off)
  if (thr != thr || thr == -INFINITY || thr == INFINITY) return thr;
  float x = thr / c;
  for (int i = 0; i < 4; ++i) {
    const float y = nextafterf(x, -INFINITY);
    if (y * c >= thr) x = y; else break;
  }
  for (int i = 0; i < 4 && !(x * c >= thr); ++i) x = nextafterf(x, INFINITY);
  return x;
}

// 16 bytes per lane from global memory straight into LDS, lane l's bytes at lds_base + 16 l
// (global_load_lds_dwordx4; lds_base is wave-uniform and goes to M0).  Issued through inline
// assembly so that the compiler does not track it as an LDS write: its own wait insertion would
// otherwise drain every copy in flight (s_waitcnt vmcnt(0)) in front of the next LDS read and
// serialise a multi-buffered copy pipeline.  Callers order the copies themselves with explicit
// s_waitcnt vmcnt and barriers.
__device__ __forceinline__ void copy16_to_lds(const void* gsrc, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gsrc), "{m0}"(lds_base) : "memory");
}
// the same copy with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset (lane
// l's 16 bytes from sbase + voff): one offset register serves every copy of a wave
__device__ __forceinline__ void copy16_to_lds_s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// Slots from an LDS counter for the lanes of a wave that take one: one atomic per wave instead of
// one per lane (same-address LDS atomics serialise).  Every active lane of the wave must call it;
// a taking lane gets its index, the others -1.
__device__ __forceinline__ int wave_alloc(bool take, int* counter) {
  const unsigned long long mask = __ballot(take);
  if (mask == 0ull) return -1;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll(mask) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(counter, __popcll(mask));
  base = __builtin_amdgcn_readlane(base, leader);
  const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
  return take ? base + below : -1;
}

// Wave-wide scans and reductions on DPP lane moves (within rows of 16 lanes, then row broadcasts
// and lane reads): no LDS round trip.  Every lane of the wave must be active.
// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31, rows 2 and 3
  return x;
}

// the sum over the 64 lanes, uniform
__device__ __forceinline__ int wave_sum(int x) { return __builtin_amdgcn_readlane(wave_incl_sum(x), 63); }

// the sum over each aligned group of 8 lanes, in every lane of the group (the xor-1, xor-2
// butterfly within quads, then the other quad of the group: the same additions as the
// xor-1/2/4 butterfly).  Every lane's source is inside its row, so bound_ctrl changes no value;
// with it set the compiler folds each move into its add (v_add_f32_dpp).
__device__ __forceinline__ float group8_sum(float x) {
  x = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xb1, 0xf, 0xf, true)) + x;
  x = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4e, 0xf, 0xf, true)) + x;
  x = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xf, 0xf, true)) + x;
  return x;
}

// the max of the two 8-lane halves of each 16-lane row (row_mirror pairs lane i with 15 - i)
__device__ __forceinline__ float halves16_max(float x) {
  return fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xf, 0xf, false)));
}

// the fp32 max over the 64 lanes (NaN lanes skipped), uniform
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false)));
  const int x = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 48))));
}

// the max over the 64 lanes, uniform
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  int x = (int)v;
  x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xb1, 0xf, 0xf, false));    // quad_perm 1,0,3,2
  x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4e, 0xf, 0xf, false));    // quad_perm 2,3,0,1
  x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, false));   // row_half_mirror
  x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x140, 0xf, 0xf, false));   // row_mirror
  return max(max((uint32_t)__builtin_amdgcn_readlane(x, 0), (uint32_t)__builtin_amdgcn_readlane(x, 16)),
             max((uint32_t)__builtin_amdgcn_readlane(x, 32), (uint32_t)__builtin_amdgcn_readlane(x, 48)));
}

__device__ __forceinline__ float wave_shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ int wave_shfl_xor(int v, int m) { return __shfl_xor(v, m, 64); }

}  // namespace sta
