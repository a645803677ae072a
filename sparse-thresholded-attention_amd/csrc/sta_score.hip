// sta_score.hip -- selection-geometry RoPE pre-kernel and the two score passes.
//
// Reference: shared_selection_triton_exact_2.py:50-140 (_select_vote_kernel).  The reference
// re-rotates Q and K inside both passes; here the rotation runs once per (row, head) and writes
// the rotated rows in MFMA operand order.  The reference's score dots are fp32 (exact_2.py:100,
// 118); here each rotated fp32 row is split into bf16 hi + lo parts and every score is
//   hi(q).hi(k) + hi(q).lo(k) + lo(q).hi(k)   (three bf16 MFMAs, fp32 accumulation),
// whose error against the fp32 dot is below 3 * 2^-16 * sum|q_i k_i| -- well inside the 1e-3
// selection band -- instead of the ~2^-8 a single bf16 product would give.
//
// Fragment layout (one unit = 8 bf16 = 16 bytes, u32x4):
//   frag[head][rb][s][hl][lane]   rb = row/32, s = dim/16 (16-wide k step), hl = 0 hi / 1 lo,
//   lane = row%32 + 32*((dim%16)/8), holding dims 8*(lane/32) .. +7 of step s.
// A 32-row block's operand for one k step is one contiguous 1 KB load per wave.
#include "sta_device.h"
#include "sta_kernels.h"
#include "sta_fp6.h"

#include <float.h>
#include <stdlib.h>

#include <type_traits>

namespace sta {

// ------------------------------------------------------------------------------------------
// RoPE pre-kernel: rotate rows in the selection geometry, split hi/lo, write fragments.
// angle = fl(fl(float(pos) * pos_scale) * inv_freq[i])          (exact_2.py:79, 95)
// c, s  = fl(cos(angle) * rope_scale), fl(sin(angle) * rope_scale)   (exact_2.py:80-81)
// r1 = fl(fl(x1*c) - fl(x2*s)), r2 = fl(fl(x2*c) + fl(x1*s))   (exact_2.py:82-83)
// Rows >= N (tile padding, and the zero "phantom" keys the reference's masked loads produce
// when q_pos_base > 0) are written as zeros.  Each row's (||hi||, ||lo||) goes to `norms`: the
// screened pass 1 of the score kernel bounds its single-product error with them.
// ------------------------------------------------------------------------------------------
// A thread takes one row and 8 frequencies i0..i0+7 (both rotation halves, dims i0.. and
// D/2+i0..) for ROPE_HG consecutive heads: the 8 sin / cos pairs depend on (row, i) only, so
// they are computed once and reused for every head of the group.
constexpr int ROPE_HG = 4;

// The fp6 correction operands (sta_fp6.h): the row's vector [hi | x - hi] is cut into 32-element
// blocks, each rounded to e2m3 under its own E8M0 scale.  Block b of a 32-row block's row r sits
// in unit b / 2, lane r + 32 (b % 2): 32 elements of 6 bits, element p at bits 6p .. 6p + 5 of
// the lane's 24 bytes, stored as three planes of 64 lanes x 8 bytes (unit = 1536 bytes), so that
// an MFMA operand is three conflict-free 8-byte LDS reads.  The lane's scale dword holds the scale
// of block 2m + (b % 2) in byte m.  Per row: (||Q6(hi) - hi||, ||Q6(x - hi) - (x - hi)||).
//
// A row's C2 threads (one wave holds whole rows) each computed 8 dims of both rotation halves;
// they trade them through the wave's LDS rows so that thread c holds all of block c, which
// v_cvt_scalef32_2xpk16_fp6_f32 rounds to nearest even in one instruction (element 2i from its
// first source, 2i + 1 from its second; checked on an MI355X against sta_fp6.h's software
// encoder), and v_cvt_scalef32_pk32_f32_fp6 decodes for the error norm.  Both go through inline
// assembly with an early-clobber result: the compiler's builtin may place the result over the
// second source, and the instruction then reads back part of its own result.
typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef float f32x32v __attribute__((ext_vector_type(32)));
typedef int i32x6v __attribute__((ext_vector_type(6)));
__device__ __forceinline__ i32x6v cvt_fp6x32(const f32x16v& even, const f32x16v& odd, float scale) {
  i32x6v r;
  asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(r) : "v"(even), "v"(odd), "v"(scale));
  return r;
}
__device__ __forceinline__ f32x32v dec_fp6x32(const i32x6v& codes, float scale) {
  f32x32v r;
  asm volatile("v_cvt_scalef32_pk32_f32_fp6 %0, %1, %2" : "=&v"(r) : "v"(codes), "v"(scale));
  return r;
}
// LDS per wave: its rows' [hi | x - hi] vectors, element p of block b at (p / 4 * NB + b) * 4 +
// p % 4 (the reads of a block's 16-byte groups by consecutive threads are then contiguous), rows
// 2D + 32 floats apart (two rows in one 16-lane read phase fall on different banks)
template <int D>
struct Fp6Rows {
  static constexpr int NB = D / 16;                 // 32-element blocks per row
  static constexpr int RS = 2 * D + 32;             // row stride in floats
  static constexpr int ROWS = 64 / (D / 16);        // rows per wave
  __device__ static __forceinline__ int at(int b, int p) { return ((p >> 2) * NB + b) * 4 + (p & 3); }
};
template <int D>
__device__ __forceinline__ void write_fp6(const float* o1, const float* o2, const u32x4& hi1, const u32x4& hi2, int c,
                                          int row, int head, int rows_pad, float* wlds, uint64_t* planes6,
                                          uint32_t* scales6, float2* dnorms6) {
#pragma clang fp contract(off)
  using R = Fp6Rows<D>;
  constexpr int C2 = D / 16, NB = R::NB;
  const int lane = threadIdx.x & 63;
  float* rl = wlds + (lane / C2) * R::RS;
  {
    // this thread's 8 dims of each half: block b0 (+ D/64 for the second half, + D/32 for the
    // residuals), positions 8 (c % 4) ..
    float hv[2][8], rv[2][8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hv[0][2 * e] = __uint_as_float(hi1[e] << 16);
      hv[0][2 * e + 1] = __uint_as_float(hi1[e] & 0xffff0000u);
      hv[1][2 * e] = __uint_as_float(hi2[e] << 16);
      hv[1][2 * e + 1] = __uint_as_float(hi2[e] & 0xffff0000u);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rv[0][e] = o1[e] - hv[0][e];   // exact
      rv[1][e] = o2[e] - hv[1][e];
    }
    const int b0 = (c * 8) / 32, p0 = 8 * (c & 3);
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int bh = b0 + half * (D / 64), br = bh + D / 32, p = p0 + 4 * k;
        *(float4*)(rl + R::at(bh, p)) = make_float4(hv[half][4 * k], hv[half][4 * k + 1], hv[half][4 * k + 2], hv[half][4 * k + 3]);
        *(float4*)(rl + R::at(br, p)) = make_float4(rv[half][4 * k], rv[half][4 * k + 1], rv[half][4 * k + 2], rv[half][4 * k + 3]);
      }
  }
  // the wave's LDS operations complete in order: its rows are whole before the reads below
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  // thread c takes block c of its row
  const int b = c;
  f32x16v ev, od;
  float bm = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float4 v = *(const float4*)(rl + R::at(b, 4 * k));
    ev[2 * k] = v.x;
    od[2 * k] = v.y;
    ev[2 * k + 1] = v.z;
    od[2 * k + 1] = v.w;
    bm = fmaxf(bm, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  __builtin_amdgcn_wave_barrier();   // the next head's writes follow every read of this one
  const int ex = e2m3_block_exp(bm);
  const float scale = __uint_as_float((uint32_t)(ex + 127) << 23);
  const i32x6v codes = cvt_fp6x32(ev, od, scale);
  const f32x32v dq = dec_fp6x32(codes, scale);
  float d2 = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float d0 = dq[2 * i] - ev[i], d1 = dq[2 * i + 1] - od[i];
    d2 = fmaf(d0, d0, d2);
    d2 = fmaf(d1, d1, d2);
  }
  const int rb = row >> 5, lr = row & 31;
  const int64_t u = (((int64_t)head * (rows_pad >> 5) + rb) * (D / 32) + (b >> 1)) * 192 + lr + 32 * (b & 1);
#pragma unroll
  for (int j = 0; j < 3; ++j)
    planes6[u + 64 * j] = (uint64_t)(uint32_t)codes[2 * j] | ((uint64_t)(uint32_t)codes[2 * j + 1] << 32);
  ((uint8_t*)scales6)[(((int64_t)head * (rows_pad >> 5) + rb) * 64 + lr + 32 * (b & 1)) * 4 + (b >> 1)] = (uint8_t)(ex + 127);
  // per row: the hi blocks' and the residual blocks' squared errors
  float dh = b < NB / 2 ? d2 : 0.0f, dr = b < NB / 2 ? 0.0f : d2;
#pragma unroll
  for (int o = 1; o < C2; o <<= 1) {
    dh += __shfl_xor(dh, o, 64);
    dr += __shfl_xor(dr, o, 64);
  }
  if (c == 0) dnorms6[(int64_t)head * rows_pad + row] = make_float2(sqrtf(dh), sqrtf(dr));
}

template <int DT, int D, bool W6>
__global__ __launch_bounds__(256) void rope_frag_kernel(const void* __restrict__ x, int64_t head_stride,
                                                        int64_t tok_stride, int heads, int N, int rows_pad,
                                                        int pos_base, float pos_scale, float rope_scale,
                                                        const float* __restrict__ inv_freq,
                                                        u32x4* __restrict__ frag, float2* __restrict__ norms,
                                                        uint64_t* __restrict__ planes6, uint32_t* __restrict__ scales6,
                                                        float2* __restrict__ dnorms6, float2* __restrict__ trig) {
#pragma clang fp contract(off)
  constexpr int C2 = D / 16;                 // threads per row
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // the fp6 operands' row exchange (LDS, per wave: rows never span waves)
  __shared__ float lds6[4][W6 ? Fp6Rows<D>::ROWS * Fp6Rows<D>::RS : 1];
  if (gid >= (int64_t)rows_pad * C2) return;
  const int c = (int)(gid % C2);
  const int row = (int)(gid / C2);
  const int h0 = blockIdx.y * ROPE_HG;
  const int h1 = h0 + ROPE_HG < heads ? h0 + ROPE_HG : heads;
  const int i0 = c * 8;
  const bool live = row < N;
  float cs[8], sn[8];
  if (live) {
    const float pf = (float)(pos_base + row) * pos_scale;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ang = pf * inv_freq[i0 + e];
      sincosf(ang, &sn[e], &cs[e]);
      cs[e] = cs[e] * rope_scale;
      sn[e] = sn[e] * rope_scale;
    }
    // the row's (cos, sin) table, written once (first head group): the screened pass 1 rebuilds
    // a candidate key's fragments from its raw row and this table, 2 + 4 cache lines per key
    if (trig && blockIdx.y == 0) {
      float4* t = (float4*)(trig + (int64_t)row * (D / 2) + i0);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = make_float4(cs[2 * e], sn[2 * e], cs[2 * e + 1], sn[2 * e + 1]);
    }
  }
  const int rb = row >> 5, lr = row & 31, g = c & 1;
  for (int head = h0; head < h1; ++head) {
    float o1[8], o2[8];
    if (live) {
      float a[8], b[8];
      const int64_t base = (int64_t)head * head_stride + (int64_t)row * tok_stride;
      load8<DT>(x, base + i0, a);
      load8<DT>(x, base + D / 2 + i0, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p1 = a[e] * cs[e], q1 = b[e] * sn[e];
        o1[e] = p1 - q1;
        const float p2 = b[e] * cs[e], q2 = a[e] * sn[e];
        o2[e] = p2 + q2;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o1[e] = o2[e] = 0.0f;
    }
    u32x4 hi1, lo1, hi2, lo2;
    split_bf16x8(o1, hi1, lo1);
    split_bf16x8(o2, hi2, lo2);
    // dims i0.. sit in k step i0/16, dims D/2+i0.. in step (D/2+i0)/16, both in half g of the step
    const int64_t rbase = ((int64_t)head * (rows_pad >> 5) + rb) * (D / 16);
    const int64_t u1 = (rbase + (i0 >> 4)) * 2 * 64 + lr + 32 * g;
    const int64_t u2 = (rbase + ((D / 2 + i0) >> 4)) * 2 * 64 + lr + 32 * g;
    frag[u1] = hi1;
    frag[u1 + 64] = lo1;
    frag[u2] = hi2;
    frag[u2 + 64] = lo2;
    // squared norms of the row's hi and lo parts: this thread's 16 elements, then the C2 threads
    // of the row (consecutive lanes of one wave; a row's threads all pass or all fail the bounds)
    float sh = 0.0f, sl = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h0a = __uint_as_float(hi1[e] << 16), h1a = __uint_as_float(hi1[e] & 0xffff0000u);
      const float l0a = __uint_as_float(lo1[e] << 16), l1a = __uint_as_float(lo1[e] & 0xffff0000u);
      const float h0b = __uint_as_float(hi2[e] << 16), h1b = __uint_as_float(hi2[e] & 0xffff0000u);
      const float l0b = __uint_as_float(lo2[e] << 16), l1b = __uint_as_float(lo2[e] & 0xffff0000u);
      sh = fmaf(h0a, h0a, sh);
      sh = fmaf(h1a, h1a, sh);
      sh = fmaf(h0b, h0b, sh);
      sh = fmaf(h1b, h1b, sh);
      sl = fmaf(l0a, l0a, sl);
      sl = fmaf(l1a, l1a, sl);
      sl = fmaf(l0b, l0b, sl);
      sl = fmaf(l1b, l1b, sl);
    }
#pragma unroll
    for (int o = 1; o < C2; o <<= 1) {
      sh += __shfl_xor(sh, o, 64);
      sl += __shfl_xor(sl, o, 64);
    }
    if (c == 0) norms[(int64_t)head * rows_pad + row] = make_float2(sqrtf(sh), sqrtf(sl));
    if constexpr (W6) write_fp6<D>(o1, o2, hi1, hi2, c, row, head, rows_pad, lds6[threadIdx.x >> 6], planes6, scales6, dnorms6);
  }
}

// per head: the maxima of (||hi||, ||lo||) over its rows_pad rows (rows_pad even); 1024 threads
// read two rows per 16-byte load, several loads in flight per thread.  blockIdx.y picks one of two
// (norms, out) pairs, so the fp6 rounding norms take the same launch.
__global__ __launch_bounds__(1024) void norm_max_kernel(const float2* __restrict__ norms0, float2* __restrict__ out0,
                                                        const float2* __restrict__ norms1, float2* __restrict__ out1,
                                                        int rows_pad) {
  __shared__ float red[2][16];
  const int head = blockIdx.x, tid = threadIdx.x;
  const float2* norms = blockIdx.y == 0 ? norms0 : norms1;
  float2* out = blockIdx.y == 0 ? out0 : out1;
  const float4* p = (const float4*)(norms + (int64_t)head * rows_pad);
  const int n4 = rows_pad / 2;
  float mh = 0.0f, ml = 0.0f;
#pragma unroll 4
  for (int r = tid; r < n4; r += 1024) {
    const float4 v = p[r];
    mh = fmaxf(mh, fmaxf(v.x, v.z));
    ml = fmaxf(ml, fmaxf(v.y, v.w));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mh = fmaxf(mh, __shfl_xor(mh, o, 64));
    ml = fmaxf(ml, __shfl_xor(ml, o, 64));
  }
  if ((tid & 63) == 0) { red[0][tid >> 6] = mh; red[1][tid >> 6] = ml; }
  __syncthreads();
  if (tid < 64) {
    mh = tid < 16 ? red[0][tid] : 0.0f;
    ml = tid < 16 ? red[1][tid] : 0.0f;
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
      mh = fmaxf(mh, __shfl_xor(mh, o, 64));
      ml = fmaxf(ml, __shfl_xor(ml, o, 64));
    }
    if (tid == 0) out[head] = make_float2(mh, ml);
  }
}

// ------------------------------------------------------------------------------------------
// Score kernel: pass 1 (exact row max) and pass 2 (keep + votes), exact_2.py:87-140.
//
// One workgroup = one head and 256 consecutive query rows in four waves of 64 rows, one wave per
// SIMD.  A wave holds its rows' Q fragments in registers, so each K fragment it reads from LDS
// feeds two 32x32 products per k step.  Key chunks of 128 rows are copied from global memory
// straight into LDS (global_load_lds: no register staging), double-buffered, and read by all four
// waves, so each K byte fetched from L2 feeds 256 queries.  Row maxima complete inside a wave, and
// so do a tile's votes (a wave holds one 64-row tile or two 32-row tiles): one byte plane per tile.
//
// Chunks whose keys are causal for every query of the workgroup (all but the last one or two)
// take a fully unrolled path that software-pipelines the per-block epilogue (row max in pass 1,
// threshold + vote count in pass 2) of 32-key block n into the MFMA stream of block n + 1; the
// chunks on the diagonal take a per-block path with causal masking.
//
// Pass 2 compares the raw accumulator against x0 = the smallest float with fl(x0 * sm_scale)
// >= m - tau.  fl(x * c) is monotone in x for c > 0, so acc >= x0 <=> fl(acc * sm_scale) >=
// fl(m - tau), exactly the reference's keep test (exact_2.py:121), with one compare per score.
// ------------------------------------------------------------------------------------------

#define STA_GLOBAL(p) ((const __attribute__((address_space(1))) void*)(p))
#define STA_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// PQ 6 stops after pass 1: each row's keep threshold x0 on the raw dot goes to ScoreArgs.xthr
// (the fused PQ Stream sweep applies it itself).
// PQ selects the pass-2 epilogue: 0 = byte votes (shared selection); 1..3 = the per-query
// variant (tile 32): packed keep bits per key, plus weighted votes for PQ 2 (margin,
// sum of fl(s - fl(m - tau))) and PQ 3 (expmass, sum of exp(fl(s - m))) over the keeping rows
// (shared_selection_triton_perquery.py:181-217); 4 / 5 = shared selection with byte votes plus
// the tile's margin / expmass weighted votes (WMODE 1 / 2, shared_selection_triton_exact_2.py:
// 126-138).
// MODE 1 runs only the screened pass 1 (hi products, half the registers and LDS of the full
// kernel, two waves per SIMD) and leaves each row's exact maximum, or the workgroup's fallback
// flag, for MODE 0, which runs pass 2 (and the three-product pass 1 where the screen fell back).
// Waves per workgroup.  The screen: 4 (one per SIMD, two workgroups per CU).  Pass 2 with plain
// votes: 8 (two per SIMD sharing each LDS chunk; each block's epilogue follows its own MFMAs and
// the SIMD's other wave fills the gap).  Pass 2 with per-query bits, weighted votes or row counts
// needs more registers: 4 waves, each overlapping a block's epilogue with the next block's MFMAs.
template <bool RC, int PQ, int MODE>
constexpr int score_waves() { return MODE == 1 ? 4 : ((PQ == 0 && !RC) ? 8 : 4); }

template <int D, int T, bool RC, int PQ, int RB, int MODE>
__global__ __launch_bounds__((64 * score_waves<RC, PQ, MODE>()), (MODE == 1 ? 2 : 1))
void score_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  // RB 32-row blocks per wave (RB = 2: 64 query rows, RB = 4: 128); four waves, one per SIMD
  constexpr int NW = score_waves<RC, PQ, MODE>();
  constexpr bool FUSED = NW == 4;                // a block's epilogue overlaps the next one's MFMAs
  constexpr bool PLAIN = PQ == 0 && !RC;         // pass 2 writes byte votes only
  constexpr int WG_ROWS = NW * 32 * RB;          // query rows per workgroup
  constexpr int NTW = 32 * RB / T;               // tiles per wave
  constexpr int S = D / 16;                      // k steps of 16
  constexpr int CK = 64;                         // keys per LDS chunk
  constexpr int NBUF = 4;                        // chunk buffers: copies run NBUF - 1 chunks ahead
  constexpr int SBC = CK / 32;                   // 32-key blocks per chunk
  constexpr int CHUNK_UNITS = SBC * S * 2 * 64;  // u32x4 units per chunk
  constexpr int LOADS = CHUNK_UNITS / (64 * NW); // 1 KB copies per wave per chunk
  static_assert(LOADS * (NBUF - 2) < 64, "vmcnt range");
  constexpr int PER = 16 * RB / S;               // epilogue elements finished per k step
  static_assert(PER * S == 16 * RB, "epilogue split");
  static_assert(RB == 2 || RB == 4, "row blocks per wave");
  static_assert(T == 32 || T == 64, "tile");
  static_assert(PQ == 0 || PQ >= 4 || T == 32, "per-query bits pack one 32-row tile");
  constexpr bool BITS = PQ >= 1 && PQ <= 3;                          // per-query keep bits
  constexpr int WM = (PQ == 2 || PQ == 4) ? 1 : ((PQ == 3 || PQ == 5) ? 2 : 0);   // weighted votes
  // the screen keeps only the hi halves of each chunk, packed: (block, k step) unit b at b * 64;
  // after its sweep the buffers hold its candidate lists (about 50 KB)
  constexpr int LDS_UNITS = MODE == 1 ? (CHUNK_UNITS / 2 > 808 ? CHUNK_UNITS / 2 : 808) : CHUNK_UNITS;
  __shared__ u32x4 lds[NBUF][LDS_UNITS];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // +inf hidden from the optimiser: med3(x, y, pinf) = max(x, y) stays one v_med3_f32, where a
  // literal +inf is rewritten into a max with two canonicalisations
  float pinf = INFINITY;
  asm volatile("" : "+s"(pinf));
  const int rows_total = a.nt * T;               // == q_rows_pad
  const int ngroups = (rows_total + WG_ROWS - 1) / WG_ROWS;
  int h, g;
  {
    const int bid = blockIdx.x;
    if ((a.H & 7) == 0) {  // XCD-aware: workgroup i runs on XCD i % 8; keep a head on one XCD
      const int hpx = a.H >> 3;
      const int r = bid >> 3;
      h = (bid & 7) * hpx + r % hpx;
      g = ngroups - 1 - r / hpx;
    } else {
      h = bid % a.H;
      g = ngroups - 1 - bid / a.H;
    }
  }
  // plain votes: the workgroups the fp6 pass-2 kernel served are done
  if constexpr (MODE == 0 && PLAIN) {
    if (fast6_serves(a, h, g, D, WG_ROWS)) return;
  }
  const int kvh = h / (a.H / a.Hkv);
  const int wrow0 = g * WG_ROWS + wave * 32 * RB;  // first row of this wave
  const bool active = wrow0 < rows_total;
  const int hi_max = a.q_pos_base + min(g * WG_ROWS + WG_ROWS, rows_total);
  const int qpos0 = a.q_pos_base + wrow0;          // position of the wave's first row
  const int hi_w = qpos0 + 32 * RB;                // keys past the wave's last query are masked
  const int nchunks = (hi_max + CK - 1) / CK;
  // chunks entirely below N whose keys are causal for every query of the workgroup
  const int nfull = min(min(nchunks, (a.q_pos_base + g * WG_ROWS + 1) / CK), a.N / CK);
  const float tau = a.tau[h];
  // the wave's tiles j = 0 .. NTW-1 start at row wrow0 + j T; one store instruction writes two
  // tiles' rows of a key (lanes 0-31 tile j, lanes 32-63 tile j + 1)
  const int64_t trow0 = (int64_t)h * a.nt + wrow0 / T;
  uint8_t* vrow = a.votes + trow0 * a.votes_stride;
  uint32_t* brow = a.bits + trow0 * a.votes_stride;
  uint32_t* wrow = (uint32_t*)a.wvotes + trow0 * a.votes_stride;
  auto tile_ok = [&](int j) { return wrow0 + j * T < rows_total; };

  // ---- Q fragments of this wave's rows (kept in AGPRs: they are only MFMA operands) ----
  u32x4 qhi[RB][S], qlo[RB][S];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const bool ok = wrow0 + 32 * rb < rows_total;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int64_t u = (((int64_t)h * (a.q_rows_pad >> 5) + wrow0 / 32 + rb) * S + s) * 128 + lane;
      qhi[rb][s] = ok ? a.qfrag[u] : u32x4{0, 0, 0, 0};
      if constexpr (MODE == 0) asm volatile("" : "+a"(qhi[rb][s]));
      if constexpr (MODE == 0) {
        qlo[rb][s] = ok ? a.qfrag[u + 64] : u32x4{0, 0, 0, 0};
        asm volatile("" : "+a"(qlo[rb][s]));
      }
    }
  }
  const u32x4* kbase = a.kfrag + (int64_t)kvh * (a.k_rows_pad >> 5) * S * 128;
  // copy key chunk c into dst: 1 KB per instruction, lane l's 16 bytes land at dst + 16 l
  auto issue = [&](int c, u32x4* dst) {
    const u32x4* src = kbase + (int64_t)c * CHUNK_UNITS + lane;
#pragma unroll
    for (int e = 0; e < LOADS; ++e) {
      const int u = (e * NW + wave) * 64;
      copy16_to_lds(src + u, lds_addr(dst + u));
    }
  };
  // wait until at most n chunks' copies of this wave are in flight.  Vector memory operations
  // complete in issue order, so this leaves only the n most recently issued chunks pending (vote
  // stores issued in between only make the wait stricter).
  auto wait_copies = [&](int n) {
    constexpr int E = (7 << 4) | (15 << 8);   // expcnt / lgkmcnt: no wait
    constexpr int L1 = LOADS, L2 = 2 * LOADS;
    if (n <= 0) __builtin_amdgcn_s_waitcnt(E);
    else if (n == 1) __builtin_amdgcn_s_waitcnt(E | (L1 & 15) | ((L1 >> 4) << 14));
    else __builtin_amdgcn_s_waitcnt(E | (L2 & 15) | ((L2 >> 4) << 14));
  };
  static_assert(NBUF == 4, "wait_copies covers up to two newer chunks");

  // per-query epilogue of one score: bit `row` of the key's mask, and its weighted vote
  // (i indexes the lane's 16 accumulator rows of a 32-row block: row = (i/4)*8 + 4*(lane/32) +
  // i%4; the lane half's 4-row offset is applied when the mask is stored)
  auto pq_acc = [&](int keep, float v, float ref, int i, uint32_t& bm, float& w) {
#pragma clang fp contract(off)
    if constexpr (BITS) bm |= (uint32_t)keep << ((i >> 2) * 8 + (i & 3));
    if constexpr (WM == 1) {
      const float qk = v * a.sm_scale;
      const float c = qk - ref;
      w += keep ? c : 0.0f;
    } else if constexpr (WM == 2) {
      const float qk = v * a.sm_scale;
      const float e = __expf(qk - ref);
      w += keep ? e : 0.0f;
    }
  };
  // pass-2 accumulation of one score: the vote count, and bits / weighted votes
  auto acc2 = [&](int keep, float v, float ref, int i, int& cnt, uint32_t& bm, float& w) {
    if constexpr (!BITS) cnt += keep;
    if constexpr (PQ != 0) pq_acc(keep, v, ref, i, bm, w);
  };
  // the key's pass-2 results of this wave's rows -> votes (exact_2.py:123) or bits + weighted
  // votes; lanes 0-31 and 32-63 hold complementary rows of the same key
  auto store_key = [&](int key, bool check, const int* cnt, const uint32_t* bm, const float* w) {
    const bool key_ok = !check || key < a.N;
    if constexpr (!BITS) {
      int tot[NTW];
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        int c = 0;
#pragma unroll
        for (int rb = j * T / 32; rb < (j + 1) * T / 32; ++rb) c += cnt[rb];
        tot[j] = c + __shfl_xor(c, 32, 64);
      }
      float wt[NTW];   // the tile's weighted vote (WMODE 1 / 2), summed like the counts
      if constexpr (WM > 0) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          float x = 0.0f;
#pragma unroll
          for (int rb = j * T / 32; rb < (j + 1) * T / 32; ++rb) x += w[rb];
          wt[j] = x + __shfl_xor(x, 32, 64);
        }
      }
      if constexpr (NTW == 1) {
        if (lane < 32 && active && key_ok) {
          vrow[key] = (uint8_t)tot[0];
          if constexpr (WM > 0) wrow[key] = __float_as_uint(wt[0]);
        }
      } else {
#pragma unroll
        for (int j2 = 0; j2 < NTW; j2 += 2) {
          const int j = j2 + (lane >> 5);
          if (tile_ok(j) && key_ok) {
            vrow[j * a.votes_stride + key] = (uint8_t)(lane < 32 ? tot[j2] : tot[j2 + 1]);
            if constexpr (WM > 0) wrow[j * a.votes_stride + key] = __float_as_uint(lane < 32 ? wt[j2] : wt[j2 + 1]);
          }
        }
      }
    } else {   // tile 32: one tile per row block
      uint32_t b[RB];
      float ww[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        b[rb] = bm[rb] << (4 * (lane >> 5));   // rows of the upper lane half sit 4 bits higher
        b[rb] |= __shfl_xor(b[rb], 32, 64);
        ww[rb] = w[rb];
        if constexpr (WM > 0) ww[rb] += __shfl_xor(w[rb], 32, 64);
      }
#pragma unroll
      for (int j2 = 0; j2 < RB; j2 += 2) {
        const int j = j2 + (lane >> 5);
        if (tile_ok(j) && key_ok) {
          brow[j * a.votes_stride + key] = lane < 32 ? b[j2] : b[j2 + 1];
          if constexpr (WM > 0) wrow[j * a.votes_stride + key] = __float_as_uint(lane < 32 ? ww[j2] : ww[j2 + 1]);
        }
      }
    }
  };

  float mx[RB][16];   // pass 1: running max of the raw dot per row slot; pass 2: the keep
                      // threshold x0 on the raw dot
  float ref[RB][16];  // pass 2, weighted votes: fl(m - tau) / m of the row, the weight's origin
  int rc[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) { ref[rb][i] = 0.0f; rc[rb][i] = 0; }

  // 32 keys x this wave's rows, one k step: hi.hi + hi.lo + lo.hi, small terms first
  auto mfma3 = [&](u32x4 bh, u32x4 bl, int s, floatx16* acc) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qlo[rb][s], bh, acc[rb]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bl, acc[rb]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bh, acc[rb]);
  };
  auto ldb = [&](const u32x4* buf, int sb, int s, int hl) { return buf[(sb * S + s) * 128 + 64 * hl + lane]; };
  // Instruction schedule of one 32-key block (S k steps): the K fragments of step s + 1 are read
  // while step s's MFMAs run, and the VALU work available (the previous block's epilogue) is
  // interleaved between the MFMAs.  One wave per SIMD has no other wave to hide LDS latency.  The
  // reads for step s + 2 follow step s + 1's first MFMA, so the LDS wait in front of that MFMA
  // covers only reads issued a whole step earlier.
  auto block_schedule = [&](auto valuc) {
    constexpr int valu_per_mfma = decltype(valuc)::value;
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);        // reads of steps 0 and 1
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int m = 0; m < 3 * RB; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
        if (m == 0 && s >= 1 && s + 1 < S) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // step s + 1
        if constexpr (valu_per_mfma > 0) __builtin_amdgcn_sched_group_barrier(0x002, valu_per_mfma, 0);
      }
    }
  };
  // all k steps of block sb, with the next step's K fragments read ahead
  auto mfma_block = [&](const u32x4* buf, int sb, floatx16* acc) {
    u32x4 bh = ldb(buf, sb, 0, 0), bl = ldb(buf, sb, 0, 1);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      u32x4 nh = bh, nl = bl;
      if (s + 1 < S) { nh = ldb(buf, sb, s + 1, 0); nl = ldb(buf, sb, s + 1, 1); }
      mfma3(bh, bl, s, acc);
      bh = nh;
      bl = nl;
    }
    block_schedule(std::integral_constant<int, 0>{});
  };
  // epilogue of one (unmasked) score
  auto epi = [&](auto passc, float v, int rb, int i, int* cnt, uint32_t* bm, float* w) {
    constexpr int pass = decltype(passc)::value;
    if constexpr (pass == 0) {
      mx[rb][i] = __builtin_amdgcn_fmed3f(v, mx[rb][i], pinf);   // max; scores are finite
    } else if constexpr (PLAIN) {
      // rows dropped: the sign of v - x0 (exact: two distinct floats never subtract to zero,
      // equal ones give +0; x0 = +inf on padded rows), counted with one shift-add
      cnt[rb] += (int)(__float_as_uint(v - mx[rb][i]) >> 31);
    } else {
      const int keep = v >= mx[rb][i];
      acc2(keep, v, ref[rb][i], i, cnt[rb], bm[rb], w[rb]);
      if constexpr (RC) rc[rb][i] += keep;
    }
  };
  // MFMAs of block sb into accN; when HAS_PREV, the epilogue of the previous (unmasked) block
  // accO at keys keyO.. is finished in slices between the k steps
  auto fused_block = [&](auto passc, auto prevc, const u32x4* buf, int sb, floatx16* accN,
                         const floatx16* accO, int keyO) {
    constexpr int pass = decltype(passc)::value;
    constexpr bool HAS_PREV = decltype(prevc)::value;
    int cnt[RB] = {};
    uint32_t bm[RB] = {};
    float w[RB] = {};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) accN[rb] = floatx16{};
    u32x4 bh = ldb(buf, sb, 0, 0), bl = ldb(buf, sb, 0, 1);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      u32x4 nh = bh, nl = bl;
      if (s + 1 < S) { nh = ldb(buf, sb, s + 1, 0); nl = ldb(buf, sb, s + 1, 1); }
      mfma3(bh, bl, s, accN);
      bh = nh;
      bl = nl;
      if constexpr (HAS_PREV) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int idx = s * PER + e, rb = idx / 16, i = idx % 16;
          epi(passc, accO[rb][i], rb, i, cnt, bm, w);
        }
      }
    }
    if constexpr (HAS_PREV && pass == 1) {
      if constexpr (PLAIN) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) cnt[rb] = 16 - cnt[rb];   // dropped -> kept of the 16 rows
      }
      store_key(keyO + (lane & 31), false, cnt, bm, w);
    }
    block_schedule(std::integral_constant<int, HAS_PREV ? 2 : 0>{});
  };
  // Pass 2 of the 8-wave workgroups on fully causal chunks: one row block's MFMAs at a time, the
  // other row block's vote epilogue interleaved between them (two accumulators; the epilogue of
  // the block's first row block runs under its second's MFMAs, that of the second under the next
  // block's first).  A per-chunk barrier starts both waves of a SIMD in the same phase, so the
  // epilogue has to hide inside each wave's own MFMA stream.
  constexpr int NE = 16 / S;                   // epilogue scores per k step (16 rows per slot set)
  static_assert(NE * S == 16, "epilogue slices");
  auto half_block = [&](const u32x4* buf, int sb, int rbn, floatx16& acc, const floatx16& accE,
                        int rbe, int& dropped) {
    acc = floatx16{};
    u32x4 bh = ldb(buf, sb, 0, 0), bl = ldb(buf, sb, 0, 1);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      u32x4 nh = bh, nl = bl;
      if (s + 1 < S) { nh = ldb(buf, sb, s + 1, 0); nl = ldb(buf, sb, s + 1, 1); }
      acc = mfma32(qlo[rbn][s], bh, acc);
      acc = mfma32(qhi[rbn][s], bl, acc);
      acc = mfma32(qhi[rbn][s], bh, acc);
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int i = s * NE + e;
        dropped += (int)(__float_as_uint(accE[i] - mx[rbe][i]) >> 31);
      }
      bh = nh;
      bl = nl;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);        // reads of step 0
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
        if (m == 0 && s + 1 < S) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // step s + 1
        __builtin_amdgcn_sched_group_barrier(0x002, 2 * NE / 3 + 1, 0);
      }
    }
  };
  // the last block's epilogue when nothing follows it
  auto flush = [&](auto passc, const floatx16* acc, int key0) {
    constexpr int pass = decltype(passc)::value;
    int cnt[RB] = {};
    uint32_t bm[RB] = {};
    float w[RB] = {};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) epi(passc, acc[rb][i], rb, i, cnt, bm, w);
    if constexpr (pass == 1) {
      if constexpr (PLAIN) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) cnt[rb] = 16 - cnt[rb];
      }
      store_key(key0 + (lane & 31), false, cnt, bm, w);
    }
  };

  // ---- screened pass 1 ----------------------------------------------------------------------
  // The sweep computes only s1 = hi(q).hi(k), one product instead of three.  With x = hi + lo per
  // operand, the three-product score differs from s1 by the cross terms, so by Cauchy-Schwarz
  //   |x(q).x(k) - s1| <= ||q_hi|| ||k_lo|| + ||q_lo|| ||k_hi|| + ||q_lo|| ||k_lo|| + (rounding),
  // and with E that bound (maximised over the head's keys), only keys whose s1 lies within 2 E of
  // the row's largest s1 can hold the row's exact maximum.  Each accumulator slot (one row, the
  // keys of one lane column) keeps its three largest s1 values with the 32-key block index packed
  // into the low `ib` mantissa bits (a relative change below 2^(ib-23), added to E).  After the
  // sweep the candidates -- slot values within 2 E of the row maximum -- are evaluated exactly as
  // fp32 dot products of the (hi + lo) operands, and the row maximum is their maximum.  A slot
  // whose third value is a candidate may hide a fourth: then every key of that slot is evaluated
  // (a few hundred keys; about 5% of workgroups meet one on Gaussian inputs).  A wave that
  // collects more than FMAX candidates sends its workgroup to the three-product sweep instead
  // (inputs with many tied scores).
  constexpr int FMAX = 1536;                     // candidate (row, key) pairs per wave
  constexpr int LOADS_H = LOADS / 2;             // 1 KB copies per wave per chunk, hi halves only
  static_assert(LOADS_H * NW * 2 * 64 == CHUNK_UNITS, "hi-half copies");
  // wave-uniform chunk bases in SGPRs and one lane offset: per-lane 64-bit addresses would hold
  // VGPRs through the sweep
  const uint32_t loff_h = (uint32_t)lane * 16u;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto issue_hi = [&](int c, u32x4* dst) {
    const u32x4* src = kbase + (int64_t)c * CHUNK_UNITS;
#pragma unroll
    for (int e = 0; e < LOADS_H; ++e) {
      const int b = e * NW + wave_s;           // (32-key block, k step) b: its hi units, packed
      copy16_to_lds_s(src + 128 * b, loff_h, lds_addr(dst + 64 * b));
    }
  };
  auto ldbh = [&](const u32x4* buf, int sb, int s) { return buf[(sb * S + s) * 64 + lane]; };
  auto wait_hi = [&](int n) {
    constexpr int E = (7 << 4) | (15 << 8);
    constexpr int L1 = LOADS_H, L2 = 2 * LOADS_H;
    if (n <= 0) __builtin_amdgcn_s_waitcnt(E);
    else if (n == 1) __builtin_amdgcn_s_waitcnt(E | (L1 & 15) | ((L1 >> 4) << 14));
    else __builtin_amdgcn_s_waitcnt(E | (L2 & 15) | ((L2 >> 4) << 14));
  };
  float t1[RB][16], t2[RB][16], t3[RB][16];
  const uint32_t blk_mask = (1u << a.ib) - 1u;
  // fold one score into its slot's top three (v finite; masked scores arrive as -FLT_MAX); blk
  // sits in a VGPR so that the packing is one v_and_or_b32 with the mask in an SGPR
  auto sepi = [&](float v, int rb, int i, uint32_t blk) {
    const float p = __uint_as_float((__float_as_uint(v) & ~blk_mask) | blk);
    t3[rb][i] = __builtin_amdgcn_fmed3f(t2[rb][i], t3[rb][i], p);
    t2[rb][i] = __builtin_amdgcn_fmed3f(t1[rb][i], t2[rb][i], p);
    t1[rb][i] = __builtin_amdgcn_fmed3f(t1[rb][i], p, pinf);
  };
  auto vgpr = [](uint32_t x) {
    asm("" : "+v"(x));
    return x;
  };
  auto s_schedule = [&](auto valuc) {
    constexpr int V = decltype(valuc)::value;
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);        // reads of steps 0 and 1
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int m = 0; m < RB; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
        if (m == 0 && s >= 1 && s + 1 < S) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // step s + 1
        if constexpr (V > 0) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
      }
    }
  };
  // hi.hi products of block sb into accN; with HAS_PREV the previous (unmasked) block accO of
  // 32-key block index blkO is folded into the top threes between the k steps
  auto s_block = [&](auto prevc, const u32x4* buf, int sb, floatx16* accN, const floatx16* accO, uint32_t blkO) {
    constexpr bool HAS_PREV = decltype(prevc)::value;
    const uint32_t bv = HAS_PREV ? vgpr(blkO) : 0u;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) accN[rb] = floatx16{};
    u32x4 bh = ldbh(buf, sb, 0);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      u32x4 nh = bh;
      if (s + 1 < S) nh = ldbh(buf, sb, s + 1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) accN[rb] = mfma32(qhi[rb][s], bh, accN[rb]);
      bh = nh;
      if constexpr (HAS_PREV) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int idx = s * PER + e;
          sepi(accO[idx / 16][idx % 16], idx / 16, idx % 16, bv);
        }
      }
    }
    s_schedule(std::integral_constant<int, HAS_PREV ? 4 * PER / RB : 0>{});
  };
  auto s_flush = [&](const floatx16* acc, uint32_t blk) {
    const uint32_t bv = vgpr(blk);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) sepi(acc[rb][i], rb, i, bv);
  };
  // returns true when the workgroup has to run the three-product sweep; otherwise mx holds every
  // row's exact raw maximum
  auto run_screened = [&]() -> bool {
    constexpr std::integral_constant<bool, true> kPrev{};
    const float lowest = __uint_as_float(0xff7fffffu & ~blk_mask);   // -FLT_MAX, block 0
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) { t1[rb][i] = lowest; t2[rb][i] = lowest; t3[rb][i] = lowest; }
    static_assert(MODE != 1 || 32 * RB == 64, "one wave row per lane");
    // the norm part of row (wave row `lane`)'s error bound E, loaded before the sweep: the
    // candidate phase reads it with a lane shuffle instead of one dependent load per slot
    const float2 kn = a.knorm_max[kvh];
    // 2^-14 covers the fp32 accumulation of s1 and of the exact dots; 2^(ib-23) the packing
    const float gam = 0x1p-14f + __uint_as_float((uint32_t)(127 + a.ib - 23) << 23);
    float ebase = 0.0f;
    if (active && wrow0 + lane < a.N) {
      const float2 qn = a.qnorm[(int64_t)h * a.q_rows_pad + wrow0 + lane];
      ebase = 1.001f * (qn.x * kn.y + qn.y * kn.x + qn.y * kn.y + gam * qn.x * kn.x);
    }
    // nothing the compiler tracks is in flight past this point: its own waits then stay out of
    // the sweep, whose copies it does not see
    __builtin_amdgcn_s_waitcnt(0);
    for (int c = 0; c < NBUF - 1; ++c) issue_hi(min(c, nchunks - 1), lds[c]);
    wait_hi(NBUF - 2);
    __syncthreads();
    floatx16 accA[RB], accB[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) accB[rb][i] = lowest;
    // one loop per kind of chunk, each with a single path through its body (loop-carried top
    // threes then keep their registers instead of being copied at every join)
    // Every step issues one chunk's copies: past the last chunk it copies the last chunk again
    // into the buffer no later step reads, which keeps the body branch-free and the waits fixed
    // (the stray copies are drained before the buffers are reused).
    auto step_begin = [&](int c) {
      issue_hi(min(c + NBUF - 1, nchunks - 1), lds[(c + NBUF - 1) % NBUF]);
    };
    auto step_end = [&](int c) {   // chunk c + 1's copies have landed, every wave is done with c
      (void)c;
      wait_hi(NBUF - 2);
      __syncthreads();
    };
    int c = 0;
    if (active) {
      for (; c < nfull; ++c) {
        step_begin(c);
        const u32x4* buf = lds[c % NBUF];
        const uint32_t blk0 = (uint32_t)(c * SBC);
        // accB: the previous chunk's second block (before the first chunk: `lowest`, a no-op)
        s_block(kPrev, buf, 0, accA, accB, c > 0 ? blk0 - 1 : 0u);
        s_block(kPrev, buf, 1, accB, accA, blk0);
        step_end(c);
      }
      s_flush(accB, nfull > 0 ? (uint32_t)(nfull * SBC - 1) : 0u);
      for (; c < nchunks; ++c) {
        step_begin(c);
        const u32x4* buf = lds[c % NBUF];
        for (int sb = 0; sb < SBC; ++sb) {
          const int key0 = c * CK + sb * 32;
          if (key0 >= hi_w) break;
          floatx16 acc[RB];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) acc[rb] = floatx16{};
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const u32x4 bh = ldbh(buf, sb, s);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bh, acc[rb]);
          }
          // key <= qpos0 + row, with the slot's row split into a lane part and a constant
          const int dk = key0 + (lane & 31) - qpos0 - (lane >> 5) * 4;
          const bool diag = key0 + 31 > qpos0;
          const uint32_t bv = vgpr((uint32_t)(key0 >> 5));
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const bool causal = !diag || dk <= rb * 32 + (i >> 2) * 8 + (i & 3);   // exact_2.py:101
              sepi(causal ? acc[rb][i] : -FLT_MAX, rb, i, bv);
            }
        }
        step_end(c);
      }
    } else {
      for (; c < nchunks; ++c) {
        step_begin(c);
        step_end(c);
      }
    }
    wait_hi(0);        // the stray copies past the last chunk
    __syncthreads();

    // ---- candidates: per row, slot values within 2 E of the row's largest s1, into one flat
    // (row, key) list per wave ----
    constexpr int WR = 32 * RB;                                // rows of a wave
    static_assert(MODE != 1 || (2 + 2 * WR + 2 * FMAX) * 4 * NW <= (int)sizeof(lds), "candidate lists fit the chunk buffers");
    int* wl = (int*)&lds[0][0] + wave * (2 + 2 * WR + 2 * FMAX);
    int* nflat = wl;                                           // list length
    uint32_t* rowbest = (uint32_t*)(wl + 2);                  // WR rows: order key of the max
    int* rowcnt = wl + 2 + WR;                                 // WR rows: candidates, then fill points
    int* frow = wl + 2 + 2 * WR;                               // FMAX rows
    int* fkey = frow + FMAX;                                   // FMAX keys
    if (lane == 0) nflat[0] = 0;
    for (int r = lane; r < WR; r += 64) {
      rowbest[r] = 0u;
      rowcnt[r] = 0;
    }
    bool amb = false;
    __syncthreads();
    float thr[RB][16];
    const int col = lane & 31;
    auto slot_keys = [&](int row) {
      const int qpos = a.q_pos_base + wrow0 + row;
      return qpos >= col ? (qpos - col) / 32 + 1 : 0;
    };
    // the number of list entries of a slot: every key of the slot when its third value is a
    // candidate (a fourth may hide behind it; its column's causal keys j <= the row's position),
    // otherwise its values within the threshold
    auto slot_count = [&](int rb, int i) {
      const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      const float th = thr[rb][i];
      const int n3 = (int)(t1[rb][i] >= th) + (int)(t2[rb][i] >= th) + (int)(t3[rb][i] >= th);
      return t3[rb][i] >= th ? slot_keys(row) : n3;
    };
    if (active) {
      // row maxima and thresholds of all slots first, with no control flow: the 32 butterfly
      // reductions interleave instead of waiting out one shuffle latency after another
      // (lane-to-lane moves in registers: DPP within 16-lane rows, then a swap of row pairs)
      auto dpp = [](float v, auto ctrlc) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), decltype(ctrlc)::value, 0xF, 0xF, false));
      };
      auto row32_max = [&](float v) {
        v = __builtin_amdgcn_fmed3f(v, dpp(v, std::integral_constant<int, 0xB1>{}), pinf);    // lane ^ 1
        v = __builtin_amdgcn_fmed3f(v, dpp(v, std::integral_constant<int, 0x4E>{}), pinf);    // lane ^ 2
        v = __builtin_amdgcn_fmed3f(v, dpp(v, std::integral_constant<int, 0x141>{}), pinf);   // 7 - lane in 8
        v = __builtin_amdgcn_fmed3f(v, dpp(v, std::integral_constant<int, 0x140>{}), pinf);   // 15 - lane in 16
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __builtin_amdgcn_fmed3f(__uint_as_float(r[0]), __uint_as_float(r[1]), pinf);  // rows 2k, 2k+1
      };
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float v = row32_max(t1[rb][i]);
          const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          const int r0 = rb * 32 + (i >> 2) * 8 + (i & 3);     // the row of lanes 0-31; lanes 32-63: + 4
          const float e0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ebase), r0));
          const float e1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ebase), r0 + 4));
          const float E = (lane < 32 ? e0 : e1) + 0x1p-20f * fabsf(v);
          const float th = v - 2.0f * E;
          // padded rows never vote: their maximum is unused (no value reaches +inf)
          const bool valid = wrow0 + row < a.N;
          amb |= valid && !(th > -1e38f);
          thr[rb][i] = valid ? th : INFINITY;
        }
      // the list is ordered by row (neighbouring pairs share the Q fragments' cache lines):
      // per-row counts first
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int n = slot_count(rb, i);
          if (n > 0) atomicAdd(&rowcnt[rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3)], n);
        }
    }
    __syncthreads();
    if (active) {   // row starts: an exclusive scan of the wave's 64 row counts, lane = row
      const int c = rowcnt[lane];
      int incl = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      rowcnt[lane] = incl - c;
      if (lane == 63) nflat[0] = incl;
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int n = slot_count(rb, i);
          if (n > 0) {
            const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            const float th = thr[rb][i];
            int f = atomicAdd(&rowcnt[row], n);
            if (t3[rb][i] >= th) {
              for (int b = 0; b < n; ++b, ++f)
                if (f < FMAX) {
                  frow[f] = row;
                  fkey[f] = col + 32 * b;
                }
            } else {
              const float tv[3] = {t1[rb][i], t2[rb][i], t3[rb][i]};
#pragma unroll
              for (int k3 = 0; k3 < 3; ++k3) {
                if (tv[k3] >= th) {
                  if (f < FMAX) {
                    frow[f] = row;
                    fkey[f] = (int)(((__float_as_uint(tv[k3]) & blk_mask) << 5) | (uint32_t)col);
                  }
                  ++f;
                }
              }
            }
          }
        }
    }
    __syncthreads();
    const int total = nflat[0];
    amb |= total > FMAX;
    if (__syncthreads_or(amb)) return true;

    // ---- exact scores of the candidates on the matrix cores, 32 list entries per round: entry
    // f's key is B column f (lanes f and f + 32 load its two dims halves: the fragment layout),
    // the wave's rows are the A operands (qhi held since the sweep, qlo loaded here in the same
    // layout), and the four products hi.hi + hi.lo + lo.hi + lo.lo over a 32-row block give each
    // (row, key) score of the round in fp32 (every product exact, the sums rounded within the
    // 2^-14 allowance of E); entry f reads its own (row, key) score from the result block.  The
    // next round's key fragments load while a round's scores are read out. ----
    if (active) {
      const int g = lane >> 5;
      // the rows' lo fragments, loaded per round for the row block it needs (from the L2: the
      // wave reads the same 16 KB every round) rather than held through the phase
      auto load_qlo = [&](int rb, u32x4* ql) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int64_t u = (((int64_t)h * (a.q_rows_pad >> 5) + wrow0 / 32 + rb) * S + s) * 128 + lane;
          ql[s] = a.qfrag[u + 64];
        }
      };
      u32x4 kh[S], kl[S];
      // a key's hi / lo operands of k steps s (dims s * 16 + 8 g ..) for this lane's half g: from
      // its raw row and (cos, sin) table row with the rope pre-kernel's own arithmetic (the same
      // fp32 rotation and split, so the same bits as its fragments), or from the fragments
      auto load8_rt = [&](int64_t i, float* out) {
        if (a.kraw_dt == DT_BF16) load8<DT_BF16>(a.kraw, i, out);
        else if (a.kraw_dt == DT_F16) load8<DT_F16>(a.kraw, i, out);
        else load8<DT_F32>(a.kraw, i, out);
      };
      auto load_keys = [&](int key) {
        if (a.ktrig) {
          const float4* tp = (const float4*)(a.ktrig + (int64_t)key * (D / 2));
          const int64_t rbase = (int64_t)kvh * a.kraw_hs + (int64_t)key * a.kraw_ts;
#pragma unroll
          for (int s = 0; s < S / 2; ++s) {
            const int d0 = s * 16 + g * 8;       // dims d0.. in step s, D/2 + d0.. in step s + S/2
            float x1[8], x2[8], o1[8], o2[8];
            load8_rt(rbase + d0, x1);
            load8_rt(rbase + D / 2 + d0, x2);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float4 t = tp[d0 / 2 + e];   // (cos, sin) of dims d0 + 2e and d0 + 2e + 1
              const float c2[2] = {t.x, t.z}, s2[2] = {t.y, t.w};
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const float xa = x1[2 * e + j], xb = x2[2 * e + j];
                const float p1 = xa * c2[j], q1 = xb * s2[j];
                o1[2 * e + j] = p1 - q1;
                const float p2 = xb * c2[j], q2 = xa * s2[j];
                o2[2 * e + j] = p2 + q2;
              }
            }
            split_bf16x8(o1, kh[s], kl[s]);
            split_bf16x8(o2, kh[s + S / 2], kl[s + S / 2]);
          }
        } else {
          const u32x4* kp = kbase + (int64_t)(key >> 5) * S * 128 + (key & 31) + 32 * g;
#pragma unroll
          for (int s = 0; s < S; ++s) {
            kh[s] = kp[s * 128];
            kl[s] = kp[s * 128 + 64];
          }
        }
      };
      auto scores = [&](int rb) {
        u32x4 ql[S];
        load_qlo(rb, ql);
        floatx16 acc = {};
#pragma unroll
        for (int s = 0; s < S; ++s) {
          acc = mfma32(qhi[rb][s], kh[s], acc);
          acc = mfma32(qhi[rb][s], kl[s], acc);
          acc = mfma32(ql[s], kh[s], acc);
          acc = mfma32(ql[s], kl[s], acc);
        }
        return acc;
      };
      int f = col;
      bool valid = f < total;
      int row = valid ? frow[f] : 0;
      load_keys(valid ? fkey[f] : 0);          // key 0 stands in for a padding entry
      for (int it = 0; it * 32 < total; ++it) {
        const int rbr = row >> 5;
        // rows are listed in order, so a round's entries mostly share one row block
        const bool in0 = __ballot(valid && rbr == 0) != 0, in1 = __ballot(valid && rbr == 1) != 0;
        floatx16 acc0 = {}, acc1 = {};
        if (in0) acc0 = scores(0);
        if (in1) acc1 = scores(RB - 1);
        const int fn = f + 32;
        const bool validn = fn < total;
        const int rown = validn ? frow[fn] : 0;
        if ((it + 1) * 32 < total) load_keys(validn ? fkey[fn] : 0);
        // (row r, column col) of a 32x32 block: lane col + 32 ((r >> 2) & 1), element (r >> 3) * 4 + (r & 3)
        const int rr = row & 31;
        const int e0 = (rr >> 3) * 4 + (rr & 3);
        float v = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) v = e == e0 ? (rbr == 0 ? acc0[e] : acc1[e]) : v;
        // order-preserving key of an fp32 value (every key of a real value is nonzero)
        const uint32_t tb = __float_as_uint(v + 0.0f);
        const uint32_t okey = (tb & 0x80000000u) ? ~tb : (tb | 0x80000000u);
        if (valid && ((rr >> 2) & 1) == g) atomicMax(&rowbest[row], okey);
        f = fn;
        valid = validn;
        row = rown;
      }
    }
    __syncthreads();
    if (active) {
      // every slot takes its row's exact maximum
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t k = rowbest[rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3)];
          const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
          mx[rb][i] = k ? __uint_as_float(b) : 0.0f;   // 0: a padded row, never used
        }
    }
    __syncthreads();   // the candidate lists are read before the next sweep's copies land
    return false;
  };

  // row max over the 32 lanes holding a row's keys (mx: the raw dot's running max per row slot),
  // then the keep threshold x0 on the raw dot, and the weighted-vote origins.
  // screened: the maximum came from the screen's four-product fp32 scores of the (hi + lo)
  // operands, which differ from pass 2's three-product value of the same key by the lo.lo term
  // and the two summation orders.  For tau >= 0 the threshold is then capped at max - delta, with delta a
  // bound on that difference, so the row's best key keeps its vote (the reference's two passes
  // share one dot, exact_2.py:100, 118, so qk == m passes whenever tau >= 0); for tau above
  // delta * scale (1e-5 at unit-scale rows) the cap changes nothing.  A negative tau keeps no key
  // in the reference, and no cap applies.
  auto finish1 = [&](bool screened) {
    const float2 knm = a.knorm_max[kvh];
    if (active) {
      // complete the row max over the 32 lanes holding a row's keys, then the threshold
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float v = mx[rb][i];
          v = fmaxf(v, __shfl_xor(v, 1, 64));
          v = fmaxf(v, __shfl_xor(v, 2, 64));
          v = fmaxf(v, __shfl_xor(v, 4, 64));
          v = fmaxf(v, __shfl_xor(v, 8, 64));
          v = fmaxf(v, __shfl_xor(v, 16, 64));
          const float m = v * a.sm_scale;   // fl(max * c) == max of fl(s * c) for c > 0
          const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          const bool ok = wrow0 + row < a.N;   // padded rows never vote (exact_2.py:121)
          float x0 = ok ? min_arg_for(m - tau, a.sm_scale) : INFINITY;
          if (screened && ok && tau >= 0.0f) {
            const float2 qn = a.qnorm[(int64_t)h * a.q_rows_pad + wrow0 + row];
            const float delta = 1.001f * (qn.y * knm.y + 0x1p-15f * (qn.x + qn.y) * (knm.x + knm.y));
            x0 = fminf(x0, v - delta);
          }
          mx[rb][i] = x0;
          if constexpr (WM == 1) ref[rb][i] = m - tau;   // perquery.py:210; exact_2.py:130
          if constexpr (WM == 2) ref[rb][i] = m;         // perquery.py:215; exact_2.py:135
          if (a.row_max && (lane & 31) == 0 && ok) a.row_max[(int64_t)h * a.N + wrow0 + row] = m;
        }
    }
  };

  auto run_pass = [&](auto passc) {
    constexpr int pass = decltype(passc)::value;
    constexpr std::integral_constant<bool, true> kPrev{};
    constexpr std::integral_constant<bool, false> kNoPrev{};
    if constexpr (pass == 0) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx[rb][i] = -INFINITY;
    }
    // nothing the compiler tracks is in flight past this point: its own waits then stay out of
    // the sweep, whose copies it does not see
    __builtin_amdgcn_s_waitcnt(0);
    for (int c = 0; c < NBUF - 1 && c < nchunks; ++c) issue(c, lds[c]);
    wait_copies(min(nchunks, NBUF - 1) - 1);
    __syncthreads();
    floatx16 accA[RB], accB[RB];
    bool pendingB = false;   // accB holds an unmasked block whose epilogue is still due
    int keyB = 0;
    // the buffer chunk c + NBUF - 1 lands in was last read in chunk c - 1, before the barrier
    auto chunk_begin = [&](int c) {
      if (c + NBUF - 1 < nchunks) issue(c + NBUF - 1, lds[(c + NBUF - 1) % NBUF]);
    };
    // chunk c + 1's copies have landed in LDS and every wave is done with chunk c
    auto chunk_end = [&](int c) {
      if (c + 1 < nchunks) wait_copies(min(nchunks - 1, c + NBUF - 1) - (c + 1));
      __syncthreads();
    };
    int c = 0;
    // the row-block pipeline (8-wave pass 2) over the fully causal chunks: pacc1 holds the
    // pending block's second row block, pdrop0 its first one's dropped-row count
    constexpr bool PIPE = !FUSED && PLAIN && pass == 1 && RB == 2;
    if constexpr (PIPE) {
      floatx16 pacc0 = floatx16{}, pacc1 = floatx16{};
      int pdrop0 = 0, pkey = 0;
      auto pipe_store = [&](int drop1) {
        int cnt[RB];
        cnt[0] = 16 - pdrop0;
        cnt[RB - 1] = 16 - drop1;
        uint32_t bm[RB] = {};
        float w[RB] = {};
        store_key(pkey + (lane & 31), false, cnt, bm, w);
      };
      for (; c < nfull; ++c) {
        chunk_begin(c);
        const u32x4* buf = lds[c % NBUF];
        if (active) {
#pragma unroll
          for (int sb = 0; sb < SBC; ++sb) {
            int d1 = 0, d0 = 0;
            half_block(buf, sb, 0, pacc0, pacc1, RB - 1, d1);     // row block 0; previous block's 1
            if (c > 0 || sb > 0) pipe_store(d1);
            half_block(buf, sb, RB - 1, pacc1, pacc0, 0, d0);     // row block 1; this block's 0
            pdrop0 = d0;
            pkey = c * CK + sb * 32;
          }
        }
        chunk_end(c);
      }
      if (active && nfull > 0) {
        int d1 = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) d1 += (int)(__float_as_uint(pacc1[i] - mx[RB - 1][i]) >> 31);
        pipe_store(d1);
      }
    }
    for (; c < nchunks; ++c) {
      chunk_begin(c);
      const u32x4* buf = lds[c % NBUF];
      if (active) {
        if (FUSED && c < nfull) {
          if (c == 0) fused_block(passc, kNoPrev, buf, 0, accA, accB, 0);
          else fused_block(passc, kPrev, buf, 0, accA, accB, keyB);
          fused_block(passc, kPrev, buf, 1, accB, accA, c * CK);
          pendingB = true;
          keyB = c * CK + 32;
        } else {
          if (pendingB) flush(passc, accB, keyB);
          pendingB = false;
          for (int sb = 0; sb < SBC; ++sb) {
            const int key0 = c * CK + sb * 32;
            if (key0 >= hi_w) break;
            floatx16 acc[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = floatx16{};
            mfma_block(buf, sb, acc);
            const int key = key0 + (lane & 31);
            const int dk = key - qpos0 - (lane >> 5) * 4;   // causal: dk <= the slot's row constant
            const bool diag = key0 + 31 > qpos0;
            int cnt[RB] = {};
            uint32_t bm[RB] = {};
            float w[RB] = {};
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const bool causal = !diag || dk <= rb * 32 + (i >> 2) * 8 + (i & 3);   // exact_2.py:101, 119
                const float v = acc[rb][i];
                if constexpr (pass == 0) {
                  if (causal && v > mx[rb][i]) mx[rb][i] = v;
                } else if constexpr (PLAIN) {
                  cnt[rb] += causal ? (int)(__float_as_uint(v - mx[rb][i]) >> 31) : 1;
                } else {
                  const int keep = causal && v >= mx[rb][i];
                  acc2(keep, v, ref[rb][i], i, cnt[rb], bm[rb], w[rb]);
                  if constexpr (RC) rc[rb][i] += keep;
                }
              }
            if constexpr (pass == 1) {
              if constexpr (PLAIN) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) cnt[rb] = 16 - cnt[rb];
              }
              store_key(key, true, cnt, bm, w);
            }
          }
        }
      }
      chunk_end(c);
    }
    if (active && pendingB) flush(passc, accB, keyB);
    if constexpr (pass == 0) finish1(false);
  };
  if constexpr (MODE == 1) {
    // the screen: each row's exact raw maximum, or the workgroup's fallback flag
    const bool fallback = run_screened();
    if (threadIdx.x == 0) a.sflags[h * ngroups + g] = fallback ? 1 : 0;
    if (!fallback && active && (lane & 31) == 0) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // a wave's rows may run past q_rows_pad (a multiple of the tile, not of 64)
          const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          if (row < rows_total) a.srmax[(int64_t)h * a.q_rows_pad + row] = mx[rb][i];
        }
    }
    return;
  } else {
    // pass 1: the screen's row maxima, or the three-product sweep where it fell back or is off
    // the screen's workgroups covering this one's rows (4 waves of 32 RB rows each)
    bool exact1 = true;
    bool screen_ok = a.screened;
    {
      constexpr int SG = score_waves<false, 0, 1>() * 32 * RB;
      const int ng_s = (rows_total + SG - 1) / SG;
      for (int gs = g * WG_ROWS / SG; gs < min((g + 1) * WG_ROWS / SG, ng_s); ++gs)
        screen_ok = screen_ok && a.sflags[h * ng_s + gs] == 0;
    }
    if (screen_ok) {
      exact1 = false;
      if (active) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            mx[rb][i] = row < rows_total ? a.srmax[(int64_t)h * a.q_rows_pad + row] : 0.0f;
          }
      }
    }
    if (exact1) run_pass(std::integral_constant<int, 0>{});
    else finish1(true);
    if constexpr (PQ == 6) {
      // thresholds only: every row's x0, replicated over the 32 lanes holding its keys
      if (active && (lane & 31) == 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            if (row < rows_total) a.xthr[(int64_t)h * a.q_rows_pad + row] = mx[rb][i];
          }
      }
      return;
    } else {
      run_pass(std::integral_constant<int, 1>{});
    }
  }

  if constexpr (RC) {
    if (active) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          int v = rc[rb][i];
          v += __shfl_xor(v, 1, 64);
          v += __shfl_xor(v, 2, 64);
          v += __shfl_xor(v, 4, 64);
          v += __shfl_xor(v, 8, 64);
          v += __shfl_xor(v, 16, 64);
          const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          if ((lane & 31) == 0 && wrow0 + row < a.N) a.row_counts[(int64_t)h * a.N + wrow0 + row] = v;
        }
    }
  }
}

// ------------------------------------------------------------------------------------------
// host launchers
// ------------------------------------------------------------------------------------------
template <int DT, int D>
static hipError_t launch_rope_frag_t(const void* x, int64_t hs, int64_t ts, int heads, int N, int rows_pad,
                                     int pos_base, float pos_scale, float rope_scale, const float* inv_freq,
                                     u32x4* frag, hipStream_t st, bool want6, float2* trig) {
  const int64_t total = (int64_t)rows_pad * (D / 16);
  const int64_t blocks = (total + 255) / 256;
  float2* norms = frag_norms(frag, heads, rows_pad, D);
  uint64_t* planes6 = want6 ? frag6_planes(frag, heads, rows_pad, D) : nullptr;
  uint32_t* scales6 = frag6_scales(frag, heads, rows_pad, D);
  float2* dn6 = frag6_dnorms(frag, heads, rows_pad, D);
  const dim3 grid((unsigned)blocks, (unsigned)((heads + ROPE_HG - 1) / ROPE_HG));
  if (want6)
    hipLaunchKernelGGL((rope_frag_kernel<DT, D, true>), grid, dim3(256), 0, st, x, hs, ts, heads, N,
                       rows_pad, pos_base, pos_scale, rope_scale, inv_freq, frag, norms, planes6, scales6, dn6, trig);
  else
    hipLaunchKernelGGL((rope_frag_kernel<DT, D, false>), grid, dim3(256), 0, st, x, hs, ts, heads, N,
                       rows_pad, pos_base, pos_scale, rope_scale, inv_freq, frag, norms, planes6, scales6, dn6, trig);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the row norms' maxima, and with the fp6 planes their rounding norms' in the same launch
  hipLaunchKernelGGL(norm_max_kernel, dim3(heads, want6 ? 2 : 1), dim3(1024), 0, st, (const float2*)norms,
                     frag_norm_max(frag, heads, rows_pad, D), (const float2*)dn6,
                     frag6_dnorm_max(frag, heads, rows_pad, D), rows_pad);
  return hipGetLastError();
}

hipError_t launch_rope_frag(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N,
                            int rows_pad, int pos_base, float pos_scale, float rope_scale,
                            const float* inv_freq, u32x4* frag, hipStream_t st, bool want6, float2* trig) {
#define STA_RF(DT_, D_) \
  if (dtype == DT_ && D == D_) return launch_rope_frag_t<DT_, D_>(x, hs, ts, heads, N, rows_pad, pos_base, pos_scale, rope_scale, inv_freq, frag, st, want6, trig);
  STA_RF(DT_F32, 64) STA_RF(DT_F32, 128) STA_RF(DT_BF16, 64) STA_RF(DT_BF16, 128)
  STA_RF(DT_F16, 64) STA_RF(DT_F16, 128)
#undef STA_RF
  return hipErrorInvalidValue;
}

// STA_EXACT_PASS1=1 in the environment (read at every launch) makes every workgroup run the
// three-product pass 1 sweep, for comparisons against the screened sweep; STA_EXACT_PASS2=1 keeps
// every workgroup on the three-product pass 2 (no fp6 correction kernel)
static int exact_pass1_forced() {
  const char* e = getenv("STA_EXACT_PASS1");
  return e && e[0] == '1' ? 1 : 0;
}
// STA_SCREEN_GATHER=1: the screen gathers its candidate keys from the K fragments even where the
// (cos, sin) table is there, for comparisons
static int screen_gather_forced() {
  const char* e = getenv("STA_SCREEN_GATHER");
  return e && e[0] == '1' ? 1 : 0;
}
static int exact_pass2_forced() {
  const char* e = getenv("STA_EXACT_PASS2");
  return e && e[0] == '1' ? 1 : 0;
}

template <int D, int T, bool RC, int PQ>
static hipError_t launch_score_t(const ScoreArgs& a0, hipStream_t st) {
  constexpr int RB = 2;   // 64 query rows per wave (128-row waves spill and balance worse)
  ScoreArgs a = a0;
  // block indices of the screened pass 1 need ib bits; its packing error 2^(ib-23) stays small
  // for ib <= 13 (up to 262144 keys), longer rows take the three-product sweep
  int ib = 1;
  while ((1 << ib) < a.k_rows_pad / 32) ++ib;
  a.ib = (ib <= 13 && a.qnorm && a.knorm_max) ? ib : 0;
  a.exact_pass1 = exact_pass1_forced();
  if (screen_gather_forced()) a.ktrig = nullptr;
  const int rows = a.nt * T;
  constexpr int WS = score_waves<false, 0, 1>(), W2 = score_waves<RC, PQ, 0>();
  const int ng_s = (rows + 32 * RB * WS - 1) / (32 * RB * WS);
  const int ng_2 = (rows + 32 * RB * W2 - 1) / (32 * RB * W2);
  // the screen's results sit behind the Q fragments' norms in the fragment region
  a.srmax = frag_rowmax(a.qfrag, a.H, a.q_rows_pad, D);
  a.sflags = frag_flags(a.qfrag, a.H, a.q_rows_pad, D);
  a.screened = a.ib != 0 && !a.exact_pass1;
  // plain votes from 16-bit inputs: the fp6 pass-2 kernel first (the workgroups whose screen
  // resolved and whose head passes the error guard), the three-product kernel for the rest
  constexpr bool PLAIN = PQ == 0 && !RC;
  a.fast6 = (PLAIN && a.screened && a.want_fast6 && !exact_pass2_forced()) ? 1 : 0;
  if (a.fast6) {
    a.qnorm_max = frag_norm_max(a.qfrag, a.H, a.q_rows_pad, D);
    a.q6 = frag6_planes(a.qfrag, a.H, a.q_rows_pad, D);
    a.q6sc = frag6_scales(a.qfrag, a.H, a.q_rows_pad, D);
    a.q6dn = frag6_dnorms(a.qfrag, a.H, a.q_rows_pad, D);
    a.q6dmax = frag6_dnorm_max(a.qfrag, a.H, a.q_rows_pad, D);
    a.k6 = frag6_planes(a.kfrag, a.Hkv, a.k_rows_pad, D);
    a.k6sc = frag6_scales(a.kfrag, a.Hkv, a.k_rows_pad, D);
    a.k6dmax = frag6_dnorm_max(a.kfrag, a.Hkv, a.k_rows_pad, D);
  }
  if (a.screened) {
    // the screen is the same for every pass-2 epilogue: one instance per (D, T)
    hipLaunchKernelGGL((score_kernel<D, T, false, 0, RB, 1>), dim3(a.H * ng_s), dim3(64 * WS), 0, st, a);
  }
  if (a.fast6) {
    const hipError_t e = launch_score6(D, T, a, st);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((score_kernel<D, T, RC, PQ, RB, 0>), dim3(a.H * ng_2), dim3(64 * W2), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_score(int D, int tile, const ScoreArgs& a, hipStream_t st) {
  const bool rc = a.row_counts != nullptr;
#define STA_SC(D_, T_) \
  if (D == D_ && tile == T_) return rc ? launch_score_t<D_, T_, true, 0>(a, st) : launch_score_t<D_, T_, false, 0>(a, st);
  STA_SC(64, 32) STA_SC(64, 64) STA_SC(128, 32) STA_SC(128, 64)
#undef STA_SC
  return hipErrorInvalidValue;
}

hipError_t launch_score_weighted(int D, int tile, int wmode, const ScoreArgs& a, hipStream_t st) {
  const bool rc = a.row_counts != nullptr;
#define STA_SW(D_, T_, PQ_) \
  if (D == D_ && tile == T_ && wmode + 3 == PQ_) return rc ? launch_score_t<D_, T_, true, PQ_>(a, st) : launch_score_t<D_, T_, false, PQ_>(a, st);
  STA_SW(64, 32, 4) STA_SW(64, 32, 5) STA_SW(64, 64, 4) STA_SW(64, 64, 5)
  STA_SW(128, 32, 4) STA_SW(128, 32, 5) STA_SW(128, 64, 4) STA_SW(128, 64, 5)
#undef STA_SW
  return hipErrorInvalidValue;
}

hipError_t launch_score_thresholds(int D, const ScoreArgs& a, hipStream_t st) {
  if (D == 64) return launch_score_t<64, 32, false, 6>(a, st);
  if (D == 128) return launch_score_t<128, 32, false, 6>(a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_score_pq(int D, int wmode, const ScoreArgs& a, hipStream_t st) {
  const bool rc = a.row_counts != nullptr;
#define STA_SP(D_, PQ_) \
  if (D == D_ && wmode + 1 == PQ_) return rc ? launch_score_t<D_, 32, true, PQ_>(a, st) : launch_score_t<D_, 32, false, PQ_>(a, st);
  STA_SP(64, 1) STA_SP(64, 2) STA_SP(64, 3) STA_SP(128, 1) STA_SP(128, 2) STA_SP(128, 3)
#undef STA_SP
  return hipErrorInvalidValue;
}

}  // namespace sta
