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

#include <type_traits>

namespace sta {

// ------------------------------------------------------------------------------------------
// RoPE pre-kernel: rotate rows in the selection geometry, split hi/lo, write fragments.
// angle = fl(fl(float(pos) * pos_scale) * inv_freq[i])          (exact_2.py:79, 95)
// c, s  = fl(cos(angle) * rope_scale), fl(sin(angle) * rope_scale)   (exact_2.py:80-81)
// r1 = fl(fl(x1*c) - fl(x2*s)), r2 = fl(fl(x2*c) + fl(x1*s))   (exact_2.py:82-83)
// Rows >= N (tile padding, and the zero "phantom" keys the reference's masked loads produce
// when q_pos_base > 0) are written as zeros.
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(256) void rope_frag_kernel(const void* __restrict__ x, int64_t head_stride,
                                                        int64_t tok_stride, int heads, int N, int rows_pad,
                                                        int pos_base, float pos_scale, float rope_scale,
                                                        const float* __restrict__ inv_freq,
                                                        u32x4* __restrict__ frag) {
#pragma clang fp contract(off)
  constexpr int C = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)heads * rows_pad * C;
  if (gid >= total) return;
  const int c = (int)(gid % C);
  const int64_t hr = gid / C;
  const int row = (int)(hr % rows_pad);
  const int head = (int)(hr / rows_pad);
  const int d0 = c * 8;
  float out[8];
  if (row < N) {
    const bool first = d0 < D / 2;
    const int i0 = first ? d0 : d0 - D / 2;
    float a[8], b[8];
    const int64_t base = (int64_t)head * head_stride + (int64_t)row * tok_stride;
    load8<DT>(x, base + i0, a);
    load8<DT>(x, base + D / 2 + i0, b);
    const float pf = (float)(pos_base + row) * pos_scale;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ang = pf * inv_freq[i0 + e];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      cs = cs * rope_scale;
      sn = sn * rope_scale;
      if (first) {
        const float p = a[e] * cs, q = b[e] * sn;
        out[e] = p - q;
      } else {
        const float p = b[e] * cs, q = a[e] * sn;
        out[e] = p + q;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = 0.0f;
  }
  u32x4 hi, lo;
  split_bf16x8(out, hi, lo);
  const int rb = row >> 5, lr = row & 31, s = d0 >> 4, g = (d0 & 15) >> 3;
  const int64_t unit = (((int64_t)head * (rows_pad >> 5) + rb) * (D / 16) + s) * 2 * 64 + lr + 32 * g;
  frag[unit] = hi;
  frag[unit + 64] = lo;
}

// ------------------------------------------------------------------------------------------
// Score kernel: pass 1 (exact row max) and pass 2 (keep + votes), exact_2.py:87-140.
//
// One workgroup = one head and 256 consecutive query rows in eight waves of 32 rows (two waves
// per SIMD, so one wave's epilogue and LDS reads overlap the other's MFMAs).  A wave holds its
// rows' Q fragments in registers.  Key chunks of 128 rows are staged once in LDS and read by all
// eight waves, so each K byte fetched from L2 feeds 256 queries.  Row maxima complete inside a
// wave; a 64-row tile's votes are the sum of its two waves' counts, which are stored as two byte
// planes and added by the selection kernel.
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

// PQ selects the pass-2 epilogue: 0 = byte votes (shared selection); 1..3 = the per-query
// variant (tile 32): packed keep bits per key, plus weighted votes for PQ 2 (margin,
// sum of fl(s - fl(m - tau))) and PQ 3 (expmass, sum of exp(fl(s - m))) over the keeping rows
// (shared_selection_triton_perquery.py:181-217).
template <int D, int T, bool RC, int PQ>
__global__ __launch_bounds__(512, 1) void score_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  constexpr int RB = 1;                          // 32-row blocks per wave
  constexpr int NTH = 512;                       // eight waves
  constexpr int HALVES = T / 32;                 // waves (vote planes) per tile
  constexpr int TPW = 8 / HALVES;                // tiles per workgroup
  constexpr int S = D / 16;                      // k steps of 16
  constexpr int CHUNK_UNITS = 4 * S * 2 * 64;    // u32x4 units per 128-key chunk
  constexpr int PF = CHUNK_UNITS / NTH;          // units per thread per chunk
  constexpr int PER = 16 * RB / S;               // epilogue elements finished per k step
  static_assert(PER * S == 16 * RB, "epilogue split");
  static_assert(PQ == 0 || T == 32, "per-query bits pack one 32-row tile");
  extern __shared__ u32x4 lds[];                 // 2 x CHUNK_UNITS

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ngroups = (a.nt + TPW - 1) / TPW;
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
  const int kvh = h / (a.H / a.Hkv);
  const int t = g * TPW + wave / HALVES;
  const int hv = wave % HALVES;                    // which 32 rows of the tile
  const bool active = t < a.nt;
  const int t_last = min(g * TPW + TPW - 1, a.nt - 1);
  const int hi_max = a.q_pos_base + (t_last + 1) * T;
  const int row0 = t * T + 32 * hv;                // first row of this wave
  const int qpos0 = a.q_pos_base + row0;           // its position
  const int hi_w = qpos0 + 32;                     // keys past the wave's last query are masked
  const int nchunks = (hi_max + 127) >> 7;
  // chunks entirely below N whose keys are causal for every query of the workgroup
  const int nfull = min(min(nchunks, (a.q_pos_base + g * TPW * T + 1) >> 7), a.N >> 7);
  const float tau = a.tau[h];
  uint8_t* vrow = a.votes + (((int64_t)h * a.nt + t) * HALVES + hv) * a.votes_stride;
  uint32_t* brow = a.bits + ((int64_t)h * a.nt + t) * a.votes_stride;
  uint32_t* wrow = (uint32_t*)a.wvotes + ((int64_t)h * a.nt + t) * a.votes_stride;
  // one store per key and lane half: lanes 0-31 the bits, lanes 32-63 the weighted vote
  auto store_pq = [&](int key, uint32_t bm, float w) {
    bm <<= 4 * (lane >> 5);                 // rows of the upper lane half sit 4 bits higher
    bm |= __shfl_xor(bm, 32, 64);
    if constexpr (PQ >= 2) w += __shfl_xor(w, 32, 64);
    if (lane < 32) brow[key] = bm;
    else if constexpr (PQ >= 2) wrow[key] = __float_as_uint(w);
  };

  // ---- Q fragments of this wave's tile ----
  u32x4 qhi[RB][S], qlo[RB][S];
  if (active) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int64_t u = (((int64_t)h * (a.q_rows_pad >> 5) + row0 / 32 + rb) * S + s) * 128 + lane;
        qhi[rb][s] = a.qfrag[u];
        qlo[rb][s] = a.qfrag[u + 64];
      }
  } else {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int s = 0; s < S; ++s) { qhi[rb][s] = u32x4{0, 0, 0, 0}; qlo[rb][s] = u32x4{0, 0, 0, 0}; }
  }
  const u32x4* kbase = a.kfrag + (int64_t)kvh * (a.k_rows_pad >> 5) * S * 128;

  // per-query epilogue of one score: bit `row` of the key's mask, and its weighted vote
  // (i indexes the lane's 16 accumulator rows: row = (i/4)*8 + 4*(lane/32) + i%4; the lane
  // half's 4-row offset is applied when the mask is stored)
  auto pq_acc = [&](int keep, float v, float ref, int i, uint32_t& bm, float& w) {
#pragma clang fp contract(off)
    bm |= (uint32_t)keep << ((i >> 2) * 8 + (i & 3));
    if constexpr (PQ == 2) {
      const float qk = v * a.sm_scale;
      const float c = qk - ref;
      w += keep ? c : 0.0f;
    } else if constexpr (PQ == 3) {
      const float qk = v * a.sm_scale;
      const float e = __expf(qk - ref);
      w += keep ? e : 0.0f;
    }
  };
  float mx[RB][16];   // pass 1: running max of the raw dot per row slot; pass 2 (PQ 2 / 3):
                      // fl(m - tau) / m of the row, the reference point of the weighted vote
  float x0[RB][16];   // pass 2: keep threshold on the raw dot per row slot
  int rc[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) { mx[rb][i] = -INFINITY; x0[rb][i] = INFINITY; rc[rb][i] = 0; }

  // 32 keys x this wave's rows: hi.hi + hi.lo + lo.hi, small terms first
  auto mfma_step = [&](const u32x4* buf, int sb, int s, floatx16* acc) {
    const u32x4 bh = buf[(sb * S + s) * 128 + lane];
    const u32x4 bl = buf[(sb * S + s) * 128 + 64 + lane];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qlo[rb][s], bh, acc[rb]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bl, acc[rb]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bh, acc[rb]);
  };
  // MFMAs of block sb into accN; when HAS_PREV, the epilogue of the previous (unmasked) block
  // accO at keys keyO.. is finished in slices between the k steps
  auto fused_block = [&](auto passc, auto prevc, const u32x4* buf, int sb, floatx16* accN,
                         const floatx16* accO, int keyO) {
    constexpr int pass = decltype(passc)::value;
    constexpr bool HAS_PREV = decltype(prevc)::value;
    int cnt = 0;
    uint32_t bm = 0;
    float w = 0.0f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) accN[rb] = floatx16{};
#pragma unroll
    for (int s = 0; s < S; ++s) {
      mfma_step(buf, sb, s, accN);
      if constexpr (HAS_PREV) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int idx = s * PER + e, rb = idx / 16, i = idx % 16;
          const float v = accO[rb][i];
          if constexpr (pass == 0) {
            mx[rb][i] = v > mx[rb][i] ? v : mx[rb][i];
          } else {
            const int keep = v >= x0[rb][i];
            if constexpr (PQ == 0) cnt += keep;
            else pq_acc(keep, v, mx[rb][i], i, bm, w);
            if constexpr (RC) rc[rb][i] += keep;
          }
        }
      }
    }
    if constexpr (HAS_PREV && pass == 1) {
      if constexpr (PQ == 0) {
        cnt += __shfl_xor(cnt, 32, 64);   // exact_2.py:123; both lane halves now hold the total
        vrow[keyO + (lane & 31)] = (uint8_t)cnt;
      } else {
        store_pq(keyO + (lane & 31), bm, w);
      }
    }
  };
  // the last block's epilogue when nothing follows it
  auto flush = [&](auto passc, const floatx16* acc, int key0) {
    constexpr int pass = decltype(passc)::value;
    int cnt = 0;
    uint32_t bm = 0;
    float w = 0.0f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float v = acc[rb][i];
        if constexpr (pass == 0) {
          mx[rb][i] = v > mx[rb][i] ? v : mx[rb][i];
        } else {
          const int keep = v >= x0[rb][i];
          if constexpr (PQ == 0) cnt += keep;
          else pq_acc(keep, v, mx[rb][i], i, bm, w);
          if constexpr (RC) rc[rb][i] += keep;
        }
      }
    if constexpr (pass == 1) {
      if constexpr (PQ == 0) {
        cnt += __shfl_xor(cnt, 32, 64);
        vrow[key0 + (lane & 31)] = (uint8_t)cnt;
      } else {
        store_pq(key0 + (lane & 31), bm, w);
      }
    }
  };

  u32x4 pf[PF];
  auto run_pass = [&](auto passc) {
    constexpr int pass = decltype(passc)::value;
    constexpr std::integral_constant<bool, true> kPrev{};
    constexpr std::integral_constant<bool, false> kNoPrev{};
#pragma unroll
    for (int e = 0; e < PF; ++e) pf[e] = kbase[e * NTH + threadIdx.x];
#pragma unroll
    for (int e = 0; e < PF; ++e) lds[e * NTH + threadIdx.x] = pf[e];
    __syncthreads();
    floatx16 accA[RB], accB[RB];
    bool pendingB = false;   // accB holds an unmasked block whose epilogue is still due
    int keyB = 0;
    for (int c = 0; c < nchunks; ++c) {
      const bool more = c + 1 < nchunks;
      if (more) {
        const u32x4* src = kbase + (int64_t)(c + 1) * CHUNK_UNITS;
#pragma unroll
        for (int e = 0; e < PF; ++e) pf[e] = src[e * NTH + threadIdx.x];
      }
      const u32x4* buf = lds + (c & 1) * CHUNK_UNITS;
      if (active) {
        if (c < nfull) {
          if (c == 0) fused_block(passc, kNoPrev, buf, 0, accA, accB, 0);
          else fused_block(passc, kPrev, buf, 0, accA, accB, keyB);
          fused_block(passc, kPrev, buf, 1, accB, accA, c * 128);
          fused_block(passc, kPrev, buf, 2, accA, accB, c * 128 + 32);
          fused_block(passc, kPrev, buf, 3, accB, accA, c * 128 + 64);
          pendingB = true;
          keyB = c * 128 + 96;
        } else {
          if (pendingB) flush(passc, accB, keyB);
          pendingB = false;
          for (int sb = 0; sb < 4; ++sb) {
            const int key0 = c * 128 + sb * 32;
            if (key0 >= hi_w) break;
            floatx16 acc[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = floatx16{};
#pragma unroll
            for (int s = 0; s < S; ++s) mfma_step(buf, sb, s, acc);
            const int key = key0 + (lane & 31);
            const bool diag = key0 + 31 > qpos0;
            int cnt = 0;
            uint32_t bm = 0;
            float w = 0.0f;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const int row = rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                const bool causal = !diag || key <= qpos0 + row;   // exact_2.py:101, 119
                const float v = acc[rb][i];
                if constexpr (pass == 0) {
                  if (causal && v > mx[rb][i]) mx[rb][i] = v;
                } else {
                  const int keep = causal && v >= x0[rb][i];
                  if constexpr (PQ == 0) cnt += keep;
                  else pq_acc(keep, v, mx[rb][i], i, bm, w);
                  if constexpr (RC) rc[rb][i] += keep;
                }
              }
            if constexpr (pass == 1) {
              if constexpr (PQ == 0) {
                cnt += __shfl_xor(cnt, 32, 64);
                if (lane < 32 && key < a.N) vrow[key] = (uint8_t)cnt;
              } else {
                // the shuffles inside run on every lane; only the store is guarded
                bm <<= 4 * (lane >> 5);
                bm |= __shfl_xor(bm, 32, 64);
                if constexpr (PQ >= 2) w += __shfl_xor(w, 32, 64);
                if (key < a.N) {
                  if (lane < 32) brow[key] = bm;
                  else if constexpr (PQ >= 2) wrow[key] = __float_as_uint(w);
                }
              }
            }
          }
        }
      }
      if (more) {
        u32x4* dst = lds + ((c + 1) & 1) * CHUNK_UNITS;
#pragma unroll
        for (int e = 0; e < PF; ++e) dst[e * NTH + threadIdx.x] = pf[e];
      }
      __syncthreads();
    }
    if (active && pendingB) flush(passc, accB, keyB);
    if constexpr (pass == 0) {
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
            const bool ok = row0 + row < a.N;   // padded rows never vote (exact_2.py:121)
            x0[rb][i] = ok ? min_arg_for(m - tau, a.sm_scale) : INFINITY;
            if constexpr (PQ == 2) mx[rb][i] = m - tau;   // perquery.py:210
            if constexpr (PQ == 3) mx[rb][i] = m;         // perquery.py:215
            if (a.row_max && (lane & 31) == 0 && ok) a.row_max[(int64_t)h * a.N + row0 + row] = m;
          }
      }
    }
  };
  run_pass(std::integral_constant<int, 0>{});
  run_pass(std::integral_constant<int, 1>{});

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
          if ((lane & 31) == 0 && row0 + row < a.N) a.row_counts[(int64_t)h * a.N + row0 + row] = v;
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
                                     u32x4* frag, hipStream_t st) {
  const int64_t total = (int64_t)heads * rows_pad * (D / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((rope_frag_kernel<DT, D>), dim3((unsigned)blocks), dim3(256), 0, st, x, hs, ts, heads, N,
                     rows_pad, pos_base, pos_scale, rope_scale, inv_freq, frag);
  return hipGetLastError();
}

hipError_t launch_rope_frag(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N,
                            int rows_pad, int pos_base, float pos_scale, float rope_scale,
                            const float* inv_freq, u32x4* frag, hipStream_t st) {
#define STA_RF(DT_, D_) \
  if (dtype == DT_ && D == D_) return launch_rope_frag_t<DT_, D_>(x, hs, ts, heads, N, rows_pad, pos_base, pos_scale, rope_scale, inv_freq, frag, st);
  STA_RF(DT_F32, 64) STA_RF(DT_F32, 128) STA_RF(DT_BF16, 64) STA_RF(DT_BF16, 128)
  STA_RF(DT_F16, 64) STA_RF(DT_F16, 128)
#undef STA_RF
  return hipErrorInvalidValue;
}

template <int D, int T, bool RC, int PQ>
static hipError_t launch_score_t(const ScoreArgs& a, hipStream_t st) {
  constexpr int S = D / 16;
  const size_t lds_bytes = 2 * (size_t)(4 * S * 2 * 64) * 16;
  hipError_t e = hipFuncSetAttribute((const void*)score_kernel<D, T, RC, PQ>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
  if (e != hipSuccess) return e;
  const int tpw = 256 / T;
  const int ngroups = (a.nt + tpw - 1) / tpw;
  hipLaunchKernelGGL((score_kernel<D, T, RC, PQ>), dim3(a.H * ngroups), dim3(512), lds_bytes, st, a);
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

hipError_t launch_score_pq(int D, int wmode, const ScoreArgs& a, hipStream_t st) {
  const bool rc = a.row_counts != nullptr;
#define STA_SP(D_, PQ_) \
  if (D == D_ && wmode + 1 == PQ_) return rc ? launch_score_t<D_, 32, true, PQ_>(a, st) : launch_score_t<D_, 32, false, PQ_>(a, st);
  STA_SP(64, 1) STA_SP(64, 2) STA_SP(64, 3) STA_SP(128, 1) STA_SP(128, 2) STA_SP(128, 3)
#undef STA_SP
  return hipErrorInvalidValue;
}

}  // namespace sta
