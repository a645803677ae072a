// sta_decode.hip -- the decode path: each query selects its own key set over the KV cache and
// attends it.  A batch of Q queries shares one cache of M keys; query i sits at position
// q_pos0 + i and sees the keys [0, m_i), m_i = M - (Q - 1 - i) -- the cache prefix that the
// reference's per-token loop hands to every call (shared_selection_triton_exact_2.py:743-745).
//
//   decode_qrot_kernel    the query rotated at fl(float(q_pos) * pos_scale)        (exact_2.py:250-257)
//   decode_score_kernel   per-key scores under the selection geometry            (exact_2.py:235-271)
//                         64 keys x up to 4 kv heads per workgroup: the key rotation's
//                         sin / cos is computed once per (key, frequency) and shared by the heads;
//                         the query rows are rotated in the workgroup's LDS (decode_qrot_kernel
//                         precomputes them when they outgrow it)
//   decode_select_kernel  _decode_build_sets (exact_2.py:527-604) for one query per workgroup:
//                         the scores staged in LDS as order-preserving keys, exact max, the
//                         top-pct cut and the k_max cap cut as radix selections (8-bit digits),
//                         compaction and the fp32 reposition recurrence
//   decode_attend_kernel  the attend over the selected slots (exact_2.py:608-655) split over
//                         workgroups of 64 slots, 16 lanes per slot and four slots per lane
//                         group (every row request in flight at once), each split a softmax
//                         state; decode_combine_kernel merges the splits
//   decode_attend_grouped_kernel  the per-query rule's attend for a batch (perquery.py:724-778):
//                         16 queries per workgroup, one 16-lane group per query, the dense-rank
//                         (cos, sin) table of each 64-slot block shared in LDS
#include <float.h>

#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

namespace {

// NE consecutive elements (NE in {2, 4, 8, 16}) from element index i as fp32
template <int DT, int NE>
__device__ __forceinline__ void load_n(const void* p, int64_t i, float* out) {
  if constexpr (NE >= 8) {
#pragma unroll
    for (int u = 0; u < NE / 8; ++u) load8<DT>(p, i + 8 * u, out + 8 * u);
  } else if constexpr (DT == DT_F32) {
    if constexpr (NE == 4) {
      const float4 a = *(const float4*)((const float*)p + i);
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    } else {
      const float2 a = *(const float2*)((const float*)p + i);
      out[0] = a.x; out[1] = a.y;
    }
  } else {
    uint32_t w[NE / 2];
    if constexpr (NE == 4) {
      const u32x2 x = *(const u32x2*)((const uint16_t*)p + i);
      w[0] = x[0]; w[1] = x[1];
    } else {
      w[0] = *(const uint32_t*)((const uint16_t*)p + i);
    }
#pragma unroll
    for (int e = 0; e < NE / 2; ++e) {
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

template <int DT>
__device__ __forceinline__ float load1(const void* p, int64_t i) {
  if constexpr (DT == DT_F32) return ((const float*)p)[i];
  else if constexpr (DT == DT_BF16) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  else return f16_bits_to_f32(((const uint16_t*)p)[i]);
}

// fp32 -> unsigned key with the same order (-0 folded into +0); no real value maps to 0
__device__ __forceinline__ uint32_t okey(float r) {
  const uint32_t b = __float_as_uint(r + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float okey_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

}  // namespace

// ------------------------------------------------------------------------------------------
// rotated queries (H, Q, D) fp32: angle base fl(float(q_pos0 + i) * pos_scale)   (exact_2.py:253)
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(D / 2) void decode_qrot_kernel(DecodeArgs a, float* qrot) {
#pragma clang fp contract(off)
  const int hi = blockIdx.x;                 // h * Q + i
  const int h = hi / a.Q, i = hi % a.Q;
  const int d = threadIdx.x;                 // frequency index
  const int64_t base = (int64_t)h * a.q_hs + (int64_t)i * a.q_ts;
  const float x1 = load1<DT>(a.q, base + d);
  const float x2 = load1<DT>(a.q, base + D / 2 + d);
  const float pb = (float)(a.q_pos0 + i) * a.pos_scale_a;
  const float ang = pb * a.inv_freq_a[d];
  float sn, cs;
  sincosf(ang, &sn, &cs);
  cs = cs * a.rope_scale_a;
  sn = sn * a.rope_scale_a;
  float* o = qrot + (int64_t)hi * D;
  const float p1 = x1 * cs, p2 = x2 * sn, p3 = x2 * cs, p4 = x1 * sn;
  o[d] = p1 - p2;                             // exact_2.py:256-257
  o[D / 2 + d] = p3 + p4;
}

// ------------------------------------------------------------------------------------------
// per-key scores (H, Q, M): 64 keys x HG kv heads per workgroup, 4 lanes per key.  Every head's
// key rows are requested first (kept packed in registers), then the workgroup rotates its query
// rows into LDS and computes the keys' sin / cos -- once per (key, frequency), shared by the
// heads -- while the rows are in flight.
// ------------------------------------------------------------------------------------------
constexpr int DEC_QLDS = 32 * 1024;           // LDS for rotated query rows

template <int DT>
constexpr int dec_hg() { return 4; }   // 4 kv heads: ~140 VGPRs, 3 waves per SIMD (8 heads: 2)

// kv heads of one score workgroup and whether its rotated query rows fit its LDS
int decode_score_hg(int dtype) { return dtype == DT_F32 ? dec_hg<DT_F32>() : dec_hg<DT_BF16>(); }
bool decode_qrot_in_lds(int dtype, int H, int Hkv, int Q, int D) {
  return (size_t)decode_score_hg(dtype) * (H / Hkv) * Q * D * 4 <= DEC_QLDS;
}

template <int DT, int D, bool QLDS>
__global__ __launch_bounds__(256) void decode_score_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int HG = dec_hg<DT>();
  constexpr int NP = D / 8;                   // rotation pairs per lane
  constexpr int ES = DT == DT_F32 ? 4 : 2;
  constexpr int UH = NP * ES / 16;            // 16-byte units per half row per lane
  __shared__ __align__(16) float qs[QLDS ? DEC_QLDS / 4 : 1];
  const int t = threadIdx.x & 3;
  const int j = blockIdx.x * 64 + (threadIdx.x >> 2);
  const int jc = j < a.M ? j : a.M - 1;
  const int hk0 = blockIdx.y * HG;
  const int nh = min(HG, a.Hkv - hk0);        // kv heads of this workgroup
  const int G = a.H / a.Hkv;
  u32x4 raw[HG][2 * UH];
#pragma unroll
  for (int g = 0; g < HG; ++g) {
    const int hk = hk0 + min(g, nh - 1);       // heads past Hkv reload a valid row, store nothing
    const char* row = (const char*)a.k + ((int64_t)hk * a.k_hs + (int64_t)jc * a.k_ts + t * NP) * ES;
#pragma unroll
    for (int u = 0; u < UH; ++u) {
      raw[g][u] = *(const u32x4*)(row + 16 * u);
      raw[g][UH + u] = *(const u32x4*)(row + (D / 2) * ES + 16 * u);
    }
  }
  const int R = nh * G * a.Q;                  // query rows: (kv head, q head of its group, query)
  if constexpr (QLDS) {
    // rotated at fl(float(q_pos0 + i) * pos_scale) (exact_2.py:250-257)
    for (int x = threadIdx.x; x < R * (D / 2); x += 256) {
      const int r = x / (D / 2), f = x % (D / 2);
      const int i = r % a.Q, hq = hk0 * G + r / a.Q;
      const int64_t base = (int64_t)hq * a.q_hs + (int64_t)i * a.q_ts;
      const float x1 = load1<DT>(a.q, base + f), x2 = load1<DT>(a.q, base + D / 2 + f);
      const float pb = (float)(a.q_pos0 + i) * a.pos_scale_a;
      const float ang = pb * a.inv_freq_a[f];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      cs = cs * a.rope_scale_a;
      sn = sn * a.rope_scale_a;
      const float p1 = x1 * cs, p2 = x2 * sn, p3 = x2 * cs, p4 = x1 * sn;
      qs[r * D + f] = p1 - p2;
      qs[r * D + D / 2 + f] = p3 + p4;
    }
  }
  // cos / sin of this key's frequencies t*NP .. t*NP + NP - 1
  float cs[NP], sn[NP];
  {
    const float kb = (float)j * a.pos_scale_a;                            // exact_2.py:264
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float ang = kb * a.inv_freq_a[t * NP + p];
      sincosf(ang, &sn[p], &cs[p]);
      cs[p] = cs[p] * a.rope_scale_a;
      sn[p] = sn[p] * a.rope_scale_a;
    }
  }
  if constexpr (QLDS) __syncthreads();
  const float* qsrc = QLDS ? qs : a.qrot + (int64_t)hk0 * G * a.Q * D;
#pragma unroll
  for (int g = 0; g < HG; ++g) {
    if (g >= nh) break;
    float k1[NP], k2[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {                                        // exact_2.py:266-267
      float x1, x2;
      if constexpr (DT == DT_F32) {
        x1 = __uint_as_float(raw[g][p / 4][p % 4]);
        x2 = __uint_as_float(raw[g][UH + p / 4][p % 4]);
      } else {
        const uint32_t w1 = raw[g][p / 8][(p % 8) / 2], w2 = raw[g][UH + p / 8][(p % 8) / 2];
        const uint32_t h1 = (p & 1) ? (w1 >> 16) : (w1 & 0xffffu), h2 = (p & 1) ? (w2 >> 16) : (w2 & 0xffffu);
        x1 = DT == DT_BF16 ? __uint_as_float(h1 << 16) : f16_bits_to_f32(h1);
        x2 = DT == DT_BF16 ? __uint_as_float(h2 << 16) : f16_bits_to_f32(h2);
      }
      const float u = x1 * cs[p], w = x2 * sn[p], y = x2 * cs[p], z = x1 * sn[p];
      k1[p] = u - w;
      k2[p] = y + z;
    }
    for (int r = g * G * a.Q; r < (g + 1) * G * a.Q; ++r) {
      const float* qr = qsrc + (int64_t)r * D;
      float acc = 0.0f;
#pragma unroll
      for (int p = 0; p < NP; p += 4) {
        const float4 u = *(const float4*)(qr + t * NP + p);
        const float4 w = *(const float4*)(qr + D / 2 + t * NP + p);
        acc = fmaf(u.x, k1[p], acc);
        acc = fmaf(w.x, k2[p], acc);
        acc = fmaf(u.y, k1[p + 1], acc);
        acc = fmaf(w.y, k2[p + 1], acc);
        acc = fmaf(u.z, k1[p + 2], acc);
        acc = fmaf(w.z, k2[p + 2], acc);
        acc = fmaf(u.w, k1[p + 3], acc);
        acc = fmaf(w.w, k2[p + 3], acc);
      }
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      const int i = r % a.Q, hq = hk0 * G + r / a.Q;
      const int m = a.M - (a.Q - 1 - i);
      if (t == 0 && j < m) a.scores[((int64_t)hq * a.Q + i) * a.M + j] = acc * a.sm_scale;   // :270
    }
  }
}

// ------------------------------------------------------------------------------------------
// _decode_build_sets for one query per workgroup
// ------------------------------------------------------------------------------------------
constexpr int DEC_SEL_NT = 1024;             // threads of the workspace-sizing selection instance

namespace {

template <int NW>
__device__ __forceinline__ int dsum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += tmp[w];
  __syncthreads();
  return total;
}

template <int NW>
__device__ __forceinline__ uint32_t dmax_u(uint32_t v, uint32_t* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) r = max(r, tmp[w]);
  __syncthreads();
  return r;
}

// exclusive prefix sum over the block's threads; *total (optional) receives the block sum
template <int NW>
__device__ __forceinline__ int dexcl_sum(int v, int* tmp, int* total = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int base = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    base += w < wave ? tmp[w] : 0;
    all += tmp[w];
  }
  __syncthreads();
  if (total) *total = all;
  return base + x - v;
}

template <int NW>
__device__ __forceinline__ float dexcl_max(float v, float* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (lane >= o) x = fmaxf(x, y);
  }
  float prev = __shfl_up(x, 1, 64);
  if (lane == 0) prev = -INFINITY;
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  float base = -INFINITY;
  for (int w = 0; w < wave; ++w) base = fmaxf(base, tmp[w]);
  __syncthreads();
  return fmaxf(base, prev);
}

}  // namespace

// Keys of the LDS store: per thread a contiguous range of `per` keys at the odd row stride
// per | 1 (conflict-free scans); the global store (caches too long for LDS) uses stride per.
constexpr int DEC_CAND = 128;                // keys of a bin ranked directly
// The histogram's 4096 bins: two 16-bit counters per word for rows staged in LDS (a bin never
// holds more keys than the row, and those rows are far below 65536 keys), which keeps a 16k-key
// row's workgroup under 80 KB (two per CU); 32-bit counters for the global store's long rows.
constexpr int dec_hist_words(bool gkeys) { return gkeys ? 4096 : 2048; }
constexpr size_t DEC_AUX = 2048 * 4 + DEC_SEL_NT * 4 + 256;   // histogram, candidates, scratch
// The PQ Stream rule also keeps one kept-key count per position block (nbend words, after the
// scratch); rows whose keys, histogram and block counts outgrow the LDS take the global store.
bool decode_select_in_lds(int M, int nbend) {   // the CU's 160 KB: M <= 35840 without block counts
  const int per = (M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  return (size_t)DEC_SEL_NT * (per | 1) * 4 + DEC_AUX + (size_t)nbend * 4 <= 160 * 1024;
}
size_t decode_keys_bytes(int H, int Q, int M, int nbend) {
  if (decode_select_in_lds(M, nbend)) return 0;
  const int per = (M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  return (size_t)H * Q * DEC_SEL_NT * per * 4;
}
int decode_bend_words(const DecodeArgs& a) { return a.rule == 2 ? (a.M + a.block_n - 1) / a.block_n : 0; }

// NT threads per query: 1024 for a few queries (latency), 512 for large batches (throughput)
// query i of head h's score row: key j at at(j) = p + (j / SCORE_TW) * ps + j % SCORE_TW, with
// ps = SCORE_TW for row-major (H, Q, M) scores and 64 SCORE_TW for the tiles of score_tile_row
struct ScoreRow {
  const float* p;
  int ps;
  __device__ __forceinline__ const float* at(int j) const {
    return p + (j >> SCORE_TW_LG) * ps + (j & (SCORE_TW - 1));
  }
};
__device__ __forceinline__ ScoreRow score_row_of(const DecodeArgs& a, int h, int i) {
  if (a.score_tiles) return {a.scores + score_tile_row(h, i, a.Q, a.M), 64 * SCORE_TW};
  return {a.scores + ((int64_t)h * a.Q + i) * a.M, SCORE_TW};
}

template <bool GKEYS, int NT>
__global__ __launch_bounds__(NT) void decode_select_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int NW = NT / 64;
  extern __shared__ __align__(16) uint32_t dsm[];
  const int tid = threadIdx.x;
  const int hi = blockIdx.x;
  const int h = hi / a.Q, i = hi % a.Q;
  const int m = a.M - (a.Q - 1 - i);           // keys this query sees
  const int p = a.q_pos0 + i;                  // its position (p < m)
  const int per_max = (a.M + NT - 1) / NT;
  const int per = (m + NT - 1) / NT;
  const int PS = GKEYS ? per : (per | 1);
  uint32_t* ks = GKEYS ? a.keys + (int64_t)hi * NT * per_max : dsm;
  constexpr bool HPACK = !GKEYS;                // 16-bit bins, two per word
  uint32_t* hist = dsm + (GKEYS ? 0 : NT * (per_max | 1));
  uint32_t* cand = hist + dec_hist_words(GKEYS);   // NT (16-byte aligned)
  int* tmp = (int*)(cand + NT);        // NW
  int* misc = tmp + NW;                // 8
  const int j0 = tid * per, j1 = min(j0 + per, m);
  uint32_t* myrow = ks + tid * PS;
  const ScoreRow sr = score_row_of(a, h, i);

  // ---- stage the scores as keys (coalesced reads, eight in flight per lane), exact max
  // (exact_2.py:549) ----
  const float tau_h = a.tau[h];
  uint32_t kmax = 0;
  for (int e0 = 0; e0 < per; e0 += 8) {
    float sv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = tid + (e0 + u) * NT;
      sv[u] = (e0 + u < per && j < m) ? *sr.at(j) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = tid + (e0 + u) * NT;
      if (e0 + u < per) {
        const uint32_t key = j < m ? okey(sv[u]) : 0u;
        kmax = max(kmax, key);
        const int row = j / per;
        ks[row * PS + (j - row * per)] = key;
      }
    }
  }
  kmax = dmax_u<NW>(kmax, (uint32_t*)tmp);         // the barrier inside also publishes the stores
  const float thr = okey_value(kmax) - tau_h;                          // exact_2.py:550
  const uint32_t kthr = okey(thr);

  // forced keys: [0, g) U [lo, p] (global, local window, self; exact_2.py:552-555)
  const int g = min(a.n_global, m);
  const int lo = min(max(0, p - a.n_local + 1), p);
  const int nB = p - max(lo, g) + 1;            // local keys not already global
  const int nforced = g + max(nB, 0);
  auto forced_j = [&](int f) { return f < g ? f : max(lo, g) + (f - g); };   // f < nforced

  // need-th largest key (1 <= need <= #nonzero keys) -> (V, #keys >= V).  Radix levels of 12,
  // 12 and 8 bits (LDS histograms with plain atomics); as soon as the bin holding the statistic
  // has at most DEC_CAND keys they are collected and ranked directly.
  auto kth = [&](int need) -> uint2 {
    uint32_t prefix = 0, pmask = 0;
    int ge = 0;
    for (int lv = 0; lv < 3; ++lv) {
      const int shift = lv == 0 ? 20 : (lv == 1 ? 8 : 0);
      const int nb = lv == 2 ? 256 : 4096;
      for (int b = tid; b < (HPACK ? nb / 2 : nb); b += NT) hist[b] = 0u;
      cand[tid] = 0u;                          // 0 ranks below every key
      if (tid == 0) misc[4] = 0;
      __syncthreads();
      for (int e = 0; e < per; ++e) {
        const uint32_t k = myrow[e];
        if (k != 0 && j0 + e < m && (k & pmask) == prefix) {
          const uint32_t bin = (k >> shift) & (uint32_t)(nb - 1);
          if constexpr (HPACK) atomicAdd(&hist[bin >> 1], 1u << ((bin & 1u) * 16));
          else atomicAdd(&hist[bin], 1u);
        }
      }
      __syncthreads();
      // bins in descending order, BPT per thread
      constexpr int BPT = 4096 / NT;
      const bool own = BPT * tid < nb;
      int c[BPT], sl = 0;
#pragma unroll
      for (int e = 0; e < BPT; ++e) {
        const int bb = nb - 1 - BPT * tid - e;
        c[e] = !own ? 0 : HPACK ? (int)((hist[bb >> 1] >> ((bb & 1) * 16)) & 0xffffu) : (int)hist[bb];
        sl += c[e];
      }
      const int excl = dexcl_sum<NW>(sl, tmp);
      if (own && excl < need && excl + sl >= need) {
        int acc = excl, d = nb - 1 - BPT * tid, e = 0;
        for (; e < BPT - 1; ++e) {
          if (acc + c[e] >= need) break;
          acc += c[e];
          d -= 1;
        }
        misc[0] = d;
        misc[1] = need - acc;   // how far into bin d's keys the statistic lies
        misc[2] = acc;          // keys in the bins above
        misc[3] = c[e];         // keys in bin d
      }
      __syncthreads();
      const int d = misc[0], cd = misc[3];
      need = misc[1];
      ge += misc[2];
      prefix |= (uint32_t)d << shift;
      pmask |= (uint32_t)(nb - 1) << shift;
      if (lv == 2) {            // every key of the last bin equals prefix
        ge += cd;
        __syncthreads();
        break;
      }
      if (cd <= DEC_CAND) {
        for (int e = 0; e < per; ++e) {
          const uint32_t k = myrow[e];
          const int slot = wave_alloc(k != 0 && j0 + e < m && (k & pmask) == prefix, &misc[4]);
          if (slot >= 0) cand[slot] = k;
        }
        __syncthreads();
        if (tid < cd) {
          const uint32_t v = cand[tid];
          int gt = 0, eq = 0;
          for (int u = 0; u < cd; u += 4) {
            const uint4 w = *(const uint4*)&cand[u];
            gt += (w.x > v) + (w.y > v) + (w.z > v) + (w.w > v);
            eq += (w.x == v) + (w.y == v) + (w.z == v) + (w.w == v);
          }
          if (gt < need && gt + eq >= need) {   // the keys equal to the statistic agree
            misc[5] = (int)v;
            misc[6] = gt + eq;
          }
        }
        __syncthreads();
        const uint32_t V = (uint32_t)misc[5];
        ge += misc[6];
        __syncthreads();
        return make_uint2(V, (uint32_t)ge);
      }
      __syncthreads();
    }
    return make_uint2(prefix, (uint32_t)ge);
  };
  auto key_of = [&](int j) {
    const int row = j / per;
    return ks[row * PS + (j - row * per)];
  };

  // ---- top-pct_decode% of the passers (exact_2.py:559-567) and |kept U forced| (:569-572) ----
  uint32_t kp_thr = kthr;
  int count;
  int ge;
  if (a.use_pct) {
    int c = 0;
    for (int e = 0; e < j1 - j0; ++e) c += myrow[e] >= kthr;
    const int n_pass = dsum<NW>(c, tmp);
    const float prod = a.pct_frac * (float)n_pass;                       // exact_2.py:561
    float b = ceilf(prod);
    if (b < 1.0f) b = 1.0f;
    const int need = (int)min((int64_t)b, (int64_t)m);                   // (budget_p - 1).clamp(0, M - 1)
    const uint2 r = kth(need);                                           // the need-th largest passer
    kp_thr = max(r.x, kthr);
    ge = (int)r.y;
    if (kp_thr != r.x) {                                                 // (only when need > n_pass)
      int c2 = 0;
      for (int e = 0; e < j1 - j0; ++e) c2 += myrow[e] >= kp_thr;
      ge = dsum<NW>(c2, tmp);
    }
  } else {
    int c = 0;
    for (int e = 0; e < j1 - j0; ++e) c += myrow[e] >= kp_thr;
    ge = dsum<NW>(c, tmp);
  }
  {
    int c = 0;
    for (int f = tid; f < nforced; f += NT) c += key_of(forced_j(f)) < kp_thr;
    count = ge + dsum<NW>(c, tmp);
  }

  // the per-query rule's measurement counters: |passers| and the overflow flag (perquery.py:686-688)
  const bool pq = a.rule == 1;
  const bool stream = a.rule == 2;   // PQ Stream: every passer and forced key, no cap
  if (pq && tid == 0) {
    if (a.usize) a.usize[hi] = ge;
    if (a.overflow) a.overflow[hi] = count > a.k_max ? 1 : 0;
  }

  // ---- cap by score over the non-forced keys (exact_2.py:571-585; perquery.py:690-701) ----
  uint32_t fin_thr = kp_thr;
  bool only_forced = false;
  // per-query rule: an exact budget (torch.topk, perquery.py:695-698) -- every key above the cut
  // and, of the keys equal to it, the first `quota` in key order; tie_base = this thread's first
  // tie index
  bool exact_cut = false;
  int quota = 0, tie_base = 0;
  if (count > a.k_max && !stream) {
    const int budget_c = a.k_max - nforced;
    if (budget_c <= 0) {
      only_forced = true;
    } else {
      // the non-forced kept keys are the non-forced keys >= kp_thr and they outnumber budget_c,
      // so the budget_c-th largest non-forced key is the reference's cut
      for (int f = tid; f < nforced; f += NT) {
        const int j = forced_j(f);
        const int row = j / per;
        ks[row * PS + (j - row * per)] = 0u;
      }
      __syncthreads();
      fin_thr = kth(budget_c).x;
      if (pq) {
        int c = 0, t = 0;
        for (int e = 0; e < j1 - j0; ++e) {
          c += myrow[e] > fin_thr;
          t += myrow[e] == fin_thr;
        }
        quota = budget_c - dsum<NW>(c, tmp);
        tie_base = dexcl_sum<NW>(t, tmp);
        exact_cut = true;
      }
    }
  }
  // tie: the running index of this thread's keys equal to the cut (advanced in key order)
  auto final_j = [&](int j, uint32_t k, int& tie) {
    if (j < g || (j >= lo && j <= p)) return true;
    if (only_forced) return false;
    if (!exact_cut) return k >= fin_thr;
    if (k == fin_thr) return tie++ < quota;
    return k > fin_thr;
  };

  // ---- compaction + reposition (exact_2.py:587-603); dense ranks (perquery.py:703-719) ----
  int cnt = 0;
  {
    int tie = tie_base;
    for (int e = 0; e < j1 - j0; ++e) cnt += final_j(j0 + e, myrow[e], tie);
  }
  int total;
  const int base = dexcl_sum<NW>(cnt, tmp, &total);
  float mloc = -INFINITY;
  if (!pq) {
    int rank = base - 1, tie = tie_base;
    for (int e = 0; e < j1 - j0; ++e) {
      if (final_j(j0 + e, myrow[e], tie)) {
        rank += 1;
        const float cp = (float)(j0 + e) * a.pos_scale_c;                  // exact_2.py:590
        mloc = fmaxf(mloc, cp - (float)rank);                            // :591
      }
    }
  }
  float run = pq ? 0.0f : dexcl_max<NW>(mloc, (float*)tmp);
  int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  // PQ Stream's positions (pqstream_kernel.py:736-749): aligned blocks of block_n keys walked
  // from the query backwards; key j of block b sits at dist = d[b] + (min(q_pos, end of b) - j)
  // with d[b] = kept keys after block b = total - (kept keys up to the end of b).  The inclusive
  // count at every block end goes to its own LDS region (ceil(M / block_n) words after the
  // scratch words, sized by the launcher).
  int* bend = misc + 8;
  if (stream) {
    int rank = base - 1, tie = tie_base;
    for (int e = 0; e < j1 - j0; ++e) {
      const int j = j0 + e;
      if (final_j(j, myrow[e], tie)) rank += 1;
      if ((j + 1) % a.block_n == 0 || j == m - 1) bend[j / a.block_n] = rank + 1;
    }
    __syncthreads();
  }
  {
    int rank = base - 1, tie = tie_base;
    for (int e = 0; e < j1 - j0; ++e) {
      const int j = j0 + e;
      const bool f = final_j(j, myrow[e], tie);
      if (f) {
        rank += 1;
        if (!pq) {
          const float cp = (float)j * a.pos_scale_c;
          run = fmaxf(run, cp - (float)rank);
        }
      }
      // the shared rule's reposition (exact_2.py:592), the dense rank itself (perquery.py:707),
      // or the streamed distance, negated (pqstream_kernel.py:749; -0 for the query itself)
      float np;
      if (stream) {
        const int b = j / a.block_n;
        const int hb = min(p, b * a.block_n + a.block_n - 1);
        const float dist = (float)(total - bend[b]) + (float)(hb - j);
        np = -dist;
      } else {
        np = pq ? (float)rank : (float)rank + run;
      }
      if (f && rank < a.k_max) {
        irow[rank] = j;
        if (a.newpos_k) nrow[rank] = np;       // (NULL under the per-query rule: dense ranks)
      }
      if (j == p) a.newpos_q[hi] = stream ? 0.0f : np;                   // :603; pqstream :770
    }
  }
  for (int s = min(total, a.k_max) + tid; s < a.k_max; s += NT) {   // sentinel m (:594-600)
    irow[s] = m;
    if (a.newpos_k) nrow[s] = 0.0f;
  }
  if (tid == 0 && a.set_size) a.set_size[hi] = total;
}

// ------------------------------------------------------------------------------------------
// _decode_build_sets_pq (perquery.py:651-720) for one query per workgroup, the row staged in LDS:
//   1. stage the scores as order-preserving keys and take the exact max (perquery.py:683);
//   2. one pass counts the passers s >= max - tau (:684, :688) and histograms the non-forced
//      passers into DEC_PQ_BINS bins linear in the value between the threshold and the max;
//   3. under the cap (:690-701) the bin holding the budget-th largest non-forced passer is found
//      from the histogram and its keys are ranked directly: the cut V and how many keys equal to
//      V are taken (torch.topk's exact budget; ties in ascending key order).  A bin with more
//      than DEC_PQ_CAND keys is split again by key-space bins of its own range, as often as
//      needed (each level divides the range by 4096);
//   4. one pass counts each thread's kept keys and its keys equal to V (one packed scan), one
//      pass writes idx ascending with the dense ranks (:703-719).
// Bit-identical to decode_select_kernel's rule 1, in fewer passes over the row.
// ------------------------------------------------------------------------------------------
constexpr int DEC_PQ_BINS = 4096;            // 16-bit counters, two per LDS word
constexpr int DEC_PQ_CAND = 512;             // keys of the cut bin ranked directly

size_t decode_select_pq_lds_bytes(int M, int NT) {
  const int per = (M + NT - 1) / NT;
  return (size_t)NT * (per | 1) * 4 + DEC_PQ_BINS / 2 * 4 + DEC_PQ_CAND * 4 + 256;
}

template <int NT>
__global__ __launch_bounds__(NT) void decode_select_pq_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int NW = NT / 64;
  constexpr int NB = DEC_PQ_BINS;
  extern __shared__ __align__(16) uint32_t dsm[];
  const int tid = threadIdx.x;
  const int hi = blockIdx.x;
  const int h = hi / a.Q, i = hi % a.Q;
  const int m = a.M - (a.Q - 1 - i);           // keys this query sees
  const int p = a.q_pos0 + i;                  // its position (p < m)
  const int per_max = (a.M + NT - 1) / NT;
  const int per = (m + NT - 1) / NT;
  const int PS = per | 1;                      // odd row stride: conflict-free scans
  uint32_t* ks = dsm;
  uint32_t* hist = dsm + NT * (per_max | 1);   // NB / 2 words
  uint32_t* cand = hist + NB / 2;              // DEC_PQ_CAND
  int* tmp = (int*)(cand + DEC_PQ_CAND);       // NW
  int* misc = tmp + NW;                        // 8
  const int j0 = tid * per, j1 = min(j0 + per, m);
  const int nk = max(j1 - j0, 0);
  uint32_t* myrow = ks + tid * PS;
  const ScoreRow sr = score_row_of(a, h, i);

  // ---- 1. stage the scores as keys, exact max.  16-byte reads (four keys per lane and load,
  // eight loads in flight) when the row is 16-byte aligned; the vector memory unit's cost goes
  // by load instructions ----
  uint32_t kmax = 0;
  auto put = [&](int j, float v) {             // key j < NT * per into its owner's row
    const uint32_t key = j < m ? okey(v) : 0u;
    kmax = max(kmax, key);
    const int row = j / per;
    ks[row * PS + (j - row * per)] = key;
  };
  if (((uintptr_t)sr.p & 15) == 0) {
    const int nq = (NT * per + 3) / 4;         // float4 units covering the keys of every row
    for (int e0 = 0; e0 * NT < nq; e0 += 8) {
      float4 sv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int qd = tid + (e0 + u) * NT;    // keys 4 qd .. 4 qd + 3
        sv[u] = (qd < nq && 4 * qd + 3 < m) ? *(const float4*)sr.at(4 * qd) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (qd < nq && 4 * qd < m && 4 * qd + 3 >= m) {   // the row's ragged end
          sv[u].x = *sr.at(4 * qd);
          if (4 * qd + 1 < m) sv[u].y = *sr.at(4 * qd + 1);
          if (4 * qd + 2 < m) sv[u].z = *sr.at(4 * qd + 2);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int qd = tid + (e0 + u) * NT;
        if (qd < nq) {
          const int j = 4 * qd;
          if (j < NT * per) put(j, sv[u].x);
          if (j + 1 < NT * per) put(j + 1, sv[u].y);
          if (j + 2 < NT * per) put(j + 2, sv[u].z);
          if (j + 3 < NT * per) put(j + 3, sv[u].w);
        }
      }
    }
  } else {
    for (int e0 = 0; e0 < per; e0 += 8) {
      float sv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = tid + (e0 + u) * NT;
        sv[u] = (e0 + u < per && j < m) ? *sr.at(j) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (e0 + u < per) put(tid + (e0 + u) * NT, sv[u]);
    }
  }
  for (int b = tid; b < NB / 2; b += NT) hist[b] = 0u;
  if (tid < 8) misc[tid] = 0;
  kmax = dmax_u<NW>(kmax, (uint32_t*)tmp);       // the barrier inside also publishes the stores
  const float vmax = okey_value(kmax);
  const float thr = vmax - a.tau[h];                                   // perquery.py:684
  const uint32_t kthr = okey(thr);
  // forced keys: [0, g) U [lo, p] (global, local window, self; perquery.py:676-679)
  const int g = min(a.n_global, m);
  const int lo = min(max(0, p - a.n_local + 1), p);
  const int nforced = g + max(p - max(lo, g) + 1, 0);
  auto forced = [&](int j) { return j < g || (j >= lo && j <= p); };

  // ---- 2. passers, non-forced passers with their value histogram and key range ----
  const float span0 = vmax - thr;
  const bool lin = span0 > 0.0f && span0 < INFINITY;   // value-linear bins over [thr, max]
  const float inv0 = lin ? (float)NB / span0 : 0.0f;
  int c_pass = 0, c_nf = 0;
  uint32_t kmin_nf = 0xffffffffu, kmax_nf = 0u;
  for (int e = 0; e < nk; ++e) {
    const uint32_t k = myrow[e];
    if (k >= kthr) {
      ++c_pass;
      if (!forced(j0 + e)) {
        ++c_nf;
        kmin_nf = min(kmin_nf, k);
        kmax_nf = max(kmax_nf, k);
        if (lin) {
          const int b = min((int)((okey_value(k) - thr) * inv0), NB - 1);
          atomicAdd(&hist[b >> 1], 1u << ((b & 1) * 16));
        }
      }
    }
  }
  {                                            // the range over the wave, then one atomic per wave
    const uint32_t wmin = ~wave_max_u32(~kmin_nf), wmax = wave_max_u32(kmax_nf);
    if ((tid & 63) == 0 && wmax >= wmin) {
      atomicMax((unsigned*)&misc[6], ~wmin);    // misc[6] = ~(min key): starts at 0 = ~0xffffffff
      atomicMax((unsigned*)&misc[7], wmax);
    }
  }
  const int packed = dsum<NW>(c_pass | (c_nf << 16), tmp);   // each count < 65536
  const int ge = packed & 0xffff, n_nf = packed >> 16;
  const int count = n_nf + nforced;            // |passers U forced| (perquery.py:687-688)
  if (tid == 0) {
    if (a.usize) a.usize[hi] = ge;
    if (a.overflow) a.overflow[hi] = count > a.k_max ? 1 : 0;
  }

  // ---- 3. the cap cut over the non-forced passers (perquery.py:690-701) ----
  bool only_forced = false, exact_cut = false;
  uint32_t V = 0u;
  int quota = 0;
  if (count > a.k_max) {
    const int budget = a.k_max - nforced;
    if (budget <= 0) {
      only_forced = true;
    } else {
      exact_cut = true;
      int need = budget;                       // rank from the top among the keys in range
      uint32_t rlo = ~(uint32_t)misc[6], rhi = (uint32_t)misc[7];   // key range of the level
      bool linear = lin;                       // level 0: the value bins filled in pass 2
      int shift = 0;
      for (;;) {                               // levels: each divides the range by NB
        if (!linear) {
          if (rlo == rhi) {                    // every key in range equals the cut
            V = rlo;
            quota = need;
            break;
          }
          shift = max(0, 32 - __clz(rhi - rlo) - 12);   // (rhi - rlo) >> shift < NB
          __syncthreads();
          for (int b = tid; b < NB / 2; b += NT) hist[b] = 0u;
          __syncthreads();
          for (int e = 0; e < nk; ++e) {
            const uint32_t k = myrow[e];
            if (k >= rlo && k <= rhi && !forced(j0 + e)) {
              const int b = (int)((k - rlo) >> shift);
              atomicAdd(&hist[b >> 1], 1u << ((b & 1) * 16));
            }
          }
          __syncthreads();
        }
        auto bin_of = [&](uint32_t k) {
          return linear ? min((int)((okey_value(k) - thr) * inv0), NB - 1) : (int)((k - rlo) >> shift);
        };
        // bins in descending order, BPT per thread: the bin holding the need-th largest
        constexpr int BPT = NB / NT;
        int c[BPT], sl = 0;
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
          const int bb = NB - 1 - BPT * tid - e;
          c[e] = (int)((hist[bb >> 1] >> ((bb & 1) * 16)) & 0xffffu);
          sl += c[e];
        }
        const int excl = dexcl_sum<NW>(sl, tmp);
        if (excl < need && excl + sl >= need) {
          int acc = excl, d = NB - 1 - BPT * tid, e = 0;
          for (; e < BPT - 1; ++e) {
            if (acc + c[e] >= need) break;
            acc += c[e];
            d -= 1;
          }
          misc[0] = d;
          misc[1] = need - acc;                // rank within the bin
          misc[2] = c[e];                      // keys in the bin
          misc[3] = 0;                         // collected keys
          misc[4] = 0;                         // ~(min key of the bin)
          misc[5] = 0;                         // max key of the bin
        }
        __syncthreads();
        const int dbin = misc[0], cd = misc[2];
        need = misc[1];
        auto in_bin = [&](int e, uint32_t k) {
          return k >= kthr && (linear || (k >= rlo && k <= rhi)) && !forced(j0 + e) && bin_of(k) == dbin;
        };
        if (cd <= DEC_PQ_CAND) {
          for (int e = 0; e < per; ++e) {        // (uniform trip count: the wave allocates slots)
            const uint32_t k = e < nk ? myrow[e] : 0u;
            const int slot = wave_alloc(e < nk && in_bin(e, k), &misc[3]);
            if (slot >= 0) cand[slot] = k;
          }
          __syncthreads();
          if (tid < cd) {
            const uint32_t v = cand[tid];
            int gt = 0, eq = 0;
            for (int u = 0; u < cd; ++u) {
              const uint32_t w = cand[u];
              gt += w > v;
              eq += w == v;
            }
            if (gt < need && gt + eq >= need) {   // the keys equal to the cut agree
              misc[6] = (int)v;
              misc[7] = need - gt;
            }
          }
          __syncthreads();
          V = (uint32_t)misc[6];
          quota = misc[7];
          break;
        }
        // more than DEC_PQ_CAND keys in the bin: its key range is the next level's
        uint32_t bmin = 0xffffffffu, bmax = 0u;
        for (int e = 0; e < nk; ++e) {
          const uint32_t k = myrow[e];
          if (in_bin(e, k)) {
            bmin = min(bmin, k);
            bmax = max(bmax, k);
          }
        }
        const uint32_t wmin = ~wave_max_u32(~bmin), wmax = wave_max_u32(bmax);
        if ((tid & 63) == 0 && wmax >= wmin) {
          atomicMax((unsigned*)&misc[4], ~wmin);   // ~(min key)
          atomicMax((unsigned*)&misc[5], wmax);
        }
        __syncthreads();
        rlo = ~(uint32_t)misc[4];
        rhi = (uint32_t)misc[5];
        linear = false;
      }
    }
  }
  // 0: not kept, 1: kept, 2: equal to the cut (the first `quota` of them in key order are kept)
  auto klass = [&](int j, uint32_t k) -> int {
    if (forced(j)) return 1;
    if (only_forced) return 0;
    if (!exact_cut) return k >= kthr ? 1 : 0;
    if (k == V) return 2;
    return k > V ? 1 : 0;
  };

  // ---- 4. compaction with dense ranks (perquery.py:703-719) ----
  int n1 = 0, n2 = 0;
  for (int e = 0; e < nk; ++e) {
    const int cl = klass(j0 + e, myrow[e]);
    n1 += cl == 1;
    n2 += cl == 2;
  }
  int tot;
  const int pre = dexcl_sum<NW>(n1 | (n2 << 16), tmp, &tot);    // each total < 65536
  const int pre2 = pre >> 16;
  const int total = (tot & 0xffff) + min(tot >> 16, quota);
  int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  // the kept keys are gathered in LDS (the histogram and candidate words, free now) and written
  // coalesced when k_max fits there; the slot positions are the slot indices (dense ranks)
  const bool staged = a.k_max <= NB / 2 + DEC_PQ_CAND;
  int* obuf = (int*)hist;
  __syncthreads();                             // every read of the histogram / candidates is done
  {
    int rank = (pre & 0xffff) + min(pre2, quota) - 1, tie = pre2;
    for (int e = 0; e < nk; ++e) {
      const int j = j0 + e;
      const int cl = klass(j, myrow[e]);
      const bool f = cl == 1 || (cl == 2 && tie++ < quota);
      if (f) {
        rank += 1;
        if (rank < a.k_max) {
          if (staged) {
            obuf[rank] = j;
          } else {
            irow[rank] = j;
            if (a.newpos_k) nrow[rank] = (float)rank;
          }
        }
      }
      if (j == p) a.newpos_q[hi] = (float)rank;   // the query itself is forced (:719)
    }
  }
  const int nvalid = min(total, a.k_max);
  if (staged) {
    __syncthreads();
    for (int s = tid; s < a.k_max; s += NT) {
      irow[s] = s < nvalid ? obuf[s] : m;     // sentinel m
      if (a.newpos_k) nrow[s] = s < nvalid ? (float)s : 0.0f;
    }
  } else {
    for (int s = nvalid + tid; s < a.k_max; s += NT) {   // sentinel m
      irow[s] = m;
      if (a.newpos_k) nrow[s] = 0.0f;
    }
  }
  if (tid == 0 && a.set_size) a.set_size[hi] = total;
}

// ------------------------------------------------------------------------------------------
// The same rule with the row in registers as fp32 values (rows of up to NT * 4G keys, k_max <=
// DEC_PQR_STAGE).
//   - Thread t owns the 4-key groups t, t + NT, ..., t + (G - 1) NT: every pass over the row is a
//     coalesced sweep with compile-time indexing, and no key needs a division to find its owner.
//   - The values stay floats: float comparisons order them as the LDS kernel's keys do (-0 equals
//     +0 there too), so the threshold, the bins, the cut and its ties agree bit for bit, without
//     a key conversion per pass.  Two quiet NaN payloads mark the keys past the row's end (before
//     the max, which skips NaN) and the forced keys (once their passers are counted): NaN passes
//     no comparison, so no later pass tests a key's index.  A row whose own scores hold NaN is
//     outside that agreement (its NaN keys are never taken).
//   - Level 0 bins are linear in the value over [max - tau, max], where the passers lie; a cut bin
//     holding more than DEC_PQ_CAND keys is split by key-space bins of its key range (closed-form
//     bin ranges), as often as needed.
//   - Per-key LDS updates are branch-free: every wave has passers, so a branch would be taken
//     anyway; non-passers add to, and dropped keys store into, per-lane spare words.
//   - Dense ranks come from segments of 256 consecutive keys (one wave, one group index): a wave
//     scan inside each segment and one scan over the G * NW segment totals.
//   - SH: the shared files' rule without a top-pct cut (exact_2.py:549-603), the same passers,
//     forced keys and cap by score, except that every key equal to the cut is kept (score >=
//     cut_c, :582) and the first k_max kept keys in key order take the slots; positions are the
//     reposition rank + cummax(fl(j pos_scale) - rank) over the kept keys (:587-592), a max scan
//     over the same segments.
// ------------------------------------------------------------------------------------------
constexpr int DEC_PQR_BINS = 2048;                         // level bins, 32-bit counters
constexpr int DEC_PQR_STAGE = DEC_PQR_BINS + DEC_PQ_CAND;  // histogram + cut-bin values (words)
constexpr uint32_t DEC_NAN_END = 0x7fc0beefu;              // past the row's end
constexpr uint32_t DEC_NAN_FORCED = 0x7fc0f00du;           // forced

// float max-scan over the 64 lanes (no NaN), the shifted-in lanes at -inf
__device__ __forceinline__ float wave_incl_max_f32(float x) {
  const int ninf = __builtin_bit_cast(int, -INFINITY);
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x111, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x112, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x114, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x118, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x142, 0xa, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, x), 0x143, 0xc, 0xf, false)));
  return x;
}

// 512-thread instances at 64 VGPRs (eight waves per SIMD, four rows per CU; the 8-group
// instance spills a few registers and still measured 6.91 -> 6.67 ms at config 3 as written)
template <int NT, int G, bool SH>
__global__ __launch_bounds__(NT, NT == 512 ? 8 : 4) void decode_select_pq_reg_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int NW = NT / 64;
  constexpr int NB = DEC_PQR_BINS;
  constexpr int BPT = NB / NT;                 // bins per thread in the cut search
  constexpr int NSEG = G * NW;                 // <= 64: one wave scans the segment totals
  constexpr int SPL = (NSEG + 63) / 64;        // segments per lane in the scans over them
  static_assert(NSEG <= 128 && BPT >= 1, "launch shape");
  constexpr int SPARE = DEC_PQR_STAGE;         // 64 per-lane spare words after the staging area
  __shared__ __align__(16) uint32_t lbuf[DEC_PQR_STAGE + 64];   // histogram + cut-bin values, then idx
  __shared__ int seg[NSEG];
  __shared__ float segm[SH ? NSEG : 1];       // SH: each segment's max of fl(j ps - rank)
  __shared__ float red_max[NW];
  __shared__ int red_sum[NW];
  __shared__ int red_scan[NW];
  __shared__ int misc[6];
  __shared__ float cut_v;
  __shared__ int cut_q, cut_eq, seg_total;
  uint32_t* hist = lbuf;
  float* candv = (float*)(lbuf + NB);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = blockIdx.x;
  const int h = hi / a.Q, i = hi % a.Q;
  const int m = a.M - (a.Q - 1 - i);           // keys this query sees
  const int p = a.q_pos0 + i;                  // its position (p < m)
  const ScoreRow sr = score_row_of(a, h, i);
  const float nan_end = __uint_as_float(DEC_NAN_END);
  // key (e, c) of this thread is j0 + 4 NT e + c.  Each pass takes j0 afresh (an empty asm the
  // compiler cannot see through), so that no pass keeps another pass's key indices live.
  auto fresh_j0 = [&]() {
    int j0 = 4 * tid;
    asm volatile("" : "+v"(j0));
    return j0;
  };
  auto is_forced = [](float v) { return __float_as_uint(v) == DEC_NAN_FORCED; };
  // wave 0: the segment counts in key order to exclusive prefix sums in place, and their total;
  // SPL consecutive segments per lane
  auto seg_scan = [&]() {
    int v[SPL], t = 0;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      v[k] = lane * SPL + k < NSEG ? seg[lane * SPL + k] : 0;
      t += v[k];
    }
    const int x = wave_incl_sum(t);
    int run = x - t;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      if (lane * SPL + k < NSEG) seg[lane * SPL + k] = run;
      run += v[k];
    }
    if (lane == 63) seg_total = x;
  };
  // group e of this wave holds keys [4 (e NT + 64 wave), + 256): the passes skip the groups that
  // start past the row's end (wave-uniform branches; their keys would all be past the end)
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto live = [&](int e) { return 4 * (e * NT + 64 * wave_u) < m; };
  // a value taken afresh (an empty asm): the rare passes' key conversions are not shared with
  // each other, which would keep 4G of them live
  auto fresh_f = [](float v) {
    asm volatile("" : "+v"(v));
    return v;
  };

  // ---- 1. the row's values (DEC_NAN_END past its end) and the exact max ----
  float val[G][4];
  const int js = fresh_j0();
  if (((uintptr_t)sr.p & 15) == 0) {
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const int j = js + 4 * NT * e;
      float4 v;
      if (!live(e)) {
        v = make_float4(nan_end, nan_end, nan_end, nan_end);
      } else if (j + 3 < m) {
        v = *(const float4*)sr.at(j);
      } else {
        v = make_float4(nan_end, nan_end, nan_end, nan_end);
        if (j < m) v.x = *sr.at(j);
        if (j + 1 < m) v.y = *sr.at(j + 1);
        if (j + 2 < m) v.z = *sr.at(j + 2);
      }
      val[e][0] = v.x; val[e][1] = v.y; val[e][2] = v.z; val[e][3] = v.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = js + 4 * NT * e + c;
        val[e][c] = j < m ? *sr.at(j) : nan_end;
      }
  }
  float vmax = -INFINITY;
#pragma unroll
  for (int e = 0; e < G; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) vmax = fmaxf(vmax, val[e][c]);   // (fmaxf skips NaN)
  vmax = wave_max_f32(vmax);
  if (lane == 0) red_max[wave] = vmax;
  for (int b = tid; b < NB; b += NT) hist[b] = 0u;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) vmax = fmaxf(vmax, red_max[w]);
  const float thr = vmax - a.tau[h];                                   // perquery.py:684
  // level-0 bins: linear in the value over [thr, max]; key-space bins over the passers' keys when
  // that span is not finite and positive (tau = inf, tau <= 0)
  const float vspan = vmax - thr;
  const bool lin = vspan > 0.0f && vspan < INFINITY;
  const float inv0 = lin ? (float)NB / vspan : 0.0f;
  const float boff = -(thr * inv0);            // value bin of v: fma(v, inv0, boff), monotone in v
  const uint32_t kthr = okey(thr), kmx = okey(vmax);
  const uint32_t span0 = kmx >= kthr ? kmx - kthr : 0u;
  const int shift0 = span0 == 0u ? 0 : max(0, 32 - __clz(span0) - 11);   // span0 >> shift0 < NB

  // ---- 2. forced keys (perquery.py:676-679): [0, g) U [lo, p], global, local window and self;
  // only the groups that hold one take the branch ----
  const int g = min(a.n_global, m);
  const int lo = min(max(0, p - a.n_local + 1), p);
  const int nforced = g + max(p - max(lo, g) + 1, 0);
  const float nan_forced = __uint_as_float(DEC_NAN_FORCED);
  int c_fp = 0;                                // forced passers
  {
    const int jf = fresh_j0();
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const int j0 = jf + 4 * NT * e;
      if (j0 < g || (j0 + 3 >= lo && j0 <= p)) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int j = j0 + c;
          const bool f = j < g || (j >= lo && j <= p);
          c_fp += (f && val[e][c] >= thr) ? 1 : 0;
          val[e][c] = f ? nan_forced : val[e][c];
        }
      }
    }
  }
  // ---- 3. the non-forced passers: count and level-0 histogram ----
  auto vbin = [&](float v) { return min((int)fmaf(v, inv0, boff), NB - 1); };
  int c_nf = 0;
  if (lin) {
#pragma unroll
    for (int e = 0; e < G; ++e) {
      if (!live(e)) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float v = val[e][c];
        const bool ps = v >= thr;
        c_nf += ps ? 1 : 0;
        atomicAdd(&lbuf[ps ? vbin(ps ? v : thr) : SPARE + lane], 1u);   // (spare words: never read)
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float v = fresh_f(val[e][c]);
        const bool ps = v >= thr;
        c_nf += ps ? 1 : 0;
        atomicAdd(&lbuf[ps ? (int)((okey(ps ? v : thr) - kthr) >> shift0) : SPARE + lane], ps ? 1u : 0u);
      }
  }
  int packed = wave_sum((c_fp + c_nf) | (c_nf << 16));   // each count < 65536
  if (lane == 0) red_sum[wave] = packed;
  if (tid < 6) misc[tid] = 0;
  __syncthreads();                             // (also publishes the histogram)
  packed = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) packed += red_sum[w];
  const int ge = packed & 0xffff, n_nf = packed >> 16;
  const int count = n_nf + nforced;            // |passers U forced| (perquery.py:687-688)
  if (tid == 0) {
    if (a.usize) a.usize[hi] = ge;
    if (a.overflow) a.overflow[hi] = count > a.k_max ? 1 : 0;
  }

  // ---- 4. the cap cut over the non-forced passers (perquery.py:690-701) ----
  bool only_forced = false, exact_cut = false;
  bool ties_all = true;                        // every key equal to the cut is kept
  float V = 0.0f;
  int quota = 0;
  if (count > a.k_max) {
    const int budget = a.k_max - nforced;
    if (budget <= 0) {
      only_forced = true;
    } else {
      exact_cut = true;
      int need = budget;                       // rank from the top among the level's keys
      uint32_t rlo = kthr, rhi = kmx;          // the key-space level's key range
      int shift = shift0;
      bool linear = lin;                       // level 0 in value bins
      int range_n = n_nf;                      // keys in the level's range
      for (int level = 0;; ++level) {          // each key-space level divides the range by 2^11
        if (level > 0) {
          if (rlo == rhi) {                    // every key in range equals the cut
            V = okey_value(rlo);
            quota = need;
            ties_all = need == range_n;
            break;
          }
          shift = max(0, 32 - __clz(rhi - rlo) - 11);
          __syncthreads();                     // the previous level's histogram is read
          for (int b = tid; b < NB; b += NT) hist[b] = 0u;
          if (tid == 0) misc[3] = 0;
          __syncthreads();
#pragma unroll
          for (int e = 0; e < G; ++e)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const float v = fresh_f(val[e][c]);
              const uint32_t k = v >= thr ? okey(v) : 0u;   // (rlo >= the threshold key > 0)
              const bool in = k - rlo <= rhi - rlo;
              atomicAdd(&lbuf[in ? (k - rlo) >> shift : SPARE + lane], in ? 1u : 0u);
            }
          __syncthreads();
        }
        // bins in descending order, BPT per thread: the bin holding the need-th largest
        int cb[BPT], sl = 0;
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
          cb[e] = (int)hist[NB - 1 - BPT * tid - e];
          sl += cb[e];
        }
        const int x = wave_incl_sum(sl);
        if (lane == 63) red_scan[wave] = x;
        __syncthreads();
        int excl = x - sl;
#pragma unroll
        for (int w = 0; w < NW; ++w) excl += w < wave ? red_scan[w] : 0;
        if (excl < need && excl + sl >= need) {
          int acc = excl, d = NB - 1 - BPT * tid, e = 0;
          for (; e < BPT - 1; ++e) {
            if (acc + cb[e] >= need) break;
            acc += cb[e];
            d -= 1;
          }
          misc[0] = d;
          misc[1] = need - acc;                // rank within the bin
          misc[2] = cb[e];                     // keys in the bin
        }
        __syncthreads();
        const int d = misc[0], cd = misc[2];
        need = misc[1];
        // the cut bin's keys: the value bin d, or the key range [blo, bhi]
        const uint32_t blo = rlo + ((uint32_t)d << shift);
        const uint32_t bw = (1u << shift) - 1u;
        const uint32_t bhi = rhi - blo <= bw ? rhi : blo + bw;
        // (the threshold and scale taken afresh: the per-key bins are not hoisted out of the
        // level loop, where 32 of them would stay live)
        float thr_l = thr, inv_l = inv0, boff_l = boff;
        asm volatile("" : "+v"(thr_l), "+v"(inv_l), "+v"(boff_l));
        auto in_bin = [&](float v) {
          const bool ps = v >= thr_l;
          return linear ? (ps && min((int)fmaf(ps ? v : thr_l, inv_l, boff_l), NB - 1) == d)
                        : (ps && okey(v) - blo <= bhi - blo);
        };
        if (cd <= DEC_PQ_CAND) {
          // The bin as a value interval [lo_b, hi_b): in key space from its key range; in value
          // bins by searching the first value of bin d and of bin d + 1 within +-32 ulps of
          // their nominal edges, one candidate per lane (the bins are monotone in the value).
          // A search that does not bracket its edge falls back to the bin test per key.
          float lo_b = okey_value(blo), hi_b = okey_value(bhi + 1u);   // (bhi + 1 = 0: NaN)
          bool bounded = true;
          if (linear) {
            auto first_of = [&](int dd, float& out) {   // the least v >= thr in a bin >= dd
              if (dd >= NB) {                  // past the clamped top bin: none
                out = __uint_as_float(DEC_NAN_END);
                return true;
              }
              const float x0 = thr_l + (float)dd / inv_l;
              const float cv = okey_value(okey(x0) + (uint32_t)(lane - 32));
              const bool ge = cv >= thr_l && min((int)fmaf(cv, inv_l, boff_l), NB - 1) >= dd;
              const unsigned long long msk = __ballot(ge);
              const int first = __ffsll(msk) - 1;  // the values rise with the lane
              if (first <= 0 || (msk >> first) != (~0ull >> first)) return false;
              out = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), first));
              return true;
            };
            if (d == 0) lo_b = thr_l;
            else bounded = first_of(d, lo_b);
            bounded = bounded && first_of(d + 1, hi_b);
          }
          if (bounded) {
#pragma unroll
            for (int e = 0; e < G; ++e) {
              if (!live(e)) continue;
#pragma unroll
              for (int c = 0; c < 4; ++c) {    // slots by wave; most waves have none
                const float v = val[e][c];
                const bool in = v >= lo_b && !(v >= hi_b);
                const int slot = wave_alloc(in, &misc[3]);
                if (in && slot < DEC_PQ_CAND) candv[slot] = v;   // (slot < cd)
              }
            }
          } else {
#pragma unroll
            for (int e = 0; e < G; ++e) {
              if (!live(e)) continue;
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                const float v = fresh_f(val[e][c]);
                const bool in = in_bin(v);
                const int slot = wave_alloc(in, &misc[3]);
                if (in && slot < DEC_PQ_CAND) candv[slot] = v;   // (slot < cd)
              }
            }
          }
          __syncthreads();
          if (tid < cd) {
            const float v = candv[tid];
            int gt = 0, eq = 0;
            for (int u = 0; u < cd; ++u) {
              const float w = candv[u];
              gt += w > v;
              eq += w == v;
            }
            if (gt < need && gt + eq >= need) {   // the values equal to the cut agree
              cut_v = v;
              cut_q = need - gt;
              cut_eq = eq;
            }
          }
          __syncthreads();
          V = cut_v;
          quota = cut_q;
          ties_all = cut_q == cut_eq;
          break;
        }
        // more than DEC_PQ_CAND keys: the next level splits the bin's key range
        if (linear) {                          // (the value bin's keys: their min and max)
          uint32_t bmin = 0xffffffffu, bmax = 0u;
#pragma unroll
          for (int e = 0; e < G; ++e)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const float v = fresh_f(val[e][c]);
              const bool in = in_bin(v);
              const uint32_t k = okey(in ? v : thr);
              bmin = min(bmin, in ? k : 0xffffffffu);
              bmax = max(bmax, in ? k : 0u);
            }
          const uint32_t wmin = ~wave_max_u32(~bmin), wmax = wave_max_u32(bmax);
          if (lane == 0 && wmax >= wmin) {
            atomicMax((unsigned*)&misc[4], ~wmin);   // ~(min key): starts at 0 = ~0xffffffff
            atomicMax((unsigned*)&misc[5], wmax);
          }
          __syncthreads();
          rlo = ~(uint32_t)misc[4];
          rhi = (uint32_t)misc[5];
        } else {
          rlo = blo;
          rhi = bhi;
        }
        linear = false;
        range_n = cd;
      }
    }
  }

  if constexpr (SH) ties_all = true;           // every key equal to the cut (exact_2.py:582)

  // ---- 5. compaction with dense ranks (perquery.py:703-719) ----
  // kept: forced, or above the cut (at or above the threshold when nothing is cut); ties: equal
  // to the cut, the first `quota` of them in key order kept.  Per segment (e, wave) the lanes'
  // packed (kept | ties << 16) counts, scanned over the wave.
  float keep_lo = thr, tie_v = __uint_as_float(DEC_NAN_END);   // (NaN: no value ties)
  if (exact_cut) {
    // v > V  <=>  v >= the least float above V (+inf: a NaN bound, which nothing passes)
    const uint32_t vb = __float_as_uint(V);
    keep_lo = (vb & 0x7fffffffu) == 0u ? __uint_as_float(1u)
                                       : __uint_as_float((vb & 0x80000000u) ? vb - 1u : vb + 1u);
    tie_v = V;
  }
  if (only_forced) keep_lo = __uint_as_float(DEC_NAN_END);   // nothing passes a NaN bound
  asm volatile("" : "+v"(keep_lo), "+v"(tie_v));   // (fresh: no pass-3 lane masks kept live)
  int* obuf = (int*)lbuf;
  int rq = -1, total = 0;
  if (ties_all) {
    // every tie kept (or none to cut): kept = forced or at or above one bound, one bit per key
    const float kb = exact_cut ? V : keep_lo;
    float keep_b = kb;
    asm volatile("" : "+v"(keep_b));
    int lpre1[G];
    auto kept1 = [&](float x) { return is_forced(x) || x >= keep_b; };
#pragma unroll
    for (int e = 0; e < G; ++e) {
      lpre1[e] = 0;
      if (!live(e)) {
        if (lane == 63) seg[e * NW + wave] = 0;
        continue;
      }
      int v = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) v += kept1(val[e][c]) ? 1 : 0;
      const int xs = wave_incl_sum(v);
      lpre1[e] = xs - v;
      if (lane == 63) seg[e * NW + wave] = xs;
    }
    __syncthreads();                           // every read of the histogram / cut-bin values is done
    if (wave == 0) seg_scan();                 // segments in key order: e-major, then wave
    __syncthreads();
    total = seg_total;
    const int jw = fresh_j0();
    float lexc[SH ? G : 1];                      // SH: the max over this wave's lanes before this one
#pragma unroll
    for (int e = 0; e < G; ++e) {
      if (!live(e)) {
        if constexpr (SH) {
          lexc[e] = -INFINITY;
          if (lane == 63) segm[e * NW + wave] = -INFINITY;
        }
        continue;
      }
      int rank = seg[e * NW + wave] + lpre1[e];   // kept keys before this lane's keys
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bool kp = kept1(val[e][c]);
        const int j = jw + 4 * NT * e + c;
        obuf[kp && rank < DEC_PQR_STAGE ? rank : SPARE + lane] = j;   // (rank < k_max, or past it: SH)
        if constexpr (SH) mx = kp ? fmaxf(mx, (float)j * a.pos_scale_c - (float)rank) : mx;   // :590-591
        rank += kp ? 1 : 0;
      }
      if constexpr (SH) {
        const float x = wave_incl_max_f32(mx);
        const float up = __shfl_up(x, 1, 64);
        lexc[e] = lane == 0 ? -INFINITY : up;
        if (lane == 63) segm[e * NW + wave] = x;
      }
    }
    if constexpr (SH) {
      // the segments' exclusive max in key order, then every kept key's position rank + cummax,
      // written straight to its slot (:592, :601); the query's own at key p (:603)
      __syncthreads();
      if (wave == 0) {                         // SPL consecutive segments per lane
        float v[SPL], t = -INFINITY;
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
          v[k] = lane * SPL + k < NSEG ? segm[lane * SPL + k] : -INFINITY;
          t = fmaxf(t, v[k]);
        }
        const float up = __shfl_up(wave_incl_max_f32(t), 1, 64);
        float run = lane == 0 ? -INFINITY : up;
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
          if (lane * SPL + k < NSEG) segm[lane * SPL + k] = run;
          run = fmaxf(run, v[k]);
        }
      }
      __syncthreads();
      float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
#pragma unroll
      for (int e = 0; e < G; ++e) {
        if (!live(e)) continue;
        int rank = seg[e * NW + wave] + lpre1[e];
        float run = fmaxf(segm[e * NW + wave], lexc[e]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool kp = kept1(val[e][c]);
          const int j = jw + 4 * NT * e + c;
          run = kp ? fmaxf(run, (float)j * a.pos_scale_c - (float)rank) : run;
          const float np = (float)rank + run;
          if (kp && rank < a.k_max) nrow[rank] = np;
          if (j == p) a.newpos_q[hi] = np;
          rank += kp ? 1 : 0;
        }
      }
    } else if (tid == ((p >> 2) & (NT - 1))) {
      // the query's own rank (it is forced, :719), in the thread that holds key p
      const int ep = (p >> 2) / NT, cp = p & 3;
#pragma unroll
      for (int e = 0; e < G; ++e)
        if (e == ep) {
          int r = seg[e * NW + wave] + lpre1[e];
#pragma unroll
          for (int c = 0; c < 3; ++c) r += c < cp && kept1(val[e][c]) ? 1 : 0;
          rq = r;
        }
    }
  } else {
    // ties at the cut taken in part: classes of 2 bits (kept / tie) and tie counts in the scans
    int lpre[G];
    uint32_t cls[G];                             // the four keys' classes, 2 bits each
#pragma unroll
    for (int e = 0; e < G; ++e) {
      int v = 0;
      cls[e] = 0u;
      lpre[e] = 0;
      if (!live(e)) {
        if (lane == 63) seg[e * NW + wave] = 0;
        continue;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float x = val[e][c];
        const bool k1 = is_forced(x) || x >= keep_lo;
        const bool k2 = x == tie_v;
        v += k1 ? 1 : (k2 ? 0x10000 : 0);
        cls[e] |= (k1 ? 1u : (k2 ? 2u : 0u)) << (2 * c);
      }
      const int xs = wave_incl_sum(v);
      lpre[e] = xs - v;
      if (lane == 63) seg[e * NW + wave] = xs;
    }
    __syncthreads();                             // every read of the histogram / cut-bin values is done
    if (wave == 0) seg_scan();                   // segments in key order: e-major, then wave
    __syncthreads();
    const int tot = seg_total;
    total = (tot & 0xffff) + min(tot >> 16, quota);
    const int jw = fresh_j0();
#pragma unroll
    for (int e = 0; e < G; ++e) {
      if (!live(e)) continue;
      const int base = seg[e * NW + wave] + lpre[e];
      int n1 = base & 0xffff, n2 = base >> 16;   // kept keys and cut ties before this lane's keys
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = jw + 4 * NT * e + c;
        const uint32_t cl = (cls[e] >> (2 * c)) & 3u;
        const int rank = n1 + min(n2, quota);
        const bool kept = cl == 1u || (cl == 2u && n2 < quota);
        obuf[kept && rank < DEC_PQR_STAGE ? rank : SPARE + lane] = j;   // (rank < k_max)
        rq = j == p ? rank : rq;                 // the query itself is forced (:719)
        n1 += (int)(cl & 1u);
        n2 += (int)(cl >> 1);
      }
    }
  }
  if (rq >= 0) a.newpos_q[hi] = (float)rq;
  const int nvalid = min(total, a.k_max);
  int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  __syncthreads();
  for (int s = tid; s < a.k_max; s += NT) {     // slot positions are the slot indices (SH: written
    irow[s] = s < nvalid ? obuf[s] : m;         // above); sentinel m
    if (SH ? s >= nvalid : a.newpos_k != nullptr) nrow[s] = s < nvalid ? (float)s : 0.0f;   // (NULL: not kept)
  }
  if (tid == 0 && a.set_size) a.set_size[hi] = total;
}

// ------------------------------------------------------------------------------------------
// attend: split s of query (h, i) sweeps slots [64 s, 64 s + 64); 16 lanes per slot, each lane
// NPL rotation pairs; every 16-lane group keeps its own online-softmax state, merged in LDS.
// A batch of many queries (the per-query prefill) gives each query fewer splits, down to one
// workgroup sweeping all its slots in 64-slot steps and writing the output itself: the split
// states and the merge kernel then cost nothing.
// ------------------------------------------------------------------------------------------
constexpr int DEC_SPL = 64;                    // slots per attend step

int decode_nsplit(int k_max) { return (k_max + DEC_SPL - 1) / DEC_SPL; }
// splits per query: the 64-slot steps of k_max for a single query, fewer as the batch grows
// (a function of Q and k_max only, so that a query's output does not depend on the head count)
static int decode_attend_splits(int Q, int k_max) {
  const int want = (256 + Q - 1) / Q;
  return max(1, min(decode_nsplit(k_max), want));
}

template <int DT, int D>
__global__ __launch_bounds__(256) void decode_attend_kernel(DecodeArgs a, int steps) {
#pragma clang fp contract(off)
  constexpr int NPL = D / 32;                  // pairs per lane
  __shared__ float sm_m[16], sm_l[16];
  __shared__ float sm_acc[16][D];
  const int split = blockIdx.x, hi = blockIdx.y;   // split: `steps` 64-slot steps of the query
  const int h = hi / a.Q, i = hi % a.Q;
  const int hk = h / (a.H / a.Hkv);
  const int m = a.M - (a.Q - 1 - i);
  const int p = a.q_pos0 + i;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, grp = wave * 4 + (lane >> 4);
  const int d0 = l16 * NPL;                    // this lane's frequencies d0 .. d0 + NPL - 1
  const int nslots = a.set_size ? min(a.set_size[hi], a.k_max) : a.k_max;
  const int send = min(nslots, (split + 1) * steps * DEC_SPL);
  float invf[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) invf[e] = a.inv_freq_c[d0 + e];
  // the query rotated at newpos_q
  float q1[NPL], q2[NPL];
  {
    float x1[NPL], x2[NPL];
    const int64_t qb = (int64_t)h * a.q_hs + (int64_t)i * a.q_ts + d0;
    load_n<DT, NPL>(a.q, qb, x1);
    load_n<DT, NPL>(a.q, qb + D / 2, x2);
    const float npq = a.newpos_q[hi];
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
      float sn, cs;
      fast_sincos(npq * invf[e], sn, cs);
      cs = cs * a.rope_scale_c;
      sn = sn * a.rope_scale_c;
      q1[e] = x1[e] * cs - x2[e] * sn;
      q2[e] = x2[e] * cs + x1[e] * sn;
    }
  }
  const int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  const float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  constexpr int U = DEC_SPL / 16;            // slots per group and step
  // the group's state over its steps: running max, sum and accumulators of the weights
  float mrun = -INFINITY, lrun = 0.0f, acc1[NPL], acc2[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) { acc1[e] = 0.0f; acc2[e] = 0.0f; }
  for (int s0 = split * steps * DEC_SPL; s0 < send; s0 += DEC_SPL) {
  const int s1 = min(s0 + DEC_SPL, send);
  // this group's four slots: indices first, then every K / V row request, then the arithmetic
  int jv[U];
  bool okv[U];
  float npk[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int s = s0 + grp * U + u;
    const int j = s < s1 ? irow[s] : -1;
    okv[u] = j >= 0 && j < m && (!a.causal || j <= p);   // sentinel m (exact_2.py:615; :195, 210)
    jv[u] = okv[u] ? j : 0;
    npk[u] = s < s1 ? (a.newpos_k ? nrow[s] : (float)s) : 0.0f;   // (NULL: dense ranks)
  }
  float x1[U][NPL], x2[U][NPL], v1[U][NPL], v2[U][NPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t kb = (int64_t)hk * a.k_hs + (int64_t)jv[u] * a.k_ts + d0;
    const int64_t vb = (int64_t)hk * a.v_hs + (int64_t)jv[u] * a.v_ts + d0;
    load_n<DT, NPL>(a.k, kb, x1[u]);
    load_n<DT, NPL>(a.k, kb + D / 2, x2[u]);
    load_n<DT, NPL>(a.v, vb, v1[u]);
    load_n<DT, NPL>(a.v, vb + D / 2, v2[u]);
  }
  float sc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
      float sn, cs;
      fast_sincos(npk[u] * invf[e], sn, cs);
      cs = cs * a.rope_scale_c;
      sn = sn * a.rope_scale_c;
      const float k1 = x1[u][e] * cs - x2[u][e] * sn;
      const float k2 = x2[u][e] * cs + x1[u][e] * sn;
      part = fmaf(q2[e], k2, fmaf(q1[e], k1, part));
    }
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    part += __shfl_xor(part, 4, 64);
    part += __shfl_xor(part, 8, 64);
    sc[u] = okv[u] ? part * a.sm_scale : -INFINITY;
  }
  // the step's own softmax state, then folded into the group's state (a first step is taken as
  // it is, so that a one-step split is exactly the step's state)
  float mst = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; ++u) mst = fmaxf(mst, sc[u]);
  if (mst > -INFINITY) {
    float lst = 0.0f, b1[NPL], b2[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) { b1[e] = 0.0f; b2[e] = 0.0f; }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float pw = okv[u] ? __expf(sc[u] - mst) : 0.0f;
      lst += pw;
#pragma unroll
      for (int e = 0; e < NPL; ++e) {
        b1[e] = fmaf(pw, v1[u][e], b1[e]);
        b2[e] = fmaf(pw, v2[u][e], b2[e]);
      }
    }
    if (mrun == -INFINITY) {
      mrun = mst;
      lrun = lst;
#pragma unroll
      for (int e = 0; e < NPL; ++e) { acc1[e] = b1[e]; acc2[e] = b2[e]; }
    } else {
      const float mn = fmaxf(mrun, mst);
      const float wo = __expf(mrun - mn), wn = __expf(mst - mn);
      lrun = lrun * wo + lst * wn;
#pragma unroll
      for (int e = 0; e < NPL; ++e) {
        acc1[e] = acc1[e] * wo + b1[e] * wn;
        acc2[e] = acc2[e] * wo + b2[e] * wn;
      }
      mrun = mn;
    }
  }
  }   // steps
  if (l16 == 0) { sm_m[grp] = mrun; sm_l[grp] = lrun; }
#pragma unroll
  for (int e = 0; e < NPL; ++e) { sm_acc[grp][d0 + e] = acc1[e]; sm_acc[grp][D / 2 + d0 + e] = acc2[e]; }
  __syncthreads();
  // merge the 16 group states: (max, sum, D accumulators) of the split
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < 16; ++u) M = fmaxf(M, sm_m[u]);
  float L = 0.0f;
  if (M > -INFINITY)
    for (int u = 0; u < 16; ++u)
      if (sm_m[u] > -INFINITY) L += sm_l[u] * __expf(sm_m[u] - M);
  float* part = a.part + ((int64_t)hi * gridDim.x + split) * (D + 2);
  for (int d = threadIdx.x; d < D; d += 256) {
    float A = 0.0f;
    if (M > -INFINITY)
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (sm_m[u] > -INFINITY) A += sm_acc[u][d] * __expf(sm_m[u] - M);
    if (gridDim.x == 1) {     // the only split: the output (as the merge kernel writes it)
      const float o = L > 0.0f ? A / L : 0.0f;
      const int64_t oi = (int64_t)hi * D + d;
      if constexpr (DT == DT_F32) ((float*)a.out)[oi] = o;
      else ((uint16_t*)a.out)[oi] = (uint16_t)(DT == DT_BF16 ? f32_to_bf16_bits(o) : f32_to_f16_bits(o));
    } else {
      part[d] = A;
    }
  }
  if (threadIdx.x == 0 && gridDim.x > 1) {
    part[D] = M;
    part[D + 1] = L;
  }
}

// ------------------------------------------------------------------------------------------
// attend for a large batch under the per-query rule: 16 queries of one head per workgroup, one
// 16-lane group per query sweeping all of its slots and writing the output.  Each half of a group
// (8 lanes) takes its own slots, a lane holding D/16 rotation pairs of the slot's K and V rows, so
// every row arrives in 16-byte loads (bf16, D = 128): the vector memory pipeline bounds this
// gather, with the arithmetic close behind (bf16 scores take one dot2 per pair of K elements
// against the query's coefficients at the slot's rank, instead of rotating K).  Under
// _decode_build_sets_pq every slot s sits at its dense rank s (perquery.py:707-717: idx is
// ascending and newpos_k gathers the ranks at idx), so the (cos, sin) of slot s are the same for
// every query: the workgroup computes them once per block of DEC_TB slots into LDS.  The launcher
// takes this kernel only when the selection of the same call wrote the sets (dense_ranks); sets
// from the caller go to the split attend, which reads every slot's position.
// ------------------------------------------------------------------------------------------
constexpr int DEC_QPW = 16;                    // queries per workgroup
constexpr int DEC_TB = 32;                     // slots per table block: 16 KB of LDS at D = 128

namespace {

// NF consecutive elements of a row as raw 32-bit words (bf16 / f16 pairs or fp32)
template <int DT, int NF>
struct RowPart {
  static constexpr int NW = NF * (DT == DT_F32 ? 4 : 2) / 4;
  uint32_t w[NW];
};

template <int DT, int NF>
__device__ __forceinline__ void load_part(const void* p, int64_t i, RowPart<DT, NF>& r) {
  constexpr int NW = RowPart<DT, NF>::NW;
  const uint32_t* src = (const uint32_t*)((const char*)p + i * (DT == DT_F32 ? 4 : 2));
  if constexpr (NW % 4 == 0) {
#pragma unroll
    for (int u = 0; u < NW / 4; ++u) {
      const u32x4 x = ((const u32x4*)src)[u];
      r.w[4 * u] = x[0]; r.w[4 * u + 1] = x[1]; r.w[4 * u + 2] = x[2]; r.w[4 * u + 3] = x[3];
    }
  } else {
    static_assert(NW == 2, "row part width");
    const u32x2 x = *(const u32x2*)src;
    r.w[0] = x[0]; r.w[1] = x[1];
  }
}

template <int DT, int NF>
__device__ __forceinline__ float part_elem(const RowPart<DT, NF>& r, int e) {
  if constexpr (DT == DT_F32) return __uint_as_float(r.w[e]);
  else if constexpr (DT == DT_BF16) return __uint_as_float((e & 1) ? (r.w[e >> 1] & 0xffff0000u) : (r.w[e >> 1] << 16));
  else return f16_bits_to_f32((e & 1) ? (r.w[e >> 1] >> 16) : (r.w[e >> 1] & 0xffffu));
}

}  // namespace

constexpr int DEC_GU = 4;                      // slots per half group and step

// 16-bit instances at five waves per SIMD (96 VGPRs with a few spilled outside the slot loop;
// 18 KB of LDS for the table and the indices): 23.9 -> 23.5 ms at config 3 against four waves;
// fp32 takes what its registers allow
template <int DT, int D, bool IDX4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DT == DT_F32 ? 1 : 5)))
void decode_attend_grouped_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int HD = D / 2;
  constexpr int NF = D / 16;                   // rotation pairs per lane (8 lanes per slot)
  constexpr int U = DEC_GU;
  static_assert(U == 4 && DEC_TB % (2 * U) == 0, "a step's slots stay inside one table block");
  static_assert(256 % HD == 0 && DEC_QPW * DEC_TB / 4 <= 256, "table and index staging shapes");
  __shared__ __align__(16) float tcs[DEC_TB][HD];
  __shared__ __align__(16) float tsn[DEC_TB][HD];
  __shared__ __align__(16) int sidx[DEC_QPW][DEC_TB];   // every query's slot indices in the block
  __shared__ int gns[DEC_QPW];                          // every query's slot count
  __shared__ int wmax;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, grp = wave * 4 + (lane >> 4);
  const int half = l16 >> 3, l8 = l16 & 7;
  const int f0 = l8 * NF;                      // this lane's frequencies f0 .. f0 + NF - 1
  // workgroup -> (head, query group), the latest query groups (the largest sets) first
  const int nqg = (a.Q + DEC_QPW - 1) / DEC_QPW;
  const int h = blockIdx.x % a.H;
  const int qg = nqg - 1 - (int)(blockIdx.x / a.H);
  const int i = qg * DEC_QPW + grp;
  const bool live = i < a.Q;
  const int ic = live ? i : a.Q - 1;
  const int hi = h * a.Q + ic;
  const int hk = h / (a.H / a.Hkv);
  const int m = a.M - (a.Q - 1 - ic);
  const int p = a.q_pos0 + ic;
  // a slot's key is attended when 0 <= j < m and, causal, j <= p: one unsigned compare with jlim
  const uint32_t jlim = (uint32_t)max(0, a.causal ? min(m, p + 1) : m);
  const int nslots = !live ? 0 : (a.set_size ? min(a.set_size[hi], a.k_max) : a.k_max);
  if (threadIdx.x == 0) wmax = 0;
  __syncthreads();
  if (l16 == 0) {
    gns[grp] = nslots;
    if (nslots > 0) atomicMax(&wmax, nslots);
  }
  // the query rotated at newpos_q, this lane's pairs
  float q1[NF], q2[NF];
  {
    float x1[NF], x2[NF];
    const int64_t qb = (int64_t)h * a.q_hs + (int64_t)ic * a.q_ts + f0;
    load_n<DT, NF>(a.q, qb, x1);
    load_n<DT, NF>(a.q, qb + HD, x2);
    const float npq = a.newpos_q[hi];
#pragma unroll
    for (int e = 0; e < NF; ++e) {
      float sn, cs;
      fast_sincos(npq * a.inv_freq_c[f0 + e], sn, cs);
      cs = cs * a.rope_scale_c;
      sn = sn * a.rope_scale_c;
      q1[e] = x1[e] * cs - x2[e] * sn;
      q2[e] = x2[e] * cs + x1[e] * sn;
    }
  }
  // K / V rows by 32-bit byte offsets from the head's rows (the launcher checks that a head's
  // cache spans less than 2 GiB): one multiply-add per slot, the upper half an immediate offset
  constexpr int ESZ = DT == DT_F32 ? 4 : 2;
  const char* kbase = (const char*)a.k + (int64_t)hk * a.k_hs * ESZ;
  const char* vbase = (const char*)a.v + (int64_t)hk * a.v_hs * ESZ;
  const uint32_t kts = (uint32_t)(a.k_ts * ESZ), vts = (uint32_t)(a.v_ts * ESZ), fo = (uint32_t)(f0 * ESZ);
  // the query's running max (the same in both halves) and each half's sum and accumulators
  float mrun = -INFINITY, lrun = 0.0f, acc1[NF], acc2[NF];
#pragma unroll
  for (int e = 0; e < NF; ++e) { acc1[e] = 0.0f; acc2[e] = 0.0f; }
  const float tf = a.inv_freq_c[threadIdx.x % HD];   // this thread's frequency in the table
  __syncthreads();
  const int nall = wmax;
  for (int s0 = 0; s0 < nall; s0 += DEC_TB) {
    if (s0 > 0) __syncthreads();               // every group is done with the previous block
    for (int x = threadIdx.x; x < DEC_TB * HD; x += 256) {
      const int r = x / HD, f = x % HD;
      float sn, cs;
      fast_sincos((float)(s0 + r) * tf, sn, cs);
      tcs[r][f] = cs * a.rope_scale_c;
      tsn[r][f] = sn * a.rope_scale_c;
    }
    // the block's slot indices of every query, four per thread (16-byte loads when the rows are
    // 16-byte aligned and k_max % 4 == 0: s + 3 < k_max); the steps read them from LDS
    if (threadIdx.x < DEC_QPW * DEC_TB / 4) {
      const int g = threadIdx.x / (DEC_TB / 4), c = 4 * (threadIdx.x % (DEC_TB / 4)), s = s0 + c;
      const int ns = gns[g];                   // 0 for a query past Q
      int4 iv = make_int4(-1, -1, -1, -1);
      if (s < ns) {
        const int32_t* row = a.idx + ((int64_t)h * a.Q + qg * DEC_QPW + g) * a.k_max + s;
        if constexpr (IDX4) {
          iv = *(const int4*)row;
        } else {
          iv.x = row[0];
          if (s + 1 < ns) iv.y = row[1];
          if (s + 2 < ns) iv.z = row[2];
          if (s + 3 < ns) iv.w = row[3];
        }
      }
      *(int4*)&sidx[g][c] = iv;
    }
    __syncthreads();
    const int send = min(nslots, s0 + DEC_TB);
    for (int t0 = s0; t0 < send; t0 += 2 * U) {
      const int sb = t0 + half * U;            // this half's U slots sb .. sb + U - 1
      const int4 iv = *(const int4*)&sidx[grp][sb - s0];   // sb - s0 is a multiple of 4
      const int jr[U] = {iv.x, iv.y, iv.z, iv.w};
      int jv[U];
      bool okv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = sb + u < send ? jr[u] : -1;
        okv[u] = (uint32_t)j < jlim;            // sentinel m and j = -1 fail it (perquery.py:739)
        jv[u] = okv[u] ? j : 0;
      }
      RowPart<DT, NF> k1r[U], k2r[U], v1r[U], v2r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t ko = (uint32_t)jv[u] * kts + fo, vo = (uint32_t)jv[u] * vts + fo;
        load_part<DT, NF>(kbase + ko, 0, k1r[u]);
        load_part<DT, NF>(kbase + ko, HD, k2r[u]);
        load_part<DT, NF>(vbase + vo, 0, v1r[u]);
        load_part<DT, NF>(vbase + vo, HD, v2r[u]);
      }
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = sb + u - s0;              // the slot's dense rank in the block's table (< DEC_TB)
        float part = 0.0f;
        if constexpr (DT == DT_BF16) {
          // q . rot(k) = k1 (q1 cs + q2 sn) + k2 (q2 cs - q1 sn): the query's coefficients at the
          // slot's rank, rounded to bf16 as the rotated operands of Kernel C's dot are to TF32
          // (perquery.py:294), and one dot2 per pair of raw bf16 K elements, fp32 accumulation
#pragma unroll
          for (int w = 0; w < NF / 2; ++w) {
            const int e = 2 * w;
            const float c0 = tcs[r][f0 + e], c1 = tcs[r][f0 + e + 1];
            const float n0 = tsn[r][f0 + e], n1 = tsn[r][f0 + e + 1];
            const float a0 = fmaf(q1[e], c0, q2[e] * n0), a1 = fmaf(q1[e + 1], c1, q2[e + 1] * n1);
            const float b0 = fmaf(q2[e], c0, -(q1[e] * n0)), b1 = fmaf(q2[e + 1], c1, -(q1[e + 1] * n1));
            part = dot2_dt<DT>(k1r[u].w[w], pack2_dt<DT>(a0, a1), part);
            part = dot2_dt<DT>(k2r[u].w[w], pack2_dt<DT>(b0, b1), part);
          }
        } else {
#pragma unroll
          for (int e = 0; e < NF; ++e) {
            const float cs = tcs[r][f0 + e], sn = tsn[r][f0 + e];
            const float x1 = part_elem(k1r[u], e), x2 = part_elem(k2r[u], e);
            const float k1 = fmaf(x1, cs, -(x2 * sn));
            const float k2 = fmaf(x2, cs, x1 * sn);
            part = fmaf(q2[e], k2, fmaf(q1[e], k1, part));
          }
        }
        part = group8_sum(part);                // the slot's 8 lanes
        sc[u] = okv[u] ? part * a.sm_scale : -INFINITY;
      }
      // the step's max over both halves' slots, then each half folds its own slots in
      float mst = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) mst = fmaxf(mst, sc[u]);
      mst = halves16_max(mst);
      if (mst > -INFINITY) {
        const float mn = fmaxf(mrun, mst);
        if (mn > mrun) {                       // the max moved: rescale (wo = 1 otherwise)
          const float wo = mrun == -INFINITY ? 0.0f : __expf(mrun - mn);
          lrun = lrun * wo;
#pragma unroll
          for (int e = 0; e < NF; ++e) {
            acc1[e] = acc1[e] * wo;
            acc2[e] = acc2[e] * wo;
          }
        }
        if constexpr (DT == DT_F32) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const float pw = okv[u] ? __expf(sc[u] - mn) : 0.0f;
            lrun += pw;
#pragma unroll
            for (int e = 0; e < NF; ++e) {
              acc1[e] = fmaf(pw, part_elem(v1r[u], e), acc1[e]);
              acc2[e] = fmaf(pw, part_elem(v2r[u], e), acc2[e]);
            }
          }
        } else {
          // P.V with the weights in the value dtype, as Kernel C's tl.dot(p.to(v.dtype), v)
          // (perquery.py:315): two slots per dot2 over a (slot u, slot u + 1) pair of values
#pragma unroll
          for (int u = 0; u < U; u += 2) {
            const float p0 = okv[u] ? __expf(sc[u] - mn) : 0.0f;
            const float p1 = okv[u + 1] ? __expf(sc[u + 1] - mn) : 0.0f;
            lrun += p0;
            lrun += p1;
            const uint32_t pp = pack2_dt<DT>(p0, p1);
#pragma unroll
            for (int w = 0; w < RowPart<DT, NF>::NW; ++w) {
              acc1[2 * w] = dot2_dt<DT>(__builtin_amdgcn_perm(v1r[u + 1].w[w], v1r[u].w[w], 0x05040100u), pp, acc1[2 * w]);
              acc1[2 * w + 1] = dot2_dt<DT>(__builtin_amdgcn_perm(v1r[u + 1].w[w], v1r[u].w[w], 0x07060302u), pp, acc1[2 * w + 1]);
              acc2[2 * w] = dot2_dt<DT>(__builtin_amdgcn_perm(v2r[u + 1].w[w], v2r[u].w[w], 0x05040100u), pp, acc2[2 * w]);
              acc2[2 * w + 1] = dot2_dt<DT>(__builtin_amdgcn_perm(v2r[u + 1].w[w], v2r[u].w[w], 0x07060302u), pp, acc2[2 * w + 1]);
            }
          }
        }
        mrun = mn;
      }
    }
  }
  // both halves' sums and accumulators; half 0 writes the first D/2 dims, half 1 the rest
  lrun += __shfl_xor(lrun, 8, 64);
  float o[NF];
#pragma unroll
  for (int e = 0; e < NF; ++e) {
    const float x1 = acc1[e] + __shfl_xor(acc1[e], 8, 64);
    const float x2 = acc2[e] + __shfl_xor(acc2[e], 8, 64);
    const float x = half ? x2 : x1;
    o[e] = lrun > 0.0f ? x / lrun : 0.0f;      // no valid slot: zeros
  }
  if (!live) return;
  const int64_t ob = (int64_t)hi * D + half * HD + f0;
#pragma unroll
  for (int e = 0; e < NF; ++e) {
    if constexpr (DT == DT_F32) ((float*)a.out)[ob + e] = o[e];
    else ((uint16_t*)a.out)[ob + e] = (uint16_t)(DT == DT_BF16 ? f32_to_bf16_bits(o[e]) : f32_to_f16_bits(o[e]));
  }
}

// merge the splits of one query: 256 threads, 256 / D per dim
template <int DT, int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a, int ns) {
  __shared__ float msplit[1024], lsplit[1024], wsplit[1024];   // ns <= 1024: k_max <= 65536
  __shared__ float red[256 / D][D];
  const int hi = blockIdx.x;
  const float* parts = a.part + (int64_t)hi * ns * (D + 2);
  for (int u = threadIdx.x; u < ns; u += 256) {
    msplit[u] = parts[u * (D + 2) + D];
    lsplit[u] = parts[u * (D + 2) + D + 1];
  }
  __syncthreads();
  float Mx = -INFINITY;
  for (int u = 0; u < ns; ++u) Mx = fmaxf(Mx, msplit[u]);
  for (int u = threadIdx.x; u < ns; u += 256)
    wsplit[u] = (Mx > -INFINITY && msplit[u] > -INFINITY) ? __expf(msplit[u] - Mx) : 0.0f;
  __syncthreads();
  float L = 0.0f;
  for (int u = 0; u < ns; ++u) L += lsplit[u] * wsplit[u];
  constexpr int NH = 256 / D;
  const int dd = threadIdx.x % D, hf = threadIdx.x / D;
  float A = 0.0f;
#pragma unroll 8
  for (int u = hf; u < ns; u += NH) A += parts[u * (D + 2) + dd] * wsplit[u];
  red[hf][dd] = A;
  __syncthreads();
  if (hf == 0) {
    float At = 0.0f;
#pragma unroll
    for (int u = 0; u < NH; ++u) At += red[u][dd];
    const float o = L > 0.0f ? At / L : 0.0f;      // no valid slot: zeros
    const int64_t oi = (int64_t)hi * D + dd;
    if constexpr (DT == DT_F32) ((float*)a.out)[oi] = o;
    else ((uint16_t*)a.out)[oi] = (uint16_t)(DT == DT_BF16 ? f32_to_bf16_bits(o) : f32_to_f16_bits(o));
  }
}


// ------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------
template <int DT, int D>
static hipError_t launch_scores_t(const DecodeArgs& a0, float* qrot, hipStream_t st) {
  DecodeArgs a = a0;
  dim3 grid((a.M + 63) / 64, (a.Hkv + dec_hg<DT>() - 1) / dec_hg<DT>());
  if (decode_qrot_in_lds(DT, a.H, a.Hkv, a.Q, D)) {
    hipLaunchKernelGGL((decode_score_kernel<DT, D, true>), grid, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((decode_qrot_kernel<DT, D>), dim3(a.H * a.Q), dim3(D / 2), 0, st, a, qrot);
    a.qrot = qrot;
    hipLaunchKernelGGL((decode_score_kernel<DT, D, false>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_decode_scores(int dtype, int D, const DecodeArgs& a, float* qrot, hipStream_t st) {
#define STA_DS(DT_, D_) if (dtype == DT_ && D == D_) return launch_scores_t<DT_, D_>(a, qrot, st);
  STA_DS(DT_F32, 64) STA_DS(DT_F32, 128) STA_DS(DT_BF16, 64) STA_DS(DT_BF16, 128)
  STA_DS(DT_F16, 64) STA_DS(DT_F16, 128)
#undef STA_DS
  return hipErrorInvalidValue;
}

template <int NT>
static hipError_t launch_select_t(const DecodeArgs& a, hipStream_t st) {
  const int per = (a.M + NT - 1) / NT;
  const int nbend = decode_bend_words(a);
  const bool in_lds = decode_select_in_lds(a.M, nbend);   // (the 1024-thread bound covers 512 threads)
  const size_t lds = (in_lds ? (size_t)NT * (per | 1) * 4 : 0) + (size_t)dec_hist_words(!in_lds) * 4 + NT * 4 + 256 +
                     (size_t)nbend * 4;
  if (in_lds) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_select_kernel<false, NT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_select_kernel<false, NT>), dim3(a.H * a.Q), dim3(NT), lds, st, a);
  } else {
    if (!a.keys) return hipErrorInvalidValue;   // decode_keys_bytes (1024 threads) bounds NT * per
    hipError_t e = hipFuncSetAttribute((const void*)decode_select_kernel<true, NT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_select_kernel<true, NT>), dim3(a.H * a.Q), dim3(NT), lds, st, a);
  }
  return hipGetLastError();
}

template <int NT>
static hipError_t launch_select_pq_t(const DecodeArgs& a, hipStream_t st) {
  const size_t lds = decode_select_pq_lds_bytes(a.M, NT);
  hipError_t e = hipFuncSetAttribute((const void*)decode_select_pq_kernel<NT>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_select_pq_kernel<NT>), dim3(a.H * a.Q), dim3(NT), lds, st, a);
  return hipGetLastError();
}

template <int NT, int G, bool SH>
static hipError_t launch_select_pq_reg_t(const DecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((decode_select_pq_reg_kernel<NT, G, SH>), dim3(a.H * a.Q), dim3(NT), 0, st, a);
  return hipGetLastError();
}

// the register-resident selection: the smallest instance whose NT x 4G keys hold the row, or
// nullptr past 16384 keys in a batch and 32768 keys otherwise (those rows take the LDS store)
template <bool SH>
static hipError_t (*select_reg_for(int M, bool batch))(const DecodeArgs&, hipStream_t) {
  const int g = (M + (batch ? 2047 : 4095)) / (batch ? 2048 : 4096);   // 4-key groups per thread
  if (batch) {
    if (g <= 1) return launch_select_pq_reg_t<512, 1, SH>;
    if (g <= 2) return launch_select_pq_reg_t<512, 2, SH>;
    if (g <= 3) return launch_select_pq_reg_t<512, 3, SH>;
    if (g <= 4) return launch_select_pq_reg_t<512, 4, SH>;
    if (g <= 6) return launch_select_pq_reg_t<512, 6, SH>;
    if (g <= 8) return launch_select_pq_reg_t<512, 8, SH>;
    return nullptr;
  }
  if (g <= 1) return launch_select_pq_reg_t<1024, 1, SH>;
  if (g <= 2) return launch_select_pq_reg_t<1024, 2, SH>;
  if (g <= 3) return launch_select_pq_reg_t<1024, 3, SH>;
  if (g <= 4) return launch_select_pq_reg_t<1024, 4, SH>;
  if (g <= 6) return launch_select_pq_reg_t<1024, 6, SH>;
  if (g <= 8) return launch_select_pq_reg_t<1024, 8, SH>;
  return nullptr;
}

hipError_t launch_decode_select(const DecodeArgs& a, hipStream_t st) {
  // a batch that fills the chip twice over takes the 512-thread instance: more queries per CU
  // and half the waves in each block reduction (per-query prefill: 39.6 -> 31.4 ms at config 3);
  // a few queries keep 1024 threads, whose shorter per-thread ranges finish each query sooner
  const bool batch = (int64_t)a.H * a.Q >= 512;
  // the per-query rule takes its own kernels (fewer passes): the row in registers up to 16384
  // keys in a batch and 32768 otherwise (k_max within the LDS staging), in LDS beyond while it
  // fits; the shared rule without a top-pct cut takes the register kernel too (c1d's selection
  // 29.1 -> 15.1 us)
  if (a.rule == 1 && !a.use_pct) {
    if (a.k_max <= DEC_PQR_STAGE)
      if (auto f = select_reg_for<false>(a.M, batch)) return f(a, st);
    if (decode_select_pq_lds_bytes(a.M, batch ? 512 : 1024) <= 160 * 1024)
      return batch ? launch_select_pq_t<512>(a, st) : launch_select_pq_t<1024>(a, st);
  }
  if (a.rule == 0 && !a.use_pct && a.k_max <= DEC_PQR_STAGE)
    if (auto f = select_reg_for<true>(a.M, batch)) return f(a, st);
  if (batch) return launch_select_t<512>(a, st);
  return launch_select_t<1024>(a, st);
}

template <int DT, int D>
static hipError_t launch_attend_t(const DecodeArgs& a, hipStream_t st) {
  // per-query rule, a batch: grouped queries (their rows by 32-bit offsets within a head)
  const int64_t esz = DT == DT_F32 ? 4 : 2;
  const bool span32 = (int64_t)a.M * std::max(a.k_ts, a.v_ts) * esz + (int64_t)D * esz < (1LL << 31);
  if (a.dense_ranks && a.Q >= DEC_QPW && span32) {
    const int nqg = (a.Q + DEC_QPW - 1) / DEC_QPW;
    if (a.k_max % 4 == 0 && (uintptr_t)a.idx % 16 == 0)
      hipLaunchKernelGGL((decode_attend_grouped_kernel<DT, D, true>), dim3(a.H * nqg), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((decode_attend_grouped_kernel<DT, D, false>), dim3(a.H * nqg), dim3(256), 0, st, a);
    return hipGetLastError();
  }
  const int nmax = decode_nsplit(a.k_max);
  if (nmax > 1024) return hipErrorInvalidValue;   // the merge kernel's split capacity: k_max <= 65536
  const int ns = decode_attend_splits(a.Q, a.k_max);
  const int steps = (nmax + ns - 1) / ns;
  const int ng = (nmax + steps - 1) / steps;     // splits that hold slots
  hipLaunchKernelGGL((decode_attend_kernel<DT, D>), dim3(ng, a.H * a.Q), dim3(256), 0, st, a, steps);
  if (ng > 1) hipLaunchKernelGGL((decode_combine_kernel<DT, D>), dim3(a.H * a.Q), dim3(256), 0, st, a, ng);
  return hipGetLastError();
}

hipError_t launch_decode_attend(int dtype, int D, const DecodeArgs& a, hipStream_t st) {
#define STA_DA(DT_, D_) if (dtype == DT_ && D == D_) return launch_attend_t<DT_, D_>(a, st);
  STA_DA(DT_F32, 64) STA_DA(DT_F32, 128) STA_DA(DT_BF16, 64) STA_DA(DT_BF16, 128)
  STA_DA(DT_F16, 64) STA_DA(DT_F16, 128)
#undef STA_DA
  return hipErrorInvalidValue;
}

}  // namespace sta
