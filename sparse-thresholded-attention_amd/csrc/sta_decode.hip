// sta_decode.hip -- the decode path: each query selects its own key set over the KV cache and
// attends it.  A batch of Q queries shares one cache of M keys; query i sits at position
// q_pos0 + i and sees the keys [0, m_i), m_i = M - (Q - 1 - i) -- the cache prefix that the
// reference's per-token loop hands to every call (shared_selection_triton_exact_2.py:743-745).
//
//   decode_qrot_kernel    the query rotated at fl(float(q_pos) * pos_scale)        (exact_2.py:250-257)
//   decode_score_kernel   per-key scores under the selection geometry            (exact_2.py:235-271)
//                         64 keys x up to 8 kv heads per workgroup: the key rotation's
//                         sin / cos is computed once per (key, frequency) and shared by the heads
//   decode_select_kernel  _decode_build_sets (exact_2.py:527-604) for one query per workgroup:
//                         the scores staged in LDS as order-preserving keys, exact max, the
//                         top-pct cut and the k_max cap cut as radix selections (8-bit digits),
//                         compaction and the fp32 reposition recurrence
//   decode_attend_kernel  the attend over the selected slots (exact_2.py:608-655) split over
//                         workgroups of 64 slots, 16 lanes per slot, each split an online
//                         softmax state; decode_combine_kernel merges the splits
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
  const float pb = (float)(a.q_pos0 + i) * a.pos_scale;
  const float ang = pb * a.inv_freq[d];
  float sn, cs;
  sincosf(ang, &sn, &cs);
  cs = cs * a.rope_scale;
  sn = sn * a.rope_scale;
  float* o = qrot + (int64_t)hi * D;
  const float p1 = x1 * cs, p2 = x2 * sn, p3 = x2 * cs, p4 = x1 * sn;
  o[d] = p1 - p2;                             // exact_2.py:256-257
  o[D / 2 + d] = p3 + p4;
}

// ------------------------------------------------------------------------------------------
// per-key scores (H, Q, M): 64 keys x HG kv heads per workgroup, 4 lanes per key
// ------------------------------------------------------------------------------------------
constexpr int DEC_HG = 8;   // kv heads per score workgroup

template <int DT, int D>
__global__ __launch_bounds__(256) void decode_score_kernel(DecodeArgs a, const float* qrot) {
#pragma clang fp contract(off)
  constexpr int NP = D / 8;                  // rotation pairs per lane
  const int t = threadIdx.x & 3;
  const int j = blockIdx.x * 64 + (threadIdx.x >> 2);
  const bool valid = j < a.M;
  const int jc = valid ? j : a.M - 1;
  const int hk0 = blockIdx.y * DEC_HG;
  const int G = a.H / a.Hkv;
  // cos / sin of this key's frequencies t*NP .. t*NP + NP - 1, shared by the heads
  float cs[NP], sn[NP];
  {
    const float kb = (float)j * a.pos_scale;                            // exact_2.py:264
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float ang = kb * a.inv_freq[t * NP + p];
      sincosf(ang, &sn[p], &cs[p]);
      cs[p] = cs[p] * a.rope_scale;
      sn[p] = sn[p] * a.rope_scale;
    }
  }
  for (int g = 0; g < DEC_HG; ++g) {
    const int hk = hk0 + g;
    if (hk >= a.Hkv) break;
    float x1[NP], x2[NP], k1[NP], k2[NP];
    const int64_t kb = (int64_t)hk * a.k_hs + (int64_t)jc * a.k_ts + t * NP;
    load_n<DT, NP>(a.k, kb, x1);
    load_n<DT, NP>(a.k, kb + D / 2, x2);
#pragma unroll
    for (int p = 0; p < NP; ++p) {                                        // exact_2.py:266-267
      const float u = x1[p] * cs[p], w = x2[p] * sn[p], y = x2[p] * cs[p], z = x1[p] * sn[p];
      k1[p] = u - w;
      k2[p] = y + z;
    }
    for (int hq = hk * G; hq < hk * G + G; ++hq) {
      for (int i = 0; i < a.Q; ++i) {
        const float* qr = qrot + ((int64_t)hq * a.Q + i) * D;
        float q1[NP], q2[NP];
#pragma unroll
        for (int p = 0; p < NP; p += 4) {
          const float4 u = *(const float4*)(qr + t * NP + p);
          const float4 w = *(const float4*)(qr + D / 2 + t * NP + p);
          q1[p] = u.x; q1[p + 1] = u.y; q1[p + 2] = u.z; q1[p + 3] = u.w;
          q2[p] = w.x; q2[p + 1] = w.y; q2[p + 2] = w.z; q2[p + 3] = w.w;
        }
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < NP; ++p) acc = fmaf(q2[p], k2[p], fmaf(q1[p], k1[p], acc));
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        const int m = a.M - (a.Q - 1 - i);
        if (t == 0 && j < m) a.scores[((int64_t)hq * a.Q + i) * a.M + j] = acc * a.sm_scale;   // :270
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// _decode_build_sets for one query per workgroup
// ------------------------------------------------------------------------------------------
constexpr int DEC_SEL_NT = 1024;             // threads of a selection workgroup
constexpr int DEC_SEL_NW = DEC_SEL_NT / 64;

namespace {

__device__ __forceinline__ int dsum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < DEC_SEL_NW; ++w) total += tmp[w];
  __syncthreads();
  return total;
}

__device__ __forceinline__ uint32_t dmax_u(uint32_t v, uint32_t* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int w = 0; w < DEC_SEL_NW; ++w) r = max(r, tmp[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ int dexcl_sum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += tmp[w];
  __syncthreads();
  return base + x - v;
}

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
bool decode_select_in_lds(int M) {   // up to 144 KB of the CU's 160 KB (M <= 35840)
  const int per = (M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  return (size_t)DEC_SEL_NT * (per | 1) * 4 + 2048 <= 144 * 1024;
}
size_t decode_select_lds_bytes(int M) {
  const int per = (M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  return (decode_select_in_lds(M) ? (size_t)DEC_SEL_NT * (per | 1) * 4 : 0) + 2048;
}
size_t decode_keys_bytes(int H, int Q, int M) {
  if (decode_select_in_lds(M)) return 0;
  const int per = (M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  return (size_t)H * Q * DEC_SEL_NT * per * 4;
}

template <bool GKEYS>
__global__ __launch_bounds__(DEC_SEL_NT) void decode_select_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t dsm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = blockIdx.x;
  const int h = hi / a.Q, i = hi % a.Q;
  const int m = a.M - (a.Q - 1 - i);           // keys this query sees
  const int p = a.q_pos0 + i;                  // its position (p < m)
  const int per_max = (a.M + DEC_SEL_NT - 1) / DEC_SEL_NT;
  const int per = (m + DEC_SEL_NT - 1) / DEC_SEL_NT;
  const int PS = GKEYS ? per : (per | 1);
  uint32_t* ks = GKEYS ? a.keys + (int64_t)hi * DEC_SEL_NT * per_max : dsm;
  int* hist = (int*)(dsm + (GKEYS ? 0 : DEC_SEL_NT * (per_max | 1)));   // 256
  int* tmp = hist + 256;                       // DEC_SEL_NW
  int* misc = tmp + DEC_SEL_NW;                // 8
  const int j0 = tid * per, j1 = min(j0 + per, m);
  uint32_t* myrow = ks + tid * PS;
  const float* srow = a.scores + (int64_t)hi * a.M;

  // ---- stage the scores as keys (coalesced reads), exact max (exact_2.py:549) ----
  uint32_t kmax = 0;
  for (int j = tid; j < DEC_SEL_NT * per; j += DEC_SEL_NT) {
    uint32_t key = 0;
    if (j < m) {
      key = okey(srow[j]);
      kmax = max(kmax, key);
    }
    const int row = j / per;
    ks[row * PS + (j - row * per)] = key;
  }
  kmax = dmax_u(kmax, (uint32_t*)tmp);         // the barrier inside also publishes the stores
  const float thr = okey_value(kmax) - a.tau[h];                       // exact_2.py:550
  const uint32_t kthr = okey(thr);

  // forced keys: [0, g) U [lo, p] (global, local window, self; exact_2.py:552-555)
  const int g = min(a.n_global, m);
  const int lo = min(max(0, p - a.n_local + 1), p);
  const int nB = p - max(lo, g) + 1;            // local keys not already global
  const int nforced = g + max(nB, 0);
  auto forced_j = [&](int f) { return f < g ? f : max(lo, g) + (f - g); };   // f < nforced

  // need-th largest key (1 <= need <= #nonzero keys) -> (V, #keys >= V), 8-bit digits
  auto kth = [&](int need) -> uint2 {
    uint32_t prefix = 0, pmask = 0;
    int ge = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += DEC_SEL_NT) hist[b] = 0;
      __syncthreads();
      if (shift == 24) {
        // the top digit (sign and high exponent bits) takes few values: one LDS atomic per
        // distinct digit of a wave
        for (int e = 0; e < per; ++e) {
          const uint32_t k = myrow[e];
          bool act = k != 0 && j0 + e < m;
          const int d = (int)(k >> 24);
          uint64_t msk = __ballot(act);
          while (msk) {
            const int leader = __ffsll((unsigned long long)msk) - 1;
            const int dl = __shfl(d, leader, 64);
            const uint64_t same = __ballot(act && d == dl);
            if (lane == leader) atomicAdd(&hist[dl], (int)__popcll(same));
            if (act && d == dl) act = false;
            msk &= ~same;
          }
        }
      } else {
        for (int e = 0; e < per; ++e) {
          const uint32_t k = myrow[e];
          if (k != 0 && j0 + e < m && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1);
        }
      }
      __syncthreads();
      if (wave == 0) {
        // lane l holds bins 255-4l .. 252-4l (descending)
        int c[4], sl = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[e] = hist[255 - 4 * lane - e]; sl += c[e]; }
        int incl = sl;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o, 64);
          if (lane >= o) incl += y;
        }
        const uint64_t hit = __ballot(incl >= need);
        const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
        if (lane == first) {
          int acc = incl - sl, d = 255 - 4 * lane, e = 0;
          for (; e < 3; ++e) {
            if (acc + c[e] >= need) break;
            acc += c[e];
            d -= 1;
          }
          misc[0] = d;
          misc[1] = need - acc;
          misc[2] = acc;
          misc[3] = c[e];
        }
      }
      __syncthreads();
      prefix |= (uint32_t)misc[0] << shift;
      ge += misc[2];
      need = misc[1];
      if (shift == 0) ge += misc[3];
      pmask |= 255u << shift;
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
    const int n_pass = dsum(c, tmp);
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
      ge = dsum(c2, tmp);
    }
  } else {
    int c = 0;
    for (int e = 0; e < j1 - j0; ++e) c += myrow[e] >= kp_thr;
    ge = dsum(c, tmp);
  }
  {
    int c = 0;
    for (int f = tid; f < nforced; f += DEC_SEL_NT) c += key_of(forced_j(f)) < kp_thr;
    count = ge + dsum(c, tmp);
  }

  // ---- cap by score over the non-forced keys (exact_2.py:571-585) ----
  uint32_t fin_thr = kp_thr;
  bool only_forced = false;
  if (count > a.k_max) {
    const int budget_c = a.k_max - nforced;
    if (budget_c <= 0) {
      only_forced = true;
    } else {
      // the non-forced kept keys are the non-forced keys >= kp_thr and they outnumber budget_c,
      // so the budget_c-th largest non-forced key is the reference's cut
      for (int f = tid; f < nforced; f += DEC_SEL_NT) {
        const int j = forced_j(f);
        const int row = j / per;
        ks[row * PS + (j - row * per)] = 0u;
      }
      __syncthreads();
      fin_thr = kth(budget_c).x;
    }
  }
  auto final_j = [&](int j, uint32_t k) {
    return j < g || (j >= lo && j <= p) || (!only_forced && k >= fin_thr);
  };

  // ---- compaction + reposition (exact_2.py:587-603) ----
  int cnt = 0;
  for (int e = 0; e < j1 - j0; ++e) cnt += final_j(j0 + e, myrow[e]);
  const int base = dexcl_sum(cnt, tmp);
  const int total = dsum(cnt, tmp);
  float mloc = -INFINITY;
  {
    int rank = base - 1;
    for (int e = 0; e < j1 - j0; ++e) {
      if (final_j(j0 + e, myrow[e])) {
        rank += 1;
        const float cp = (float)(j0 + e) * a.pos_scale;                  // exact_2.py:590
        mloc = fmaxf(mloc, cp - (float)rank);                            // :591
      }
    }
  }
  float run = dexcl_max(mloc, (float*)tmp);
  int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  {
    int rank = base - 1;
    for (int e = 0; e < j1 - j0; ++e) {
      const int j = j0 + e;
      const bool f = final_j(j, myrow[e]);
      if (f) {
        rank += 1;
        const float cp = (float)j * a.pos_scale;
        run = fmaxf(run, cp - (float)rank);
      }
      const float np = (float)rank + run;                                // exact_2.py:592
      if (f && rank < a.k_max) {
        irow[rank] = j;
        nrow[rank] = np;
      }
      if (j == p) a.newpos_q[hi] = np;                                   // :603
    }
  }
  for (int s = min(total, a.k_max) + tid; s < a.k_max; s += DEC_SEL_NT) {   // sentinel m (:594-600)
    irow[s] = m;
    nrow[s] = 0.0f;
  }
  if (tid == 0 && a.set_size) a.set_size[hi] = total;
}

// ------------------------------------------------------------------------------------------
// attend: split s of query (h, i) sweeps slots [64 s, 64 s + 64); 16 lanes per slot, each lane
// NPL rotation pairs; every 16-lane group keeps its own online-softmax state, merged in LDS
// ------------------------------------------------------------------------------------------
constexpr int DEC_SPL = 64;                    // slots per attend workgroup

int decode_nsplit(int k_max) { return (k_max + DEC_SPL - 1) / DEC_SPL; }

template <int DT, int D>
__global__ __launch_bounds__(256) void decode_attend_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
  constexpr int NPL = D / 32;                  // pairs per lane
  __shared__ float sm_m[16], sm_l[16];
  __shared__ float sm_acc[16][D];
  const int split = blockIdx.x, hi = blockIdx.y;
  const int h = hi / a.Q, i = hi % a.Q;
  const int hk = h / (a.H / a.Hkv);
  const int m = a.M - (a.Q - 1 - i);
  const int p = a.q_pos0 + i;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, grp = wave * 4 + (lane >> 4);
  const int d0 = l16 * NPL;                    // this lane's frequencies d0 .. d0 + NPL - 1
  const int nslots = a.set_size ? min(a.set_size[hi], a.k_max) : a.k_max;
  const int s0 = split * DEC_SPL, s1 = min(s0 + DEC_SPL, nslots);
  float invf[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) invf[e] = a.inv_freq[d0 + e];
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
      cs = cs * a.rope_scale;
      sn = sn * a.rope_scale;
      q1[e] = x1[e] * cs - x2[e] * sn;
      q2[e] = x2[e] * cs + x1[e] * sn;
    }
  }
  float mrun = -INFINITY, lrun = 0.0f, acc1[NPL], acc2[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) { acc1[e] = 0.0f; acc2[e] = 0.0f; }
  const int32_t* irow = a.idx + (int64_t)hi * a.k_max;
  const float* nrow = a.newpos_k + (int64_t)hi * a.k_max;
  for (int sb = s0; sb < s1; sb += 16) {
    const int s = sb + grp;
    const int j = s < s1 ? irow[s] : -1;
    const bool ok = j >= 0 && j < m && (!a.causal || j <= p);   // sentinel m (exact_2.py:615; :195, 210)
    const int jc = ok ? j : 0;
    float x1[NPL], x2[NPL], v1[NPL], v2[NPL];
    const int64_t kb = (int64_t)hk * a.k_hs + (int64_t)jc * a.k_ts + d0;
    const int64_t vb = (int64_t)hk * a.v_hs + (int64_t)jc * a.v_ts + d0;
    load_n<DT, NPL>(a.k, kb, x1);
    load_n<DT, NPL>(a.k, kb + D / 2, x2);
    load_n<DT, NPL>(a.v, vb, v1);
    load_n<DT, NPL>(a.v, vb + D / 2, v2);
    const float npk = ok ? nrow[s] : 0.0f;
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
      float sn, cs;
      fast_sincos(npk * invf[e], sn, cs);
      cs = cs * a.rope_scale;
      sn = sn * a.rope_scale;
      const float k1 = x1[e] * cs - x2[e] * sn;
      const float k2 = x2[e] * cs + x1[e] * sn;
      part = fmaf(q2[e], k2, fmaf(q1[e], k1, part));
    }
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    part += __shfl_xor(part, 4, 64);
    part += __shfl_xor(part, 8, 64);
    if (ok) {
      const float sc = part * a.sm_scale;
      const float mnew = fmaxf(mrun, sc);
      const float alpha = __expf(mrun - mnew);        // 0 on the group's first slot
      const float pw = __expf(sc - mnew);
      lrun = lrun * alpha + pw;
#pragma unroll
      for (int e = 0; e < NPL; ++e) {
        acc1[e] = acc1[e] * alpha + pw * v1[e];
        acc2[e] = acc2[e] * alpha + pw * v2[e];
      }
      mrun = mnew;
    }
  }
  if (l16 == 0) { sm_m[grp] = mrun; sm_l[grp] = lrun; }
#pragma unroll
  for (int e = 0; e < NPL; ++e) { sm_acc[grp][d0 + e] = acc1[e]; sm_acc[grp][D / 2 + d0 + e] = acc2[e]; }
  __syncthreads();
  // merge the 16 group states: (max, sum, D accumulators) of the split
  float* part = a.part + ((int64_t)hi * gridDim.x + split) * (D + 2);
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < 16; ++u) M = fmaxf(M, sm_m[u]);
  for (int d = threadIdx.x; d < D; d += 256) {
    float A = 0.0f;
    if (M > -INFINITY)
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (sm_m[u] > -INFINITY) A += sm_acc[u][d] * __expf(sm_m[u] - M);
    part[d] = A;
  }
  if (threadIdx.x == 0) {
    float L = 0.0f;
    if (M > -INFINITY)
      for (int u = 0; u < 16; ++u)
        if (sm_m[u] > -INFINITY) L += sm_l[u] * __expf(sm_m[u] - M);
    part[D] = M;
    part[D + 1] = L;
  }
}

template <int DT, int D>
__global__ __launch_bounds__(D) void decode_combine_kernel(DecodeArgs a, int nsplit) {
  const int hi = blockIdx.x, d = threadIdx.x;
  const float* part = a.part + (int64_t)hi * nsplit * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part[s * (D + 2) + D]);
  float A = 0.0f, L = 0.0f;
  if (M > -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ms = part[s * (D + 2) + D];
      if (ms == -INFINITY) continue;
      const float w = __expf(ms - M);
      A += part[s * (D + 2) + d] * w;
      L += part[s * (D + 2) + D + 1] * w;
    }
  }
  const float o = L > 0.0f ? A / L : 0.0f;      // no valid slot: zeros
  const int64_t oi = (int64_t)hi * D + d;
  if constexpr (DT == DT_F32) ((float*)a.out)[oi] = o;
  else ((uint16_t*)a.out)[oi] = (uint16_t)(DT == DT_BF16 ? f32_to_bf16_bits(o) : f32_to_f16_bits(o));
}

// ------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------
template <int DT, int D>
static hipError_t launch_scores_t(const DecodeArgs& a, float* qrot, hipStream_t st) {
  hipLaunchKernelGGL((decode_qrot_kernel<DT, D>), dim3(a.H * a.Q), dim3(D / 2), 0, st, a, qrot);
  dim3 grid((a.M + 63) / 64, (a.Hkv + DEC_HG - 1) / DEC_HG);
  hipLaunchKernelGGL((decode_score_kernel<DT, D>), grid, dim3(256), 0, st, a, (const float*)qrot);
  return hipGetLastError();
}

hipError_t launch_decode_scores(int dtype, int D, const DecodeArgs& a, float* qrot, hipStream_t st) {
#define STA_DS(DT_, D_) if (dtype == DT_ && D == D_) return launch_scores_t<DT_, D_>(a, qrot, st);
  STA_DS(DT_F32, 64) STA_DS(DT_F32, 128) STA_DS(DT_BF16, 64) STA_DS(DT_BF16, 128)
  STA_DS(DT_F16, 64) STA_DS(DT_F16, 128)
#undef STA_DS
  return hipErrorInvalidValue;
}

hipError_t launch_decode_select(const DecodeArgs& a, hipStream_t st) {
  const size_t lds = decode_select_lds_bytes(a.M);
  if (decode_select_in_lds(a.M)) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_select_kernel<false>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(decode_select_kernel<false>, dim3(a.H * a.Q), dim3(DEC_SEL_NT), lds, st, a);
  } else {
    if (!a.keys) return hipErrorInvalidValue;
    hipLaunchKernelGGL(decode_select_kernel<true>, dim3(a.H * a.Q), dim3(DEC_SEL_NT), lds, st, a);
  }
  return hipGetLastError();
}

template <int DT, int D>
static hipError_t launch_attend_t(const DecodeArgs& a, hipStream_t st) {
  const int ns = decode_nsplit(a.k_max);
  hipLaunchKernelGGL((decode_attend_kernel<DT, D>), dim3(ns, a.H * a.Q), dim3(256), 0, st, a);
  hipLaunchKernelGGL((decode_combine_kernel<DT, D>), dim3(a.H * a.Q), dim3(D), 0, st, a, ns);
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
