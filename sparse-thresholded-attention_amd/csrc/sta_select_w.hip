// sta_select_w.hip -- per-(head, tile) key-set selection ranked by weighted votes, the device
// form of _build_sets with select_score "margin" / "expmass".
//
// Reference: shared_selection_triton_exact_2.py:277-426 with wvotes.  The ranking metric is the
// weighted vote with frequency as an epsilon tiebreak, rank = fl(wvotes + fl(1e-6 votes))
// (:299-302); the union size U = #(votes > 0) and the budgets ceil(fl(p/100 * U)) stay
// frequency-based (:296, :329).  The order statistic the reference reads from topk (:321, :330)
// is the budget-th largest rank value; here it is a radix select over the tile's rank values
// staged in LDS (order-preserving 32-bit keys, 8-bit digits) that finds the cuts of all fallback
// steps in one traversal, and the set sizes follow from its last histograms: #(rank >= cut) is
// the keys above the cut plus those equal to it.  The forced
// keys with a rank below the cut are counted directly.  The 30 -> 25 -> 20 fallback, the pct = 0
// case, the measure loop, compaction and the fp32 reposition recurrence are those of the
// frequency-ranked select kernel.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

namespace {

// one workgroup per (head, tile): W_NT threads in W_NW waves
constexpr int W_NT = 512;
constexpr int W_NW = W_NT / 64;

__device__ __forceinline__ int w_block_sum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < W_NW; ++w) total += tmp[w];
  __syncthreads();
  return total;
}

__device__ __forceinline__ int w_block_exclusive_sum(int v, int* tmp) {
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

__device__ __forceinline__ float w_block_exclusive_max(float v, float* tmp) {
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

// budget = ceil(fl(float32(p/100.0) * float32(U))).clamp(min=1)   (exact_2.py:329)
__device__ __forceinline__ int64_t w_budget_of(int p, int64_t usize) {
#pragma clang fp contract(off)
  const float frac = (float)((double)p / 100.0);
  const float prod = frac * (float)usize;
  float b = ceilf(prod);
  if (b < 1.0f) b = 1.0f;
  return (int64_t)b;
}

// fp32 -> unsigned key with the same order (-0 folded into +0 first); key 0 marks "no key"
__device__ __forceinline__ uint32_t order_key(float r) {
  const uint32_t b = __float_as_uint(r + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// KB keys of this thread's row from index i0 on (0 past `per`), read together so that one wait
// covers them all
constexpr int W_KB = 8;
__device__ __forceinline__ void w_load_keys(const uint32_t* row, int i0, int per, uint32_t (&k)[W_KB]) {
#pragma unroll
  for (int e = 0; e < W_KB; ++e) k[e] = i0 + e < per ? row[i0 + e] : 0u;
}

}  // namespace

// LDS: per thread a contiguous key range of `per` keys at an odd row stride (conflict-free
// scans), unless the keys are read from the vote rows at every pass (global_keys)
size_t select_w_lds_bytes(int N, int k_max, bool global_keys) {
  const size_t per = (size_t)(N + W_NT - 1) / W_NT;
  const size_t keys = global_keys ? 0 : W_NT * (per | 1) * 4;
  return keys + (3 * 256 + 16 + 16 + 16) * 4 + 256 * 4 + (size_t)k_max * 8;
}

// GK = false: the tile's rank keys are staged in LDS once.  GK = true (rows too long for LDS):
// every pass recomputes each key from the vote and weighted-vote rows in the workspace (L2
// resident for the workgroups in flight), with the same fp32 operations as the staging.
template <typename VT, bool GK>
__global__ __launch_bounds__(W_NT) void select_w_kernel(SelectArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t wsm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int N = a.N, T = a.T;
  // the longest key ranges (the last tiles) start first
  const int h = (int)(blockIdx.x % a.H);
  const int t = a.nt - 1 - (int)(blockIdx.x / a.H);
  const int64_t tstart = (int64_t)a.q_pos_base + (int64_t)t * T;          // exact_2.py:291
  const int64_t lo = tstart - a.n_local + 1, hi_l = tstart + T - 1;
  const int hi_keys = a.votes_dense ? N : (int)min((int64_t)N, tstart + T);
  // Keys at or past R carry no votes and are not forced: rank value 0, order key ZK.  They are not
  // staged: they lie below every cut as long as at least `need` staged keys rank above zero, which
  // the staging counts; a tile where that fails stages all N keys instead.
  constexpr uint32_t ZK = 0x80000000u;                   // order_key(0.0f)
  int R = a.votes_dense ? N : (int)min((int64_t)N, max(tstart + T, (int64_t)a.n_global));
  const int PSMAX = GK ? 0 : ((N + W_NT - 1) / W_NT) | 1;
  uint32_t* rkb = wsm;                                   // W_NT rows x PS order keys (LDS staging)
  int* hist = (int*)(rkb + W_NT * PSMAX);                // 3 x 256
  int* tmp = hist + 3 * 256;                             // 16
  int* misc = tmp + 16;                                  // 16
  float* tmpf = (float*)(misc + 16);                     // 16
  float* qnp = tmpf + 16;                                // T (<= 256)
  int32_t* sidx = (int32_t*)(qnp + 256);                 // k_max
  float* snp = (float*)(sidx + a.k_max);                 // k_max

  const int64_t roff = ((int64_t)h * a.nt + t) * a.votes_stride;
  const VT* vrow = (const VT*)a.votes + roff;
  const float* wrow = a.wvotes + roff;
  auto is_forced = [&](int j) { return j < a.n_global || (j >= lo && j <= hi_l); };   // exact_2.py:290-293

  // ---- stage the rank keys of [0, R) (coalesced: key j by thread j % W_NT), U = #(votes > 0) and
  //      the keys ranked above zero; SU loads of each array in flight per lane ----
  int per = 0, PS = 1, cu = 0, cpos = 0;
  uint32_t inv_per = 0;
  constexpr int SU = 8;
  auto stage = [&]() {
    per = (R + W_NT - 1) / W_NT;
    PS = per | 1;
    inv_per = per > 1 ? (uint32_t)((0x100000000ull + per - 1) / per) : 0u;
    cu = 0;
    cpos = 0;
    for (int jb = 0; jb < W_NT * per; jb += W_NT * SU) {
      int vv[SU];
      float wv[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int j = jb + u * W_NT + tid;
        const bool ok = j < hi_keys;
        vv[u] = ok ? (int)vrow[j] : 0;
        wv[u] = ok ? wrow[j] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int j = jb + u * W_NT + tid;
        if (j >= W_NT * per) break;
        uint32_t key = 0;
        if (j < R) {
          const int v = vv[u];
          const float w = wv[u];
          cu += v > 0;                                                       // exact_2.py:296
          const float tb = 1e-6f * (float)v;                                 // exact_2.py:302
          key = order_key(w + tb);
          cpos += key > ZK;
        }
        if constexpr (!GK) {
          const uint32_t row = per == 1 ? (uint32_t)j : __umulhi((uint32_t)j, inv_per);
          rkb[row * PS + (j - row * per)] = key;
        }
      }
    }
    __syncthreads();
  };
  stage();
  const int64_t usize = w_block_sum(cu, tmp);   // no votes past R
  {
    // the largest order statistic any step asks for (exact_2.py:329-330): the first step's
    int64_t need = w_budget_of(a.steps[0], usize);
    need = need > a.K_ord ? a.K_ord : need;
    if (R < N && (int64_t)w_block_sum(cpos, tmp) < need) {
      R = N;
      stage();
    }
  }
  if (a.votes_out || a.wvotes_out) {
    // the reference's dense (H, nt, N) votes / wvotes, zero past the tile's causal end
    for (int j = tid; j < N; j += W_NT) {
      const bool ok = j < hi_keys;
      if (a.votes_out) a.votes_out[((int64_t)h * a.nt + t) * N + j] = ok ? (int)vrow[j] : 0;
      if (a.wvotes_out) a.wvotes_out[((int64_t)h * a.nt + t) * N + j] = ok ? wrow[j] : 0.0f;
    }
  }
  uint32_t* myrow = rkb + tid * PS;                      // keys j0 .. j0 + per - 1 (LDS staging)
  const int j0 = tid * per, j1 = min(j0 + per, R);
  // the rank key of key j from the vote rows (GK): the staging's operations, 0 past R
  auto gkey = [&](int j) -> uint32_t {
    if (j >= R) return 0u;
    const bool ok = j < hi_keys;
    const int v = ok ? (int)vrow[j] : 0;
    const float w = ok ? wrow[j] : 0.0f;
    const float tb = 1e-6f * (float)v;
    return order_key(w + tb);
  };
  // this thread's keys i0 .. i0 + W_KB - 1 of its contiguous range [j0, j0 + per)
  auto range_keys = [&](int i0, uint32_t (&kk)[W_KB]) {
    if constexpr (GK) {
#pragma unroll
      for (int e = 0; e < W_KB; ++e) kk[e] = i0 + e < per ? gkey(j0 + i0 + e) : 0u;
    } else {
      w_load_keys(myrow, i0, per, kk);
    }
  };

  // Order statistics for up to three targets at once: target t is the need[t]-th largest key
  // (1 <= need[t] <= N).  The targets walk the radix tree together, one pass over the keys per
  // 8-bit digit; targets whose prefixes coincide share a histogram (at most three distinct
  // prefixes, and a key matches at most one of them).  Results: V[t] the key, GE[t] = #(keys >= V[t]).
  auto kth_multi = [&](int ntarg, const int* need_in, uint32_t* V, int* GE) {
    uint32_t prefix[3], pmask = 0;
    int need[3], ge[3], hid[3];
#pragma unroll
    for (int u = 0; u < 3; ++u) { prefix[u] = 0; need[u] = u < ntarg ? need_in[u] : 1; ge[u] = 0; hid[u] = 0; }
    for (int shift = 24; shift >= 0; shift -= 8) {
      // distinct prefixes of this level -> histogram slots
      // (fixed-bound loops: the small arrays stay in registers)
      int nh = 0;
      uint32_t hp[3] = {0u, 0u, 0u};
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (u < ntarg) {
          int f = -1;
#pragma unroll
          for (int w = 0; w < 3; ++w) f = (f < 0 && w < nh && hp[w] == prefix[u]) ? w : f;
          if (f < 0) {
#pragma unroll
            for (int w = 0; w < 3; ++w) hp[w] = w == nh ? prefix[u] : hp[w];
            f = nh++;
          }
          hid[u] = f;
        }
      }
      for (int i = tid; i < 256 * nh; i += W_NT) hist[i] = 0;
      __syncthreads();
      // plain LDS atomics on every level, the top digit included (a per-wave aggregation of the
      // top digit's few distinct values by ballots measured slower)
      for (int i0 = 0; i0 < per; i0 += W_KB) {
        uint32_t kk[W_KB];
        if constexpr (GK) {
          // the histograms ignore key order: key (i0 + e) * W_NT + tid, coalesced
#pragma unroll
          for (int e = 0; e < W_KB; ++e) kk[e] = i0 + e < per ? gkey((i0 + e) * W_NT + tid) : 0u;
        } else {
          w_load_keys(myrow, i0, per, kk);
        }
#pragma unroll
        for (int e = 0; e < W_KB; ++e) {
          const uint32_t k = kk[e];
          if (k == 0 || (!GK && j0 + i0 + e >= R)) continue;
          const uint32_t kp = k & pmask;
#pragma unroll
          for (int w = 0; w < 3; ++w)
            if (w < nh && kp == hp[w]) atomicAdd(&hist[w * 256 + ((k >> shift) & 255u)], 1);
        }
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (u < ntarg && tid < 64) {
          // wave 0 finds target u's digit: lane l holds bins 255-4l .. 252-4l (descending)
          const int* hu = hist + hid[u] * 256;
          int c[4], sl = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) { c[e] = hu[255 - 4 * lane - e]; sl += c[e]; }
          int incl = sl;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
          }
          const uint64_t hit = __ballot(incl >= need[u]);
          const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
          if (lane == first) {
            int acc = incl - sl, d = 255 - 4 * lane, e = 0;
            for (; e < 3; ++e) {
              if (acc + c[e] >= need[u]) break;
              acc += c[e];
              d -= 1;
            }
            misc[4 * u + 0] = d;
            misc[4 * u + 1] = need[u] - acc;   // how far into digit d's keys the statistic lies
            misc[4 * u + 2] = acc;             // keys with a larger digit (above the prefix range)
            misc[4 * u + 3] = c[e];            // keys with digit d
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (u >= ntarg) continue;
        prefix[u] |= (uint32_t)misc[4 * u] << shift;
        ge[u] += misc[4 * u + 2];
        need[u] = misc[4 * u + 1];
        if (shift == 0) ge[u] += misc[4 * u + 3];   // the last digit's bin: the keys equal to V
      }
      pmask |= 255u << shift;
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 3; ++u)
      if (u < ntarg) { V[u] = prefix[u]; GE[u] = ge[u]; }
  };
  auto kth = [&](int need) {
    uint32_t V;
    int GE;
    kth_multi(1, &need, &V, &GE);
    return make_int2((int)V, GE);
  };
  // forced keys whose rank lies below a cut (exact_2.py:332: kept = shared | forced)
  const int gA = min(a.n_global, N);
  const int bl = (int)max(lo, (int64_t)gA);
  const int bh = (int)min(hi_l, (int64_t)N - 1);
  const int nB = bh >= bl ? bh - bl + 1 : 0;
  auto key_of = [&](int j) -> uint32_t {
    if constexpr (GK) {
      return gkey(j);
    } else {
      const uint32_t row = per == 1 ? (uint32_t)j : __umulhi((uint32_t)j, inv_per);
      return rkb[row * PS + (j - row * per)];
    }
  };
  auto forced_below = [&](uint32_t cut) {
    int c = 0;
    for (int i = tid; i < gA + nB; i += W_NT) {
      const int j = i < gA ? i : bl + (i - gA);
      c += key_of(j) < cut;
    }
    return w_block_sum(c, tmp);
  };
  const int nforced = gA + nB;

  // ---- the 30 -> 25 -> 20 fallback (exact_2.py:328-350): every step's cut in one traversal ----
  int resolved = 0, ch = 0, oflow = 0, forced_only = 0;
  uint32_t cut = 0;
  {
    int needs[3];
    uint32_t Vs[3];
    int GEs[3];
    for (int si = 0; si < a.nsteps; ++si) {
      int64_t need = w_budget_of(a.steps[si], usize);
      needs[si] = (int)(need > a.K_ord ? a.K_ord : need);                 // exact_2.py:330
    }
    kth_multi(a.nsteps, needs, Vs, GEs);
    for (int si = 0; si < a.nsteps; ++si) {
      const int p = a.steps[si];
      const int64_t size = (int64_t)GEs[si] + forced_below(Vs[si]);
      if (p == a.start_pct) oflow = size > a.k_max;
      if (!resolved) {
        cut = Vs[si];
        if (size <= a.k_max) { resolved = 1; ch = p; }
      }
    }
  }
  if (a.start_pct == 0) {                                                   // exact_2.py:343-346
    oflow = nforced > a.k_max;
    if (!resolved) forced_only = 1;
  }
  int kmeas = ch;
  if (a.measure && !resolved) {                                             // exact_2.py:357-371
    const int floor_pct = a.steps[a.nsteps - 1];
    for (int p = floor_pct - 1; p > 0; --p) {
      int64_t need = w_budget_of(p, usize);
      need = need > a.K_ord ? a.K_ord : need;
      const int2 r = kth((int)need);
      if ((int64_t)r.y + forced_below((uint32_t)r.x) <= a.k_max) { kmeas = p; break; }
    }
  }

  // ---- compaction + reposition (exact_2.py:383-412) ----
  auto kept_of = [&](int j, uint32_t k) { return is_forced(j) || (!forced_only && k >= cut); };
  int cnt = 0, csh = 0;
  for (int i0 = 0; i0 < per; i0 += W_KB) {
    uint32_t kk[W_KB];
    range_keys(i0, kk);
#pragma unroll
    for (int e = 0; e < W_KB; ++e) {
      const int j = j0 + i0 + e;
      if (j < j1) {
        cnt += kept_of(j, kk[e]);
        csh += !forced_only && kk[e] >= cut;
      }
    }
  }
  const int base = w_block_exclusive_sum(cnt, tmp);
  const int kept_total = w_block_sum(cnt, tmp);
  const int shared_total = w_block_sum(csh, tmp);
  float mloc = -INFINITY;
  {
    int rank = base - 1;
    for (int i0 = 0; i0 < per; i0 += W_KB) {
      uint32_t kk[W_KB];
      range_keys(i0, kk);
#pragma unroll
      for (int e = 0; e < W_KB; ++e) {
        const int j = j0 + i0 + e;
        if (j < j1 && kept_of(j, kk[e])) {
          rank += 1;
          const float cp = (float)j * a.pos_scale;        // exact_2.py:384
          mloc = fmaxf(mloc, cp - (float)rank);           // exact_2.py:385
        }
      }
    }
  }
  float run = w_block_exclusive_max(mloc, tmpf);
  const int qlo = (int)min(tstart, (int64_t)N - 1);
  const int qhi = (int)min(tstart + T - 1, (int64_t)N - 1);
  {
    int rank = base - 1;
    for (int i0 = 0; i0 < per; i0 += W_KB) {
      uint32_t kk[W_KB];
      range_keys(i0, kk);
#pragma unroll
      for (int e = 0; e < W_KB; ++e) {
        const int j = j0 + i0 + e;
        if (j < j1) {
          const bool kept = kept_of(j, kk[e]);
          if (kept) {
            rank += 1;
            const float cp = (float)j * a.pos_scale;
            run = fmaxf(run, cp - (float)rank);
          }
          const float np = (float)rank + run;              // exact_2.py:386
          if (kept && rank < a.k_max) { sidx[rank] = j; snp[rank] = np; }
          if (j >= qlo && j <= qhi) qnp[j - qlo] = np;
        }
      }
    }
  }
  __syncthreads();
  const int nvalid = min(kept_total, a.k_max);
  int32_t* irow = a.idx + ((int64_t)h * a.nt + t) * a.k_max;
  float* nkrow = a.newpos_k + ((int64_t)h * a.nt + t) * a.k_max;
  for (int s = tid; s < a.k_max; s += W_NT) {         // exact_2.py:401-408
    irow[s] = s < nvalid ? sidx[s] : N;
    nkrow[s] = s < nvalid ? snp[s] : 0.0f;
  }
  float* nqrow = a.newpos_q + ((int64_t)h * a.nt + t) * T;
  for (int i = tid; i < T; i += W_NT) {                 // exact_2.py:410-412
    const int qp = (int)min(tstart + i, (int64_t)N - 1);
    nqrow[i] = qnp[qp - qlo];
  }
  if (tid == 0) {
    const int o = h * a.nt + t;
    a.shared_size[o] = shared_total;
    a.kept_size[o] = kept_total;
    a.chosen[o] = ch;
    a.orig_overflow[o] = (uint8_t)oflow;
    a.overflow20[o] = (uint8_t)(oflow && !resolved);   // exact_2.py:354
    a.kpct_meas[o] = kmeas;
  }
}

template <typename VT, bool GK>
static hipError_t launch_select_w_t(const SelectArgs& a, size_t lds, hipStream_t st) {
  hipError_t e = hipFuncSetAttribute((const void*)select_w_kernel<VT, GK>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((select_w_kernel<VT, GK>), dim3(a.H * a.nt), dim3(W_NT), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_select_weighted(const SelectArgs& a, int vote_bytes, hipStream_t st) {
  if (a.T > 256 || !a.wvotes) return hipErrorInvalidValue;
  // the rank keys in LDS while they fit, else read from the vote rows at every pass
  const bool gk = select_w_lds_bytes(a.N, a.k_max, false) > 160 * 1024;
  const size_t lds = select_w_lds_bytes(a.N, a.k_max, gk);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  if (vote_bytes == 1)
    return gk ? launch_select_w_t<uint8_t, true>(a, lds, st) : launch_select_w_t<uint8_t, false>(a, lds, st);
  return gk ? launch_select_w_t<int32_t, true>(a, lds, st) : launch_select_w_t<int32_t, false>(a, lds, st);
}

}  // namespace sta
