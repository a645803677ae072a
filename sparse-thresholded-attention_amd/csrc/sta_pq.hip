// sta_pq.hip -- per-(head, tile) set construction of the per-query variant (PQ Union).
//
// Reference: shared_selection_triton_perquery.py:363-453 (_build_sets_pq).  The reference builds
// the tile's union of per-query keep sets (votes > 0), adds the forced global / local columns,
// and when |union U forced| > k_max keeps the forced keys plus the top (k_max - n_forced)
// candidates by rank value (expmass or margin weighted vote + 1e-6 votes, or votes) through a
// full-width torch.topk; positions are dense ranks over the kept set and every slot carries the
// key's per-query bits (forced columns: all bits).
//
// Here one workgroup owns one (head, tile) and scans only the keys the tile can keep: the causal
// range plus the global keys (all N keys for caller-given dense votes).  The tile's rank values
// are staged in LDS as order-preserving unsigned keys and the budget cut -- the budget-th largest key V, every candidate above V and the first
// (in key order) of those equal to V -- is a radix select:
//   level 1 (during staging): an 11-bit digit per candidate, the vote count itself for frequency
//     ranking (exact) or the sign and bits 30..20 of weighted rank values;
//   weighted: the keys of the statistic's level-1 bin (a few percent of the candidates) are
//     gathered into an LDS list and the remaining 20 bits are resolved on the list;
//   a bin too large for the list (or a vote count >= 2047) resolves the remaining bits over all
//     keys instead.
// torch.topk leaves the choice among ties unspecified; ascending key order is the rule here.
// Compaction is a block prefix sum; the dense rank of slot s is s itself.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

// one workgroup per (head, tile): PQ_NT threads in PQ_NW waves
constexpr int PQ_NT = 512;
constexpr int PQ_NW = PQ_NT / 64;

// inclusive block scan of one int per thread; returns the exclusive prefix and the block total
// through *total
__device__ __forceinline__ int pq_block_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < PQ_NW; ++w) {
    base += w < wave ? tmp[w] : 0;
    tot += tmp[w];
  }
  *total = tot;
  __syncthreads();
  return base + x - v;
}

// three block sums in one exchange (tmp holds 3 * PQ_NW ints)
__device__ __forceinline__ void pq_block_sum3(int x, int y, int z, int* tmp, int* sx, int* sy, int* sz) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    x += __shfl_xor(x, o, 64);
    y += __shfl_xor(y, o, 64);
    z += __shfl_xor(z, o, 64);
  }
  if (lane == 0) {
    tmp[wave] = x;
    tmp[PQ_NW + wave] = y;
    tmp[2 * PQ_NW + wave] = z;
  }
  __syncthreads();
  int a = 0, b = 0, c = 0;
#pragma unroll
  for (int w = 0; w < PQ_NW; ++w) {
    a += tmp[w];
    b += tmp[PQ_NW + w];
    c += tmp[2 * PQ_NW + w];
  }
  *sx = a;
  *sy = b;
  *sz = c;
  __syncthreads();
}

// KB keys of this thread's row from index i0 on (0 past `per`), read together so that one wait
// covers them all
constexpr int PQ_KB = 8;
__device__ __forceinline__ void pq_load_keys(const uint32_t* row, int i0, int per, uint32_t (&k)[PQ_KB]) {
#pragma unroll
  for (int e = 0; e < PQ_KB; ++e) k[e] = i0 + e < per ? row[i0 + e] : 0u;
}

// The digit holding the need-th largest count of a histogram of PQ_NT * B bins (descending),
// and how many of its keys are still needed: misc[0], misc[1].  Thread t owns bins
// PQ_NT*B-1-Bt .. PQ_NT*B-B-Bt.  Requires need >= 1 and at least `need` counts in the histogram.
template <int B>
__device__ __forceinline__ void pq_find_digit(const int* hist, int need, int* tmp, int* misc) {
  const int tid = threadIdx.x;
  const int top = PQ_NT * B - 1 - B * tid;
  int c[B], sl = 0;
#pragma unroll
  for (int e = 0; e < B; ++e) {
    c[e] = hist[top - e];
    sl += c[e];
  }
  int total;
  const int excl = pq_block_scan(sl, tmp, &total);
  if (excl < need && excl + sl >= need) {
    int acc = excl, d = top;
    bool found = false;
#pragma unroll
    for (int e = 0; e < B - 1; ++e) {
      found = found || acc + c[e] >= need;
      if (!found) {
        acc += c[e];
        d -= 1;
      }
    }
    misc[0] = d;
    misc[1] = need - acc;
  }
  __syncthreads();
}

// fp32 -> unsigned key of the same order (-0 folded into +0); never 0, which marks "not a candidate"
__device__ __forceinline__ uint32_t pq_order_key(float r) {
  const uint32_t b = __float_as_uint(r + 0.0f);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return k ? k : 1u;
}

// GK = false: the tile's rank keys are staged in LDS once.  GK = true (rows too long for LDS):
// every pass recomputes each key from the bits / votes / weighted-vote rows in the workspace
// (L2-resident for the workgroups in flight), with the staging's operations.
template <bool GK>
__global__ __launch_bounds__(PQ_NT) void pq_select_kernel(PqSelectArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t pq_smem[];
  const int tid = threadIdx.x;
  const int N = a.N, T = a.T;
  // the longest key ranges (the last tiles) start first
  const int h = (int)(blockIdx.x % a.H);
  const int t = a.nt - 1 - (int)(blockIdx.x / a.H);
  const int64_t tstart = (int64_t)a.q_pos_base + (int64_t)t * T;   // perquery.py:377
  const int64_t lo = tstart - a.n_local + 1, hi_l = tstart + T - 1;
  const int hi_keys = a.dense ? N : (int)min((int64_t)N, tstart + T);
  // keys at or past R are neither union members (no votes) nor forced
  const int R = a.dense ? N : (int)min((int64_t)N, max(tstart + T, (int64_t)a.n_global));
  const int per = (R + PQ_NT - 1) / PQ_NT;
  // thread tid scans keys [tid*per, tid*per + per); its keys sit at a row of odd stride PS so the
  // 64 lanes of a scan step fall in distinct LDS banks
  const int PS = per | 1;
  const int PSMAX = GK ? 0 : ((N + PQ_NT - 1) / PQ_NT) | 1;
  uint32_t* rkb = pq_smem;                                  // PQ_NT rows x PS rank keys (0: not a candidate)
  uint32_t* myrow = rkb + tid * PS;                         // this thread's keys j0 .. j0 + per - 1
  // j / per by a reciprocal multiply (per >= 2): exact for per <= 256 and j < 2^24
  const uint32_t inv_per = per > 1 ? (uint32_t)((0x100000000ull + per - 1) / per) : 0u;
  int* hist = (int*)(rkb + PQ_NT * PSMAX);                  // PQ_NT bins (list and fallback levels)
  int* tmp = hist + PQ_NT;                                  // 3 * PQ_NW
  int* misc = tmp + 3 * PQ_NW;                              // 8
  float* qnp = (float*)(misc + 8);                          // T (<= 64)
  // region A, max(2048, k_max) words: the level-1 histogram (2048 bins), then the list of the
  // statistic's bin, then the kept keys in rank order
  uint32_t* areg = (uint32_t*)(qnp + 64);
  int* hist1 = (int*)areg;
  uint32_t* list = areg;
  int32_t* sidx = (int32_t*)areg;
  const int list_cap = max(2048, a.k_max);

  const int64_t roff = ((int64_t)h * a.nt + t) * a.stride;
  const uint32_t* brow = a.bits + roff;
  const int j0 = tid * per, j1 = min(j0 + per, R);
  auto is_forced = [&](int j) { return j < a.n_global || (j >= lo && j <= hi_l); };
  const bool weighted = a.wvotes != nullptr;

#pragma unroll
  for (int e = 0; e < 2048 / PQ_NT; ++e) hist1[tid + PQ_NT * e] = 0;
  if (tid == 0) misc[2] = 0;
  __syncthreads();

  // ---- union, forced, candidates, their rank keys and the level-1 histogram (perquery.py:381-397) ----
  // staged with coalesced loads (key j by thread j % PQ_NT); the scans below walk contiguous ranges
  int cu = 0, cf = 0, cfo = 0;
  constexpr int U = 16;   // loads in flight per lane
  for (int jb = 0; jb < PQ_NT * per; jb += PQ_NT * U) {
    uint32_t bv[U];
    int vv[U];
    float wvv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + u * PQ_NT + tid;
      const bool ok = j < hi_keys;
      bv[u] = (ok && !a.votes) ? brow[j] : 0u;
      vv[u] = (ok && a.votes) ? a.votes[roff + j] : 0;
      wvv[u] = (ok && weighted) ? a.wvotes[roff + j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + u * PQ_NT + tid;
      uint32_t key = 0;
      if (j < R) {
        const int vt = a.votes ? vv[u] : __popc(bv[u]);
        const bool un = vt > 0, fo = is_forced(j);
        cu += un;
        cf += un || fo;
        cfo += fo;
        if (un && !fo) {
          int d1;
          if (weighted) {
            const float tb = 1e-6f * (float)vt;
            key = pq_order_key(wvv[u] + tb);
            // digit 0: negative values; 1 + bits 30..20 of a non-negative value (the top two
            // share digit 2047)
            d1 = key >= 0x80000000u ? 1 + min((int)((key & 0x7FFFFFFFu) >> 20), 2046) : 0;
          } else {
            key = pq_order_key((float)vt);
            d1 = min(vt, 2047);
          }
          atomicAdd(&hist1[d1], 1);
        }
      }
      if (!GK && j < PQ_NT * per) {
        const uint32_t row = per == 1 ? (uint32_t)j : __umulhi((uint32_t)j, inv_per);
        rkb[row * PS + (j - row * per)] = key;
      }
    }
  }
  __syncthreads();
  int usize, nfull, nforced;
  pq_block_sum3(cu, cf, cfo, tmp, &usize, &nfull, &nforced);
  const bool overflow = nfull > a.k_max;                    // perquery.py:386
  const int budget = max(a.k_max - nforced, 0);             // perquery.py:399-400
  const bool cut = overflow && budget > 0;
  // the rank key of key j from the workspace rows (GK): the staging's operations; 0 for keys past
  // R, outside the union, or forced
  auto gkey = [&](int j) -> uint32_t {
    if (j >= R || is_forced(j)) return 0u;
    const bool ok = j < hi_keys;
    const int vt = !ok ? 0 : (a.votes ? a.votes[roff + j] : __popc(brow[j]));
    if (vt <= 0) return 0u;
    if (weighted) {
      const float tb = 1e-6f * (float)vt;
      return pq_order_key(a.wvotes[roff + j] + tb);
    }
    return pq_order_key((float)vt);
  };
  // PQ_KB keys in an order the histograms and the list ignore: strided over the threads
  // (coalesced) when read from the workspace
  auto order_free_keys = [&](int i0, uint32_t (&kk)[PQ_KB]) {
    if constexpr (GK) {
#pragma unroll
      for (int e = 0; e < PQ_KB; ++e) kk[e] = i0 + e < per ? gkey((i0 + e) * PQ_NT + tid) : 0u;
    } else {
      pq_load_keys(myrow, i0, per, kk);
    }
  };
  // this thread's keys i0 .. i0 + PQ_KB - 1 of its contiguous range [j0, j0 + per)
  auto range_keys = [&](int i0, uint32_t (&kk)[PQ_KB]) {
    if constexpr (GK) {
#pragma unroll
      for (int e = 0; e < PQ_KB; ++e) kk[e] = i0 + e < per ? gkey(j0 + i0 + e) : 0u;
    } else {
      pq_load_keys(myrow, i0, per, kk);
    }
  };

  // ---- overflow: the budget-th largest rank key V and how many keys equal to V are taken ----
  uint32_t V = 0;
  int need_eq = 0;
  if (cut) {
    pq_find_digit<2048 / PQ_NT>(hist1, budget, tmp, misc);
    const int d1 = misc[0];
    int need = misc[1];
    const int bin_count = hist1[d1];
    uint32_t prefix, pmask;
    bool from_list = false;
    if (!weighted && d1 < 2047) {
      // the digit is the vote count: exact
      prefix = pq_order_key((float)d1);
      pmask = 0xFFFFFFFFu;
    } else if (weighted) {
      // the bin's keys share a prefix with the statistic; the rest from the bin's list when it fits
      if (d1 == 0) {
        prefix = 0;
        pmask = 0x80000000u;
      } else if (d1 < 2047) {
        prefix = 0x80000000u | ((uint32_t)(d1 - 1) << 20);
        pmask = 0xFFF00000u;
      } else {
        prefix = 0x80000000u | (2046u << 20);
        pmask = 0xFFE00000u;
      }
      from_list = bin_count <= list_cap;
    } else {
      // a vote count of 2047 or more holds the statistic: resolve the float keys from the top
      prefix = 0;
      pmask = 0;
      need = budget;
    }
    __syncthreads();   // every thread has read hist1 before the list overwrites it
    int cnt = 0;
    if (from_list) {
      for (int i0 = 0; i0 < per; i0 += PQ_KB) {
        uint32_t kk[PQ_KB];
        order_free_keys(i0, kk);
#pragma unroll
        for (int e = 0; e < PQ_KB; ++e) {
          const int slot = wave_alloc(kk[e] != 0 && (kk[e] & pmask) == prefix, &misc[2]);
          if (slot >= 0) list[slot] = kk[e];
        }
      }
      __syncthreads();
      cnt = misc[2];
    }
    // remaining levels: 8-bit digits below the prefix, the last one narrower when the bits run out
    while (pmask != 0xFFFFFFFFu) {
      const int nfree = 32 - __clz(~pmask);          // pmask covers the top 32 - nfree bits
      const int width = min(8, nfree), sh = nfree - width;
      const uint32_t dmask = (1u << width) - 1u;
      hist[tid] = 0;
      __syncthreads();
      if (from_list) {
        for (int i = tid; i < cnt; i += PQ_NT) {
          const uint32_t k = list[i];
          if ((k & pmask) == prefix) atomicAdd(&hist[(k >> sh) & dmask], 1);
        }
      } else {
        for (int i0 = 0; i0 < per; i0 += PQ_KB) {
          uint32_t kk[PQ_KB];
          order_free_keys(i0, kk);
#pragma unroll
          for (int e = 0; e < PQ_KB; ++e)
            if (kk[e] != 0 && (kk[e] & pmask) == prefix) atomicAdd(&hist[(kk[e] >> sh) & dmask], 1);
        }
      }
      __syncthreads();
      pq_find_digit<1>(hist, need, tmp, misc);
      prefix |= (uint32_t)misc[0] << sh;
      pmask |= dmask << sh;
      need = misc[1];
      __syncthreads();
    }
    V = prefix;
    need_eq = need;   // how many keys equal to V are taken, first in key order
  }
  __syncthreads();   // the list is dead: region A becomes sidx

  // ---- counts: kept keys strictly above the cut (and forced), keys at the cut ----
  // (forced keys hold key 0; a candidate's key is never 0)
  int cstrict = 0, ceq = 0;
  for (int i0 = 0; i0 < per; i0 += PQ_KB) {
    uint32_t kk[PQ_KB];
    range_keys(i0, kk);
#pragma unroll
    for (int e = 0; e < PQ_KB; ++e) {
      const int j = j0 + i0 + e;
      if (j < j1) {
        const uint32_t k = kk[e];
        if (is_forced(j)) {
          ++cstrict;
        } else if (k != 0) {
          if (!overflow) ++cstrict;
          else if (cut) {
            cstrict += k > V;
            ceq += k == V;
          }
        }
      }
    }
  }
  int eq_base = 0, eq_total;
  if (cut) eq_base = pq_block_scan(ceq, tmp, &eq_total);
  const int taken_eq = cut ? max(0, min(ceq, need_eq - eq_base)) : 0;
  int kept_total;
  const int base = pq_block_scan(cstrict + taken_eq, tmp, &kept_total);
  auto kept_of = [&](int j, uint32_t k, int eq_before) -> bool {
    if (is_forced(j)) return true;
    if (k == 0) return false;                 // not in the union (or forced, handled above)
    if (!overflow) return true;
    if (budget == 0) return false;
    if (k > V) return true;
    return k == V && eq_before < need_eq;
  };

  // ---- compaction: dense ranks (perquery.py:414-442) ----
  const int qlo = (int)min(tstart, (int64_t)N - 1);
  const int qhi = (int)min(tstart + T - 1, (int64_t)N - 1);
  int32_t* irow = a.idx + ((int64_t)h * a.nt + t) * a.k_max;
  float* nkrow = a.newpos_k + ((int64_t)h * a.nt + t) * a.k_max;
  int32_t* mrow = a.mask + ((int64_t)h * a.nt + t) * a.k_max;
  {
    int eq = eq_base;
    int rank = base - 1;
    for (int i0 = 0; i0 < per; i0 += PQ_KB) {
      uint32_t kk[PQ_KB];
      range_keys(i0, kk);
#pragma unroll
      for (int e = 0; e < PQ_KB; ++e) {
        const int j = j0 + i0 + e;
        if (j < j1) {
          const bool kp = kept_of(j, kk[e], eq);
          eq += cut && kk[e] == V;
          if (kp) {
            rank += 1;
            if (rank < a.k_max) sidx[rank] = j;
          }
          if (j >= qlo && j <= qhi) qnp[j - qlo] = (float)rank;   // rank0 = cumsum - 1
        }
      }
    }
  }
  __syncthreads();
  // slots in order, one per lane: coalesced stores (the ranks above are contiguous per thread,
  // which would scatter every store instruction over 64 cache lines); the kept keys ascend with
  // the slot, so the bit reads for the mask are nearly coalesced too
  const int nk = min(kept_total, a.k_max);
  for (int s0 = tid; s0 < a.k_max; s0 += 4 * PQ_NT) {
    int jj[4];
    uint32_t bb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {               // every bit read in flight before the stores
      const int s = s0 + PQ_NT * e;
      jj[e] = s < nk ? sidx[s] : N;
      bb[e] = (s < nk && !is_forced(jj[e]) && jj[e] < hi_keys) ? brow[jj[e]] : 0u;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = s0 + PQ_NT * e;
      if (s < a.k_max) {
        const bool valid = s < nk;
        irow[s] = jj[e];
        nkrow[s] = valid ? (float)s : 0.0f;
        mrow[s] = valid ? (is_forced(jj[e]) ? -1 : (int32_t)bb[e]) : 0;
      }
    }
  }
  float* nqrow = a.newpos_q + ((int64_t)h * a.nt + t) * T;
  for (int i = tid; i < T; i += PQ_NT) {
    const int qp = (int)min(tstart + i, (int64_t)N - 1);
    nqrow[i] = qnp[qp - qlo];
  }
  if (tid == 0) {
    const int o = h * a.nt + t;
    a.usize[o] = usize;
    a.kept_size[o] = kept_total;
    a.overflow[o] = (uint8_t)overflow;
  }
}

// byte-free workspace layout -> the reference's dense (H, nt, N) votes / bits / wvotes
__global__ __launch_bounds__(256) void expand_pq_kernel(const uint32_t* __restrict__ bits,
                                                        const float* __restrict__ wv, int64_t stride,
                                                        int nt, int N, int T, int q_pos_base,
                                                        int32_t* __restrict__ votes_out,
                                                        int32_t* __restrict__ bits_out,
                                                        float* __restrict__ wv_out) {
  const int ht = blockIdx.y;
  const int t = ht % nt;
  const int64_t hi = min((int64_t)N, (int64_t)q_pos_base + (int64_t)(t + 1) * T);
  for (int j = blockIdx.x * 256 + threadIdx.x; j < N; j += gridDim.x * 256) {
    const bool ok = j < hi;
    const uint32_t b = ok ? bits[(int64_t)ht * stride + j] : 0u;
    if (votes_out) votes_out[(int64_t)ht * N + j] = __popc(b);
    if (bits_out) bits_out[(int64_t)ht * N + j] = (int32_t)b;
    if (wv_out) wv_out[(int64_t)ht * N + j] = (ok && wv) ? wv[(int64_t)ht * stride + j] : 0.0f;
  }
}

size_t pq_select_lds_bytes(int N, int k_max, bool global_keys) {
  const size_t per = (size_t)(N + PQ_NT - 1) / PQ_NT;
  const size_t region_a = (size_t)(k_max > 2048 ? k_max : 2048) * 4;
  const size_t keys = global_keys ? 0 : PQ_NT * (per | 1) * 4;
  return keys + (PQ_NT + 3 * PQ_NW + 8) * 4 + 64 * 4 + region_a;
}

hipError_t launch_pq_select(const PqSelectArgs& a, hipStream_t st) {
  if (a.T > 64) return hipErrorInvalidValue;
  // the rank keys in LDS while they fit, else read from the workspace rows at every pass
  const bool gk = pq_select_lds_bytes(a.N, a.k_max, false) > 160 * 1024;
  const size_t lds = pq_select_lds_bytes(a.N, a.k_max, gk);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const void* fn = gk ? (const void*)pq_select_kernel<true> : (const void*)pq_select_kernel<false>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  if (gk) hipLaunchKernelGGL(pq_select_kernel<true>, dim3(a.H * a.nt), dim3(PQ_NT), lds, st, a);
  else hipLaunchKernelGGL(pq_select_kernel<false>, dim3(a.H * a.nt), dim3(PQ_NT), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_expand_pq(const uint32_t* bits, const float* wv, int64_t stride, int H, int nt, int N,
                            int T, int q_pos_base, int32_t* votes_out, int32_t* bits_out,
                            float* wv_out, hipStream_t st) {
  const int bx = (N + 255) / 256 < 64 ? (N + 255) / 256 : 64;
  hipLaunchKernelGGL(expand_pq_kernel, dim3(bx, H * nt), dim3(256), 0, st, bits, wv, stride, nt, N, T,
                     q_pos_base, votes_out, bits_out, wv_out);
  return hipGetLastError();
}

}  // namespace sta
