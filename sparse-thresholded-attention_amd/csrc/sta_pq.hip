// sta_pq.hip -- per-(head, tile) set construction of the per-query variant (PQ Union).
//
// Reference: shared_selection_triton_perquery.py:363-453 (_build_sets_pq).  The reference builds
// the tile's union of per-query keep sets (votes > 0), adds the forced global / local columns,
// and when |union U forced| > k_max keeps the forced keys plus the top (k_max - n_forced)
// candidates by rank value (expmass or margin weighted vote + 1e-6 votes, or votes) through a
// full-width torch.topk; positions are dense ranks over the kept set and every slot carries the
// key's per-query bits (forced columns: all bits).
//
// Here one workgroup owns one (head, tile).  The tile's rank values are staged in LDS as their
// fp32 bit patterns (all positive, so unsigned order is value order) and the cut is a 4-pass
// radix select on 8-bit digits: the budget-th largest value V, then every candidate above V and
// the first (in key order) of those equal to V.  torch.topk leaves the choice among ties
// unspecified; ascending key order is the rule here.  Compaction is a block prefix sum; the
// dense rank of slot s is s itself.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

__device__ __forceinline__ int pq_block_sum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  const int total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  __syncthreads();
  return total;
}

__device__ __forceinline__ int pq_block_exclusive_sum(int v, int* tmp) {
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

__global__ __launch_bounds__(256) void pq_select_kernel(PqSelectArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t pq_smem[];
  const int tid = threadIdx.x;
  const int h = blockIdx.x / a.nt, t = blockIdx.x % a.nt;
  const int N = a.N, T = a.T;
  const int per = (N + 255) / 256;
  // thread tid scans keys [tid*per, tid*per + per); its keys sit at a row of odd stride PS so the
  // 64 lanes of a scan step fall in distinct LDS banks
  const int PS = per | 1;
  uint32_t* rkb = pq_smem;                                  // 256 rows x PS rank keys (0: not a candidate)
  uint32_t* myrow = rkb + tid * PS;                         // this thread's keys j0 .. j0 + per - 1
  // j / per by a reciprocal multiply (per >= 2): exact for per <= 256 and j < 2^24
  const uint32_t inv_per = per > 1 ? (uint32_t)((0x100000000ull + per - 1) / per) : 0u;
  int* hist = (int*)(rkb + 256 * PS);                       // 256
  int* tmp = hist + 256;                                    // 8
  int* misc = tmp + 8;                                      // 8
  float* qnp = (float*)(misc + 8);                          // T (<= 64)
  int32_t* sidx = (int32_t*)(qnp + 64);                     // k_max: kept keys in rank order

  const int64_t tstart = (int64_t)a.q_pos_base + (int64_t)t * T;   // perquery.py:377
  const int64_t lo = tstart - a.n_local + 1, hi_l = tstart + T - 1;
  const int hi_keys = a.dense ? N : (int)min((int64_t)N, tstart + T);
  const int64_t roff = ((int64_t)h * a.nt + t) * a.stride;
  const uint32_t* brow = a.bits + roff;
  const int j0 = tid * per, j1 = min(j0 + per, N);
  auto is_forced = [&](int j) { return j < a.n_global || (j >= lo && j <= hi_l); };

  // ---- union, forced, candidates and their rank values (perquery.py:381-397) ----
  // staged with coalesced loads (key j by thread j % 256); the scans below walk contiguous ranges
  int cu = 0, cf = 0, cfo = 0;
  constexpr int U = 16;   // loads in flight per lane
  for (int jb = 0; jb < 256 * per; jb += 256 * U) {
    uint32_t bv[U];
    int vv[U];
    float wvv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + u * 256 + tid;
      const bool ok = j < hi_keys;
      bv[u] = (ok && !a.votes) ? brow[j] : 0u;
      vv[u] = (ok && a.votes) ? a.votes[roff + j] : 0;
      wvv[u] = (ok && a.wvotes) ? a.wvotes[roff + j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + u * 256 + tid;
      if (j >= 256 * per) break;
      uint32_t key = 0;
      if (j < N) {
        const int vt = a.votes ? vv[u] : __popc(bv[u]);
        const bool un = vt > 0, fo = is_forced(j);
        cu += un;
        cf += un || fo;
        cfo += fo;
        if (un && !fo) {
          float rv;
          if (a.wvotes) {
            const float tb = 1e-6f * (float)vt;
            rv = wvv[u] + tb;
          } else {
            rv = (float)vt;
          }
          key = __float_as_uint(rv);
          if (key == 0 || key >= 0x80000000u) key = 1;   // a non-positive value stays a candidate, lowest
        }
      }
      const uint32_t row = per == 1 ? (uint32_t)j : __umulhi((uint32_t)j, inv_per);
      rkb[row * PS + (j - row * per)] = key;
    }
  }
  __syncthreads();
  const int usize = pq_block_sum(cu, tmp);
  const int nfull = pq_block_sum(cf, tmp);
  const int nforced = pq_block_sum(cfo, tmp);
  const bool overflow = nfull > a.k_max;                    // perquery.py:386
  const int budget = max(a.k_max - nforced, 0);             // perquery.py:399-400

  // ---- overflow: radix select of the budget-th largest rank key, 8-bit digits ----
  // Rank values of one tile share few exponents, so the top digits of most keys coincide: that
  // pass aggregates its histogram increments per wave (one LDS atomic per distinct digit) instead
  // of 64 conflicting lane atomics.
  uint32_t V = 0;
  int need_eq = 0;
  if (overflow && budget > 0) {
    const int lane = tid & 63;
    uint32_t prefix = 0, pmask = 0;
    int need = budget;
    for (int shift = 24; shift >= 0; shift -= 8) {
      hist[tid] = 0;
      __syncthreads();
      if (shift == 24 && !a.wvotes) {
        // top digit (sign + high exponent bits) of vote counts: a handful of distinct values per
        // wave -> one atomic per distinct digit (weighted rank values spread over more exponents,
        // where plain atomics measured faster)
        for (int i = 0; i < per; ++i) {                // same trip count on every lane
          const uint32_t k = myrow[i];
          bool act = k != 0 && j0 + i < N;
          const int d = (int)(k >> 24);
          uint64_t m = __ballot(act);
          while (m) {
            const int leader = __ffsll((unsigned long long)m) - 1;
            const int dl = __shfl(d, leader, 64);
            const uint64_t same = __ballot(act && d == dl);
            if (lane == leader) atomicAdd(&hist[dl], (int)__popcll(same));
            if (act && d == dl) act = false;
            m &= ~same;
          }
        }
      } else {
        // lower digits are spread over the bins: plain LDS atomics
        for (int i = 0; i < per; ++i) {
          const uint32_t k = myrow[i];
          if (k != 0 && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1);
        }
      }
      __syncthreads();
      if (tid < 64) {
        // wave 0 finds the digit: lane l holds bins 255-4l .. 252-4l (descending)
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
          int acc = incl - sl, d = 255 - 4 * lane;
#pragma unroll
          for (int e = 0; e < 3; ++e) {
            if (acc + c[e] >= need) break;
            acc += c[e];
            d -= 1;
          }
          misc[0] = d;
          misc[1] = need - acc;
        }
      }
      __syncthreads();
      prefix |= (uint32_t)misc[0] << shift;
      pmask |= 255u << shift;
      need = misc[1];
      __syncthreads();
    }
    V = prefix;
    need_eq = need;   // how many keys equal to V are taken, first in key order
  }
  auto kept_of = [&](int j, int eq_before) -> bool {
    if (is_forced(j)) return true;
    const uint32_t k = myrow[j - j0];
    if (k == 0) return false;                 // not in the union (or forced, handled above)
    if (!overflow) return true;
    if (budget == 0) return false;
    if (k > V) return true;
    return k == V && eq_before < need_eq;
  };
  // ties at V: exclusive count of equal keys before each thread's range
  int eq_base = 0;
  if (overflow && budget > 0) {
    int ceq = 0;
    for (int j = j0; j < j1; ++j) ceq += myrow[j - j0] == V && !is_forced(j);
    eq_base = pq_block_exclusive_sum(ceq, tmp);
  }
  // ---- compaction: dense ranks (perquery.py:414-442) ----
  int ck = 0;
  {
    int eq = eq_base;
    for (int j = j0; j < j1; ++j) {
      const bool kp = kept_of(j, eq);
      eq += myrow[j - j0] == V && !is_forced(j) && overflow && budget > 0;
      ck += kp;
    }
  }
  const int base = pq_block_exclusive_sum(ck, tmp);
  const int kept_total = pq_block_sum(ck, tmp);
  const int qlo = (int)min(tstart, (int64_t)N - 1);
  const int qhi = (int)min(tstart + T - 1, (int64_t)N - 1);
  int32_t* irow = a.idx + ((int64_t)h * a.nt + t) * a.k_max;
  float* nkrow = a.newpos_k + ((int64_t)h * a.nt + t) * a.k_max;
  int32_t* mrow = a.mask + ((int64_t)h * a.nt + t) * a.k_max;
  {
    int eq = eq_base;
    int rank = base - 1;
    for (int j = j0; j < j1; ++j) {
      const bool kp = kept_of(j, eq);
      eq += myrow[j - j0] == V && !is_forced(j) && overflow && budget > 0;
      if (kp) {
        rank += 1;
        if (rank < a.k_max) sidx[rank] = j;
      }
      if (j >= qlo && j <= qhi) qnp[j - qlo] = (float)rank;   // rank0 = cumsum - 1
    }
  }
  __syncthreads();
  // slots in order, one per lane: coalesced stores (the ranks above are contiguous per thread,
  // which would scatter every store instruction over 64 cache lines); the kept keys ascend with
  // the slot, so the bit reads for the mask are nearly coalesced too
  const int nk = min(kept_total, a.k_max);
  for (int s = tid; s < a.k_max; s += 256) {
    if (s < nk) {
      const int j = sidx[s];
      irow[s] = j;
      nkrow[s] = (float)s;
      mrow[s] = is_forced(j) ? -1 : (int32_t)(j < hi_keys ? brow[j] : 0u);
    } else {
      irow[s] = N;
      nkrow[s] = 0.0f;
      mrow[s] = 0;
    }
  }
  float* nqrow = a.newpos_q + ((int64_t)h * a.nt + t) * T;
  for (int i = tid; i < T; i += 256) {
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

size_t pq_select_lds_bytes(int N, int k_max) {
  const size_t per = (size_t)(N + 255) / 256;
  return 256 * (per | 1) * 4 + (256 + 8 + 8) * 4 + 64 * 4 + (size_t)k_max * 4;
}

hipError_t launch_pq_select(const PqSelectArgs& a, hipStream_t st) {
  const size_t lds = pq_select_lds_bytes(a.N, a.k_max);
  if (lds > 160 * 1024 || a.T > 64) return hipErrorInvalidValue;
  hipError_t e = hipFuncSetAttribute((const void*)pq_select_kernel,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(pq_select_kernel, dim3(a.H * a.nt), dim3(256), lds, st, a);
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
