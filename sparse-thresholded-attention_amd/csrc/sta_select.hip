// sta_select.hip -- per-(head, tile) key-set selection, the device form of _build_sets.
//
// Reference: shared_selection_triton_exact_2.py:277-426 (freq mode).  The reference runs about
// twenty full (H, nt, N) torch passes, a topk of width ceil(0.3 N) and up to three host syncs.
// Here one workgroup owns one (head, tile): the tile's vote row is staged in LDS, and because
// votes are integers in [0, tile] the order statistic the reference reads from topk is a lookup
// in a vote histogram:
//   sv[b] (the (b+1)-th largest vote) = max{ v : #(votes >= v) >= b + 1 }.
// kept-set sizes for a cut v are #(votes >= v) + #(forced keys with vote < v), so the whole
// 30 -> 25 -> 20 fallback (exact_2.py:328-350), the pct=0 special case (343-346) and the
// measure loop (357-371) are histogram arithmetic.  Compaction (401-408) is a block prefix sum,
// and the reposition recurrence newpos = rank0 + cummax(cpos - rank0) (383-386) is a block
// prefix max over the same fp32 values the reference computes.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

// block-wide exclusive scans over 256 threads (4 waves); `tmp` holds 4 entries
__device__ __forceinline__ int block_exclusive_sum(int v, int* tmp) {
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

__device__ __forceinline__ float block_exclusive_max(float v, float* tmp) {
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
__device__ __forceinline__ int64_t budget_of(int p, int64_t usize) {
#pragma clang fp contract(off)
  const float frac = (float)((double)p / 100.0);
  const float prod = frac * (float)usize;
  float b = ceilf(prod);
  if (b < 1.0f) b = 1.0f;
  return (int64_t)b;
}

// the smallest vote v with C[v] >= need (C non-increasing, C[0] = N >= need)
__device__ __forceinline__ int cut_for(const int* C, int64_t need) {
  int lo = 0, hi = 255;  // answer in [0, 255]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)C[mid] >= need) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <typename VT>
__global__ __launch_bounds__(256) void select_kernel(SelectArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  // the longest key ranges (the last tiles) start first
  const int h = (int)(blockIdx.x % a.H);
  const int t = a.nt - 1 - (int)(blockIdx.x / a.H);
  const int T = a.T;
  const int64_t tstart = (int64_t)a.q_pos_base + (int64_t)t * T;          // exact_2.py:291
  // the key axis: [0, N); under DCA inter selection the tile's inter keys, with the budget's
  // K_ord = max(1, min(N, ceil(start_pct / 100 N))) of that axis (exact_2.py:320)
  int N = a.N;
  int64_t K_ord = a.K_ord;
  if (a.dca_L > 0) {
    const int64_t c = tstart / a.dca_L;
    N = c >= 2 ? (int)min((int64_t)a.N, (c - 1) * a.dca_L) : 0;
    K_ord = (int64_t)ceil((double)a.start_pct / 100.0 * (double)N);
    K_ord = K_ord > N ? N : (K_ord < 1 ? 1 : K_ord);
    if (N == 0) {                 // no inter keys (the first two chunks): an empty set
      const int o = h * a.nt + t;
      if (threadIdx.x == 0) {
        a.shared_size[o] = 0;
        a.kept_size[o] = 0;
        a.chosen[o] = 0;
        a.orig_overflow[o] = 0;
        a.overflow20[o] = 0;
        a.kpct_meas[o] = 0;
      }
      for (int s = threadIdx.x; s < a.k_max; s += 256) {
        a.idx[(int64_t)o * a.k_max + s] = 0;
        a.newpos_k[(int64_t)o * a.k_max + s] = 0.0f;
      }
      for (int i = threadIdx.x; i < T; i += 256) a.newpos_q[(int64_t)o * T + i] = 0.0f;
      if (a.votes_out)
        for (int j = threadIdx.x; j < a.N; j += 256) a.votes_out[(int64_t)o * a.N + j] = 0;
      return;
    }
  }
  // votes are read for keys [0, hi_keys); Kernel A leaves keys past the tile's causal end
  // unwritten (their count is 0), a caller-supplied dense tensor is read in full
  const int hi_keys = a.votes_dense ? N : (int)min((int64_t)N, tstart + T);
  // keys per thread for a scan over [0, n): a multiple of 16 (the vote bytes are read 16 at a time)
  auto per_of = [](int n) { return (((n + 255) / 256 + 15) / 16) * 16; };
  const int per = per_of(a.N);                                              // the staged row
  uint8_t* vb = smem;                                                       // 256 * per vote bytes
  int* hist = (int*)(smem + 256 * per);                                     // 256 bins -> C[v] (257)
  int* fhist = hist + 260;                                                  // 256 bins -> F[v] (257)
  int* tmpi = fhist + 260;                                                  // 8
  float* tmpf = (float*)(tmpi + 8);                                         // 8
  int* misc = (int*)(tmpf + 8);                                             // 16
  float* qnp = (float*)(misc + 16);                                         // T (<= 256)
  int32_t* sidx = (int32_t*)(qnp + 256);                                    // k_max (stage_slots)
  float* snp = (float*)(sidx + a.k_max);                                    // k_max (stage_slots)

  for (int i = tid; i < 260; i += 256) { hist[i] = 0; fhist[i] = 0; }
  if (tid == 0) misc[1] = 0;
  // ---- stage the vote row, zero past the keys the score kernel wrote (its causal range) ----
  const VT* vrow = (const VT*)a.votes + ((int64_t)h * a.nt + t) * a.votes_stride;
  if constexpr (sizeof(VT) == 1) {
    for (int wi = tid; wi < 64 * per; wi += 256) {   // four keys per word
      const int j = wi * 4;
      uint32_t w = 0;
      if (j < hi_keys) {   // j + 3 < roundup(N, 4) <= votes_stride: the word is inside the row
        w = ((const uint32_t*)vrow)[wi];
        const int valid = hi_keys - j;
        if (valid < 4) w &= (1u << (8 * valid)) - 1u;
      }
      ((uint32_t*)vb)[wi] = w;
    }
  } else {
    for (int j = tid; j < 256 * per; j += 256) vb[j] = j < hi_keys ? (uint8_t)vrow[j] : 0;
  }
  __syncthreads();
  if (a.votes_out) {
    int32_t* vo = a.votes_out + ((int64_t)h * a.nt + t) * a.N;
    for (int j = tid; j < a.N; j += 256) vo[j] = vb[j];
  }
  // Thread tid owns a contiguous key range for the histogram and one for the compaction, each
  // sized by the range the scan covers; its vote bytes are read 16 at a time.
  auto seg_bytes = [&](int jb) { return *(const u32x4*)(vb + jb); };
  auto byte_of = [](const u32x4& w, int e) { return (int)((w[e >> 2] >> (8 * (e & 3))) & 0xffu); };
  // ---- vote histogram over all N keys: the nonzero votes by LDS atomics, the zero bin by
  // subtraction (most keys of a tile have no vote, and one bin taking them all serialises) ----
  {
    const int per_h = per_of(hi_keys);
    const int jh0 = tid * per_h;
    const int jend = min(jh0 + per_h, hi_keys);
    int nz = 0;
    for (int jb = jh0; jb < jend; jb += 16) {
      const u32x4 w = seg_bytes(jb);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int b = byte_of(w, e);
        if (jb + e < jend && b != 0) {
          atomicAdd(&hist[b], 1);
          ++nz;
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) nz += __shfl_xor(nz, o, 64);
    if ((tid & 63) == 0) atomicAdd(&misc[1], nz);
  }
  // forced = [0, n_global) U [tstart - n_local + 1, tstart + T - 1]   (exact_2.py:290-293)
  const int gA = min(a.n_global, N);
  const int64_t lo = tstart - a.n_local + 1, hi_l = tstart + T - 1;
  const int bl = (int)max(lo, (int64_t)gA);
  const int bh = (int)min(hi_l, (int64_t)N - 1);
  const int nB = bh >= bl ? bh - bl + 1 : 0;
  for (int i = tid; i < gA + nB; i += 256) {
    const int j = i < gA ? i : bl + (i - gA);
    atomicAdd(&fhist[vb[j]], 1);
  }
  __syncthreads();
  if (tid == 0) hist[0] = N - misc[1];   // keys past hi_keys have no vote either
  __syncthreads();
  // ---- C[v] = #(votes >= v) (suffix sums) and F[v] = #(forced with vote < v) (prefix sums) ----
  {
    const int hv = hist[tid], fv = fhist[tid];
    __syncthreads();
    const int above = block_exclusive_sum(hv, tmpi);   // sum of hist[0..tid-1]
    const int fbelow = block_exclusive_sum(fv, tmpi + 4);
    const int total = N;
    hist[tid] = total - above;                          // C[tid] = N - #(votes < tid)
    fhist[tid] = fbelow;                                // F[tid]
    if (tid == 255) {
      hist[256] = total - above - hv;                   // C[256] = 0 for byte votes
      fhist[256] = fbelow + fv;                         // F[256] = # forced keys
    }
  }
  __syncthreads();
  const int* C = hist;
  const int* F = fhist;
  if (tid == 0) {
    const int64_t usize = C[1];                         // #(votes > 0)   (exact_2.py:296)
    int resolved = 0, ch = 0, oflow = 0, vc = 0;
    for (int si = 0; si < a.nsteps; ++si) {             // exact_2.py:328-342
      const int p = a.steps[si];
      int64_t bi = budget_of(p, usize) - 1;
      bi = bi < 0 ? 0 : (bi > K_ord - 1 ? K_ord - 1 : bi);
      const int v_cut = cut_for(C, bi + 1);             // sv[bi] (exact_2.py:330)
      const int64_t size = (int64_t)C[v_cut] + F[v_cut];
      if (p == a.start_pct) oflow = size > a.k_max;
      if (!resolved) {
        vc = v_cut;
        if (size <= a.k_max) { resolved = 1; ch = p; }
      }
    }
    if (a.start_pct == 0) {                              // exact_2.py:343-346
      oflow = F[256] > a.k_max;
      if (!resolved) vc = 256;                           // forced keys only
    }
    int kmeas = ch;
    if (a.measure && !resolved) {                        // exact_2.py:357-371
      const int floor_pct = a.steps[a.nsteps - 1];
      for (int p = floor_pct - 1; p > 0; --p) {
        int64_t bi = budget_of(p, usize) - 1;
        bi = bi < 0 ? 0 : (bi > K_ord - 1 ? K_ord - 1 : bi);
        const int v_cut = cut_for(C, bi + 1);
        if ((int64_t)C[v_cut] + F[v_cut] <= a.k_max) { kmeas = p; break; }
      }
    }
    const int o = h * a.nt + t;
    a.shared_size[o] = C[vc];
    a.kept_size[o] = C[vc] + F[vc];
    a.chosen[o] = ch;
    a.orig_overflow[o] = (uint8_t)oflow;
    a.overflow20[o] = (uint8_t)(oflow && !resolved);     // exact_2.py:354
    a.kpct_meas[o] = kmeas;
    misc[0] = vc;
  }
  __syncthreads();
  const int vc = misc[0];
  const int kept_total = C[vc] + F[vc];
  const int nvalid = min(kept_total, a.k_max);
  int32_t* irow = a.idx + ((int64_t)h * a.nt + t) * a.k_max;
  float* nkrow = a.newpos_k + ((int64_t)h * a.nt + t) * a.k_max;
  // the kept slots: gathered in LDS and written coalesced afterwards, or (long rows, where the
  // k_max slots in LDS would leave one workgroup per CU) written straight from the compaction,
  // each thread's kept keys having consecutive ranks
  int32_t* dst_i = a.stage_slots ? sidx : irow;
  float* dst_n = a.stage_slots ? snp : nkrow;
  // ---- compaction + reposition over keys [0, scan_end) ----
  const int scan_end = (vc == 0) ? N : min(N, max(hi_keys, max(gA, bh + 1)));
  const int per_c = per_of(scan_end);
  const int j0 = tid * per_c;
  const int j1 = min(j0 + per_c, scan_end);
  int cnt = 0;
  for (int jb = j0; jb < j1; jb += 16) {
    const u32x4 w = seg_bytes(jb);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = jb + e;
      const bool forced = (j < gA) || (j >= bl && j <= bh);
      cnt += j < j1 && ((byte_of(w, e) >= vc) || forced);
    }
  }
  const int base = block_exclusive_sum(cnt, tmpi);
  float mloc = -INFINITY;
  {
    int rank = base - 1;
    for (int jb = j0; jb < j1; jb += 16) {
      const u32x4 w = seg_bytes(jb);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = jb + e;
        const bool forced = (j < gA) || (j >= bl && j <= bh);
        if (j < j1 && ((byte_of(w, e) >= vc) || forced)) {
          rank += 1;
          const float cp = (float)j * a.pos_scale;      // exact_2.py:384
          mloc = fmaxf(mloc, cp - (float)rank);         // exact_2.py:385
        }
      }
    }
  }
  float run = block_exclusive_max(mloc, tmpf);
  const int qlo = (int)min(tstart, (int64_t)N - 1);
  const int qhi = (int)min(tstart + T - 1, (int64_t)N - 1);
  {
    int rank = base - 1;
    for (int jb = j0; jb < j1; jb += 16) {
      const u32x4 w = seg_bytes(jb);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = jb + e;
        if (j < j1) {
          const bool forced = (j < gA) || (j >= bl && j <= bh);
          const bool kept = (byte_of(w, e) >= vc) || forced;
          if (kept) {
            rank += 1;
            const float cp = (float)j * a.pos_scale;
            run = fmaxf(run, cp - (float)rank);
          }
          const float np = (float)rank + run;          // exact_2.py:386
          if (kept && rank < a.k_max) { dst_i[rank] = j; dst_n[rank] = np; }
          if (j >= qlo && j <= qhi) qnp[j - qlo] = np;
        }
      }
    }
  }
  __syncthreads();
  if (a.stage_slots) {
    for (int s = tid; s < a.k_max; s += 256) {        // exact_2.py:401-408
      irow[s] = s < nvalid ? sidx[s] : N;
      nkrow[s] = s < nvalid ? snp[s] : 0.0f;
    }
  } else {
    for (int s = nvalid + tid; s < a.k_max; s += 256) {   // sentinels (exact_2.py:401-408)
      irow[s] = N;
      nkrow[s] = 0.0f;
    }
  }
  float* nqrow = a.newpos_q + ((int64_t)h * a.nt + t) * T;
  for (int i = tid; i < T; i += 256) {                  // exact_2.py:410-412
    const int qp = (int)min(tstart + i, (int64_t)N - 1);
    nqrow[i] = qnp[qp - qlo];
  }
}

// byte votes (keys < min(N, tile end) valid) -> the reference's dense int32 (H, nt, N) votes, and
// the weighted votes (when wv is given) -> dense fp32 (H, nt, N)
__global__ __launch_bounds__(256) void expand_votes_kernel(const uint8_t* __restrict__ v8, int64_t stride,
                                                           int nt, int N, int T, int q_pos_base,
                                                           int32_t* __restrict__ out,
                                                           const float* __restrict__ wv,
                                                           float* __restrict__ wv_out) {
  const int ht = blockIdx.y;
  const int t = ht % nt;
  const int64_t hp = min((int64_t)N, (int64_t)q_pos_base + (int64_t)t * T + T);
  for (int j = blockIdx.x * 256 + threadIdx.x; j < N; j += gridDim.x * 256) {
    out[(int64_t)ht * N + j] = j < hp ? (int32_t)v8[(int64_t)ht * stride + j] : 0;
    if (wv_out) wv_out[(int64_t)ht * N + j] = j < hp ? wv[(int64_t)ht * stride + j] : 0.0f;
  }
}

hipError_t launch_expand_votes(const uint8_t* v8, int64_t stride, int H, int nt, int N, int T, int q_pos_base,
                               int32_t* out, const float* wv, float* wv_out, hipStream_t st) {
  const int bx = (N + 255) / 256 < 64 ? (N + 255) / 256 : 64;
  hipLaunchKernelGGL(expand_votes_kernel, dim3(bx, H * nt), dim3(256), 0, st, v8, stride, nt, N, T, q_pos_base,
                     out, wv, wv_out);
  return hipGetLastError();
}

// the LDS a row needs without the slot staging (k_max * 8 bytes more with it)
size_t select_lds_bytes(int N, int k_max) {
  (void)k_max;
  const int per = ((((N + 255) / 256) + 15) / 16) * 16;
  return (size_t)256 * per + (260 + 260 + 8) * 4 + 8 * 4 + 16 * 4 + 256 * 4;
}

hipError_t launch_select(const SelectArgs& a0, int vote_bytes, hipStream_t st) {
  SelectArgs a = a0;
  const size_t base = select_lds_bytes(a.N, a.k_max);
  if (base > 160 * 1024) return hipErrorInvalidValue;
  // stage the slots while two workgroups still fit a CU (c4's 64k rows: 3.5 ms direct against
  // 6.7 ms staged at one workgroup per CU; c1's rows: 0.127 ms staged, 0.137 ms direct)
  a.stage_slots = base + (size_t)a.k_max * 8 <= 80 * 1024 ? 1 : 0;
  const size_t lds = base + (a.stage_slots ? (size_t)a.k_max * 8 : 0);
  if (vote_bytes == 1) {
    hipError_t e = hipFuncSetAttribute((const void*)select_kernel<uint8_t>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(select_kernel<uint8_t>, dim3(a.H * a.nt), dim3(256), lds, st, a);
  } else {
    hipError_t e = hipFuncSetAttribute((const void*)select_kernel<int32_t>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(select_kernel<int32_t>, dim3(a.H * a.nt), dim3(256), lds, st, a);
  }
  return hipGetLastError();
}

}  // namespace sta
