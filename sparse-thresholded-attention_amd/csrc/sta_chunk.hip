// sta_chunk.hip -- chunk-granular set construction (the "chunk_exact" variant).
//
// Reference: shared_selection_triton_chunked.py, _build_sets_chunk (:149-243, prefill, per
// (head, tile) from Kernel A's votes / weighted votes) and _decode_build_sets_chunk (:411-489,
// per query from its scores).  Keys are grouped into fixed chunks of C; a chunk is valued by the
// sum (or the mean over its candidates) of its threshold passers' rank values; the forced global /
// local chunks are kept, and of the other visible chunks the top n_chunk by value (equal values
// in ascending chunk order -- torch.topk leaves that order unspecified); the kept chunks' keys up
// to the last query are compacted at dense ranks.  The budget is exact: at most
// (forced + n_chunk) chunks are kept.
//
// One workgroup (256 threads) owns one (head, tile) or one (head, query).  Thread t owns the
// contiguous chunks [t cpt, t cpt + cpt) and sums each chunk's keys in key order; the chunk values
// live in LDS as orderable keys (fp32 bits + 1, 0 = not a candidate), the n_chunk-th largest is
// found by a 4-pass radix select on 8-bit digits, ties are ranked by a block prefix sum in chunk
// order, and the compaction is a second prefix sum over the kept chunks' key counts.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

constexpr int CH_NT = 256;

__device__ __forceinline__ int ch_block_sum(int v, int* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  const int total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  __syncthreads();
  return total;
}

__device__ __forceinline__ int ch_block_exclusive_sum(int v, int* tmp) {
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

__device__ __forceinline__ float ch_block_max(float v, float* tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  const float m = fmaxf(fmaxf(tmp[0], tmp[1]), fmaxf(tmp[2], tmp[3]));
  __syncthreads();
  return m;
}

// a chunk value (>= 0) as an orderable nonzero key
__device__ __forceinline__ uint32_t ch_key(float v) { return __float_as_uint(v) + 1u; }

// selc[c] = 1 for the n_take largest candidate keys ck[c] != 0 (equal keys: ascending c); the
// calling thread owns chunks [c0, c1).  Returns nothing; selc must be zero on entry.
__device__ void ch_top(const uint32_t* ck, uint8_t* selc, int c0, int c1, int n_take, int* hist, int* tmp,
                       int* misc) {
  const int tid = threadIdx.x;
  if (n_take <= 0) return;
  int nl = 0;
  for (int c = c0; c < c1; ++c) nl += ck[c] != 0u;
  const int ncand = ch_block_sum(nl, tmp);
  if (ncand <= n_take) {
    for (int c = c0; c < c1; ++c) selc[c] = ck[c] != 0u;
    __syncthreads();
    return;
  }
  // the n_take-th largest key, 8 bits per pass from the top
  uint32_t prefix = 0u, pmask = 0u;
  int need = n_take;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[tid] = 0;
    __syncthreads();
    for (int c = c0; c < c1; ++c) {
      const uint32_t k = ck[c];
      if (k != 0u && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1);
    }
    __syncthreads();
    const int d = 255 - tid;                    // bins in descending order
    const int v = hist[d];
    const int above = ch_block_exclusive_sum(v, tmp);
    if (above < need && above + v >= need) {
      misc[0] = d;
      misc[1] = need - above;
    }
    __syncthreads();
    prefix |= (uint32_t)misc[0] << shift;
    pmask |= 255u << shift;
    need = misc[1];
    __syncthreads();
  }
  const uint32_t K = prefix;
  int gt = 0, eq = 0;
  for (int c = c0; c < c1; ++c) {
    gt += ck[c] > K;
    eq += ck[c] == K;
  }
  const int quota = n_take - ch_block_sum(gt, tmp);
  int tie = ch_block_exclusive_sum(eq, tmp);
  for (int c = c0; c < c1; ++c) {
    const uint32_t k = ck[c];
    if (k > K) {
      selc[c] = 1;
    } else if (k == K) {
      selc[c] = tie < quota;
      ++tie;
    }
  }
  __syncthreads();
}

// kept keys of chunk c: its keys j < lim when the chunk is kept, else `extra` alone when it falls
// in the chunk (the decode rule's own position)
__device__ __forceinline__ int ch_chunk_kept(const uint8_t* selc, int c, int C, int lim, int extra) {
  const int a = c * C, b = min((c + 1) * C, lim);
  if (b <= a) return 0;
  if (selc[c]) return b - a;
  return (extra >= a && extra < b) ? 1 : 0;
}

// ------------------------------------------------------------------------------------------
// prefill: one workgroup per (head, tile)
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(CH_NT) void chunk_select_kernel(ChunkSelectArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t ch_smem[];
  const int tid = threadIdx.x;
  const int h = blockIdx.x / a.nt, t = blockIdx.x % a.nt;
  const int N = a.N, T = a.T, C = a.C;
  const int nC = (N + C - 1) / C;
  uint32_t* ck = ch_smem;                                   // nC
  uint8_t* selc = (uint8_t*)(ck + nC);                      // nC
  int* hist = (int*)(ck + nC + (nC + 3) / 4);               // 256
  int* tmp = hist + 256;                                    // 8
  int* misc = tmp + 8;                                      // 8
  const int cpt = (nC + CH_NT - 1) / CH_NT;
  const int c0 = min(tid * cpt, nC), c1 = min(c0 + cpt, nC);

  const int64_t r0 = (int64_t)a.q_pos_base + (int64_t)t * T;
  const int64_t last_q = r0 + T - 1;
  const int lim = (int)min(last_q + 1, (int64_t)N);         // kept keys j <= min(last_q, N - 1)
  const int hi_keys = a.dense ? N : (int)min((int64_t)N, r0 + T);
  const int64_t roff = ((int64_t)h * a.nt + t) * a.stride;
  const int ng_c = (a.n_global + C - 1) / C;
  const int64_t lo_c = max((int64_t)0, r0 - a.n_local + 1) / C, hi_c = last_q / C;
  auto visible = [&](int c) { return (int64_t)c * C <= last_q; };
  auto forced = [&](int c) { return visible(c) && (c < ng_c || (c >= lo_c && c <= hi_c)); };
  auto votes_of = [&](int j) -> int {
    if (j >= hi_keys) return 0;
    return a.votes ? a.votes[roff + j] : __popc(a.bits[roff + j]);
  };

  // ---- chunk values (chunked.py:165-180) and usize (:203) ----
  int us = 0;
  for (int c = c0; c < c1; ++c) {
    float m = 0.0f;
    int cnt = 0;
    const int jend = min((c + 1) * C, N);
    for (int j = c * C; j < jend; ++j) {
      const int vt = votes_of(j);
      if (vt > 0) {
        m = m + (a.wvotes ? a.wvotes[roff + j] : (float)vt);
        ++cnt;
        us += j <= last_q;
      }
    }
    const float val = a.mean ? m / (float)max(cnt, 1) : m;
    ck[c] = (visible(c) && !forced(c)) ? ch_key(val) : 0u;
    selc[c] = 0;
  }
  __syncthreads();
  us = ch_block_sum(us, tmp);

  // ---- top n_chunk of the visible non-forced chunks, plus the forced visible ones (:184-193) ----
  ch_top(ck, selc, c0, c1, min(a.n_chunk, nC), hist, tmp, misc);
  for (int c = c0; c < c1; ++c) selc[c] |= (uint8_t)forced(c);
  __syncthreads();

  // ---- compaction at dense ranks (:198-231) ----
  int mine = 0;
  for (int c = c0; c < c1; ++c) mine += ch_chunk_kept(selc, c, C, lim, -1);
  int total;
  {
    const int excl = ch_block_exclusive_sum(mine, tmp);
    total = ch_block_sum(mine, tmp);
    mine = excl;                                            // kept keys before chunk c0
  }
  const int64_t orow = ((int64_t)h * a.nt + t) * a.k_max;
  int32_t* irow = a.idx + orow;
  float* nrow = a.newpos_k + orow;
  int pk = 0;
  {
    int r = mine;
    for (int c = c0; c < c1; ++c) {
      if (!selc[c]) continue;
      const int jend = min((c + 1) * C, lim);
      for (int j = c * C; j < jend; ++j, ++r) {
        if (r < a.k_max) {
          irow[r] = j;
          nrow[r] = (float)r;
        }
        if (a.passers_kept) pk += votes_of(j) > 0;
      }
    }
    // each query position's rank: kept keys <= qp, minus one (:228-231)
    for (int i = 0; i < T; ++i) {
      const int qp = (int)min(r0 + i, (int64_t)N - 1);
      const int cq = qp / C;
      if (cq < c0 || cq >= c1) continue;
      int before = mine;
      for (int c = c0; c < cq; ++c) before += ch_chunk_kept(selc, c, C, lim, -1);
      const int within = selc[cq] ? qp - cq * C + 1 : 0;
      a.newpos_q[((int64_t)h * a.nt + t) * T + i] = (float)(before + within - 1);
    }
  }
  for (int s = min(total, a.k_max) + tid; s < a.k_max; s += CH_NT) {
    irow[s] = N;
    nrow[s] = 0.0f;
  }
  if (a.mask)
    for (int s = tid; s < a.k_max; s += CH_NT) a.mask[orow + s] = s < total ? -1 : 0;   // pooled (:225-226)
  if (a.passers_kept) pk = ch_block_sum(pk, tmp);
  if (tid == 0) {
    const int64_t o = (int64_t)h * a.nt + t;
    a.usize[o] = us;
    a.kept_size[o] = total;
    if (a.overflow) a.overflow[o] = 0;
    if (a.passers_kept) a.passers_kept[o] = pk;
  }
}

// ------------------------------------------------------------------------------------------
// decode: one workgroup per (head, query); query i at q_pos0 + i over the keys [0, m_i)
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(CH_NT) void chunk_decode_select_kernel(ChunkDecodeArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint32_t ch_smem[];
  const int tid = threadIdx.x;
  const int h = blockIdx.x / a.Q, i = blockIdx.x % a.Q;
  const int C = a.C;
  const int m = a.M - (a.Q - 1 - i);
  const int qp = a.q_pos0 + i;
  const int nC = (m + C - 1) / C;
  const int nCmax = (a.M + C - 1) / C;
  uint32_t* ck = ch_smem;
  uint8_t* selc = (uint8_t*)(ck + nCmax);
  int* hist = (int*)(ck + nCmax + (nCmax + 3) / 4);
  int* tmp = hist + 256;
  int* misc = tmp + 8;
  const int cpt = (nC + CH_NT - 1) / CH_NT;
  const int c0 = min(tid * cpt, nC), c1 = min(c0 + cpt, nC);
  const float* row = a.scores + ((int64_t)h * a.Q + i) * a.M;

  // ---- row max and threshold (chunked.py:433-434) ----
  float mx = -INFINITY;
  for (int j = tid; j < m; j += CH_NT) mx = fmaxf(mx, row[j]);
  mx = ch_block_max(mx, (float*)tmp);
  const float thr = mx - a.tau[h];

  const int ng_c = (a.n_global + C - 1) / C;
  const int lo_c = max(0, qp - a.n_local + 1) / C, hi_c = qp / C;
  auto visible = [&](int c) { return c * C <= qp; };
  auto forced = [&](int c) { return visible(c) && (c < ng_c || (c >= lo_c && c <= hi_c)); };

  // ---- chunk values: exp(s - m) (or 1) over the kept keys (:437-445) ----
  int npass = 0;
  for (int c = c0; c < c1; ++c) {
    float s = 0.0f;
    int cnt = 0;
    const int jend = min((c + 1) * C, m);
    for (int j = c * C; j < jend; ++j) {
      const float x = row[j];
      if (x >= thr) {
        s = s + (a.weighted ? expf(x - mx) : 1.0f);
        ++cnt;
      }
    }
    npass += cnt;
    const float val = a.mean ? s / (float)max(cnt, 1) : s;
    ck[c] = (visible(c) && !forced(c)) ? ch_key(val) : 0u;
    selc[c] = 0;
  }
  __syncthreads();
  if (a.usize) npass = ch_block_sum(npass, tmp);
  ch_top(ck, selc, c0, c1, min(a.n_chunk, nC), hist, tmp, misc);
  for (int c = c0; c < c1; ++c) selc[c] |= (uint8_t)forced(c);
  __syncthreads();

  // ---- kept = the chunks' keys j <= q_pos, and q_pos itself (:460-462); dense ranks ----
  const int lim = min(qp + 1, m);
  const int extra = qp < m ? qp : -1;
  int mine = 0;
  for (int c = c0; c < c1; ++c) mine += ch_chunk_kept(selc, c, C, lim, extra);
  const int excl = ch_block_exclusive_sum(mine, tmp);
  const int total = ch_block_sum(mine, tmp);
  const int64_t orow = ((int64_t)h * a.Q + i) * a.k_max;
  int32_t* irow = a.idx + orow;
  float* nrow = a.newpos_k + orow;
  int pk = 0;
  {
    int r = excl;
    for (int c = c0; c < c1; ++c) {
      const int jend = min((c + 1) * C, lim);
      for (int j = c * C; j < jend; ++j) {
        if (!(selc[c] || j == extra)) continue;
        if (r < a.k_max) {
          irow[r] = j;
          nrow[r] = (float)r;
        }
        if (j == qp) a.newpos_q[(int64_t)h * a.Q + i] = (float)r;   // rank0[q_pos] (:477)
        if (a.passers_kept) pk += row[j] >= thr;
        ++r;
      }
    }
  }
  for (int s = min(total, a.k_max) + tid; s < a.k_max; s += CH_NT) {
    irow[s] = m;
    nrow[s] = 0.0f;
  }
  if (a.passers_kept) pk = ch_block_sum(pk, tmp);
  if (tid == 0) {
    a.kept_size[(int64_t)h * a.Q + i] = total;
    if (a.passers_kept) a.passers_kept[(int64_t)h * a.Q + i] = pk;
    if (a.usize) a.usize[(int64_t)h * a.Q + i] = npass;
  }
}

size_t chunk_select_lds_bytes(int n_keys, int C) {
  const size_t nC = ((size_t)n_keys + C - 1) / C;
  return nC * 4 + (nC + 3) / 4 * 4 + (256 + 16) * 4;
}

hipError_t launch_chunk_select(const ChunkSelectArgs& a, hipStream_t st) {
  const size_t lds = chunk_select_lds_bytes(a.N, a.C);
  hipError_t e = hipFuncSetAttribute((const void*)chunk_select_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(chunk_select_kernel, dim3(a.H * a.nt), dim3(CH_NT), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_chunk_decode_select(const ChunkDecodeArgs& a, hipStream_t st) {
  const size_t lds = chunk_select_lds_bytes(a.M, a.C);
  hipError_t e = hipFuncSetAttribute((const void*)chunk_decode_select_kernel,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(chunk_decode_select_kernel, dim3(a.H * a.Q), dim3(CH_NT), lds, st, a);
  return hipGetLastError();
}

}  // namespace sta
