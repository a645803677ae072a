/*
 * sta_oracle.c -- CPU restatement of the exact-max shared-selection thresholded attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP product path is compared against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product
 * library never links it and never falls back to it.
 *
 * It follows the reference line by line (all citations are into the reference repository):
 *   oracle_select_vote  <- shared_selection_triton_exact_2.py:50-140   (Kernel A, WMODE 0/1/2)
 *   oracle_build_sets   <- shared_selection_triton_exact_2.py:277-426  (_build_sets, freq /
 *                          margin / expmass ranking)
 *   oracle_gather_attn  <- shared_selection_triton_exact_2.py:146-225  (Kernel C)
 * The same three functions serve the YaRN and hybrid files, whose kernels are identical and whose
 * entry points differ only in the (inv_freq, pos_scale, rope_scale) triples they pass
 * (shared_selection_triton_YaRN_exact.py:442-496, shared_selection_triton_hybrid_exact.py:450-510).
 *
 * fp32 semantics kept on purpose (build with -ffp-contract=off):
 *   angle = fl(fl(float(pos) * pos_scale) * inv_freq[i])          (exact_2.py:79, 95)
 *   c, s  = fl(cosf(angle) * rope_scale), fl(sinf(angle) * rope_scale)   (exact_2.py:80-81)
 *   r1 = fl(fl(x1*c) - fl(x2*s)),  r2 = fl(fl(x2*c) + fl(x1*s))  (exact_2.py:82-83)
 *   score = fl(fl(dot(r1q,r1k) + dot(r2q,r2k)) * sm_scale)        (exact_2.py:100, 118)
 * Each half dot is accumulated in double and rounded once, i.e. an fp32 dot without the
 * accumulation-order noise of any particular BLAS.
 *   budget = ceilf(fl((float)(p/100.0) * (float)U))                (exact_2.py:329, float32 tensor op)
 *   newpos = fl(rank0 + cummax(fl(cpos - rank0)))                  (exact_2.py:383-386)
 *
 * dtype codes: 0 = fp32, 1 = bf16 (uint16 storage), 2 = fp16 (uint16 storage).
 * Tensors are contiguous (H, N, D); K and V may have Hkv heads (kv head = h / (H / Hkv)), which
 * is what repeat_kv materialises in the reference (exact_2.py:708-710).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "sta_oracle_common.h"

void oracle_round_to_dtype(const float* in, void* out, size_t n, int dtype) {
  oracle_round_to_dtype_impl(in, out, n, dtype);
}

void oracle_to_f32(const void* in, float* out, size_t n, int dtype) { oracle_to_f32_impl(in, out, n, dtype); }

void oracle_rope_rotate(const void* x, int dtype, int rows, int D, const float* posf,
                        const float* inv_freq, float rope_scale, float* out) {
  for (int r = 0; r < rows; ++r)
    rope_row(x, dtype, (size_t)r * D, D, posf[r], inv_freq, rope_scale, out + (size_t)r * D);
}

/* ------------------------------------------------------------------------------------------- */
/* Kernel A: exact row max (pass 1) + keep/votes (pass 2)       exact_2.py:50-140             */
/* ------------------------------------------------------------------------------------------- */
/*
 * votes      (H, nt, N) int32, written for every key (0 where no query keeps it)
 * row_counts (H, N)     int32 or NULL: per-query kept count (includes the zero "phantom" keys
 *                       N..hi-1 that the reference's masked loads produce when q_pos_base > 0)
 * row_max    (H, N)     fp32 or NULL: the exact max m of each query (exact_2.py:88-103)
 * band       (H, nt, N) int32 or NULL: per key, # of the tile's queries whose score lies within
 *                       band_eps of that query's threshold m - tau (the parity tolerance band)
 * band_rows  (H, N)     int32 or NULL: per query, # of its causal keys inside that band
 * keep_bits  (H, N, N)  uint8 or NULL: keep(q, k) for every pair (small shapes only)
 * wvotes     (H, nt, N) fp32 or NULL, written for wmode 1 / 2 (WMODE, exact_2.py:126-138):
 *                       wmode 1 (margin):  sum over the tile's keeping rows of fl(s - fl(m - tau))
 *                       wmode 2 (expmass): sum over the tile's keeping rows of exp(fl(s - m))
 *                       The reference sums a tile's rows in fp32 in its reduction tree's order;
 *                       here the sum is accumulated in double and rounded once (a few ulps apart).
 */
void oracle_select_vote(const void* q, const void* k, int dtype, int H, int Hkv, int N, int D,
                        const float* tau, const float* inv_freq, float pos_scale, float rope_scale,
                        float sm_scale, int tile, int q_pos_base, int32_t* votes,
                        int32_t* row_counts, float* row_max, int32_t* band, int32_t* band_rows,
                        float band_eps, uint8_t* keep_bits, int wmode, float* wvotes) {
  const int T = tile;
  const int nt = (N + T - 1) / T;
  const int group = H / Hkv;
  const int kmax_key = q_pos_base + nt * T; /* largest hi over all tiles */
  memset(votes, 0, sizeof(int32_t) * (size_t)H * nt * N);
  if (row_counts) memset(row_counts, 0, sizeof(int32_t) * (size_t)H * N);
  if (band) memset(band, 0, sizeof(int32_t) * (size_t)H * nt * N);
  if (band_rows) memset(band_rows, 0, sizeof(int32_t) * (size_t)H * N);
  if (keep_bits) memset(keep_bits, 0, (size_t)H * N * N);
  if (wvotes) memset(wvotes, 0, sizeof(float) * (size_t)H * nt * N);

  /* rotated K per kv head (keys >= N are the zero rows the reference's masked loads produce) */
  float* krot = (float*)malloc(sizeof(float) * (size_t)Hkv * kmax_key * D);
  for (int hk = 0; hk < Hkv; ++hk) {
    for (int j = 0; j < kmax_key; ++j) {
      float* dst = krot + ((size_t)hk * kmax_key + j) * D;
      if (j < N) {
        volatile float cp = (float)j * pos_scale;
        rope_row(k, dtype, ((size_t)hk * N + j) * D, D, cp, inv_freq, rope_scale, dst);
      } else {
        memset(dst, 0, sizeof(float) * D);
      }
    }
  }

#pragma omp parallel
  {
    float* qr = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* sc = (float*)malloc(sizeof(float) * (size_t)T * kmax_key);
    double* wacc = (double*)malloc(sizeof(double) * (size_t)kmax_key);
#pragma omp for schedule(dynamic, 1)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const int hk = h / group;
      const int hi = q_pos_base + (t + 1) * T; /* exact_2.py:85 */
      const float tau_h = tau[h];
      for (int j = 0; j < hi; ++j) wacc[j] = 0.0;
      for (int r = 0; r < T; ++r) {
        const int row = t * T + r;
        if (row >= N) continue;
        volatile float cp = (float)(q_pos_base + row) * pos_scale; /* exact_2.py:79 */
        rope_row(q, dtype, ((size_t)h * N + row) * D, D, cp, inv_freq, rope_scale, qr + (size_t)r * D);
      }
      for (int r = 0; r < T; ++r) {
        const int row = t * T + r;
        if (row >= N) continue; /* padded rows never vote (exact_2.py:121) */
        const int qpos = q_pos_base + row;
        float* srow = sc + (size_t)r * kmax_key;
        float m = -INFINITY;
        for (int j = 0; j < hi; ++j) { /* pass 1, exact_2.py:89-103 */
          if (qpos < j) { srow[j] = -INFINITY; continue; }
          const float s = score_of(qr + (size_t)r * D, krot + ((size_t)hk * kmax_key + j) * D, D, sm_scale);
          srow[j] = s;
          if (s > m) m = s;
        }
        if (row_max) row_max[(size_t)h * N + row] = m;
        volatile float thr = m - tau_h;
        int cnt = 0, nband = 0;
        for (int j = 0; j < hi; ++j) { /* pass 2, exact_2.py:107-125 */
          if (qpos < j) continue;
          const float s = srow[j];
          const int keep = s >= thr;
          if (fabsf(s - thr) < band_eps) {
            nband += 1;
            if (band && j < N) band[((size_t)h * nt + t) * N + j] += 1;
          }
          if (!keep) continue;
          cnt += 1;
          if (j < N) {
            /* different rows of one tile touch the same key, but one tile belongs to one thread */
            votes[((size_t)h * nt + t) * N + j] += 1;
            if (keep_bits) keep_bits[((size_t)h * N + row) * N + j] = 1;
            if (wmode == 1) { /* exact_2.py:129-131: qk - (m - tau) */
              volatile float c = s - thr;
              wacc[j] += (double)c;
            } else if (wmode == 2) { /* exact_2.py:134-136: exp(qk - m) */
              volatile float dl = s - m;
              wacc[j] += (double)expf(dl);
            }
          }
        }
        if (row_counts) row_counts[(size_t)h * N + row] = cnt;
        if (band_rows) band_rows[(size_t)h * N + row] = nband;
      }
      if (wvotes && wmode > 0)
        for (int j = 0; j < hi && j < N; ++j) wvotes[((size_t)h * nt + t) * N + j] = (float)wacc[j];
    }
    free(qr);
    free(sc);
    free(wacc);
  }
  free(krot);
}

/* ------------------------------------------------------------------------------------------- */
/* _build_sets                                                   exact_2.py:277-426            */
/* ------------------------------------------------------------------------------------------- */
static int cmp_desc_f(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}

/* budget = ceil(fl(float(p/100.0) * float(U))).clamp(min=1) in float32 (exact_2.py:329) */
static long budget_of(int p, long usize) {
  volatile float frac = (float)((double)p / 100.0);
  volatile float prod = frac * (float)usize;
  float b = ceilf(prod);
  if (b < 1.0f) b = 1.0f;
  return (long)b;
}

/*
 * votes: (H, nt, N) int32.  Outputs as in exact_2.py:418-426:
 *   idx (H,nt,k_max) int32 ascending, sentinel N; newpos_k (H,nt,k_max) fp32 (0 at sentinels);
 *   newpos_q (H,nt,T) fp32; shared_size, kept_size, chosen (H,nt) int32;
 *   orig_overflow, overflow20 (H,nt) uint8; kpct_meas (H,nt) int32.
 * start_pct = max(0, int(round(pct))) is computed by the caller (Python round semantics).
 * wvotes (H, nt, N) fp32 or NULL: with it the ranking metric is the weighted score with frequency
 * as an epsilon tiebreak, rank = fl(wvotes + fl(1e-6 * votes)) (exact_2.py:299-302); the union
 * size and budgets stay frequency-based (exact_2.py:296).  NULL ranks by votes (freq).
 * cut (H, nt) fp32 or NULL: the rank-value threshold v_cut of the step whose sets were kept
 * (exact_2.py:330, 348-350), +inf where only the forced keys are kept (pct 0).  Not a reference
 * output: the parity tests use it to tell a key moved by a shifted cut from a flipped key.
 */
void oracle_build_sets(const int32_t* votes, int H, int nt, int N, float pos_scale, int n_global,
                       int n_local, int start_pct, int T, int k_max, int q_pos_base, int measure,
                       int32_t* idx, float* newpos_k, float* newpos_q, int32_t* shared_size,
                       int32_t* kept_size, int32_t* chosen, uint8_t* orig_overflow,
                       int32_t* kpct_meas, uint8_t* overflow20, const float* wvotes, float* cut) {
  /* pct_steps = [start] + [c for c in (25, 20) if c < start]            (exact_2.py:309-310) */
  int steps[3], nsteps = 0;
  steps[nsteps++] = start_pct;
  if (25 < start_pct) steps[nsteps++] = 25;
  if (20 < start_pct) steps[nsteps++] = 20;
  int maxp = steps[0];
  for (int i = 1; i < nsteps; ++i) if (steps[i] > maxp) maxp = steps[i];
  /* K_ord = max(1, min(N, ceil(max_pct / 100.0 * N)))  in double      (exact_2.py:320) */
  long K_ord = (long)ceil((double)maxp / 100.0 * (double)N);
  if (K_ord > N) K_ord = N;
  if (K_ord < 1) K_ord = 1;
  const int floor_pct = steps[nsteps - 1];

#pragma omp parallel
  {
    float* sv = (float*)malloc(sizeof(float) * (size_t)N);
    float* rv = (float*)malloc(sizeof(float) * (size_t)N);
    uint8_t* forced = (uint8_t*)malloc((size_t)N);
    uint8_t* kept = (uint8_t*)malloc((size_t)N);
    uint8_t* shared = (uint8_t*)malloc((size_t)N);
    float* newpos_all = (float*)malloc(sizeof(float) * (size_t)N);
#pragma omp for schedule(dynamic, 4)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const int32_t* vrow = votes + ((size_t)h * nt + t) * N;
      const long tstart = (long)q_pos_base + (long)t * T; /* exact_2.py:291 */
      const long lo = tstart - n_local + 1, hi_l = tstart + T - 1;
      long usize = 0;
      const float* wrow = wvotes ? wvotes + ((size_t)h * nt + t) * N : NULL;
      for (int j = 0; j < N; ++j) {
        forced[j] = (j < n_global) || (j >= lo && j <= hi_l); /* exact_2.py:290-293, 303 */
        if (wrow) { /* exact_2.py:302: rank_val = wvotes.float() + 1e-6 * vf, in float32 */
          volatile float tb = 1e-6f * (float)vrow[j];
          volatile float r = wrow[j] + tb;
          rv[j] = r;
        } else {
          rv[j] = (float)vrow[j]; /* exact_2.py:300 */
        }
        sv[j] = rv[j];
        if (vrow[j] > 0) usize += 1; /* exact_2.py:296 */
      }
      /* topk(K_ord, sorted) == first K_ord entries of a descending sort (exact_2.py:321) */
      qsort(sv, (size_t)N, sizeof(float), cmp_desc_f);

      int resolved = 0, ch = 0;
      int oflow = 0;
      float cut_final = 0.0f; /* threshold of the chosen (or last tried) step */
      int use_forced_only = 0;
      for (int si = 0; si < nsteps; ++si) { /* exact_2.py:328-342 */
        const int p = steps[si];
        const long budget = budget_of(p, usize);
        long bi = budget - 1;
        if (bi < 0) bi = 0;
        if (bi > K_ord - 1) bi = K_ord - 1;
        const float v_cut = sv[bi]; /* exact_2.py:330 */
        long size = 0;
        for (int j = 0; j < N; ++j) size += (rv[j] >= v_cut) || forced[j];
        if (p == start_pct) oflow = size > k_max; /* exact_2.py:333-334 */
        if (!resolved) {
          /* unresolved tiles keep the last step's sets (exact_2.py:347-350) */
          cut_final = v_cut;
          if (size <= k_max) {
            resolved = 1;
            ch = p;
          }
        }
      }
      if (start_pct == 0) { /* exact_2.py:343-346: the pct=0 special case */
        long nf = 0;
        for (int j = 0; j < N; ++j) nf += forced[j];
        oflow = nf > k_max;
        if (!resolved) use_forced_only = 1;
      }
      const int ovf20 = oflow && !resolved; /* exact_2.py:354 */
      int kmeas = ch;                       /* exact_2.py:355 */
      if (measure && !resolved) {           /* exact_2.py:357-371 */
        for (int p = floor_pct - 1; p > 0; --p) {
          const long budget = budget_of(p, usize);
          long bi = budget - 1;
          if (bi < 0) bi = 0;
          if (bi > K_ord - 1) bi = K_ord - 1;
          const float v_cut = sv[bi];
          long size = 0;
          for (int j = 0; j < N; ++j) size += (rv[j] >= v_cut) || forced[j];
          if (size <= k_max) {
            kmeas = p;
            break;
          }
        }
      }

      long nshared = 0, nkept = 0;
      for (int j = 0; j < N; ++j) {
        shared[j] = use_forced_only ? 0 : (rv[j] >= cut_final);
        kept[j] = shared[j] || forced[j];
        nshared += shared[j];
        nkept += kept[j];
      }

      /* positions: newpos = rank0 + cummax(where(kept, cpos - rank0, -inf))  exact_2.py:383-386 */
      long rank = -1;
      float run = -INFINITY;
      for (int j = 0; j < N; ++j) {
        if (kept[j]) rank += 1;
        const float r0 = (float)rank;
        if (kept[j]) {
          volatile float cp = (float)j * pos_scale;
          volatile float d = cp - r0;
          if (d > run) run = d;
        }
        volatile float np = r0 + run;
        newpos_all[j] = np;
      }

      /* compaction: slots rank0 < k_max, ascending positions, sentinel N  exact_2.py:401-408 */
      int32_t* irow = idx + ((size_t)h * nt + t) * k_max;
      float* nkrow = newpos_k + ((size_t)h * nt + t) * k_max;
      for (int s = 0; s < k_max; ++s) {
        irow[s] = N;
        nkrow[s] = 0.0f;
      }
      long slot = 0;
      for (int j = 0; j < N && slot < k_max; ++j) {
        if (!kept[j]) continue;
        irow[slot] = j;
        nkrow[slot] = newpos_all[j];
        slot += 1;
      }
      /* newpos_q: gather at clamp(qpos, N-1)                                exact_2.py:410-412 */
      float* nqrow = newpos_q + ((size_t)h * nt + t) * T;
      for (int i = 0; i < T; ++i) {
        long qp = tstart + i;
        if (qp > N - 1) qp = N - 1;
        nqrow[i] = newpos_all[qp];
      }
      const size_t o = (size_t)h * nt + t;
      shared_size[o] = (int32_t)nshared;
      kept_size[o] = (int32_t)nkept;
      chosen[o] = ch;
      orig_overflow[o] = (uint8_t)oflow;
      overflow20[o] = (uint8_t)ovf20;
      kpct_meas[o] = kmeas;
      if (cut) cut[o] = use_forced_only ? INFINITY : cut_final;
    }
    free(sv);
    free(rv);
    free(forced);
    free(kept);
    free(shared);
    free(newpos_all);
  }
}

/* ------------------------------------------------------------------------------------------- */
/* Kernel C: gather + repositioned attention                    exact_2.py:146-225             */
/* ------------------------------------------------------------------------------------------- */
/*
 * out: (H, N, D) fp32 = the accumulator before the final cast to the input dtype
 * (exact_2.py:223-225); rows >= N are not written.  block_k is the slot block of the online
 * softmax (the reference's BLOCK_K); it matters only through the cast of P to the input dtype.
 */
static void gather_core(const void* q, const void* k, const void* v, int dtype, int H, int Hkv,
                        int N, int D, const float* inv_freq, float rope_scale, float sm_scale,
                        int tile, int k_max, int block_k, int q_pos_base, const int32_t* idx,
                        const float* newpos_k, const float* newpos_q, const int32_t* mask,
                        float* out) {
  const int T = tile;
  const int nt = (N + T - 1) / T;
  const int group = H / Hkv;
#pragma omp parallel
  {
    float* qr = (float*)malloc(sizeof(float) * (size_t)D);
    float* kr = (float*)malloc(sizeof(float) * (size_t)k_max * D); /* rotated slots of one tile */
    float* sblk = (float*)malloc(sizeof(float) * (size_t)block_k);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    double* dotv = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const int hk = h / group;
      const int32_t* irow = idx + ((size_t)h * nt + t) * k_max;
      const float* nkrow = newpos_k + ((size_t)h * nt + t) * k_max;
      const float* nqrow = newpos_q + ((size_t)h * nt + t) * T;
      /* K rotated at newpos_k once per slot (exact_2.py:199-207); shared by the tile's rows */
      for (int s = 0; s < k_max; ++s) {
        const int j = irow[s];
        if (j < N) rope_row(k, dtype, ((size_t)hk * N + j) * D, D, nkrow[s], inv_freq, rope_scale,
                            kr + (size_t)s * D);
      }
      for (int r = 0; r < T; ++r) {
        const int row = t * T + r;
        if (row >= N) continue;
        const long qpos = (long)q_pos_base + row;
        rope_row(q, dtype, ((size_t)h * N + row) * D, D, nqrow[r], inv_freq, rope_scale, qr);
        float mR = -INFINITY, l = 0.0f;
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int s0 = 0; s0 < k_max; s0 += block_k) { /* exact_2.py:191-221 */
          const int nb = (k_max - s0) < block_k ? (k_max - s0) : block_k;
          float bmax = -INFINITY;
          for (int b = 0; b < block_k; ++b) {
            sblk[b] = -INFINITY;
            if (b >= nb) continue; /* slots >= K_MAX load the sentinel (exact_2.py:193-195) */
            const int j = irow[s0 + b];
            if (j >= N) continue;           /* padding slot */
            if (qpos < j) continue;         /* causal on ORIGINAL positions (exact_2.py:210) */
            /* per-query bit test of the PQ Union gather (perquery.py:296-297) */
            if (mask && !(((uint32_t)mask[((size_t)h * nt + t) * k_max + s0 + b] >> r) & 1u)) continue;
            const float s = score_of(qr, kr + (size_t)(s0 + b) * D, D, sm_scale);
            sblk[b] = s;
            if (s > bmax) bmax = s;
          }
          const float mnew = mR > bmax ? mR : bmax;           /* exact_2.py:213 */
          const float msafe = (mnew == -INFINITY) ? 0.0f : mnew; /* :214 */
          volatile float alpha = expf(mR - msafe);           /* :216 */
          double psum = 0.0;
          for (int d = 0; d < D; ++d) dotv[d] = 0.0;
          for (int b = 0; b < block_k; ++b) {
            volatile float dlt = sblk[b] - msafe;
            const float p = expf(dlt); /* :215 */
            psum += p;
            if (p == 0.0f) continue;
            const float pc = round_to_dtype(p, dtype); /* p.to(vv.dtype), :220 */
            const int j = irow[s0 + b];
            for (int d = 0; d < D; ++d)
              dotv[d] += (double)pc * (double)load_elem(v, dtype, ((size_t)hk * N + j) * D + d);
          }
          volatile float la = l * alpha;
          l = la + (float)psum; /* :217 */
          for (int d = 0; d < D; ++d) {
            volatile float aa = acc[d] * alpha;
            acc[d] = aa + (float)dotv[d]; /* :220 */
          }
          mR = mnew;
        }
        float* orow = out + ((size_t)h * N + row) * D;
        for (int d = 0; d < D; ++d) orow[d] = acc[d] / l; /* :223 */
      }
    }
    free(qr);
    free(kr);
    free(sblk);
    free(acc);
    free(dotv);
  }
}

void oracle_gather_attn(const void* q, const void* k, const void* v, int dtype, int H, int Hkv,
                        int N, int D, const float* inv_freq, float rope_scale, float sm_scale,
                        int tile, int k_max, int block_k, int q_pos_base, const int32_t* idx,
                        const float* newpos_k, const float* newpos_q, float* out) {
  gather_core(q, k, v, dtype, H, Hkv, N, D, inv_freq, rope_scale, sm_scale, tile, k_max, block_k,
              q_pos_base, idx, newpos_k, newpos_q, NULL, out);
}

/* Kernel C of the PQ Union file: the same gather with the per-slot query bitmask
 * (shared_selection_triton_perquery.py:226-312); mask (H, nt, k_max) int32, bit r = row r. */
void oracle_gather_attn_mask(const void* q, const void* k, const void* v, int dtype, int H, int Hkv,
                             int N, int D, const float* inv_freq, float rope_scale, float sm_scale,
                             int tile, int k_max, int block_k, int q_pos_base, const int32_t* idx,
                             const float* newpos_k, const float* newpos_q, const int32_t* mask,
                             float* out) {
  gather_core(q, k, v, dtype, H, Hkv, N, D, inv_freq, rope_scale, sm_scale, tile, k_max, block_k,
              q_pos_base, idx, newpos_k, newpos_q, mask, out);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
