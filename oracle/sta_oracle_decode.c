/*
 * sta_oracle_decode.c -- CPU restatement of the decode path: one query per call selects its own
 * key set over the cache and attends it.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it; the product library never links it and never falls back to it.
 *
 *   oracle_decode_scores     <- shared_selection_triton_exact_2.py:235-271 (_decode_select_kernel),
 *                               :505-525 (_decode_scores_kernel); torch twin :541-546
 *   oracle_decode_build_sets <- shared_selection_triton_exact_2.py:527-604 (_decode_build_sets)
 *   oracle_decode_attend     <- shared_selection_triton_exact_2.py:608-623 (_decode_attend_torch);
 *                               with causal != 0 the slot rule of Kernel C as
 *                               _decode_attend_kernelC runs it (:626-655, key <= q_pos); with
 *                               rope_scale 1 and the dense ranks of the per-query rule it is
 *                               shared_selection_triton_perquery.py:723-740 (_decode_attend_torch_pq)
 *                               and :743-778 (_decode_attend_kernelC_pq)
 *   oracle_decode_build_sets_pqs <- pqstream_kernel.py:695-797 (_decode_build_sets_pqs): every
 *                               passer and forced key, streamed positions over aligned blocks
 *   oracle_decode_build_sets_pq <- shared_selection_triton_perquery.py:651-720
 *                               (_decode_build_sets_pq): no top-pct cut, the k_max cap as forced +
 *                               the top-(k_max - n_forced) non-forced keys by score with an exact
 *                               budget, dense-rank positions
 *
 * A batch of Q queries shares one cache of M keys: query i sits at position q_pos0 + i and sees
 * the keys [0, m_i), m_i = M - (Q - 1 - i) -- the cache prefix K[:, :P + 1] that spi_forward's
 * per-token loop hands to each call (exact_2.py:743-745) when q_pos0 + Q == M.  With Q = 1 it is
 * one call of the reference on M keys at q_pos = q_pos0.
 *
 * fp32 semantics (build with -ffp-contract=off):
 *   query angle base fl(float(q_pos) * pos_scale), key angle base fl(float(j) * pos_scale)
 *   (exact_2.py:253, 264), then rope_row's fp32 rotation (exact_2.py:254-257, 265-268)
 *   score = fl(fl(dot over all D) * sm_scale), the dot accumulated in double and rounded once
 *   (exact_2.py:270)
 *   thr = fl(max - tau); keep = s >= thr (:549-550)
 *   budget_p = max(1, ceilf(fl(float(pct/100) * float(n_pass)))) (:561), the float32 tensor op
 *   rank0 / cpos / newpos as fp32 (:589-592)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "sta_oracle_common.h"

/* fl(fl(dot(a, b)) * sm_scale) with the dot over all D accumulated in double */
static inline float score_full(const float* a, const float* b, int D, float sm_scale) {
  double d = 0.0;
  for (int i = 0; i < D; ++i) d += (double)a[i] * (double)b[i];
  volatile float f = (float)d;
  return f * sm_scale;
}

/* scores (H, Q, M) fp32; entries j >= m_i of row (h, i) are set to NaN */
void oracle_decode_scores(const void* q, const void* k, int dtype, int H, int Hkv, int Q, int M, int D,
                          const float* inv_freq, float pos_scale, float rope_scale, float sm_scale,
                          int q_pos0, float* scores) {
  const int group = H / Hkv;
#pragma omp parallel
  {
    float* qr = (float*)malloc(sizeof(float) * (size_t)D);
    float* kr = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int hi = 0; hi < H * Q; ++hi) {
      const int h = hi / Q, i = hi % Q;
      const int hk = h / group;
      const int m = M - (Q - 1 - i);
      volatile float qbase = (float)(q_pos0 + i) * pos_scale;              /* exact_2.py:253 */
      rope_row(q, dtype, ((size_t)h * Q + i) * D, D, qbase, inv_freq, rope_scale, qr);
      float* srow = scores + ((size_t)h * Q + i) * M;
      for (int j = 0; j < M; ++j) {
        if (j >= m) {
          srow[j] = NAN;
          continue;
        }
        volatile float kbase = (float)j * pos_scale;                        /* exact_2.py:264 */
        rope_row(k, dtype, ((size_t)hk * M + j) * D, D, kbase, inv_freq, rope_scale, kr);
        srow[j] = score_full(qr, kr, D, sm_scale);                          /* exact_2.py:270 */
      }
    }
    free(qr);
    free(kr);
  }
}

static int cmp_desc(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}

/*
 * _decode_build_sets from given scores (H, Q, M).  Outputs per (h, i): idx (k_max) ascending
 * kept positions padded with the sentinel m_i, newpos_k (k_max) (0 at sentinels), newpos_q, and
 * set_size = |final set| before the truncation to k_max (not returned by the reference; the
 * count its idx sort truncates).
 */
void oracle_decode_build_sets(const float* scores, int H, int Q, int M, const float* tau, int q_pos0,
                              float pos_scale, int n_global, int n_local, int k_max, double pct_decode,
                              int32_t* idx, float* newpos_k, float* newpos_q, int32_t* set_size) {
#pragma omp parallel
  {
    float* sp = (float*)malloc(sizeof(float) * (size_t)M);
    uint8_t* fin = (uint8_t*)malloc((size_t)M);
    uint8_t* kp = (uint8_t*)malloc((size_t)M);
    uint8_t* forced = (uint8_t*)malloc((size_t)M);
    float* newpos = (float*)malloc(sizeof(float) * (size_t)M);
#pragma omp for schedule(dynamic, 1)
    for (int hi = 0; hi < H * Q; ++hi) {
      const int h = hi / Q, i = hi % Q;
      const int m = M - (Q - 1 - i);
      const int p = q_pos0 + i;
      const float* s = scores + ((size_t)h * Q + i) * M;
      /* exact max and threshold (exact_2.py:549-550) */
      float mx = -INFINITY;
      for (int j = 0; j < m; ++j) mx = s[j] > mx ? s[j] : mx;
      volatile float thr = mx - tau[h];
      /* forced: global, local window, self (:552-556) */
      const int g = n_global < m ? n_global : m;
      int lo = p - n_local + 1;
      if (lo < 0) lo = 0;
      int n_forced = 0;
      for (int j = 0; j < m; ++j) {
        forced[j] = (uint8_t)(j < g || (j >= lo && j <= p) || j == p);
        n_forced += forced[j];
      }
      /* top-pct_decode% of the passers by score (:559-567) */
      float cut_p = -INFINITY;
      int use_pct = pct_decode < 100.0;
      if (use_pct) {
        long n_pass = 0;
        for (int j = 0; j < m; ++j) n_pass += s[j] >= thr;
        volatile float frac = (float)(pct_decode / 100.0);
        volatile float prod = frac * (float)n_pass;
        float b = ceilf(prod);
        if (b < 1.0f) b = 1.0f;
        long budget = (long)b;
        for (int j = 0; j < m; ++j) sp[j] = s[j] >= thr ? s[j] : -INFINITY;
        qsort(sp, (size_t)m, sizeof(float), cmp_desc);
        long ci = budget - 1;
        if (ci < 0) ci = 0;
        if (ci > m - 1) ci = m - 1;
        cut_p = sp[ci];
      }
      int count = 0;
      for (int j = 0; j < m; ++j) {
        const int keep = s[j] >= thr && (!use_pct || s[j] >= cut_p);
        kp[j] = (uint8_t)(keep || forced[j]);                               /* :569 */
        count += kp[j];
      }
      /* cap by score over the non-forced keys (:571-585) */
      const int budget_c = k_max - n_forced;
      if (count > k_max) {
        for (int j = 0; j < m; ++j) sp[j] = (kp[j] && !forced[j]) ? s[j] : -INFINITY;
        qsort(sp, (size_t)m, sizeof(float), cmp_desc);
        int ci = budget_c - 1;
        if (ci < 0) ci = 0;
        if (ci > m - 1) ci = m - 1;
        const float cut_c = sp[ci];
        for (int j = 0; j < m; ++j) {
          const int nf = kp[j] && !forced[j];
          const int kept_nf = budget_c > 0 && nf && s[j] >= cut_c;
          fin[j] = (uint8_t)(forced[j] || kept_nf);
        }
      } else {
        memcpy(fin, kp, (size_t)m);
      }
      /* reposition: newpos = rank0 + cummax(cpos - rank0) over kept keys (:587-592) */
      int rank = -1, total = 0;
      float run = -INFINITY;
      for (int j = 0; j < m; ++j) {
        if (fin[j]) {
          rank += 1;
          volatile float cp = (float)j * pos_scale;
          volatile float cr = cp - (float)rank;
          run = cr > run ? cr : run;
        }
        volatile float np = (float)rank + run;
        newpos[j] = np;
        total += fin[j];
      }
      /* ascending kept positions, first k_max, sentinel m (:594-602) */
      int32_t* irow = idx + ((size_t)h * Q + i) * k_max;
      float* nrow = newpos_k + ((size_t)h * Q + i) * k_max;
      int r = 0;
      for (int j = 0; j < m && r < k_max; ++j)
        if (fin[j]) {
          irow[r] = j;
          nrow[r] = newpos[j];
          ++r;
        }
      for (; r < k_max; ++r) {
        irow[r] = m;
        nrow[r] = 0.0f;
      }
      newpos_q[(size_t)h * Q + i] = newpos[p];                              /* :603 */
      if (set_size) set_size[(size_t)h * Q + i] = total;
    }
    free(sp);
    free(fin);
    free(kp);
    free(forced);
    free(newpos);
  }
}

/*
 * Attend over the selected slots: out (H, Q, D) fp32 before the cast to the model dtype.
 * A slot is valid when idx < m_i (the sentinel test) and, with causal != 0, idx <= q_pos0 + i.
 * Softmax and the weighted sum in double; no valid slot gives zeros.
 */
void oracle_decode_attend(const void* q, const void* k, const void* v, int dtype, int H, int Hkv, int Q,
                          int M, int D, const float* inv_freq, float rope_scale, float sm_scale, int q_pos0,
                          int k_max, const int32_t* idx, const float* newpos_k, const float* newpos_q,
                          int causal, float* out) {
  const int group = H / Hkv;
#pragma omp parallel
  {
    float* qr = (float*)malloc(sizeof(float) * (size_t)D);
    float* kr = (float*)malloc(sizeof(float) * (size_t)D);
    float* sc = (float*)malloc(sizeof(float) * (size_t)k_max);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int hi = 0; hi < H * Q; ++hi) {
      const int h = hi / Q, i = hi % Q;
      const int hk = h / group;
      const int m = M - (Q - 1 - i);
      const int p = q_pos0 + i;
      const int32_t* irow = idx + ((size_t)h * Q + i) * k_max;
      const float* nrow = newpos_k + ((size_t)h * Q + i) * k_max;
      rope_row(q, dtype, ((size_t)h * Q + i) * D, D, newpos_q[(size_t)h * Q + i], inv_freq, rope_scale, qr);
      float mx = -INFINITY;
      for (int r = 0; r < k_max; ++r) {
        const int j = irow[r];
        sc[r] = -INFINITY;
        if (j < 0 || j >= m || (causal && j > p)) continue;
        rope_row(k, dtype, ((size_t)hk * M + j) * D, D, nrow[r], inv_freq, rope_scale, kr);
        sc[r] = score_full(qr, kr, D, sm_scale);
        mx = sc[r] > mx ? sc[r] : mx;
      }
      double l = 0.0;
      for (int d = 0; d < D; ++d) acc[d] = 0.0;
      if (mx > -INFINITY) {
        for (int r = 0; r < k_max; ++r) {
          if (sc[r] == -INFINITY) continue;
          const double w = exp((double)sc[r] - (double)mx);
          l += w;
          const int j = irow[r];
          for (int d = 0; d < D; ++d) acc[d] += w * (double)load_elem(v, dtype, ((size_t)hk * M + j) * D + d);
        }
      }
      float* orow = out + ((size_t)h * Q + i) * D;
      for (int d = 0; d < D; ++d) orow[d] = l > 0.0 ? (float)(acc[d] / l) : 0.0f;
    }
    free(qr);
    free(kr);
    free(sc);
    free(acc);
  }
}

/* (score, key) pairs in descending score, ties in ascending key order */
typedef struct {
  float s;
  int j;
} scored_key;

static int cmp_scored_desc(const void* a, const void* b) {
  const scored_key* x = (const scored_key*)a;
  const scored_key* y = (const scored_key*)b;
  if (x->s != y->s) return (x->s < y->s) - (x->s > y->s);
  return (x->j > y->j) - (x->j < y->j);
}

/*
 * _decode_build_sets_pq (shared_selection_triton_perquery.py:651-720) from given scores (H, Q, M),
 * batched like oracle_decode_build_sets (query i at q_pos0 + i over the keys [0, m_i)).
 *   thr = fl(max - tau); keep = s >= thr                                   (:676-677)
 *   forced = global [0, n_global) U local [q_pos - n_local + 1, q_pos] U self (:679-683)
 *   usize = |keep|, over = |keep U forced| > k_max                         (:686-688)
 *   over: forced U the top-(k_max - n_forced) non-forced kept keys by score (:690-701); the
 *   reference takes them with torch.topk, whose order among equal scores is unspecified: here
 *   equal scores at the cut are taken in ascending key order
 *   positions: dense ranks over the final set (rank0 = cumsum - 1), newpos_q = rank0[q_pos]
 *   (:703-719); idx ascending, first k_max, sentinel m_i, newpos_k 0 at sentinels.
 * set_size = |final set|; usize and overflow are the reference's measurement counters
 * (_ovf_accumulate(over, usize, "decode"), :688); each output pointer may be NULL.
 */
void oracle_decode_build_sets_pq(const float* scores, int H, int Q, int M, const float* tau, int q_pos0,
                                 int n_global, int n_local, int k_max, int32_t* idx, float* newpos_k,
                                 float* newpos_q, int32_t* set_size, int32_t* usize, uint8_t* overflow) {
#pragma omp parallel
  {
    scored_key* cand = (scored_key*)malloc(sizeof(scored_key) * (size_t)M);
    uint8_t* fin = (uint8_t*)malloc((size_t)M);
    uint8_t* forced = (uint8_t*)malloc((size_t)M);
    int32_t* rank0 = (int32_t*)malloc(sizeof(int32_t) * (size_t)M);
#pragma omp for schedule(dynamic, 1)
    for (int hi = 0; hi < H * Q; ++hi) {
      const int h = hi / Q, i = hi % Q;
      const int m = M - (Q - 1 - i);
      const int p = q_pos0 + i;
      const float* s = scores + ((size_t)h * Q + i) * M;
      float mx = -INFINITY;
      for (int j = 0; j < m; ++j) mx = s[j] > mx ? s[j] : mx;
      volatile float thr = mx - tau[h];
      const int g = n_global < m ? n_global : m;
      int lo = p - n_local + 1;
      if (lo < 0) lo = 0;
      int n_forced = 0, n_keep = 0, count = 0;
      for (int j = 0; j < m; ++j) {
        forced[j] = (uint8_t)(j < g || (j >= lo && j <= p) || j == p);
        const int keep = s[j] >= thr;
        n_forced += forced[j];
        n_keep += keep;
        fin[j] = (uint8_t)(keep || forced[j]);
        count += fin[j];
      }
      const int over = count > k_max;
      if (over) {
        const int budget = k_max - n_forced > 0 ? k_max - n_forced : 0;
        int nc = 0;
        for (int j = 0; j < m; ++j)
          if (fin[j] && !forced[j]) {
            cand[nc].s = s[j];
            cand[nc].j = j;
            ++nc;
          }
        qsort(cand, (size_t)nc, sizeof(scored_key), cmp_scored_desc);
        for (int j = 0; j < m; ++j) fin[j] = forced[j];
        for (int c = 0; c < nc && c < budget; ++c) fin[cand[c].j] = 1;
      }
      int rank = -1, total = 0;
      for (int j = 0; j < m; ++j) {
        if (fin[j]) rank += 1;
        rank0[j] = rank;
        total += fin[j];
      }
      int32_t* irow = idx + ((size_t)h * Q + i) * k_max;
      float* nrow = newpos_k + ((size_t)h * Q + i) * k_max;
      int r = 0;
      for (int j = 0; j < m && r < k_max; ++j)
        if (fin[j]) {
          irow[r] = j;
          nrow[r] = (float)rank0[j];
          ++r;
        }
      for (; r < k_max; ++r) {
        irow[r] = m;
        nrow[r] = 0.0f;
      }
      newpos_q[(size_t)h * Q + i] = (float)rank0[p];
      if (set_size) set_size[(size_t)h * Q + i] = total;
      if (usize) usize[(size_t)h * Q + i] = n_keep;
      if (overflow) overflow[(size_t)h * Q + i] = (uint8_t)over;
    }
    free(cand);
    free(fin);
    free(forced);
    free(rank0);
  }
}

/*
 * _decode_build_sets_pqs (pqstream_kernel.py:695-797) from given scores (H, Q, M), batched like
 * oracle_decode_build_sets (query i at q_pos0 + i over the keys [0, m_i)).
 *   keep = s >= fl(max - tau), plus the forced global / local / self keys; no cap   (:727-734)
 *   streamed positions (:736-749): blocks of block_n keys aligned at 0; c[b] = kept keys of block
 *   b; d[b] = kept keys of the blocks after b (nearer the query); a key j of block b sits at
 *   dist = d[b] + (min(q_pos, b block_n + block_n - 1) - j), newpos_k = -dist (fp32, -0 for the
 *   query itself), newpos_q = 0
 *   idx: every kept key ascending, then the sentinel m_i up to k_max slots (the reference's kbuf)
 * set_size (H, Q) = kept count; span (H, Q) fp32 = the largest dist among kept keys; skipped (H, Q)
 * = blocks without a kept key (the reference's decode counters, :786-791).  Pointers after
 * newpos_q may be NULL.
 */
void oracle_decode_build_sets_pqs(const float* scores, int H, int Q, int M, const float* tau, int q_pos0,
                                  int n_global, int n_local, int block_n, int k_max, int32_t* idx,
                                  float* newpos_k, float* newpos_q, int32_t* set_size, float* span,
                                  int32_t* skipped) {
#pragma omp parallel
  {
    uint8_t* kp = (uint8_t*)malloc((size_t)M);
    int32_t* cnt = (int32_t*)malloc(sizeof(int32_t) * ((size_t)M / (block_n > 0 ? block_n : 1) + 2));
#pragma omp for schedule(dynamic, 1)
    for (int hi = 0; hi < H * Q; ++hi) {
      const int h = hi / Q, i = hi % Q;
      const int m = M - (Q - 1 - i);
      const int p = q_pos0 + i;
      const float* s = scores + ((size_t)h * Q + i) * M;
      float mx = -INFINITY;
      for (int j = 0; j < m; ++j) mx = s[j] > mx ? s[j] : mx;
      volatile float thr = mx - tau[h];
      const int g = n_global < m ? n_global : m;
      int lo = p - n_local + 1;
      if (lo < 0) lo = 0;
      const int nblk = (m + block_n - 1) / block_n;
      for (int b = 0; b < nblk; ++b) cnt[b] = 0;
      int total = 0;
      for (int j = 0; j < m; ++j) {
        kp[j] = (uint8_t)(s[j] >= thr || j < g || (j >= lo && j <= p) || j == p);
        cnt[j / block_n] += kp[j];
        total += kp[j];
      }
      int32_t* irow = idx + ((size_t)h * Q + i) * k_max;
      float* nrow = newpos_k + ((size_t)h * Q + i) * k_max;
      int after = 0, r = total, skip = 0;
      float sp = 0.0f;
      /* descending blocks: d[b] = kept keys of the blocks after b */
      for (int b = nblk - 1; b >= 0; --b) {
        skip += cnt[b] == 0;
        const int hb = (b * block_n + block_n - 1) < p ? b * block_n + block_n - 1 : p;
        const int j1 = (b * block_n + block_n) < m ? b * block_n + block_n : m;
        for (int j = j1 - 1; j >= b * block_n; --j) {
          if (!kp[j]) continue;
          --r;
          volatile float dist = (float)after + (float)(hb - j);
          if (dist > sp) sp = dist;
          if (r < k_max) {
            irow[r] = j;
            nrow[r] = -dist;
          }
        }
        after += cnt[b];
      }
      for (int u = total; u < k_max; ++u) {
        irow[u] = m;
        nrow[u] = 0.0f;
      }
      newpos_q[(size_t)h * Q + i] = 0.0f;
      if (set_size) set_size[(size_t)h * Q + i] = total;
      if (span) span[(size_t)h * Q + i] = sp;
      if (skipped) skipped[(size_t)h * Q + i] = skip;
    }
    free(kp);
    free(cnt);
  }
}
