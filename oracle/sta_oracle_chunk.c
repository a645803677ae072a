/*
 * sta_oracle_chunk.c -- CPU restatement of the chunk-granular selection of
 * shared_selection_triton_chunked.py (TEST INFRASTRUCTURE ONLY: the checker of the HIP kernels,
 * never linked into or called by the product path).
 *
 * _build_sets_chunk (chunked.py:149-243), prefill, per (head, tile):
 *   - a key is a candidate when its votes are > 0; its rank value is its weighted vote
 *     (select_score margin / expmass) or its vote count (freq), zero for non-candidates (:168-171);
 *   - chunk c = keys [cC, cC + C) is valued by the sum of its keys' values, or their mean over
 *     its candidates ("mean", clamp 1) (:173-180);
 *   - forced chunks: the global chunks c < ceil(n_global / C) and the local chunks
 *     floor(max(0, r0 - n_local + 1) / C) .. floor(last_q / C); visible chunks: cC <= last_q;
 *     forced = (global | local) & visible, with r0 = q_pos_base + tT the tile's first query and
 *     last_q = r0 + T - 1.  The reference takes this mask from chunk_recall_core.forced_chunk_mask,
 *     a module absent from the reference tree; the rule here is the one its own golden,
 *     chunk_attention_torch, states (:368-376);
 *   - the top min(n_chunk, nC) visible non-forced chunks by value are selected (torch.topk,
 *     :188-192; equal values in ascending chunk order here, the order topk leaves unspecified),
 *     and the forced visible chunks are added (:193);
 *   - kept keys: the selected chunks' keys, trimmed to j <= min(last_q, N - 1) (:198-201);
 *     kept_size, usize = candidates j <= last_q (:202-203); dense ranks over the kept set
 *     (:211); idx ascending with sentinel N, newpos_k the ranks (0 at sentinels), newpos_q the
 *     rank-before-or-at each query position min(r0 + i, N - 1) (:228-231), mask -1 on valid slots
 *     (pooled attention, :225-226); passers_kept = candidates among the kept keys (the measure
 *     counter, :205-208).
 *
 * _decode_build_sets_chunk (chunked.py:411-489), one query at q_pos over M keys:
 *   keep = s >= m - tau with m the row max (:433-434); rank value 1 (freq) or exp(s - m) for kept
 *   keys (:437-438); chunk values as above over nC = ceil(M / C) chunks; forced = global chunks
 *   and chunks floor(max(0, q_pos - n_local + 1) / C) .. floor(q_pos / C), visible cC <= q_pos
 *   (:448-452); top min(n_chunk, nC) as above; kept = selected chunks' keys j <= q_pos, plus
 *   q_pos itself (:460-462); dense ranks; idx (sentinel M), newpos_k, newpos_q = rank of q_pos
 *   (:468-477).
 *
 * Sums run in key order in fp32; the chunk order statistic is exact.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  float v;
  int c;
} chunk_val;

static int cmp_chunk_desc(const void* a, const void* b) {
  const chunk_val* x = (const chunk_val*)a;
  const chunk_val* y = (const chunk_val*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return x->c - y->c;
}

/* sel[c] = 1 for the top n_take candidates (cand[c]) by val, ties in ascending c; returns the count */
static int top_chunks(const float* val, const uint8_t* cand, int nC, int n_take, uint8_t* sel, chunk_val* buf) {
  int n = 0;
  for (int c = 0; c < nC; ++c) {
    sel[c] = 0;
    if (cand[c]) {
      buf[n].v = val[c];
      buf[n].c = c;
      ++n;
    }
  }
  qsort(buf, (size_t)n, sizeof(chunk_val), cmp_chunk_desc);
  const int take = n < n_take ? n : n_take;
  for (int r = 0; r < take; ++r) sel[buf[r].c] = 1;
  return take;
}

/* Dense ranks over the kept keys [0, lim) of the kept chunks; writes idx / newpos_k (k_max slots,
 * sentinel `sentinel`) and returns kept_size.  kept_key(j) decides membership. */
static int compact(const uint8_t* keptc, int C, int lim, int extra_key, int k_max, int sentinel, int32_t* idx,
                   float* npk) {
  int r = 0;
  for (int j = 0; j < lim; ++j) {
    if (keptc[j / C] || j == extra_key) {
      if (r < k_max) {
        idx[r] = j;
        npk[r] = (float)r;
      }
      ++r;
    }
  }
  for (int s = r; s < k_max; ++s) {
    idx[s] = sentinel;
    npk[s] = 0.0f;
  }
  return r;
}

void oracle_build_sets_chunk(const int32_t* votes, const float* wvotes, int H, int nt, int N, int T, int k_max,
                             int C, int n_chunk, int q_pos_base, int n_global, int n_local, int weighted,
                             int mean, int32_t* idx, float* newpos_k, float* newpos_q, int32_t* mask,
                             int32_t* usize, int32_t* kept_size, int32_t* passers_kept) {
  const int nC = (N + C - 1) / C;
  const int n_take = n_chunk < nC ? n_chunk : nC;
  const int ng_c = (n_global + C - 1) / C;
#pragma omp parallel
  {
    float* val = (float*)malloc(sizeof(float) * (size_t)nC);
    uint8_t* cand = (uint8_t*)malloc((size_t)nC);
    uint8_t* sel = (uint8_t*)malloc((size_t)nC);
    chunk_val* buf = (chunk_val*)malloc(sizeof(chunk_val) * (size_t)nC);
#pragma omp for schedule(dynamic, 4)
    for (int x = 0; x < H * nt; ++x) {
      const int t = x % nt;
      const int32_t* vr = votes + (size_t)x * N;
      const float* wr = wvotes ? wvotes + (size_t)x * N : NULL;
      const int64_t r0 = (int64_t)q_pos_base + (int64_t)t * T;
      const int64_t last_q = r0 + T - 1;
      const int lim = (int)(last_q < N - 1 ? last_q + 1 : N);     /* keys j <= min(last_q, N - 1) */
      const int64_t lo_c = (r0 - n_local + 1 > 0 ? r0 - n_local + 1 : 0) / C, hi_c = last_q / C;
      int us = 0;
      for (int c = 0; c < nC; ++c) {
        float m = 0.0f;
        int cnt = 0;
        for (int j = c * C; j < (c + 1) * C && j < N; ++j) {
          if (vr[j] > 0) {
            m += weighted ? wr[j] : (float)vr[j];
            ++cnt;
          }
        }
        val[c] = mean ? m / (float)(cnt > 1 ? cnt : 1) : m;
        const int vis = (int64_t)c * C <= last_q;
        const int forced = vis && (c < ng_c || (c >= lo_c && c <= hi_c));
        cand[c] = (uint8_t)(vis && !forced);
      }
      for (int j = 0; j < N && j <= last_q; ++j) us += vr[j] > 0;
      top_chunks(val, cand, nC, n_take, sel, buf);
      for (int c = 0; c < nC; ++c) {
        const int vis = (int64_t)c * C <= last_q;
        const int forced = vis && (c < ng_c || (c >= lo_c && c <= hi_c));
        sel[c] = (uint8_t)(sel[c] || forced);
      }
      int32_t* ir = idx + (size_t)x * k_max;
      float* nr = newpos_k + (size_t)x * k_max;
      const int ks = compact(sel, C, lim, -1, k_max, N, ir, nr);
      int pk = 0;
      for (int j = 0; j < lim; ++j) pk += sel[j / C] && vr[j] > 0;
      for (int s = 0; s < k_max; ++s) mask[(size_t)x * k_max + s] = s < ks ? -1 : 0;
      /* rank0 at each query position: (kept keys <= qpos) - 1 */
      for (int i = 0; i < T; ++i) {
        int64_t qp = r0 + i;
        if (qp > N - 1) qp = N - 1;
        int cntk = 0;
        for (int j = 0; j <= qp && j < lim; ++j) cntk += sel[j / C];
        newpos_q[(size_t)x * T + i] = (float)(cntk - 1);
      }
      usize[x] = us;
      kept_size[x] = ks;
      if (passers_kept) passers_kept[x] = pk;
    }
    free(val);
    free(cand);
    free(sel);
    free(buf);
  }
}

/*
 * Decode: scores (H, Q, M) fp32; query i at q_pos0 + i sees the keys [0, M - (Q - 1 - i)) (the
 * batched decode contract: m_i keys, the chunk grid over them, sentinel m_i).
 */
void oracle_decode_build_sets_chunk(const float* scores, int H, int Q, int M, const float* tau, int q_pos0,
                                    int n_global, int n_local, int k_max, int C, int n_chunk, int weighted,
                                    int mean, int32_t* idx, float* newpos_k, float* newpos_q, int32_t* kept_size,
                                    int32_t* passers_kept) {
  const int ng_c = (n_global + C - 1) / C;
#pragma omp parallel
  {
    const int nCmax = (M + C - 1) / C;
    float* val = (float*)malloc(sizeof(float) * (size_t)nCmax);
    uint8_t* cand = (uint8_t*)malloc((size_t)nCmax);
    uint8_t* sel = (uint8_t*)malloc((size_t)nCmax);
    chunk_val* buf = (chunk_val*)malloc(sizeof(chunk_val) * (size_t)nCmax);
#pragma omp for schedule(dynamic, 4)
    for (int x = 0; x < H * Q; ++x) {
      const int h = x / Q, i = x % Q;
      const int m = M - (Q - 1 - i);
      const int qp = q_pos0 + i;
      const float* row = scores + (size_t)x * M;
      float mx = -INFINITY;
      for (int j = 0; j < m; ++j) mx = row[j] > mx ? row[j] : mx;
      const float thr = mx - tau[h];                                   /* fp32, :434 */
      const int nC = (m + C - 1) / C;
      const int n_take = n_chunk < nC ? n_chunk : nC;
      const int64_t lo_c = (qp - n_local + 1 > 0 ? qp - n_local + 1 : 0) / C, hi_c = qp / C;
      for (int c = 0; c < nC; ++c) {
        float s = 0.0f;
        int cnt = 0;
        for (int j = c * C; j < (c + 1) * C && j < m; ++j) {
          if (row[j] >= thr) {
            s += weighted ? expf(row[j] - mx) : 1.0f;
            ++cnt;
          }
        }
        val[c] = mean ? s / (float)(cnt > 1 ? cnt : 1) : s;
        const int vis = (int64_t)c * C <= qp;
        const int forced = vis && (c < ng_c || (c >= lo_c && c <= hi_c));
        cand[c] = (uint8_t)(vis && !forced);
      }
      top_chunks(val, cand, nC, n_take, sel, buf);
      for (int c = 0; c < nC; ++c) {
        const int vis = (int64_t)c * C <= qp;
        const int forced = vis && (c < ng_c || (c >= lo_c && c <= hi_c));
        sel[c] = (uint8_t)(sel[c] || forced);
      }
      const int lim = qp + 1 < m ? qp + 1 : m;
      int32_t* ir = idx + (size_t)x * k_max;
      float* nr = newpos_k + (size_t)x * k_max;
      const int ks = compact(sel, C, lim, qp, k_max, m, ir, nr);
      int rq = -1, pk = 0;
      for (int j = 0; j < lim; ++j) {
        const int kept = sel[j / C] || j == qp;
        rq += kept && j <= qp;
        pk += kept && row[j] >= thr;
      }
      newpos_q[x] = (float)rq;
      kept_size[x] = ks;
      if (passers_kept) passers_kept[x] = pk;
    }
    free(val);
    free(cand);
    free(sel);
    free(buf);
  }
}
