/*
 * sta_oracle_pq.c -- CPU restatement of the two per-query variants: PQ Union and PQ Stream.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP product path is compared against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product
 * library never links it and never falls back to it.
 *
 * It follows the reference line by line (all citations are into the reference repository):
 *   oracle_select_bits    <- shared_selection_triton_perquery.py:119-218  (_select_bits_kernel)
 *   oracle_build_sets_pq  <- shared_selection_triton_perquery.py:363-453  (_build_sets_pq)
 *   oracle_gather_attn_mask (in sta_oracle.c) <- perquery.py:226-312      (_gather_attn_pq_kernel)
 *   oracle_pqstream       <- pqstream_kernel.py:174-368                    (_pqstream_kernel)
 *
 * fp32 rounding points are those of sta_oracle.c (build with -ffp-contract=off).  The weighted
 * votes (margin / expmass) are sums over a tile's rows; the reference sums them in fp32 in the
 * order of its reduction tree, here they are accumulated in double and rounded once, so they
 * agree with the reference to a few fp32 ulps, not bit for bit.
 *
 * Ties in the overflow ranking.  The reference keeps the top-budget candidates by torch.topk
 * (perquery.py:404-406), whose choice among equal rank values is unspecified.  Here equal rank
 * values are taken in ascending key order; tests compare modulo the tied keys at the cut.
 */
#include "sta_oracle_common.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------- */
/* Kernel A of PQ Union: keep + votes + packed per-query bits + weighted votes                 */
/* ------------------------------------------------------------------------------------------- */
/*
 * votes      (H, nt, N) int32     # of the tile's queries keeping key j           (perquery.py:197)
 * bits       (H, nt, N) int32     bit i = keep(row i of the tile, key j)          (:200-203)
 * wvotes     (H, nt, N) fp32/NULL wmode 1: sum of fl(s - fl(m - tau)) over keeping rows (:208-212)
 *                                 wmode 2: sum of exp(fl(s - m)) over keeping rows      (:213-217)
 * row_counts (H, N) int32/NULL, row_max (H, N) fp32/NULL, band (H, nt, N) int32/NULL and
 * band_rows (H, N) int32/NULL as in oracle_select_vote.
 * tile <= 32 (the reference asserts tile == 32 at its entry point, perquery.py:470).
 */
void oracle_select_bits(const void* q, const void* k, int dtype, int H, int Hkv, int N, int D,
                        const float* tau, const float* inv_freq, float pos_scale, float rope_scale,
                        float sm_scale, int tile, int q_pos_base, int wmode, int32_t* votes,
                        int32_t* bits, float* wvotes, int32_t* row_counts, float* row_max,
                        int32_t* band, int32_t* band_rows, float band_eps) {
  const int T = tile;
  const int nt = (N + T - 1) / T;
  const int group = H / Hkv;
  const int kmax_key = q_pos_base + nt * T;
  memset(votes, 0, sizeof(int32_t) * (size_t)H * nt * N);
  memset(bits, 0, sizeof(int32_t) * (size_t)H * nt * N);
  if (wvotes) memset(wvotes, 0, sizeof(float) * (size_t)H * nt * N);
  if (row_counts) memset(row_counts, 0, sizeof(int32_t) * (size_t)H * N);
  if (band) memset(band, 0, sizeof(int32_t) * (size_t)H * nt * N);
  if (band_rows) memset(band_rows, 0, sizeof(int32_t) * (size_t)H * N);

  float* krot = (float*)malloc(sizeof(float) * (size_t)Hkv * kmax_key * D);
  for (int hk = 0; hk < Hkv; ++hk)
    for (int j = 0; j < kmax_key; ++j) {
      float* dst = krot + ((size_t)hk * kmax_key + j) * D;
      if (j < N) {
        volatile float cp = (float)j * pos_scale;
        rope_row(k, dtype, ((size_t)hk * N + j) * D, D, cp, inv_freq, rope_scale, dst);
      } else {
        memset(dst, 0, sizeof(float) * D);
      }
    }

#pragma omp parallel
  {
    float* qr = (float*)malloc(sizeof(float) * (size_t)D);
    float* srow = (float*)malloc(sizeof(float) * (size_t)kmax_key);
    double* wacc = (double*)malloc(sizeof(double) * (size_t)kmax_key);
#pragma omp for schedule(dynamic, 1)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const int hk = h / group;
      const int hi = q_pos_base + (t + 1) * T; /* perquery.py:161 */
      const float tau_h = tau[h];
      for (int j = 0; j < hi; ++j) wacc[j] = 0.0;
      for (int r = 0; r < T; ++r) {
        const int row = t * T + r;
        if (row >= N) continue; /* padded rows never vote (perquery.py:195) */
        const int qpos = q_pos_base + row;
        volatile float cp = (float)qpos * pos_scale;
        rope_row(q, dtype, ((size_t)h * N + row) * D, D, cp, inv_freq, rope_scale, qr);
        float m = -INFINITY;
        for (int j = 0; j < hi; ++j) { /* pass 1, perquery.py:164-179 */
          if (qpos < j) { srow[j] = -INFINITY; continue; }
          const float s = score_of(qr, krot + ((size_t)hk * kmax_key + j) * D, D, sm_scale);
          srow[j] = s;
          if (s > m) m = s;
        }
        if (row_max) row_max[(size_t)h * N + row] = m;
        volatile float thr = m - tau_h;
        int cnt = 0, nband = 0;
        for (int j = 0; j < hi; ++j) { /* pass 2, perquery.py:181-217 */
          if (qpos < j) continue;
          const float s = srow[j];
          if (fabsf(s - thr) < band_eps) {
            nband += 1;
            if (band && j < N) band[((size_t)h * nt + t) * N + j] += 1;
          }
          if (!(s >= thr)) continue;
          cnt += 1;
          if (j >= N) continue;
          const size_t o = ((size_t)h * nt + t) * N + j;
          votes[o] += 1;
          bits[o] = (int32_t)((uint32_t)bits[o] | (1u << r));
          if (wmode == 1) {
            volatile float c = s - thr;
            wacc[j] += (double)c;
          } else if (wmode == 2) {
            volatile float dl = s - m;
            wacc[j] += (double)expf(dl);
          }
        }
        if (row_counts) row_counts[(size_t)h * N + row] = cnt;
        if (band_rows) band_rows[(size_t)h * N + row] = nband;
      }
      if (wvotes && wmode > 0)
        for (int j = 0; j < hi && j < N; ++j) wvotes[((size_t)h * nt + t) * N + j] = (float)wacc[j];
    }
    free(qr);
    free(srow);
    free(wacc);
  }
  free(krot);
}

/* ------------------------------------------------------------------------------------------- */
/* _build_sets_pq                                                 perquery.py:363-453           */
/* ------------------------------------------------------------------------------------------- */
typedef struct { float v; int j; } rank_item;

static int cmp_rank_desc(const void* a, const void* b) {
  const rank_item* x = (const rank_item*)a;
  const rank_item* y = (const rank_item*)b;
  if (x->v != y->v) return (x->v < y->v) - (x->v > y->v);
  return (x->j > y->j) - (x->j < y->j); /* equal values: ascending key */
}

/*
 * votes, bits (H, nt, N) int32; wvotes (H, nt, N) fp32 or NULL; rank_mode 0 = freq (rank by
 * votes), otherwise rank by fl(wvotes + fl(1e-6 * votes)) (perquery.py:394-397).
 * Outputs as perquery.py:446-453: idx (H,nt,k_max) int32 ascending, sentinel N; newpos_k
 * (H,nt,k_max) fp32 dense ranks (0 at sentinels); newpos_q (H,nt,T) fp32; mask (H,nt,k_max)
 * int32 (bits at idx, forced -> -1, sentinels -> 0); usize, kept_size (H,nt) int32; overflow
 * (H,nt) uint8.
 */
void oracle_build_sets_pq(const int32_t* votes, const int32_t* bits, const float* wvotes, int H,
                          int nt, int N, int n_global, int n_local, int T, int k_max,
                          int q_pos_base, int rank_mode, int32_t* idx, float* newpos_k,
                          float* newpos_q, int32_t* mask, int32_t* usize, int32_t* kept_size,
                          uint8_t* overflow) {
#pragma omp parallel
  {
    uint8_t* forced = (uint8_t*)malloc((size_t)N);
    uint8_t* kept = (uint8_t*)malloc((size_t)N);
    float* rank0 = (float*)malloc(sizeof(float) * (size_t)N);
    rank_item* cand = (rank_item*)malloc(sizeof(rank_item) * (size_t)N);
#pragma omp for schedule(dynamic, 4)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const size_t row = ((size_t)h * nt + t) * N;
      const long tstart = (long)q_pos_base + (long)t * T;  /* perquery.py:377 */
      const long lo = tstart - n_local + 1, hi = tstart + T - 1;
      long nu = 0, nfull = 0, nforced = 0;
      for (int j = 0; j < N; ++j) {
        forced[j] = (j < n_global) || (j >= lo && j <= hi); /* perquery.py:376-381 */
        const int u = votes[row + j] > 0;                     /* :383 */
        nu += u;
        kept[j] = u || forced[j];                             /* :385 */
        nfull += kept[j];
        nforced += forced[j];
      }
      const int ovf = nfull > k_max;                          /* :386 */
      if (ovf) {                                              /* :393-410 */
        long budget = (long)k_max - nforced;
        if (budget < 0) budget = 0;
        int nc = 0;
        for (int j = 0; j < N; ++j) {
          if (!(votes[row + j] > 0) || forced[j]) continue;   /* cand = union & ~forced */
          float rv;
          if (rank_mode == 0 || !wvotes) {
            rv = (float)votes[row + j];
          } else {
            volatile float tb = 1e-6f * (float)votes[row + j];
            volatile float s = wvotes[row + j] + tb;
            rv = s;
          }
          cand[nc].v = rv;
          cand[nc].j = j;
          nc += 1;
        }
        qsort(cand, (size_t)nc, sizeof(rank_item), cmp_rank_desc);
        for (int j = 0; j < N; ++j) kept[j] = forced[j];
        for (int c = 0; c < nc && c < budget; ++c) kept[cand[c].j] = 1;
      }
      long rank = -1, nk = 0;
      for (int j = 0; j < N; ++j) { /* rank0 = cumsum(kept) - 1   perquery.py:414 */
        if (kept[j]) { rank += 1; nk += 1; }
        rank0[j] = (float)rank;
      }
      int32_t* irow = idx + ((size_t)h * nt + t) * k_max;
      float* nkrow = newpos_k + ((size_t)h * nt + t) * k_max;
      int32_t* mrow = mask + ((size_t)h * nt + t) * k_max;
      for (int s = 0; s < k_max; ++s) { irow[s] = N; nkrow[s] = 0.0f; mrow[s] = 0; }
      long slot = 0;
      for (int j = 0; j < N && slot < k_max; ++j) { /* scatter compaction, :423-433 */
        if (!kept[j]) continue;
        irow[slot] = j;
        nkrow[slot] = rank0[j];
        mrow[slot] = forced[j] ? -1 : bits[row + j]; /* :437-442 */
        slot += 1;
      }
      float* nqrow = newpos_q + ((size_t)h * nt + t) * T;
      for (int i = 0; i < T; ++i) { /* :444-446 */
        long qp = tstart + i;
        if (qp > N - 1) qp = N - 1;
        nqrow[i] = rank0[qp];
      }
      usize[(size_t)h * nt + t] = (int32_t)nu;
      kept_size[(size_t)h * nt + t] = (int32_t)nk;
      overflow[(size_t)h * nt + t] = (uint8_t)ovf;
    }
    free(forced);
    free(kept);
    free(rank0);
    free(cand);
  }
}

/* ------------------------------------------------------------------------------------------- */
/* PQ Stream: fused exact max + per-query keep + streamed positions + attend                  */
/* ------------------------------------------------------------------------------------------- */
/*
 * pqstream_kernel.py:174-368, prefill (q_pos_base 0).  One (head, 32-query tile) at a time:
 *   P_top = min(last row of the tile, N-1), nblk = ceil((P_top+1)/BN)
 *   pass 1: m_i = exact max of the select-geometry scores over causal keys
 *   pass 2: blocks t = 0..nblk-1 at start = (nblk-1-t)*BN (descending), hi_t = min(P_top, start+BN-1)
 *     keep_ij = (s_ij >= m_i - tau | forced_j) & causal & row < N & key < N
 *     adv = max_i c_i (adv_full: hi_t - start + 1); skipped when adv == 0 and use_skip
 *     npk_j = -(d + (hi_t - j)), npq_i = qpos_i - P_top, base RoPE (inv_freq_c, scale 1)
 *     online softmax over kept keys, P cast to the input dtype before P.V; d += adv
 * out (H, N, D) fp32 accumulator before the final cast; span, blocks, skipped (H, nt) fp32;
 * kept (H, N) int32 (kept keys per query); band_rows (H, N) int32 or NULL: per query, # of its
 * causal non-forced keys whose select score lies within band_eps of m - tau.
 * bits_in (H, nt, N) int32 or NULL: when given, the threshold decision s >= m - tau of row i for
 * key j is bit i of bits_in[h, t, j] instead of the scores computed here (forced keys, the
 * causal mask and everything after the decision are unchanged).
 */
void oracle_pqstream(const void* q, const void* k, const void* v, int dtype, int H, int Hkv, int N,
                     int D, const float* tau, const float* inv_freq_a, const float* inv_freq_c,
                     float pos_scale_a, float rope_scale_a, float sm_scale, int n_global,
                     int n_local, int tile, int block_n, int adv_full, int use_skip,
                     const int32_t* bits_in, float* out, float* span, int32_t* kept, float* blocks,
                     float* skipped, int32_t* band_rows, float band_eps) {
  const int T = tile, BN = block_n;
  const int nt = (N + T - 1) / T;
  const int group = H / Hkv;
  /* select-geometry keys, rotated once per kv head */
  float* ks = (float*)malloc(sizeof(float) * (size_t)Hkv * N * D);
  for (int hk = 0; hk < Hkv; ++hk)
    for (int j = 0; j < N; ++j) {
      volatile float cp = (float)j * pos_scale_a;
      rope_row(k, dtype, ((size_t)hk * N + j) * D, D, cp, inv_freq_a, rope_scale_a,
               ks + ((size_t)hk * N + j) * D);
    }
  if (band_rows) memset(band_rows, 0, sizeof(int32_t) * (size_t)H * N);

#pragma omp parallel
  {
    float* qs = (float*)malloc(sizeof(float) * (size_t)T * D);   /* select geometry */
    float* qa = (float*)malloc(sizeof(float) * (size_t)T * D);   /* attend geometry */
    float* m = (float*)malloc(sizeof(float) * (size_t)T);
    float* sel = (float*)malloc(sizeof(float) * (size_t)T * BN);
    uint8_t* keep = (uint8_t*)malloc((size_t)T * BN);
    float* kra = (float*)malloc(sizeof(float) * (size_t)BN * D);
    float* mR = (float*)malloc(sizeof(float) * (size_t)T);
    float* l = (float*)malloc(sizeof(float) * (size_t)T);
    float* acc = (float*)malloc(sizeof(float) * (size_t)T * D);
    int32_t* kr = (int32_t*)malloc(sizeof(int32_t) * (size_t)T);
    double* dotv = (double*)malloc(sizeof(double) * (size_t)D);
    float* sblk = (float*)malloc(sizeof(float) * (size_t)BN);
#pragma omp for schedule(dynamic, 1)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt;
      const int hk = h / group;
      const int r0 = t * T;
      const int P_top = (r0 + T - 1 < N - 1) ? r0 + T - 1 : N - 1; /* :203-204 */
      const int hi = P_top + 1;
      const int nblk = (hi + BN - 1) / BN;
      const float tau_h = tau[h];
      for (int r = 0; r < T; ++r) {
        const int row = r0 + r;
        m[r] = -INFINITY;
        mR[r] = -INFINITY;
        l[r] = 0.0f;
        kr[r] = 0;
        for (int d = 0; d < D; ++d) acc[(size_t)r * D + d] = 0.0f;
        if (row >= N) continue;
        volatile float cp = (float)row * pos_scale_a;                 /* :215 */
        rope_row(q, dtype, ((size_t)h * N + row) * D, D, cp, inv_freq_a, rope_scale_a, qs + (size_t)r * D);
        volatile float npq = (float)(row - P_top);                    /* :222 */
        rope_row(q, dtype, ((size_t)h * N + row) * D, D, npq, inv_freq_c, 1.0f, qa + (size_t)r * D);
        if (bits_in && !band_rows) continue;                          /* decisions are given */
        for (int j = 0; j <= row; ++j) {                              /* pass 1, :229-244 */
          const float s = score_of(qs + (size_t)r * D, ks + ((size_t)hk * N + j) * D, D, sm_scale);
          if (s > m[r]) m[r] = s;
        }
      }
      const long loc_lo = (long)r0 - n_local + 1, loc_hi = (long)r0 + T - 1; /* :260-261 */
      float d = 0.0f;
      int n_used = 0;
      for (int tb = 0; tb < nblk; ++tb) {                             /* :264-358 */
        const int start = (nblk - 1 - tb) * BN;
        const int hi_t = (P_top < start + BN - 1) ? P_top : start + BN - 1;
        int cmax = 0;
        for (int r = 0; r < T; ++r) {
          const int row = r0 + r;
          int c = 0;
          for (int b = 0; b < BN; ++b) {
            const int j = start + b;
            keep[r * BN + b] = 0;
            if (row >= N || j >= N || j > row) continue;              /* causal, row_ok, n_ok */
            const int forced = (j < n_global) || (j >= loc_lo && j <= loc_hi);
            int pass;
            if (bits_in && !band_rows) {
              pass = ((uint32_t)bits_in[((size_t)h * nt + t) * N + j] >> r) & 1u;
            } else {
              const float s = score_of(qs + (size_t)r * D, ks + ((size_t)hk * N + j) * D, D, sm_scale);
              volatile float thr = m[r] - tau_h;
              if (!forced && band_rows && fabsf(s - thr) < band_eps) band_rows[(size_t)h * N + row] += 1;
              pass = bits_in ? (int)(((uint32_t)bits_in[((size_t)h * nt + t) * N + j] >> r) & 1u) : (s >= thr);
            }
            const int kp = pass || forced;                            /* :285-286 */
            keep[r * BN + b] = (uint8_t)kp;
            c += kp;
          }
          sel[r] = (float)c;
          if (c > cmax) cmax = c;
        }
        const float adv = adv_full ? (float)(hi_t - start + 1) : (float)cmax; /* :303-306 */
        if (use_skip && !(adv > 0.0f)) continue;                      /* :319-322 */
        /* attend-geometry keys of this block at npk_j = -(d + o_j), o_j = hi_t - j  (:270, 325-332) */
        for (int b = 0; b < BN; ++b) {
          const int j = start + b;
          if (j >= N) { memset(kra + (size_t)b * D, 0, sizeof(float) * D); continue; }
          volatile float o = (float)(hi_t - j);
          volatile float dpo = d + o;
          const float npk = -dpo;
          rope_row(k, dtype, ((size_t)hk * N + j) * D, D, npk, inv_freq_c, 1.0f, kra + (size_t)b * D);
        }
        for (int r = 0; r < T; ++r) {                                 /* :334-344 */
          const int row = r0 + r;
          float bmax = -INFINITY;
          for (int b = 0; b < BN; ++b) {
            sblk[b] = -INFINITY;
            if (row >= N || !keep[r * BN + b]) continue;
            const float s = score_of(qa + (size_t)r * D, kra + (size_t)b * D, D, sm_scale);
            sblk[b] = s;
            if (s > bmax) bmax = s;
          }
          const float mnew = mR[r] > bmax ? mR[r] : bmax;
          const float msafe = (mnew == -INFINITY) ? 0.0f : mnew;
          volatile float alpha = expf(mR[r] - msafe);
          double psum = 0.0;
          for (int e = 0; e < D; ++e) dotv[e] = 0.0;
          for (int b = 0; b < BN; ++b) {
            volatile float dl = sblk[b] - msafe;
            const float p = expf(dl);
            psum += p;
            if (p == 0.0f) continue;
            const float pc = round_to_dtype(p, dtype);               /* :345 */
            const int j = start + b;
            for (int e = 0; e < D; ++e)
              dotv[e] += (double)pc * (double)load_elem(v, dtype, ((size_t)hk * N + j) * D + e);
          }
          volatile float la = l[r] * alpha;
          l[r] = la + (float)psum;
          for (int e = 0; e < D; ++e) {
            volatile float aa = acc[(size_t)r * D + e] * alpha;
            acc[(size_t)r * D + e] = aa + (float)dotv[e];
          }
          mR[r] = mnew;
          kr[r] += (int32_t)sel[r];                                   /* :347 */
        }
        d = d + adv;                                                  /* :348 */
        n_used += 1;
      }
      for (int r = 0; r < T; ++r) {
        const int row = r0 + r;
        if (row >= N) continue;
        for (int e = 0; e < D; ++e) out[((size_t)h * N + row) * D + e] = acc[(size_t)r * D + e] / l[r];
        kept[(size_t)h * N + row] = kr[r];
      }
      span[(size_t)h * nt + t] = d;
      blocks[(size_t)h * nt + t] = (float)nblk;
      skipped[(size_t)h * nt + t] = (float)(nblk - n_used);
    }
    free(qs); free(qa); free(m); free(sel); free(keep); free(kra); free(mR); free(l); free(acc);
    free(kr); free(dotv); free(sblk);
  }
  free(ks);
}

/* ------------------------------------------------------------------------------------------- */
/* DCA: dense attention with dual-chunk positions                 dca_kernel.py:166-231, 278-366, */
/*                                                                 372-489 (prefill branch)      */
/* ------------------------------------------------------------------------------------------- */
/*
 * Tables (ChunkLlamaRotaryEmbedding._set_cos_sin_cache, dca_kernel.py:166-231): for a position
 * value t, cos/sin of fl(t * inv_freq[i]) in fp32, times mscale in fp32, then cast to the model
 * dtype.  Keys sit at j mod L (L = chunk_size - local_window); queries at i mod L (intra chunk),
 * min(i mod L + L, chunk_size) (one chunk back) and min(2L - 1, chunk_size) (further back).
 * Rotation x*cos + rotate_half(x)*sin in the model dtype, each product and the sum rounded
 * (dca_kernel.py:278-286).  Attention: one softmax over every causal key (the reference's three
 * blocks merged by log-sum-exp, :372-400, 453-489), scores and weights in double, scale `scale`.
 * rows: the query rows to compute (n_rows of them; NULL = all N).  out (H, N, D) fp32, only
 * those rows written.
 */
static void dca_table(float t, const float* inv_freq, int D, float mscale, int dtype, float* c, float* s) {
  const int half = D / 2;
  for (int i = 0; i < half; ++i) {
    /* cos / sin of the fp32 angle correctly rounded to fp32 (through double), then the fp32
     * product with mscale: the table is rounded to the model dtype next, where a one-ulp
     * difference between fp32 cosine implementations could flip a bf16 entry */
    volatile float ang = t * inv_freq[i];
    volatile float c32 = (float)cos((double)ang), s32 = (float)sin((double)ang);
    volatile float cc = c32 * mscale;
    volatile float ss = s32 * mscale;
    c[i] = round_to_dtype(cc, dtype);
    s[i] = round_to_dtype(ss, dtype);
  }
}

static void dca_rotate(const void* x, int dtype, size_t off, int D, const float* c, const float* s, float* out) {
  const int half = D / 2;
  for (int i = 0; i < half; ++i) {
    const float x1 = load_elem(x, dtype, off + i), x2 = load_elem(x, dtype, off + half + i);
    volatile float a = round_to_dtype(x1 * c[i], dtype);
    volatile float b = round_to_dtype(-x2 * s[i], dtype);
    volatile float e = round_to_dtype(x2 * c[i], dtype);
    volatile float f = round_to_dtype(x1 * s[i], dtype);
    out[i] = round_to_dtype(a + b, dtype);
    out[half + i] = round_to_dtype(e + f, dtype);
  }
}

void oracle_dca(const void* q, const void* k, const void* v, int dtype, int H, int Hkv, int N, int D,
                const float* inv_freq, int chunk_size, int local_window, float mscale, float scale,
                const int32_t* rows, int n_rows, float* out) {
  const int L = chunk_size - local_window;
  const int half = D / 2;
  const int group = H / Hkv;
  const int nr = rows ? n_rows : N;
  float* kr = (float*)malloc(sizeof(float) * (size_t)Hkv * N * D);
  {
    float* c = (float*)malloc(sizeof(float) * half);
    float* s = (float*)malloc(sizeof(float) * half);
    for (int j = 0; j < N; ++j) {
      dca_table((float)(j % L), inv_freq, D, mscale, dtype, c, s);     /* keys: j mod L (:187-190) */
      for (int hk = 0; hk < Hkv; ++hk)
        dca_rotate(k, dtype, ((size_t)hk * N + j) * D, D, c, s, kr + ((size_t)hk * N + j) * D);
    }
    free(c);
    free(s);
  }
#pragma omp parallel
  {
    float* c = (float*)malloc(sizeof(float) * half);
    float* s = (float*)malloc(sizeof(float) * half);
    float* qv = (float*)malloc(sizeof(float) * 3 * D);
    double* sc = (double*)malloc(sizeof(double) * (size_t)N);
    double* acc = (double*)malloc(sizeof(double) * D);
#pragma omp for schedule(dynamic, 1)
    for (int x = 0; x < H * nr; ++x) {
      const int h = x / nr;
      const int i = rows ? rows[x % nr] : x % nr;
      const int hk = h / group;
      const int pid = i % L;
      const int cq = i / L;
      /* intra (:181-182), succ (:185-186), inter at the clamped index L-1 (:464-467) */
      const int pos_succ = (pid + L) < chunk_size ? pid + L : chunk_size;
      const int pos_inter = (2 * L - 1) < chunk_size ? 2 * L - 1 : chunk_size;
      dca_table((float)pid, inv_freq, D, mscale, dtype, c, s);
      dca_rotate(q, dtype, ((size_t)h * N + i) * D, D, c, s, qv);
      dca_table((float)pos_succ, inv_freq, D, mscale, dtype, c, s);
      dca_rotate(q, dtype, ((size_t)h * N + i) * D, D, c, s, qv + D);
      dca_table((float)pos_inter, inv_freq, D, mscale, dtype, c, s);
      dca_rotate(q, dtype, ((size_t)h * N + i) * D, D, c, s, qv + 2 * D);
      double mx = -INFINITY;
      for (int j = 0; j <= i; ++j) {
        const int di = cq - j / L;
        const float* qq = qv + (di == 0 ? 0 : (di == 1 ? D : 2 * D));
        const float* kk = kr + ((size_t)hk * N + j) * D;
        double d = 0.0;
        for (int e = 0; e < D; ++e) d += (double)qq[e] * (double)kk[e];
        sc[j] = d * (double)scale;
        if (sc[j] > mx) mx = sc[j];
      }
      double l = 0.0;
      for (int e = 0; e < D; ++e) acc[e] = 0.0;
      for (int j = 0; j <= i; ++j) {
        const double p = exp(sc[j] - mx);
        l += p;
        for (int e = 0; e < D; ++e) acc[e] += p * (double)load_elem(v, dtype, ((size_t)hk * N + j) * D + e);
      }
      for (int e = 0; e < D; ++e) out[((size_t)h * N + i) * D + e] = (float)(acc[e] / l);
    }
    free(c);
    free(s);
    free(qv);
    free(sc);
    free(acc);
  }
  free(kr);
}

/* ------------------------------------------------------------------------------------------- */
/* Config 4: DCA positions with exact-max selection over the inter-chunk keys                 */
/* ------------------------------------------------------------------------------------------- */
/*
 * No reference file combines the two; the build defines the composition from reference parts:
 *   - positions and rotations of dca_kernel.py (keys at j mod L, queries at intra / succ / inter
 *     positions, model-dtype tables and rotation, :166-231, 278-286, 456-489);
 *   - for a query of chunk c >= 2, the inter keys [0, (c - 1) L) -- the keys DCA's inter block
 *     attends at the constant query position (:481-487) -- are scored, thresholded at the exact
 *     row max minus tau and voted per 64-query tile as Kernel A does
 *     (shared_selection_triton_exact_2.py:87-125: s = fl(fl(dot) * scale), keep s >= fl(m - tau));
 *   - each tile's inter votes, as a key axis of length (c - 1) L, go through _build_sets
 *     (exact_2.py:277-426, here oracle_build_sets with that length and the tile's start as
 *     q_pos_base, so its local window lies past the axis and only the global keys are forced);
 *   - each query attends its tile's selected inter keys at the inter position plus every key of
 *     its own and the previous chunk (intra / succ positions), in one softmax.
 * Kernel-A-style scores here are dots of the model-dtype rotated vectors accumulated in double
 * and rounded once to fp32.
 */
void oracle_build_sets(const int32_t* votes, int H, int nt, int N, float pos_scale, int n_global,
                       int n_local, int start_pct, int T, int k_max, int q_pos_base, int measure,
                       int32_t* idx, float* newpos_k, float* newpos_q, int32_t* shared_size,
                       int32_t* kept_size, int32_t* chosen, uint8_t* orig_overflow,
                       int32_t* kpct_meas, uint8_t* overflow20, const float* wvotes, float* cut);

/* rotated keys (Hkv, N, D) and the three query variants (3, H, N, D) as fp32 values */
static void dca_rotate_all(const void* q, const void* k, int dtype, int H, int Hkv, int N, int D,
                           const float* inv_freq, int chunk_size, int L, float mscale, float* kr, float* qr) {
  const int half = D / 2;
#pragma omp parallel
  {
    float* c = (float*)malloc(sizeof(float) * half);
    float* s = (float*)malloc(sizeof(float) * half);
#pragma omp for schedule(static)
    for (int j = 0; j < N; ++j) {
      dca_table((float)(j % L), inv_freq, D, mscale, dtype, c, s);
      for (int hk = 0; hk < Hkv; ++hk)
        dca_rotate(k, dtype, ((size_t)hk * N + j) * D, D, c, s, kr + ((size_t)hk * N + j) * D);
      const int pid = j % L;
      const int pos[3] = {pid, (pid + L) < chunk_size ? pid + L : chunk_size,
                          (2 * L - 1) < chunk_size ? 2 * L - 1 : chunk_size};
      for (int var = 0; var < 3; ++var) {
        dca_table((float)pos[var], inv_freq, D, mscale, dtype, c, s);
        for (int h = 0; h < H; ++h)
          dca_rotate(q, dtype, ((size_t)h * N + j) * D, D, c, s, qr + (((size_t)var * H + h) * N + j) * D);
      }
    }
    free(c);
    free(s);
  }
}

static inline float dot_f32(const float* a, const float* b, int D) {
  double d = 0.0;
  for (int e = 0; e < D; ++e) d += (double)a[e] * (double)b[e];
  return (float)d;
}

/*
 * Inter votes: votes (H, nt, N) int32 (0 past each tile's inter keys), row_max (H, N) fp32 (-inf
 * for rows without inter keys), band (H, nt, N) int32 or NULL (# of the tile's rows whose score for
 * the key lies within band_eps of that row's threshold).  T = 64.  tile_mask (nt bytes) or NULL:
 * only the tiles with a nonzero entry are evaluated (for sampled checks at long lengths); the
 * others keep zero votes and a NaN row max.
 */
void oracle_dca_inter_votes(const void* q, const void* k, int dtype, int H, int Hkv, int N, int D,
                            const float* inv_freq, int chunk_size, int local_window, float mscale, float scale,
                            const float* tau, int T, float band_eps, int32_t* votes, float* row_max,
                            int32_t* band, const uint8_t* tile_mask) {
  const int L = chunk_size - local_window;
  const int group = H / Hkv;
  const int nt = (N + T - 1) / T;
  float* kr = (float*)malloc(sizeof(float) * (size_t)Hkv * N * D);
  float* qr = (float*)malloc(sizeof(float) * (size_t)3 * H * N * D);
  dca_rotate_all(q, k, dtype, H, Hkv, N, D, inv_freq, chunk_size, L, mscale, kr, qr);
  memset(votes, 0, sizeof(int32_t) * (size_t)H * nt * N);
  if (band) memset(band, 0, sizeof(int32_t) * (size_t)H * nt * N);
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)N);
#pragma omp for schedule(dynamic, 1)
    for (int ht = 0; ht < H * nt; ++ht) {
      const int h = ht / nt, t = ht % nt, hk = h / group;
      const int c = (t * T) / L;
      const int ext = c >= 2 ? (c - 1) * L : 0;
      int32_t* vrow = votes + (size_t)ht * N;
      int32_t* brow = band ? band + (size_t)ht * N : NULL;
      if (tile_mask && !tile_mask[t]) {
        for (int i = t * T; i < t * T + T && i < N; ++i) row_max[(size_t)h * N + i] = NAN;
        continue;
      }
      for (int i = t * T; i < t * T + T && i < N; ++i) {
        const float* qq = qr + (((size_t)2 * H + h) * N + i) * D;
        float mx = -INFINITY;
        for (int j = 0; j < ext; ++j) {
          volatile float d = dot_f32(qq, kr + ((size_t)hk * N + j) * D, D);
          volatile float s = d * scale;
          sc[j] = s;
          mx = s > mx ? s : mx;
        }
        row_max[(size_t)h * N + i] = ext > 0 ? mx : -INFINITY;
        if (ext == 0) continue;
        volatile float thr = mx - tau[h];
        for (int j = 0; j < ext; ++j) {
          vrow[j] += sc[j] >= thr;
          if (brow && fabsf(sc[j] - thr) <= band_eps) brow[j] += 1;
        }
      }
    }
    free(sc);
  }
  free(kr);
  free(qr);
}

/*
 * _build_sets over each tile's inter keys: idx (H, nt, k_max) (sentinel: the tile's inter key
 * count), shared_size / kept_size / chosen / kpct_meas (H, nt) int32, orig_overflow / overflow20
 * (H, nt) uint8, cut (H, nt) fp32 or NULL.  Tiles without inter keys get an empty set (all
 * statistics 0, idx 0).
 */
void oracle_dca_build_sets(const int32_t* votes, int H, int N, int chunk_size, int local_window, int T,
                           int n_global, int start_pct, int k_max, int measure, int32_t* idx,
                           int32_t* shared_size, int32_t* kept_size, int32_t* chosen, uint8_t* orig_overflow,
                           int32_t* kpct_meas, uint8_t* overflow20, float* cut) {
  const int L = chunk_size - local_window;
  const int nt = (N + T - 1) / T;
  float* npk = (float*)malloc(sizeof(float) * (size_t)k_max);
  float* npq = (float*)malloc(sizeof(float) * (size_t)T);
  for (int ht = 0; ht < H * nt; ++ht) {
    const int t = ht % nt;
    const int c = (t * T) / L;
    const int ext = c >= 2 ? (c - 1) * L : 0;
    int32_t* irow = idx + (size_t)ht * k_max;
    if (ext == 0) {
      for (int s = 0; s < k_max; ++s) irow[s] = 0;
      shared_size[ht] = kept_size[ht] = chosen[ht] = kpct_meas[ht] = 0;
      orig_overflow[ht] = overflow20[ht] = 0;
      if (cut) cut[ht] = INFINITY;
      continue;
    }
    oracle_build_sets(votes + (size_t)ht * N, 1, 1, ext, 1.0f, n_global, 0, start_pct, T, k_max, t * T,
                      measure, irow, npk, npq, shared_size + ht, kept_size + ht, chosen + ht,
                      orig_overflow + ht, kpct_meas + ht, overflow20 + ht, NULL, cut ? cut + ht : NULL);
  }
  free(npk);
  free(npq);
}

/*
 * Attention given the selection: out (H, N, D) fp32 for the listed rows (all when rows is NULL),
 * the softmax over the tile's selected inter keys idx[h][t][0 .. min(kept, k_max)) at the inter
 * position and the keys [max(0, (c - 1) L), i] at the intra / succ positions, in double.
 */
void oracle_dca_select_attn(const void* q, const void* k, const void* v, int dtype, int H, int Hkv, int N, int D,
                            const float* inv_freq, int chunk_size, int local_window, float mscale, float scale,
                            int T, const int32_t* idx, const int32_t* kept_size, int k_max, const int32_t* rows,
                            int n_rows, float* out) {
  const int L = chunk_size - local_window;
  const int group = H / Hkv;
  const int nt = (N + T - 1) / T;
  const int nr = rows ? n_rows : N;
  float* kr = (float*)malloc(sizeof(float) * (size_t)Hkv * N * D);
  float* qr = (float*)malloc(sizeof(float) * (size_t)3 * H * N * D);
  dca_rotate_all(q, k, dtype, H, Hkv, N, D, inv_freq, chunk_size, L, mscale, kr, qr);
#pragma omp parallel
  {
    double* sc = (double*)malloc(sizeof(double) * ((size_t)k_max + 2 * (size_t)L + 64));
    int32_t* key = (int32_t*)malloc(sizeof(int32_t) * ((size_t)k_max + 2 * (size_t)L + 64));
    double* acc = (double*)malloc(sizeof(double) * D);
#pragma omp for schedule(dynamic, 1)
    for (int x = 0; x < H * nr; ++x) {
      const int h = x / nr;
      const int i = rows ? rows[x % nr] : x % nr;
      const int hk = h / group, t = i / T, c = i / L;
      const int lo = c >= 2 ? (c - 1) * L : 0;
      int n = 0;
      double mx = -INFINITY;
      const int ks = kept_size[(size_t)h * nt + t];
      const int nsel = ks < k_max ? ks : k_max;
      const int32_t* irow = idx + ((size_t)h * nt + t) * k_max;
      for (int s = 0; s < nsel; ++s) {                  /* selected inter keys, inter position */
        const int j = irow[s];
        key[n] = j;
        sc[n] = (double)dot_f32(qr + (((size_t)2 * H + h) * N + i) * D, kr + ((size_t)hk * N + j) * D, D) * scale;
        mx = sc[n] > mx ? sc[n] : mx;
        ++n;
      }
      for (int j = lo; j <= i; ++j) {                   /* local keys, succ / intra positions */
        const int var = (j / L == c) ? 0 : 1;
        key[n] = j;
        sc[n] = (double)dot_f32(qr + (((size_t)var * H + h) * N + i) * D, kr + ((size_t)hk * N + j) * D, D) *
                scale;
        mx = sc[n] > mx ? sc[n] : mx;
        ++n;
      }
      double l = 0.0;
      for (int e = 0; e < D; ++e) acc[e] = 0.0;
      for (int u = 0; u < n; ++u) {
        const double p = exp(sc[u] - mx);
        l += p;
        for (int e = 0; e < D; ++e) acc[e] += p * (double)load_elem(v, dtype, ((size_t)hk * N + key[u]) * D + e);
      }
      for (int e = 0; e < D; ++e) out[((size_t)h * N + i) * D + e] = (float)(acc[e] / l);
    }
    free(sc);
    free(key);
    free(acc);
  }
  free(kr);
  free(qr);
}

/* ------------------------------------------------------------------------------------------- */
/* DCA at decode (dca_kernel.py:491-522) and the rotated key cache (:434-435)                   */
/* ------------------------------------------------------------------------------------------- */
/*
 * oracle_dca_rotate_keys: raw keys (heads, N, D) at positions pos0 .. pos0 + N - 1 rotated with
 * the cyclic key table (:187-190, 198-206): table position (pos mod L), model-dtype table and
 * rotation as in the prefill.  out (heads, N, D) fp32 holding model-dtype values.
 */
void oracle_dca_rotate_keys(const void* k, int dtype, int heads, int N, int D, int pos0, const float* inv_freq,
                            int chunk_size, int local_window, float mscale, float* out) {
  const int L = chunk_size - local_window;
  float* c = (float*)malloc(sizeof(float) * (D / 2));
  float* s = (float*)malloc(sizeof(float) * (D / 2));
  for (int j = 0; j < N; ++j) {
    dca_table((float)((pos0 + j) % L), inv_freq, D, mscale, dtype, c, s);
    for (int h = 0; h < heads; ++h)
      dca_rotate(k, dtype, ((size_t)h * N + j) * D, D, c, s, out + ((size_t)h * N + j) * D);
  }
  free(c);
  free(s);
}

/*
 * oracle_dca_decode: the decode branch.  q (H, D) raw at position cur = M - 1; krot (Hkv, M, D)
 * the cached keys, already rotated (model dtype); v (Hkv, M, D).  The query is rotated at
 * pid = cur mod L (intra, :497), at min(pid + L, s) (succ, :510) and at min(2L - 1, s) (inter:
 * the clamped table index L - 1, :504-505).  Keys [0, inter_end) are scored with the inter
 * variant, [inter_end, chunk_start) with succ, [chunk_start, M) with intra (:494-495, 502-517).
 * Every matmul of the reference runs in the model dtype: each dot accumulates in fp32 (in key
 * dimension order here) and is rounded to the dtype, the scale product is rounded to the dtype
 * (:506-517); the softmax is fp32 (max, then exp(s - max) / sum) and its weights are cast to
 * the dtype (:520-521); P.V accumulates in fp32 (in key order) and is rounded (:522).
 * out (H, D) fp32 holding model-dtype values.
 */
void oracle_dca_decode(const void* q, const void* krot, const void* v, int dtype, int H, int Hkv, int M, int D,
                       const float* inv_freq, int chunk_size, int local_window, float mscale, float scale,
                       float* out) {
  const int L = chunk_size - local_window;
  const int half = D / 2;
  const int group = H / Hkv;
  const int cur = M - 1;
  const int chunk_start = (cur / L) * L;
  const int inter_end = chunk_start - L > 0 ? chunk_start - L : 0;
  const int pid = cur % L;
  const int pos[3] = {pid, pid + L < chunk_size ? pid + L : chunk_size, 2 * L - 1 < chunk_size ? 2 * L - 1 : chunk_size};
  float* c = (float*)malloc(sizeof(float) * half);
  float* s = (float*)malloc(sizeof(float) * half);
  float* qv = (float*)malloc(sizeof(float) * 3 * D);
  float* sc = (float*)malloc(sizeof(float) * (size_t)M);
  float* acc = (float*)malloc(sizeof(float) * D);
  for (int h = 0; h < H; ++h) {
    const int hk = h / group;
    for (int var = 0; var < 3; ++var) {
      dca_table((float)pos[var], inv_freq, D, mscale, dtype, c, s);
      dca_rotate(q, dtype, (size_t)h * D, D, c, s, qv + var * D);
    }
    float mx = -INFINITY;
    for (int j = 0; j < M; ++j) {
      const float* qq = qv + (j < inter_end ? 2 : (j < chunk_start ? 1 : 0)) * D;
      float d = 0.0f;
      for (int e = 0; e < D; ++e) {
        volatile float prod = qq[e] * load_elem(krot, dtype, ((size_t)hk * M + j) * D + e);
        d = d + prod;
      }
      volatile float sd = round_to_dtype(d, dtype) * scale;
      sc[j] = round_to_dtype(sd, dtype);
      if (sc[j] > mx) mx = sc[j];
    }
    float l = 0.0f;
    for (int j = 0; j < M; ++j) l += expf(sc[j] - mx);
    for (int e = 0; e < D; ++e) acc[e] = 0.0f;
    for (int j = 0; j < M; ++j) {
      volatile float pj = expf(sc[j] - mx) / l;
      const float p = round_to_dtype(pj, dtype);
      for (int e = 0; e < D; ++e) {
        volatile float prod = p * load_elem(v, dtype, ((size_t)hk * M + j) * D + e);
        acc[e] = acc[e] + prod;
      }
    }
    for (int e = 0; e < D; ++e) out[(size_t)h * D + e] = round_to_dtype(acc[e], dtype);
  }
  free(c);
  free(s);
  free(qv);
  free(sc);
  free(acc);
}
