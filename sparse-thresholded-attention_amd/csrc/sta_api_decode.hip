// sta_api_decode.hip -- the C ABI of the decode path (include/sta.h, sta_decode_*).
#include <string.h>

#include "../../include/sta.h"
#include "sta_api_util.h"
#include "sta_kernels.h"

using namespace sta;
using namespace sta_api;

namespace {

// batches of at least this many queries take their scores from the matrix cores (RoPE fragments +
// score_rows_kernel); smaller ones from the decode score kernel's fp32 dots
constexpr int ROWS_MIN_Q = 64;

struct DecLayout {
  int nsplit;
  bool rows;                                          // scores through the fragments
  int q_rows_pad, k_rows_pad;
  size_t qrot_off, scores_off, keys_off, size_off, part_off, qfrag_off, kfrag_off, total;
};

// the PQ Stream rule's block-end counts in the selection's LDS (decode_bend_words)
int dec_bend_words(const sta_decode_args* a) {
  return a->rule == STA_RULE_STREAM && a->block_n >= 1 ? (a->M + a->block_n - 1) / a->block_n : 0;
}

DecLayout dec_layout_of(const sta_decode_args* a) {
  DecLayout L;
  L.nsplit = decode_nsplit(a->k_max);
  L.rows = a->Q >= ROWS_MIN_Q;
  L.q_rows_pad = (a->Q + 31) / 32 * 32;
  L.k_rows_pad = (a->M + 31) / 32 * 32;
  const size_t hq = (size_t)a->H * a->Q;
  size_t off = 0;
  L.qrot_off = off;                                   // rotated queries (H, Q, D) fp32
  off = align256(off + hq * a->D * 4);
  L.scores_off = off;                                 // scores when not an output: (H, Q, M), or
                                                      // 64 x 32 tiles from the score rows kernel
  off = align256(off + (L.rows ? (size_t)a->H * score_tiles_per_head(a->Q, a->M) : hq * a->M) * 4);
  L.keys_off = off;                                   // key store of long caches
  off = align256(off + decode_keys_bytes(a->H, a->Q, a->M, dec_bend_words(a)));
  L.size_off = off;                                   // set sizes (H, Q) when not an output
  off = align256(off + hq * 4);
  L.part_off = off;                                   // attend split states
  off = align256(off + hq * L.nsplit * (a->D + 2) * 4);
  L.qfrag_off = L.kfrag_off = off;                    // rotated hi / lo fragments (rows mode)
  if (L.rows) {
    off = align256(off + frag_region_bytes(a->H, L.q_rows_pad, a->D));
    L.kfrag_off = off;
    off = align256(off + frag_region_bytes(a->Hkv, L.k_rows_pad, a->D));
  }
  L.total = off;
  return L;
}

// need_pos: the entry point selects or attends, so every query's position must lie inside its
// key range (forced[q_pos], exact_2.py:555); the scores alone take any position
int dec_check(const sta_decode_args* a, bool need_pos = true) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  if (a->dtype != STA_DTYPE_F32 && a->dtype != STA_DTYPE_BF16 && a->dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", a->dtype);
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->D != 64 && a->D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", a->D);
  if (a->M < 1 || a->M >= (1 << 24)) return fail(STA_ERR_INVALID_ARG, "M=%d out of range [1, 2^24)", a->M);
  if (a->Q < 1) return fail(STA_ERR_INVALID_ARG, "Q=%d must be >= 1", a->Q);
  if (a->q_pos0 < 0 || (need_pos && (int64_t)a->q_pos0 + a->Q > a->M))
    return fail(STA_ERR_INVALID_ARG, "need 0 <= q_pos0 (%d) and q_pos0 + Q (%d) <= M (%d)", a->q_pos0, a->Q, a->M);
  if (a->k_max < 1 || a->k_max > 65536)
    return fail(STA_ERR_UNSUPPORTED, "k_max=%d outside [1, 65536]", a->k_max);
  if (a->n_global < 0 || a->n_local < 0)
    return fail(STA_ERR_UNSUPPORTED, "n_global=%d / n_local=%d must be >= 0", a->n_global, a->n_local);
  if ((size_t)a->H * a->Q >= (1u << 31)) return fail(STA_ERR_INVALID_ARG, "H * Q too large");
  if (a->rule != STA_RULE_SHARED && a->rule != STA_RULE_PQ && a->rule != STA_RULE_STREAM)
    return fail(STA_ERR_INVALID_ARG, "rule %d is not STA_RULE_SHARED, STA_RULE_PQ or STA_RULE_STREAM", a->rule);
  if (a->rule == STA_RULE_STREAM) {
    if (a->block_n < 1) return fail(STA_ERR_INVALID_ARG, "stream rule: block_n=%d must be >= 1", a->block_n);
    // one block-end count per position block in the selection's LDS (16 KB at most)
    if ((a->M + a->block_n - 1) / a->block_n > 4096)
      return fail(STA_ERR_UNSUPPORTED, "stream rule: M=%d over block_n=%d exceeds 4096 blocks", a->M, a->block_n);
  }
  if (a->rule == STA_RULE_PQ && (int64_t)a->n_global + a->n_local > a->k_max)
    return fail(STA_ERR_INVALID_ARG, "per-query rule: n_global (%d) + n_local (%d) exceeds k_max (%d)",
                a->n_global, a->n_local, a->k_max);
  return STA_OK;
}

int dec_check_ws(const sta_decode_args* a, const DecLayout& L) {
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0) return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return STA_OK;
}

DecodeArgs dec_args_of(const sta_decode_args* a, const DecLayout& L) {
  char* ws = (char*)a->workspace;
  DecodeArgs d{};
  d.q = a->q;
  d.q_hs = a->q_head_stride;
  d.q_ts = a->q_tok_stride;
  d.k = a->k;
  d.k_hs = a->k_head_stride;
  d.k_ts = a->k_tok_stride;
  d.v = a->v;
  d.v_hs = a->v_head_stride;
  d.v_ts = a->v_tok_stride;
  d.H = a->H;
  d.Hkv = a->Hkv;
  d.Q = a->Q;
  d.M = a->M;
  d.q_pos0 = a->q_pos0;
  d.inv_freq_a = a->inv_freq_a;
  d.pos_scale_a = a->pos_scale_a;
  d.rope_scale_a = a->rope_scale_a;
  d.pos_scale_c = a->pos_scale_c;
  d.inv_freq_c = a->inv_freq_c;
  d.rope_scale_c = a->rope_scale_c;
  d.sm_scale = a->sm_scale;
  d.tau = a->tau;
  d.n_global = a->n_global;
  d.n_local = a->n_local;
  d.k_max = a->k_max;
  d.rule = a->rule;
  d.block_n = a->rule == STA_RULE_STREAM ? a->block_n : 0;
  d.usize = a->rule == STA_RULE_PQ ? a->usize : nullptr;
  d.overflow = a->rule == STA_RULE_PQ ? a->overflow : nullptr;
  // the per-query rule keeps every passer (perquery.py:651-720 has no top-pct cut)
  d.use_pct = a->rule == STA_RULE_SHARED && a->pct_decode < 100.0;   // exact_2.py:559 (the others keep
                                                                     // every passer)
  d.pct_frac = (float)(a->pct_decode / 100.0);                    // the float32 scalar of :561
  d.scores = a->scores ? a->scores : (float*)(ws + L.scores_off);
  d.keys = decode_select_in_lds(a->M, dec_bend_words(a)) ? nullptr : (uint32_t*)(ws + L.keys_off);
  d.idx = a->idx;
  d.newpos_k = a->newpos_k;
  d.newpos_q = a->newpos_q;
  d.set_size = a->set_size;
  d.causal = a->causal ? 1 : 0;
  d.part = (float*)(ws + L.part_off);
  d.qrot = nullptr;
  d.out = a->out;
  return d;
}

int dec_scores(const sta_decode_args* a, const DecLayout& L, DecodeArgs d, float* scores, hipStream_t st) {
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride, a->k_tok_stride, 0, 0};
  int rc = check_qkv_ptrs(a->dtype, a->q, a->k, nullptr, strides, false);
  if (rc != STA_OK) return rc;
  if (!a->inv_freq_a) return fail(STA_ERR_INVALID_ARG, "inv_freq_a must be non-NULL");
  if (!scores) return fail(STA_ERR_INVALID_ARG, "scores must be non-NULL");
  d.scores = scores;
  if (!L.rows) {
    hipError_t e = launch_decode_scores(a->dtype, a->D, d, (float*)((char*)a->workspace + L.qrot_off), st);
    return e == hipSuccess ? STA_OK : hip_fail(e, "decode scores");
  }
  // a batch of queries: rotate queries (at q_pos0 + i) and keys once into hi / lo fragments under
  // the selection geometry, then one matrix product per head
  char* ws = (char*)a->workspace;
  u32x4* qfrag = (u32x4*)(ws + L.qfrag_off);
  u32x4* kfrag = (u32x4*)(ws + L.kfrag_off);
  hipError_t e = launch_rope_frag(a->dtype, a->D, a->q, a->q_head_stride, a->q_tok_stride, a->H, a->Q,
                                  L.q_rows_pad, a->q_pos0, a->pos_scale_a, a->rope_scale_a, a->inv_freq_a,
                                  qfrag, st);
  if (e != hipSuccess) return hip_fail(e, "decode scores: rope pre-kernel (q)");
  e = launch_rope_frag(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->M, L.k_rows_pad, 0,
                       a->pos_scale_a, a->rope_scale_a, a->inv_freq_a, kfrag, st);
  if (e != hipSuccess) return hip_fail(e, "decode scores: rope pre-kernel (k)");
  RowsArgs r{};
  r.qfrag = qfrag;
  r.kfrag = kfrag;
  r.H = a->H;
  r.Hkv = a->Hkv;
  r.Q = a->Q;
  r.M = a->M;
  r.q_pos0 = a->q_pos0;
  r.q_rows_pad = L.q_rows_pad;
  r.k_rows_pad = L.k_rows_pad;
  r.sm_scale = a->sm_scale;
  r.scores = scores;
  r.tiles = d.score_tiles;
  e = launch_score_rows(a->D, r, st);
  return e == hipSuccess ? STA_OK : hip_fail(e, "decode scores: score rows");
}

// newpos_k may be NULL under STA_RULE_PQ: its positions are the slot indices (dense ranks)
bool newpos_k_ok(const sta_decode_args* a) { return a->newpos_k || a->rule == STA_RULE_PQ; }

int dec_select(const sta_decode_args* a, DecodeArgs d, const float* scores, hipStream_t st) {
  if (!a->tau || !a->idx || !newpos_k_ok(a) || !a->newpos_q)
    return fail(STA_ERR_INVALID_ARG, "tau, idx, newpos_k (unless STA_RULE_PQ) and newpos_q must be non-NULL");
  if (!scores) return fail(STA_ERR_INVALID_ARG, "scores must be non-NULL");
  d.scores = (float*)scores;
  hipError_t e = launch_decode_select(d, st);
  return e == hipSuccess ? STA_OK : hip_fail(e, "decode selection");
}

int dec_attend(const sta_decode_args* a, const DecodeArgs& d, hipStream_t st) {
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride,
                              a->k_tok_stride, a->v_head_stride, a->v_tok_stride};
  int rc = check_qkv_ptrs(a->dtype, a->q, a->k, a->v, strides, true);
  if (rc != STA_OK) return rc;
  if (!a->inv_freq_c || !a->out || !a->idx || !newpos_k_ok(a) || !a->newpos_q)
    return fail(STA_ERR_INVALID_ARG,
                "inv_freq_c, out, idx, newpos_k (unless STA_RULE_PQ) and newpos_q must be non-NULL");
  hipError_t e = launch_decode_attend(a->dtype, a->D, d, st);
  return e == hipSuccess ? STA_OK : hip_fail(e, "decode attend");
}

}  // namespace

extern "C" {

size_t sta_decode_workspace_size(const sta_decode_args* args) {
  if (dec_check(args, false) != STA_OK) return 0;
  return dec_layout_of(args).total;
}

int sta_decode_scores(const sta_decode_args* a, float* scores, void* stream) {
  int rc = dec_check(a, false);
  if (rc != STA_OK) return rc;
  const DecLayout L = dec_layout_of(a);
  if ((rc = dec_check_ws(a, L)) != STA_OK) return rc;
  return dec_scores(a, L, dec_args_of(a, L), scores, (hipStream_t)stream);
}

int sta_decode_build_sets(const sta_decode_args* a, const float* scores, void* stream) {
  int rc = dec_check(a);
  if (rc != STA_OK) return rc;
  const DecLayout L = dec_layout_of(a);
  if ((rc = dec_check_ws(a, L)) != STA_OK) return rc;
  return dec_select(a, dec_args_of(a, L), scores, (hipStream_t)stream);
}

int sta_decode_build_sets_chunk(const sta_decode_args* a, const sta_chunk_params* cp, int32_t select_score,
                                const float* scores, void* stream) {
  int rc = dec_check(a);
  if (rc != STA_OK) return rc;
  if (!cp) return fail(STA_ERR_INVALID_ARG, "chunk params are NULL");
  if (!scores) return fail(STA_ERR_INVALID_ARG, "scores must be non-NULL");
  if (cp->chunk_size < 1 || cp->n_chunk < 1)
    return fail(STA_ERR_INVALID_ARG, "chunk_size=%d and n_chunk=%d must be >= 1", cp->chunk_size, cp->n_chunk);
  if (cp->chunk_agg != STA_CHUNK_SUM && cp->chunk_agg != STA_CHUNK_MEAN)
    return fail(STA_ERR_INVALID_ARG, "chunk_agg %d is not STA_CHUNK_SUM or STA_CHUNK_MEAN", cp->chunk_agg);
  if (select_score < STA_SCORE_FREQ || select_score > STA_SCORE_EXPMASS)
    return fail(STA_ERR_INVALID_ARG, "select_score %d is not one of STA_SCORE_*", select_score);
  if (chunk_select_lds_bytes(a->M, cp->chunk_size) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "M=%d in chunks of %d needs more than 160 KB of LDS", a->M, cp->chunk_size);
  if (!a->tau || !a->idx || !a->newpos_k || !a->newpos_q || !a->set_size)
    return fail(STA_ERR_INVALID_ARG, "tau, idx, newpos_k, newpos_q and set_size must be non-NULL");
  ChunkDecodeArgs d{};
  d.scores = scores;
  d.tau = a->tau;
  d.H = a->H;
  d.Q = a->Q;
  d.M = a->M;
  d.q_pos0 = a->q_pos0;
  d.k_max = a->k_max;
  d.n_global = a->n_global;
  d.n_local = a->n_local;
  d.C = cp->chunk_size;
  d.n_chunk = cp->n_chunk;
  d.weighted = select_score != STA_SCORE_FREQ;
  d.mean = cp->chunk_agg == STA_CHUNK_MEAN;
  d.idx = a->idx;
  d.newpos_k = a->newpos_k;
  d.newpos_q = a->newpos_q;
  d.kept_size = a->set_size;
  d.passers_kept = cp->passers_kept;
  d.usize = a->usize;
  hipError_t e = launch_chunk_decode_select(d, (hipStream_t)stream);
  return e == hipSuccess ? STA_OK : hip_fail(e, "chunk decode select kernel");
}

int sta_decode_attend(const sta_decode_args* a, void* stream) {
  int rc = dec_check(a);
  if (rc != STA_OK) return rc;
  const DecLayout L = dec_layout_of(a);
  if ((rc = dec_check_ws(a, L)) != STA_OK) return rc;
  return dec_attend(a, dec_args_of(a, L), (hipStream_t)stream);
}

int sta_decode_attention(const sta_decode_args* a, void* stream) {
  int rc = dec_check(a);
  if (rc != STA_OK) return rc;
  const DecLayout L = dec_layout_of(a);
  if ((rc = dec_check_ws(a, L)) != STA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  DecodeArgs d = dec_args_of(a, L);
  // the attend sweeps only the selected slots: the set sizes always exist (output or workspace)
  if (!d.set_size) d.set_size = (int32_t*)((char*)a->workspace + L.size_off);
  // scores that only this call's selection reads leave the score rows kernel in 64 x 32 tiles
  d.score_tiles = L.rows && !a->scores ? 1 : 0;
  if ((rc = mark_event(a->stage_events, 0, st)) != STA_OK) return rc;
  if ((rc = dec_scores(a, L, d, d.scores, st)) != STA_OK) return rc;
  if ((rc = mark_event(a->stage_events, 1, st)) != STA_OK) return rc;
  if ((rc = dec_select(a, d, d.scores, st)) != STA_OK) return rc;
  if ((rc = mark_event(a->stage_events, 2, st)) != STA_OK) return rc;
  // the per-query rule's selection just wrote newpos_k = the slot index of every slot
  d.dense_ranks = a->rule == STA_RULE_PQ ? 1 : 0;
  if ((rc = dec_attend(a, d, st)) != STA_OK) return rc;
  return mark_event(a->stage_events, 3, st);
}

}  // extern "C"
