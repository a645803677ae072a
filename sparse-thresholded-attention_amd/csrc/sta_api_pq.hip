// sta_api_pq.hip -- the C ABI of the per-query variant, PQ Union (include/sta.h, sta_pq_*).
//
// Same kernels as the shared path where the work is the same: the selection-geometry RoPE
// pre-kernel, the two score passes (with the per-query epilogue: packed keep bits and weighted
// votes per key), and the gather (with the per-slot query bitmask and dense-rank positions under
// base RoPE).  Set construction is its own kernel (sta_pq.hip).
#include <string.h>

#include "../../include/sta.h"
#include "sta_api_util.h"
#include "sta_kernels.h"

using namespace sta;
using namespace sta_api;

namespace {

struct PqLayout {
  int nt, q_rows_pad, k_rows_pad;
  int64_t stride;
  size_t qfrag_off, kfrag_off, ktrig_off, bits_off, wv_off, total;
};

PqLayout pq_layout_of(const sta_pq_args* a) {
  PqLayout L;
  L.nt = (a->N + a->tile - 1) / a->tile;
  L.q_rows_pad = L.nt * a->tile;
  const int64_t kneed = (int64_t)a->q_pos_base + (int64_t)L.nt * a->tile;
  L.k_rows_pad = (int)(((kneed > a->N ? kneed : a->N) + 127) / 128 * 128);
  L.stride = ((int64_t)a->N + 15) / 16 * 16;
  size_t off = 0;
  L.qfrag_off = off;
  off = align256(off + frag_region_bytes(a->H, L.q_rows_pad, a->D));
  L.kfrag_off = off;
  off = align256(off + frag_region_bytes(a->Hkv, L.k_rows_pad, a->D));
  L.ktrig_off = off;   // the K rotation's (cos, sin) per key row, for the screened pass 1
  off = align256(off + (size_t)L.k_rows_pad * (a->D / 2) * sizeof(float2));
  L.bits_off = off;
  off = align256(off + (size_t)a->H * L.nt * L.stride * 4);
  L.wv_off = off;
  off = align256(off + (size_t)a->H * L.nt * L.stride * 4);
  L.total = off;
  return L;
}

int pq_check_common(const sta_pq_args* a) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  if (a->dtype != STA_DTYPE_F32 && a->dtype != STA_DTYPE_BF16 && a->dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", a->dtype);
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->N < 1 || a->N >= (1 << 24)) return fail(STA_ERR_INVALID_ARG, "N=%d out of range [1, 2^24)", a->N);
  if (a->D != 64 && a->D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", a->D);
  // perquery.py:470: per-query keep bits pack into one int32 per key
  if (a->tile != 32) return fail(STA_ERR_INVALID_ARG, "tile %d: the per-query variant needs tile 32", a->tile);
  if (a->k_max < 1) return fail(STA_ERR_INVALID_ARG, "k_max=%d must be >= 1", a->k_max);
  if (a->q_pos_base < 0) return fail(STA_ERR_INVALID_ARG, "q_pos_base=%d must be >= 0", a->q_pos_base);
  if (a->n_global < 0 || a->n_local < 0)
    return fail(STA_ERR_INVALID_ARG, "n_global=%d / n_local=%d must be >= 0", a->n_global, a->n_local);
  if (a->select_score < STA_SCORE_FREQ || a->select_score > STA_SCORE_EXPMASS)
    return fail(STA_ERR_INVALID_ARG, "select_score %d is not one of STA_SCORE_*", a->select_score);
  if (pq_select_lds_bytes(a->N, a->k_max, true) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "k_max=%d needs more than 160 KB of LDS for per-query selection",
                a->k_max);
  return STA_OK;
}

int pq_check_qkv(const sta_pq_args* a, bool need_v) {
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride,
                              a->k_tok_stride, a->v_head_stride, a->v_tok_stride};
  return check_qkv_ptrs(a->dtype, a->q, a->k, a->v, strides, need_v);
}

int pq_check_workspace(const sta_pq_args* a, const PqLayout& L) {
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0) return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return STA_OK;
}

int pq_check_set_outputs(const sta_pq_args* a) {
  if (!a->idx || !a->newpos_k || !a->newpos_q || !a->mask || !a->usize || !a->kept_size || !a->overflow)
    return fail(STA_ERR_INVALID_ARG, "a selection output pointer is NULL");
  return STA_OK;
}

// RoPE pre-kernels + the two score passes with the per-query epilogue
int pq_run_kernel_a(const sta_pq_args* a, const PqLayout& L, hipStream_t st) {
  char* ws = (char*)a->workspace;
  u32x4* qfrag = (u32x4*)(ws + L.qfrag_off);
  u32x4* kfrag = (u32x4*)(ws + L.kfrag_off);
  int rc = mark_event(a->stage_events, 0, st);
  if (rc != STA_OK) return rc;
  hipError_t e = launch_rope_frag(a->dtype, a->D, a->q, a->q_head_stride, a->q_tok_stride, a->H, a->N,
                                  L.q_rows_pad, a->q_pos_base, a->pos_scale_a, a->rope_scale_a,
                                  a->inv_freq_a, qfrag, st);
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (q)");
  e = launch_rope_frag(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->N,
                       L.k_rows_pad, 0, a->pos_scale_a, a->rope_scale_a, a->inv_freq_a, kfrag, st, false,
                       (float2*)(ws + L.ktrig_off));
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (k)");
  if ((rc = mark_event(a->stage_events, 1, st)) != STA_OK) return rc;
  ScoreArgs sa{};
  sa.qfrag = qfrag;
  sa.kfrag = kfrag;
  sa.qnorm = frag_norms(qfrag, a->H, L.q_rows_pad, a->D);
  sa.knorm_max = frag_norm_max(kfrag, a->Hkv, L.k_rows_pad, a->D);
  sa.ktrig = (const float2*)(ws + L.ktrig_off);
  sa.kraw = a->k;
  sa.kraw_hs = a->k_head_stride;
  sa.kraw_ts = a->k_tok_stride;
  sa.kraw_dt = a->dtype;
  sa.H = a->H;
  sa.Hkv = a->Hkv;
  sa.N = a->N;
  sa.nt = L.nt;
  sa.q_rows_pad = L.q_rows_pad;
  sa.k_rows_pad = L.k_rows_pad;
  sa.q_pos_base = a->q_pos_base;
  sa.tau = a->tau;
  sa.sm_scale = a->sm_scale;
  sa.votes_stride = L.stride;
  sa.bits = (uint32_t*)(ws + L.bits_off);
  sa.wvotes = (float*)(ws + L.wv_off);
  sa.row_max = a->row_max;
  sa.row_counts = a->row_counts;
  e = launch_score_pq(a->D, a->select_score, sa, st);
  if (e != hipSuccess) return hip_fail(e, "score kernel (per-query)");
  return STA_OK;
}

PqSelectArgs pq_select_args_of(const sta_pq_args* a, int nt) {
  PqSelectArgs s;
  memset(&s, 0, sizeof(s));
  s.H = a->H;
  s.nt = nt;
  s.N = a->N;
  s.T = a->tile;
  s.k_max = a->k_max;
  s.q_pos_base = a->q_pos_base;
  s.n_global = a->n_global;
  s.n_local = a->n_local;
  s.idx = a->idx;
  s.newpos_k = a->newpos_k;
  s.newpos_q = a->newpos_q;
  s.mask = a->mask;
  s.usize = a->usize;
  s.kept_size = a->kept_size;
  s.overflow = a->overflow;
  return s;
}

int pq_run_gather(const sta_pq_args* a, int nt, hipStream_t st) {
  if (gather_lds_bytes(a->dtype, a->D, a->k_max) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "k_max=%d needs more than 160 KB of LDS in the gather", a->k_max);
  GatherArgs g{};
  g.q = a->q;
  g.k = a->k;
  g.v = a->v;
  g.q_head_stride = a->q_head_stride;
  g.q_tok_stride = a->q_tok_stride;
  g.k_head_stride = a->k_head_stride;
  g.k_tok_stride = a->k_tok_stride;
  g.v_head_stride = a->v_head_stride;
  g.v_tok_stride = a->v_tok_stride;
  g.H = a->H;
  g.Hkv = a->Hkv;
  g.N = a->N;
  g.nt = nt;
  g.k_max = a->k_max;
  g.q_pos_base = a->q_pos_base;
  g.inv_freq = a->inv_freq_c;
  g.rope_scale = 1.0f;                 // perquery.py:513: Kernel C runs base RoPE, scale 1
  g.sm_scale = a->sm_scale;
  g.idx = a->idx;
  g.newpos_k = a->newpos_k;
  g.newpos_q = a->newpos_q;
  g.kept_size = a->kept_size;
  g.mask = a->mask;
  g.out = a->out;
  hipError_t e = launch_gather(a->dtype, a->D, a->tile, g, st);
  if (e != hipSuccess) return hip_fail(e, "gather kernel (per-query)");
  return STA_OK;
}

// the chunked variant's parameters and its exact budget (chunked.py:115-146, 270-278)
int chunk_check(const sta_pq_args* a, const sta_chunk_params* cp) {
  if (!cp) return fail(STA_ERR_INVALID_ARG, "chunk params are NULL");
  if (cp->chunk_size < 1) return fail(STA_ERR_INVALID_ARG, "chunk_size=%d must be >= 1", cp->chunk_size);
  if (cp->n_chunk < 1) return fail(STA_ERR_INVALID_ARG, "n_chunk=%d must be >= 1", cp->n_chunk);
  if (cp->chunk_agg != STA_CHUNK_SUM && cp->chunk_agg != STA_CHUNK_MEAN)
    return fail(STA_ERR_INVALID_ARG, "chunk_agg %d is not STA_CHUNK_SUM or STA_CHUNK_MEAN", cp->chunk_agg);
  const int64_t C = cp->chunk_size;
  const int64_t nf = (a->n_global + C - 1) / C + (a->n_local + a->tile - 1 + C - 1) / C + 1;
  const int64_t nC = (a->N + C - 1) / C;
  const int64_t chunks = nC < nf + cp->n_chunk ? nC : nf + cp->n_chunk;
  if (chunks * C > a->k_max)
    return fail(STA_ERR_INVALID_ARG, "budget overflow: min(nC=%lld, %lld forced + %d selected) * %d > k_max=%d",
                (long long)nC, (long long)nf, cp->n_chunk, cp->chunk_size, a->k_max);
  if (chunk_select_lds_bytes(a->N, cp->chunk_size) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "N=%d in chunks of %d needs more than 160 KB of LDS", a->N, cp->chunk_size);
  if (!a->idx || !a->newpos_k || !a->newpos_q || !a->mask || !a->usize || !a->kept_size)
    return fail(STA_ERR_INVALID_ARG, "a selection output pointer is NULL");
  return STA_OK;
}

ChunkSelectArgs chunk_select_args_of(const sta_pq_args* a, const sta_chunk_params* cp, int nt) {
  ChunkSelectArgs s;
  memset(&s, 0, sizeof(s));
  s.H = a->H;
  s.nt = nt;
  s.N = a->N;
  s.T = a->tile;
  s.k_max = a->k_max;
  s.q_pos_base = a->q_pos_base;
  s.n_global = a->n_global;
  s.n_local = a->n_local;
  s.C = cp->chunk_size;
  s.n_chunk = cp->n_chunk;
  s.mean = cp->chunk_agg == STA_CHUNK_MEAN;
  s.idx = a->idx;
  s.newpos_k = a->newpos_k;
  s.newpos_q = a->newpos_q;
  s.mask = a->mask;
  s.usize = a->usize;
  s.kept_size = a->kept_size;
  s.overflow = a->overflow;
  s.passers_kept = cp->passers_kept;
  return s;
}

}  // namespace

extern "C" {

size_t sta_pq_workspace_size(const sta_pq_args* args) {
  if (pq_check_common(args) != STA_OK) return 0;
  return pq_layout_of(args).total;
}

int sta_pq_attention(const sta_pq_args* args, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = pq_check_qkv(args, true)) != STA_OK) return rc;
  if (!args->tau || !args->inv_freq_a || !args->inv_freq_c || !args->out)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a, inv_freq_c and out must be non-NULL");
  // perquery.py:474-476: the forced set must fit in k_max
  if ((int64_t)args->n_global + args->n_local + args->tile - 1 > args->k_max)
    return fail(STA_ERR_INVALID_ARG, "forced set (n_global=%d + n_local=%d + tile-1=%d) exceeds k_max=%d",
                args->n_global, args->n_local, args->tile - 1, args->k_max);
  if ((rc = pq_check_set_outputs(args)) != STA_OK) return rc;
  const PqLayout L = pq_layout_of(args);
  if ((rc = pq_check_workspace(args, L)) != STA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = pq_run_kernel_a(args, L, st)) != STA_OK) return rc;
  if ((rc = mark_event(args->stage_events, 2, st)) != STA_OK) return rc;
  char* ws = (char*)args->workspace;
  PqSelectArgs s = pq_select_args_of(args, L.nt);
  s.bits = (const uint32_t*)(ws + L.bits_off);
  s.wvotes = args->select_score == STA_SCORE_FREQ ? nullptr : (const float*)(ws + L.wv_off);
  s.votes = nullptr;
  s.stride = L.stride;
  s.dense = 0;
  hipError_t e = launch_pq_select(s, st);
  if (e != hipSuccess) return hip_fail(e, "per-query select kernel");
  if (args->votes || args->bits || args->wvotes) {
    e = launch_expand_pq(s.bits, args->select_score == STA_SCORE_FREQ ? nullptr : s.wvotes, L.stride,
                         args->H, L.nt, args->N, args->tile, args->q_pos_base, args->votes, args->bits,
                         args->wvotes, st);
    if (e != hipSuccess) return hip_fail(e, "vote expansion (per-query)");
  }
  if ((rc = mark_event(args->stage_events, 3, st)) != STA_OK) return rc;
  if ((rc = pq_run_gather(args, L.nt, st)) != STA_OK) return rc;
  return mark_event(args->stage_events, 4, st);
}

int sta_pq_select_bits(const sta_pq_args* args, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = pq_check_qkv(args, false)) != STA_OK) return rc;
  if (!args->tau || !args->inv_freq_a || !args->votes || !args->bits || !args->wvotes)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a, votes, bits and wvotes must be non-NULL");
  const PqLayout L = pq_layout_of(args);
  if ((rc = pq_check_workspace(args, L)) != STA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = pq_run_kernel_a(args, L, st)) != STA_OK) return rc;
  char* ws = (char*)args->workspace;
  hipError_t e = launch_expand_pq((const uint32_t*)(ws + L.bits_off),
                                  args->select_score == STA_SCORE_FREQ ? nullptr : (const float*)(ws + L.wv_off),
                                  L.stride, args->H, L.nt, args->N, args->tile, args->q_pos_base,
                                  args->votes, args->bits, args->wvotes, st);
  if (e != hipSuccess) return hip_fail(e, "vote expansion (per-query)");
  return STA_OK;
}

int sta_pq_build_sets(const sta_pq_args* args, const int32_t* votes, const int32_t* bits,
                      const float* wvotes, int32_t num_tiles, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if (!votes || !bits) return fail(STA_ERR_INVALID_ARG, "votes and bits must be non-NULL");
  if (args->select_score != STA_SCORE_FREQ && !wvotes)
    return fail(STA_ERR_INVALID_ARG, "wvotes is NULL but select_score ranks by weighted votes");
  if (num_tiles < 1) return fail(STA_ERR_INVALID_ARG, "num_tiles=%d must be >= 1", num_tiles);
  if ((rc = pq_check_set_outputs(args)) != STA_OK) return rc;
  PqSelectArgs s = pq_select_args_of(args, num_tiles);
  s.bits = (const uint32_t*)bits;
  s.votes = votes;
  s.wvotes = args->select_score == STA_SCORE_FREQ ? nullptr : wvotes;
  s.stride = args->N;
  s.dense = 1;
  hipError_t e = launch_pq_select(s, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "per-query select kernel");
  return STA_OK;
}

int sta_pq_gather_attention(const sta_pq_args* args, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = pq_check_qkv(args, true)) != STA_OK) return rc;
  if (!args->inv_freq_c || !args->out || !args->idx || !args->newpos_k || !args->newpos_q || !args->mask)
    return fail(STA_ERR_INVALID_ARG, "inv_freq_c, out, idx, newpos_k, newpos_q and mask must be non-NULL");
  const int nt = (args->N + args->tile - 1) / args->tile;
  return pq_run_gather(args, nt, (hipStream_t)stream);   // kept_size, when given, bounds the slots
}

int sta_chunk_build_sets(const sta_pq_args* args, const sta_chunk_params* cp, const int32_t* votes,
                         const float* wvotes, int32_t num_tiles, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = chunk_check(args, cp)) != STA_OK) return rc;
  if (!votes) return fail(STA_ERR_INVALID_ARG, "votes must be non-NULL");
  if (args->select_score != STA_SCORE_FREQ && !wvotes)
    return fail(STA_ERR_INVALID_ARG, "wvotes is NULL but select_score ranks by weighted votes");
  if (num_tiles < 1) return fail(STA_ERR_INVALID_ARG, "num_tiles=%d must be >= 1", num_tiles);
  ChunkSelectArgs s = chunk_select_args_of(args, cp, num_tiles);
  s.votes = votes;
  s.wvotes = args->select_score == STA_SCORE_FREQ ? nullptr : wvotes;
  s.stride = args->N;
  s.dense = 1;
  hipError_t e = launch_chunk_select(s, (hipStream_t)stream);
  return e == hipSuccess ? STA_OK : hip_fail(e, "chunk select kernel");
}

int sta_chunk_attention(const sta_pq_args* args, const sta_chunk_params* cp, void* stream) {
  int rc = pq_check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = chunk_check(args, cp)) != STA_OK) return rc;
  if ((rc = pq_check_qkv(args, true)) != STA_OK) return rc;
  if (!args->tau || !args->inv_freq_a || !args->inv_freq_c || !args->out)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a, inv_freq_c and out must be non-NULL");
  const PqLayout L = pq_layout_of(args);
  if ((rc = pq_check_workspace(args, L)) != STA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = pq_run_kernel_a(args, L, st)) != STA_OK) return rc;
  if ((rc = mark_event(args->stage_events, 2, st)) != STA_OK) return rc;
  char* ws = (char*)args->workspace;
  ChunkSelectArgs s = chunk_select_args_of(args, cp, L.nt);
  s.bits = (const uint32_t*)(ws + L.bits_off);
  s.wvotes = args->select_score == STA_SCORE_FREQ ? nullptr : (const float*)(ws + L.wv_off);
  s.stride = L.stride;
  s.dense = 0;
  hipError_t e = launch_chunk_select(s, st);
  if (e != hipSuccess) return hip_fail(e, "chunk select kernel");
  if (args->votes || args->bits || args->wvotes) {
    e = launch_expand_pq(s.bits, s.wvotes, L.stride, args->H, L.nt, args->N, args->tile, args->q_pos_base,
                         args->votes, args->bits, args->wvotes, st);
    if (e != hipSuccess) return hip_fail(e, "vote expansion (chunked)");
  }
  if ((rc = mark_event(args->stage_events, 3, st)) != STA_OK) return rc;
  if ((rc = pq_run_gather(args, L.nt, st)) != STA_OK) return rc;
  return mark_event(args->stage_events, 4, st);
}

}  // extern "C"
