// sta_api_dca.hip -- the C ABI of the DCA prefill (include/sta.h, sta_dca_*).
#include <math.h>
#include <string.h>

#include "../../include/sta.h"
#include "sta_api_util.h"
#include "sta_kernels.h"

using namespace sta;
using namespace sta_api;

namespace {

constexpr int kDcaSelTile = 64;   // queries per selection tile (config 4)

struct DcaLayout {
  int Npad, planes, nt;
  int64_t votes_stride;
  size_t krot_off, qrot_off, votes_off, rmax_off, npk_off, npq_off, state_off, tab_off, total;
};

DcaLayout dca_layout_of(const sta_dca_args* a) {
  DcaLayout L;
  L.Npad = (a->N + 63) / 64 * 64;
  L.planes = a->dtype == STA_DTYPE_F32 ? 2 : 1;
  L.nt = (a->N + kDcaSelTile - 1) / kDcaSelTile;
  L.votes_stride = ((int64_t)a->N + 15) / 16 * 16;
  size_t off = 0;
  L.krot_off = off;
  off = align256(off + (size_t)a->Hkv * L.Npad * L.planes * a->D * 2);
  L.qrot_off = off;
  off = align256(off + (size_t)3 * a->H * L.Npad * L.planes * a->D * 2);
  L.votes_off = L.rmax_off = L.npk_off = L.npq_off = L.state_off = off;
  if (a->select) {
    L.votes_off = off;                                 // byte votes (H, nt, votes_stride)
    off = align256(off + (size_t)a->H * L.nt * L.votes_stride);
    L.rmax_off = off;                                  // raw inter row maxima (H, Npad)
    off = align256(off + (size_t)a->H * L.Npad * 4);
    L.npk_off = off;                                   // selection positions (unused by DCA)
    off = align256(off + (size_t)a->H * L.nt * a->k_max * 4);
    L.npq_off = off;
    off = align256(off + (size_t)a->H * L.nt * kDcaSelTile * 4);
    L.state_off = off;                                 // partial softmax states (H, Npad, D + 4)
    off = align256(off + (size_t)a->H * L.Npad * (a->D + 4) * 4);
  }
  L.tab_off = off;                                     // the remap's (cos, sin) table
  off = align256(off + dca_table_bytes(a->D, a->chunk_size));
  L.total = off;
  return L;
}

int dca_check(const sta_dca_args* a) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  if (a->dtype != STA_DTYPE_F32 && a->dtype != STA_DTYPE_BF16 && a->dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", a->dtype);
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->N < 1 || a->N >= (1 << 24)) return fail(STA_ERR_INVALID_ARG, "N=%d out of range [1, 2^24)", a->N);
  if (a->D != 64 && a->D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", a->D);
  // dca_kernel.py:552: 0 < w < s
  if (!(a->local_window > 0 && a->local_window < a->chunk_size))
    return fail(STA_ERR_INVALID_ARG, "need 0 < local_window(%d) < chunk_size(%d)", a->local_window, a->chunk_size);
  if (a->pretrain_len < 1) return fail(STA_ERR_INVALID_ARG, "pretrain_len=%d must be >= 1", a->pretrain_len);
  if (!(a->mscale >= 0.0f) || isinf(a->mscale))
    return fail(STA_ERR_INVALID_ARG, "mscale=%g must be finite and >= 0 (0: derived from N)", (double)a->mscale);
  // the sweep keeps its running max on the raw dots, which orders as the scaled scores only for
  // a positive scale
  if (!(a->scale > 0.0f) || isinf(a->scale))
    return fail(STA_ERR_INVALID_ARG, "scale=%g must be finite and > 0", (double)a->scale);
  const int L = a->chunk_size - a->local_window;
  if (L % 64 != 0)
    return fail(STA_ERR_UNSUPPORTED, "chunk_size - local_window = %d is not a multiple of 64", L);
  if (a->select != 0 && a->select != 1) return fail(STA_ERR_INVALID_ARG, "select=%d is not 0 or 1", a->select);
  if (a->select) {
    if (a->k_max < 1) return fail(STA_ERR_INVALID_ARG, "k_max=%d must be >= 1", a->k_max);
    if (a->n_global < 0) return fail(STA_ERR_INVALID_ARG, "n_global=%d must be >= 0", a->n_global);
    if (a->start_pct < 0) return fail(STA_ERR_INVALID_ARG, "start_pct=%d must be >= 0", a->start_pct);
    if (select_lds_bytes(a->N, a->k_max) > 160 * 1024)
      return fail(STA_ERR_UNSUPPORTED, "N=%d with k_max=%d needs more than 160 KB of LDS for selection",
                  a->N, a->k_max);
  }
  return STA_OK;
}

int check_rows(const char* what, int dtype, const void* p, int64_t hs, int64_t ts) {
  const int es = esize(dtype);
  if (!p) return fail(STA_ERR_INVALID_ARG, "%s is NULL", what);
  if (!aligned16(p)) return fail(STA_ERR_UNSUPPORTED, "%s is not 16-byte aligned", what);
  if (hs < 0 || ts < 0 || (hs * es) % 16 != 0 || (ts * es) % 16 != 0)
    return fail(STA_ERR_UNSUPPORTED, "%s strides (%lld, %lld) are negative or not 16-byte aligned", what,
                (long long)hs, (long long)ts);
  return STA_OK;
}

int check_dtype_dim(int dtype, int D) {
  if (dtype != STA_DTYPE_F32 && dtype != STA_DTYPE_BF16 && dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", dtype);
  if (D != 64 && D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", D);
  return STA_OK;
}

int check_chunks(int chunk_size, int local_window, float mscale) {
  if (!(local_window > 0 && local_window < chunk_size))
    return fail(STA_ERR_INVALID_ARG, "need 0 < local_window(%d) < chunk_size(%d)", local_window, chunk_size);
  if (!(mscale > 0.0f) || isinf(mscale)) return fail(STA_ERR_INVALID_ARG, "mscale=%g must be finite and > 0",
                                                     (double)mscale);
  return STA_OK;
}

struct DcaDecLayout {
  int nb;
  size_t qrot_off, scores_off, pmax_off, psum_off, part_off, total;
};

DcaDecLayout dca_dec_layout_of(const sta_dca_decode_args* a) {
  DcaDecLayout L;
  L.nb = dca_dec_nblocks(a->M);
  size_t off = 0;
  L.qrot_off = off;
  off = align256(off + (size_t)a->H * 3 * a->D * 4);
  L.scores_off = off;
  off = align256(off + (size_t)a->H * a->M * 4);
  L.pmax_off = off;
  off = align256(off + (size_t)a->H * L.nb * 4);
  L.psum_off = off;
  off = align256(off + (size_t)a->H * L.nb * 4);
  L.part_off = off;
  off = align256(off + (size_t)a->H * L.nb * a->D * 4);
  L.total = off;
  return L;
}

int dca_dec_check(const sta_dca_decode_args* a) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  int rc = check_dtype_dim(a->dtype, a->D);
  if (rc != STA_OK) return rc;
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->H / a->Hkv > dca_dec_max_group())
    return fail(STA_ERR_UNSUPPORTED, "H / Hkv = %d exceeds %d heads per kv head", a->H / a->Hkv,
                dca_dec_max_group());
  if (a->M < 1 || a->M >= (1 << 24)) return fail(STA_ERR_INVALID_ARG, "M=%d out of range [1, 2^24)", a->M);
  return check_chunks(a->chunk_size, a->local_window, a->mscale);
}

// config 4's selection: inter-key votes (two passes), then _build_sets over each tile's inter keys
int dca_select(const sta_dca_args* a, const DcaLayout& L, const uint16_t* krot, const uint16_t* qrot, int Lc,
               hipStream_t st) {
  if (!a->tau || !a->idx || !a->shared_size || !a->kept_size || !a->chosen || !a->orig_overflow ||
      !a->kpct_meas || !a->overflow20)
    return fail(STA_ERR_INVALID_ARG, "select: tau and the selection outputs must be non-NULL");
  char* ws = (char*)a->workspace;
  DcaVoteArgs v{};
  v.qrot = qrot;
  v.krot = krot;
  v.H = a->H;
  v.Hkv = a->Hkv;
  v.N = a->N;
  v.Npad = L.Npad;
  v.L = Lc;
  v.nt = L.nt;
  v.scale = a->scale;
  v.tau = a->tau;
  v.rmax = (float*)(ws + L.rmax_off);
  v.row_max = a->row_max;
  v.votes = (uint8_t*)(ws + L.votes_off);
  v.votes_stride = L.votes_stride;
  hipError_t e = launch_dca_votes(a->dtype, a->D, v, st);
  if (e != hipSuccess) return hip_fail(e, "dca inter votes");
  int rc = mark_event(a->stage_events, 2, st);
  if (rc != STA_OK) return rc;
  SelectArgs s;
  memset(&s, 0, sizeof(s));
  s.votes = ws + L.votes_off;
  s.votes_stride = L.votes_stride;
  s.votes_dense = 0;
  s.H = a->H;
  s.nt = L.nt;
  s.N = a->N;
  s.T = kDcaSelTile;
  s.k_max = a->k_max;
  s.q_pos_base = 0;
  s.n_global = a->n_global;
  s.n_local = 0;
  s.pos_scale = 1.0f;
  s.nsteps = 0;
  s.steps[s.nsteps++] = a->start_pct;                  // exact_2.py:309-310
  if (25 < a->start_pct) s.steps[s.nsteps++] = 25;
  if (20 < a->start_pct) s.steps[s.nsteps++] = 20;
  s.K_ord = 1;                                         // per tile under dca_L
  s.start_pct = a->start_pct;
  s.measure = a->measure;
  s.idx = a->idx;
  s.newpos_k = (float*)(ws + L.npk_off);
  s.newpos_q = (float*)(ws + L.npq_off);
  s.shared_size = a->shared_size;
  s.kept_size = a->kept_size;
  s.chosen = a->chosen;
  s.orig_overflow = a->orig_overflow;
  s.kpct_meas = a->kpct_meas;
  s.overflow20 = a->overflow20;
  s.votes_out = a->votes;
  s.dca_L = Lc;
  e = launch_select(s, 1, st);
  return e == hipSuccess ? STA_OK : hip_fail(e, "dca inter selection");
}

}  // namespace

extern "C" {

size_t sta_dca_workspace_size(const sta_dca_args* args) {
  if (dca_check(args) != STA_OK) return 0;
  return dca_layout_of(args).total;
}

int sta_dca_attention(const sta_dca_args* a, void* stream) {
  int rc = dca_check(a);
  if (rc != STA_OK) return rc;
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride,
                              a->k_tok_stride, a->v_head_stride, a->v_tok_stride};
  if ((rc = check_qkv_ptrs(a->dtype, a->q, a->k, a->v, strides, true)) != STA_OK) return rc;
  if (!a->inv_freq || !a->out) return fail(STA_ERR_INVALID_ARG, "inv_freq and out must be non-NULL");
  const DcaLayout L = dca_layout_of(a);
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0) return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)a->workspace;
  uint16_t* krot = (uint16_t*)(ws + L.krot_off);
  uint16_t* qrot = (uint16_t*)(ws + L.qrot_off);
  const int Lc = a->chunk_size - a->local_window;
  // mscale = get_mscale(N / c): 0.05 ln(N / c) + 1 when the prefill outruns c, else 1 (:163-170),
  // unless the caller passes the factor its tables were built with
  const double ratio = (double)a->N / (double)a->pretrain_len;
  const float mscale = a->mscale > 0.0f ? a->mscale : (ratio <= 1.0 ? 1.0f : (float)(0.05 * log(ratio) + 1.0));

  if ((rc = mark_event(a->stage_events, 0, st)) != STA_OK) return rc;
  float2* table = (float2*)(ws + L.tab_off);
  hipError_t e = launch_dca_table(a->dtype, a->D, a->inv_freq, mscale, a->chunk_size, table, st);
  if (e != hipSuccess) return hip_fail(e, "dca table");
  e = launch_dca_rope(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->N, L.Npad, Lc,
                      a->chunk_size, 1, table, krot, st);
  if (e != hipSuccess) return hip_fail(e, "dca rotation (k)");
  e = launch_dca_rope(a->dtype, a->D, a->q, a->q_head_stride, a->q_tok_stride, a->H, a->N, L.Npad, Lc,
                      a->chunk_size, 0, table, qrot, st);
  if (e != hipSuccess) return hip_fail(e, "dca rotation (q)");
  if ((rc = mark_event(a->stage_events, 1, st)) != STA_OK) return rc;
  if (a->select) {
    if ((rc = dca_select(a, L, krot, qrot, Lc, st)) != STA_OK) return rc;
    if ((rc = mark_event(a->stage_events, 3, st)) != STA_OK) return rc;
  }
  DcaArgs d{};
  d.qrot = qrot;
  d.krot = krot;
  d.v = a->v;
  d.v_head_stride = a->v_head_stride;
  d.v_tok_stride = a->v_tok_stride;
  d.H = a->H;
  d.Hkv = a->Hkv;
  d.N = a->N;
  d.Npad = L.Npad;
  d.L = Lc;
  d.scale = a->scale;
  d.out = a->out;
  if (a->select) {
    d.idx = a->idx;
    d.kept_size = a->kept_size;
    d.k_max = a->k_max;
    d.nt64 = L.nt;
    d.state = (float*)(ws + L.state_off);
  }
  e = launch_dca_attn(a->dtype, a->D, d, st);
  if (e != hipSuccess) return hip_fail(e, "dca attention");
  return mark_event(a->stage_events, a->select ? 4 : 2, st);
}

int sta_dca_rotate_keys(const sta_dca_rotate_args* a, void* stream) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  int rc = check_dtype_dim(a->dtype, a->D);
  if (rc != STA_OK) return rc;
  if (a->heads < 1 || a->N < 0 || a->pos0 < 0 || (int64_t)a->pos0 + a->N >= (1ll << 31))
    return fail(STA_ERR_INVALID_ARG, "heads=%d, N=%d, pos0=%d out of range", a->heads, a->N, a->pos0);
  if ((rc = check_chunks(a->chunk_size, a->local_window, a->mscale)) != STA_OK) return rc;
  if (!a->inv_freq) return fail(STA_ERR_INVALID_ARG, "inv_freq is NULL");
  if (a->N == 0) return STA_OK;
  if ((rc = check_rows("x", a->dtype, a->x, a->x_head_stride, a->x_tok_stride)) != STA_OK) return rc;
  if ((rc = check_rows("out", a->dtype, a->out, a->out_head_stride, a->out_tok_stride)) != STA_OK) return rc;
  DcaRotArgs d{};
  d.x = a->x;
  d.x_head_stride = a->x_head_stride;
  d.x_tok_stride = a->x_tok_stride;
  d.out = a->out;
  d.out_head_stride = a->out_head_stride;
  d.out_tok_stride = a->out_tok_stride;
  d.heads = a->heads;
  d.N = a->N;
  d.pos0 = a->pos0;
  d.L = a->chunk_size - a->local_window;
  d.mscale = a->mscale;
  d.inv_freq = a->inv_freq;
  hipError_t e = launch_dca_rotate_keys(a->dtype, a->D, d, (hipStream_t)stream);
  return e == hipSuccess ? STA_OK : hip_fail(e, "dca key rotation");
}

size_t sta_dca_decode_workspace_size(const sta_dca_decode_args* a) {
  if (dca_dec_check(a) != STA_OK) return 0;
  return dca_dec_layout_of(a).total;
}

int sta_dca_decode(const sta_dca_decode_args* a, void* stream) {
  int rc = dca_dec_check(a);
  if (rc != STA_OK) return rc;
  if ((rc = check_rows("q", a->dtype, a->q, a->q_head_stride, 0)) != STA_OK) return rc;
  if ((rc = check_rows("k", a->dtype, a->k, a->k_head_stride, a->k_tok_stride)) != STA_OK) return rc;
  if ((rc = check_rows("v", a->dtype, a->v, a->v_head_stride, a->v_tok_stride)) != STA_OK) return rc;
  if (!a->inv_freq || !a->out) return fail(STA_ERR_INVALID_ARG, "inv_freq and out must be non-NULL");
  const DcaDecLayout L = dca_dec_layout_of(a);
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0) return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  char* ws = (char*)a->workspace;
  DcaDecArgs d{};
  d.q = a->q;
  d.q_head_stride = a->q_head_stride;
  d.k = a->k;
  d.k_head_stride = a->k_head_stride;
  d.k_tok_stride = a->k_tok_stride;
  d.v = a->v;
  d.v_head_stride = a->v_head_stride;
  d.v_tok_stride = a->v_tok_stride;
  d.H = a->H;
  d.Hkv = a->Hkv;
  d.M = a->M;
  d.L = a->chunk_size - a->local_window;
  d.chunk_size = a->chunk_size;
  d.nb = L.nb;
  d.mscale = a->mscale;
  d.scale = a->scale;
  d.inv_freq = a->inv_freq;
  d.out = a->out;
  d.qrot = (float*)(ws + L.qrot_off);
  d.scores = (float*)(ws + L.scores_off);
  d.pmax = (float*)(ws + L.pmax_off);
  d.psum = (float*)(ws + L.psum_off);
  d.part = (float*)(ws + L.part_off);
  hipError_t e = launch_dca_decode(a->dtype, a->D, d, (hipStream_t)stream);
  return e == hipSuccess ? STA_OK : hip_fail(e, "dca decode");
}

}  // extern "C"
