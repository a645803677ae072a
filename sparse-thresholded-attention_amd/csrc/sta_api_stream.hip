// sta_api_stream.hip -- the C ABI of PQ Stream (include/sta.h, sta_pqstream_*).
//
// Launches on one stream: the selection-geometry RoPE pre-kernel (Q and K fragments), pass 1 of
// the score kernel (each query's exact row max, left as its keep threshold on the raw dot), the
// attend-geometry pre-rotation of K at absolute positions, and the stream sweep, which computes
// the keep bits itself (the fused sweep).  Where the fused sweep's staging does not fit the LDS
// (fp32 inputs with block_n 64) pass 2 of the score kernel writes the keep bits instead and the
// sweep reads them.
#include <string.h>

#include "../../include/sta.h"
#include "sta_api_util.h"
#include "sta_kernels.h"

using namespace sta;
using namespace sta_api;

namespace {

constexpr size_t kStreamBitsAuto = (size_t)4 << 30;   // 4 GiB

struct StreamLayout {
  int nt, q_rows_pad, k_rows_pad, Npad, planes;
  bool fused;
  int64_t stride;
  size_t qfrag_off, kfrag_off, ktrig_off, bits_off, xthr_off, ktil_off, total;
};

StreamLayout stream_layout_of(const sta_pqstream_args* a) {
  StreamLayout L;
  L.nt = (a->N + a->tile - 1) / a->tile;
  L.q_rows_pad = L.nt * a->tile;
  L.k_rows_pad = (a->N + 127) / 128 * 128;      // q_pos_base is 0: no keys past N are swept
  if (L.k_rows_pad < L.q_rows_pad) L.k_rows_pad = (L.q_rows_pad + 127) / 128 * 128;
  L.Npad = (a->N + 63) / 64 * 64;
  L.planes = a->dtype == STA_DTYPE_F32 ? 2 : 1;
  L.stride = ((int64_t)a->N + 15) / 16 * 16;
  size_t off = 0;
  L.qfrag_off = off;
  off = align256(off + frag_region_bytes(a->H, L.q_rows_pad, a->D));
  L.kfrag_off = off;
  off = align256(off + frag_region_bytes(a->Hkv, L.k_rows_pad, a->D));
  L.ktrig_off = off;   // the K rotation's (cos, sin) per key row, for the screened pass 1
  off = align256(off + (size_t)L.k_rows_pad * (a->D / 2) * sizeof(float2));
  // the keep-bit buffer holds H * nt * N words: the fused sweep replaces it where asked to, or
  // automatically once it would pass kStreamBitsAuto bytes
  const size_t bits_bytes = (size_t)a->H * L.nt * L.stride * 4;
  const bool can = stream_can_fuse(a->dtype, a->D, a->block_n);
  L.fused = can && (a->fused == STA_STREAM_FUSED || (a->fused == STA_STREAM_AUTO && bits_bytes > kStreamBitsAuto));
  L.bits_off = L.xthr_off = off;
  if (L.fused) off = align256(off + (size_t)a->H * L.q_rows_pad * 4);        // thresholds
  else off = align256(off + (size_t)a->H * L.nt * L.stride * 4);             // keep bits
  L.ktil_off = off;
  off = align256(off + (size_t)a->Hkv * L.Npad * L.planes * a->D * 2);
  L.total = off;
  return L;
}

int stream_check(const sta_pqstream_args* a) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  if (a->dtype != STA_DTYPE_F32 && a->dtype != STA_DTYPE_BF16 && a->dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", a->dtype);
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->N < 1 || a->N >= (1 << 24)) return fail(STA_ERR_INVALID_ARG, "N=%d out of range [1, 2^24)", a->N);
  if (a->D != 64 && a->D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", a->D);
  // the sweep keeps its running max on the raw dots, which orders as the scaled scores only for a
  // positive scale
  if (!(a->sm_scale > 0.0f && a->sm_scale < INFINITY))
    return fail(STA_ERR_INVALID_ARG, "sm_scale=%g must be finite and > 0", (double)a->sm_scale);
  // pqstream_kernel.py:509-518
  if (a->tile != 32) return fail(STA_ERR_INVALID_ARG, "tile %d: BLOCK_M is fixed at 32", a->tile);
  if (a->q_pos_base != 0)
    return fail(STA_ERR_INVALID_ARG, "pqstream prefill expects q_pos_base == 0, got %d", a->q_pos_base);
  if (a->block_n < a->tile - 1)
    return fail(STA_ERR_INVALID_ARG, "block_n=%d < tile-1=%d", a->block_n, a->tile - 1);
  if (a->block_n != 32 && a->block_n != 64)
    return fail(STA_ERR_UNSUPPORTED, "block_n %d not in {32, 64}", a->block_n);
  if (a->pos_advance != STA_ADV_MAX && a->pos_advance != STA_ADV_FULL)
    return fail(STA_ERR_INVALID_ARG, "pos_advance %d is not STA_ADV_MAX / STA_ADV_FULL", a->pos_advance);
  if (a->n_global < 0 || a->n_local < 0)
    return fail(STA_ERR_INVALID_ARG, "n_global=%d / n_local=%d must be >= 0", a->n_global, a->n_local);
  if (a->fused != STA_STREAM_AUTO && a->fused != STA_STREAM_FUSED && a->fused != STA_STREAM_UNFUSED)
    return fail(STA_ERR_INVALID_ARG, "fused=%d is not STA_STREAM_AUTO / FUSED / UNFUSED", a->fused);
  if (a->fused == STA_STREAM_FUSED && !stream_can_fuse(a->dtype, a->D, a->block_n))
    return fail(STA_ERR_UNSUPPORTED, "no fused sweep for this dtype with block_n=%d (LDS)", a->block_n);
  if (stream_lds_bytes(a->dtype, a->D, a->block_n, false) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "block_n=%d needs more than 160 KB of LDS", a->block_n);
  return STA_OK;
}

}  // namespace

extern "C" {

size_t sta_pqstream_workspace_size(const sta_pqstream_args* args) {
  if (stream_check(args) != STA_OK) return 0;
  return stream_layout_of(args).total;
}

int sta_pqstream_attention(const sta_pqstream_args* a, void* stream) {
  int rc = stream_check(a);
  if (rc != STA_OK) return rc;
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride,
                              a->k_tok_stride, a->v_head_stride, a->v_tok_stride};
  if ((rc = check_qkv_ptrs(a->dtype, a->q, a->k, a->v, strides, true)) != STA_OK) return rc;
  if (!a->tau || !a->inv_freq_a || !a->inv_freq_c || !a->out || !a->span || !a->kept || !a->blocks ||
      !a->skipped)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a/c and the outputs must be non-NULL");
  const StreamLayout L = stream_layout_of(a);
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0) return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)a->workspace;
  u32x4* qfrag = (u32x4*)(ws + L.qfrag_off);
  u32x4* kfrag = (u32x4*)(ws + L.kfrag_off);
  uint32_t* bits = L.fused ? nullptr : (uint32_t*)(ws + L.bits_off);
  float* xthr = L.fused ? (float*)(ws + L.xthr_off) : nullptr;
  uint16_t* ktil = (uint16_t*)(ws + L.ktil_off);

  if ((rc = mark_event(a->stage_events, 0, st)) != STA_OK) return rc;
  hipError_t e = launch_rope_frag(a->dtype, a->D, a->q, a->q_head_stride, a->q_tok_stride, a->H, a->N,
                                  L.q_rows_pad, 0, a->pos_scale_a, a->rope_scale_a, a->inv_freq_a, qfrag, st);
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (q)");
  e = launch_rope_frag(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->N, L.k_rows_pad, 0,
                       a->pos_scale_a, a->rope_scale_a, a->inv_freq_a, kfrag, st, false,
                       (float2*)(ws + L.ktrig_off));
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (k)");

  // pass 1 (exact row max) + keep bits s >= m - tau per (query, key): pqstream_kernel.py:229-244, 285
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
  sa.q_pos_base = 0;
  sa.tau = a->tau;
  sa.sm_scale = a->sm_scale;
  sa.votes_stride = L.stride;
  sa.bits = bits;
  sa.xthr = xthr;
  sa.row_max = a->row_max;
  if (L.fused) {
    e = launch_score_thresholds(a->D, sa, st);
    if (e != hipSuccess) return hip_fail(e, "score kernel (thresholds)");
  } else {
    e = launch_score_pq(a->D, STA_SCORE_FREQ, sa, st);
    if (e != hipSuccess) return hip_fail(e, "score kernel (keep bits)");
    if (a->bits) {
      e = launch_expand_pq(bits, nullptr, L.stride, a->H, L.nt, a->N, a->tile, 0, nullptr, a->bits, nullptr, st);
      if (e != hipSuccess) return hip_fail(e, "keep-bit copy");
    }
  }

  // keys at their absolute positions under the attend geometry
  if ((rc = mark_event(a->stage_events, 2, st)) != STA_OK) return rc;
  e = launch_abs_rope(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->N, L.Npad,
                      a->inv_freq_c, ktil, st);
  if (e != hipSuccess) return hip_fail(e, "attend pre-rotation (k)");

  if ((rc = mark_event(a->stage_events, 3, st)) != STA_OK) return rc;
  StreamArgs s{};
  s.q = a->q;
  s.q_head_stride = a->q_head_stride;
  s.q_tok_stride = a->q_tok_stride;
  s.ktil = ktil;
  s.v = a->v;
  s.v_head_stride = a->v_head_stride;
  s.v_tok_stride = a->v_tok_stride;
  s.bits = bits;
  s.bits_stride = L.fused ? a->N : L.stride;
  s.qfrag = L.fused ? qfrag : nullptr;
  s.kfrag = L.fused ? kfrag : nullptr;
  s.q_rows_pad = L.q_rows_pad;
  s.k_rows_pad = L.k_rows_pad;
  s.xthr = xthr;
  s.bits_out = L.fused ? (uint32_t*)a->bits : nullptr;
  s.inv_freq = a->inv_freq_c;
  s.sm_scale = a->sm_scale;
  s.H = a->H;
  s.Hkv = a->Hkv;
  s.N = a->N;
  s.nt = L.nt;
  s.Npad = L.Npad;
  s.n_global = a->n_global;
  s.n_local = a->n_local;
  s.adv_full = a->pos_advance == STA_ADV_FULL;
  s.use_skip = a->use_skip != 0;
  s.out = a->out;
  s.span = a->span;
  s.kept = a->kept;
  s.blocks = a->blocks;
  s.skipped = a->skipped;
  e = launch_stream(a->dtype, a->D, a->block_n, s, st);
  if (e != hipSuccess) return hip_fail(e, "stream kernel");
  return mark_event(a->stage_events, 4, st);
}

}  // extern "C"
