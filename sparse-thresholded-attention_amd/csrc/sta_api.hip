// sta_api.hip -- the C ABI (include/sta.h): argument validation, workspace layout, launches.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <mutex>
#include <string>

#include "../../include/sta.h"
#include "sta_api_util.h"
#include "sta_kernels.h"

using namespace sta;

namespace sta_api {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_qkv_ptrs(int dtype, const void* q, const void* k, const void* v, const int64_t strides[6],
                   bool need_v) {
  const int es = esize(dtype);
  const void* ptrs[3] = {q, k, v};
  for (int i = 0; i < (need_v ? 3 : 2); ++i) {
    if (!ptrs[i]) return fail(STA_ERR_INVALID_ARG, "%c is NULL", "qkv"[i]);
    if (!aligned16(ptrs[i])) return fail(STA_ERR_UNSUPPORTED, "%c is not 16-byte aligned", "qkv"[i]);
    for (int j = 0; j < 2; ++j) {
      const int64_t s = strides[2 * i + j];
      if (s < 0 || (s * es) % 16 != 0)
        return fail(STA_ERR_UNSUPPORTED, "%c %s stride %lld is negative or not 16-byte aligned",
                    "qkv"[i], j ? "token" : "head", (long long)s);
    }
  }
  return STA_OK;
}

}  // namespace sta_api

using namespace sta_api;

namespace {

struct Layout {
  int nt, q_rows_pad, k_rows_pad;
  int64_t votes_stride;
  size_t qfrag_off, kfrag_off, ktrig_off, votes_off, wv_off, total;
};

Layout layout_of(const sta_shared_args* a) {
  Layout L;
  L.nt = (a->N + a->tile - 1) / a->tile;
  L.q_rows_pad = L.nt * a->tile;
  const int64_t kneed = (int64_t)a->q_pos_base + (int64_t)L.nt * a->tile;
  L.k_rows_pad = (int)(((kneed > a->N ? kneed : a->N) + 127) / 128 * 128);
  L.votes_stride = ((int64_t)a->N + 15) / 16 * 16;
  size_t off = 0;
  // 16-bit inputs: the fragment regions carry the fp6 operands of pass 2
  const bool with6 = a->dtype != STA_DTYPE_F32;
  L.qfrag_off = off;
  off = align256(off + frag_region_bytes(a->H, L.q_rows_pad, a->D, with6));
  L.kfrag_off = off;
  off = align256(off + frag_region_bytes(a->Hkv, L.k_rows_pad, a->D, with6));
  L.ktrig_off = off;   // the K rotation's (cos, sin) per key row, for the screened pass 1
  off = align256(off + (size_t)L.k_rows_pad * (a->D / 2) * sizeof(float2));
  L.votes_off = off;
  off = align256(off + (size_t)a->H * L.nt * L.votes_stride);
  L.wv_off = off;   // weighted votes (H, nt, votes_stride) fp32, for a weighted select_score only
  if (a->select_score != STA_SCORE_FREQ) off = align256(off + (size_t)a->H * L.nt * L.votes_stride * 4);
  L.total = off;
  return L;
}

// shape / parameter checks shared by every entry point
int check_common(const sta_shared_args* a) {
  if (!a) return fail(STA_ERR_INVALID_ARG, "args is NULL");
  if (a->dtype != STA_DTYPE_F32 && a->dtype != STA_DTYPE_BF16 && a->dtype != STA_DTYPE_F16)
    return fail(STA_ERR_INVALID_ARG, "dtype %d is not one of STA_DTYPE_F32/BF16/F16", a->dtype);
  if (a->H < 1 || a->Hkv < 1 || a->H % a->Hkv != 0)
    return fail(STA_ERR_INVALID_ARG, "H=%d must be a positive multiple of Hkv=%d", a->H, a->Hkv);
  if (a->N < 1 || a->N >= (1 << 24))
    return fail(STA_ERR_INVALID_ARG, "N=%d out of range [1, 2^24)", a->N);
  if (a->D != 64 && a->D != 128) return fail(STA_ERR_UNSUPPORTED, "head_dim %d not in {64, 128}", a->D);
  if (a->tile != 32 && a->tile != 64) return fail(STA_ERR_UNSUPPORTED, "tile %d not in {32, 64}", a->tile);
  if (a->k_max < 1) return fail(STA_ERR_INVALID_ARG, "k_max=%d must be >= 1", a->k_max);
  if (a->q_pos_base < 0) return fail(STA_ERR_INVALID_ARG, "q_pos_base=%d must be >= 0", a->q_pos_base);
  if (a->n_global < 0 || a->n_local < 0)
    return fail(STA_ERR_INVALID_ARG, "n_global=%d / n_local=%d must be >= 0", a->n_global, a->n_local);
  if (a->select_score < STA_SCORE_FREQ || a->select_score > STA_SCORE_EXPMASS)
    return fail(STA_ERR_INVALID_ARG, "select_score %d is not one of STA_SCORE_*", a->select_score);
  return STA_OK;
}

int check_qkv(const sta_shared_args* a, bool need_v) {
  const int64_t strides[6] = {a->q_head_stride, a->q_tok_stride, a->k_head_stride,
                              a->k_tok_stride, a->v_head_stride, a->v_tok_stride};
  return check_qkv_ptrs(a->dtype, a->q, a->k, a->v, strides, need_v);
}

int check_workspace(const sta_shared_args* a, const Layout& L) {
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(STA_ERR_WORKSPACE, "workspace of %zu bytes at %p is smaller than the %zu needed",
                a->workspace_bytes, a->workspace, L.total);
  if (((uintptr_t)a->workspace & 255u) != 0)
    return fail(STA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return STA_OK;
}

int check_sets_outputs(const sta_shared_args* a) {
  if (!a->idx || !a->newpos_k || !a->newpos_q || !a->shared_size || !a->kept_size || !a->chosen ||
      !a->orig_overflow || !a->kpct_meas || !a->overflow20)
    return fail(STA_ERR_INVALID_ARG, "a selection output pointer is NULL");
  if (select_lds_bytes(a->N, a->k_max) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED, "N=%d with k_max=%d needs more than 160 KB of LDS for selection",
                a->N, a->k_max);
  if (a->select_score != STA_SCORE_FREQ && select_w_lds_bytes(a->N, a->k_max, true) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED,
                "weighted ranking with k_max=%d needs more than 160 KB of LDS for selection", a->k_max);
  return STA_OK;
}

SelectArgs select_args_of(const sta_shared_args* a, const Layout& L) {
  SelectArgs s;
  memset(&s, 0, sizeof(s));
  s.H = a->H;
  s.nt = L.nt;
  s.N = a->N;
  s.T = a->tile;
  s.k_max = a->k_max;
  s.q_pos_base = a->q_pos_base;
  s.n_global = a->n_global;
  s.n_local = a->n_local;
  s.pos_scale = a->pos_scale_c;
  // pct_steps = [start] + [c for c in (25, 20) if c < start]   (exact_2.py:309-310)
  s.nsteps = 0;
  s.steps[s.nsteps++] = a->start_pct;
  if (25 < a->start_pct) s.steps[s.nsteps++] = 25;
  if (20 < a->start_pct) s.steps[s.nsteps++] = 20;
  // K_ord = max(1, min(N, ceil(max_pct / 100.0 * N)))   (exact_2.py:320)
  int64_t kord = (int64_t)ceil((double)a->start_pct / 100.0 * (double)a->N);
  if (kord > a->N) kord = a->N;
  if (kord < 1) kord = 1;
  s.K_ord = kord;
  s.start_pct = a->start_pct;
  s.measure = a->measure;
  s.idx = a->idx;
  s.newpos_k = a->newpos_k;
  s.newpos_q = a->newpos_q;
  s.shared_size = a->shared_size;
  s.kept_size = a->kept_size;
  s.chosen = a->chosen;
  s.orig_overflow = a->orig_overflow;
  s.kpct_meas = a->kpct_meas;
  s.overflow20 = a->overflow20;
  s.votes_out = a->votes;
  s.wvotes_out = a->select_score != STA_SCORE_FREQ ? a->wvotes : nullptr;
  return s;
}

int mark(const sta_shared_args* a, int i, hipStream_t st) { return mark_event(a->stage_events, i, st); }

int run_kernel_a(const sta_shared_args* a, const Layout& L, hipStream_t st) {
  char* ws = (char*)a->workspace;
  u32x4* qfrag = (u32x4*)(ws + L.qfrag_off);
  u32x4* kfrag = (u32x4*)(ws + L.kfrag_off);
  int rc = mark(a, 0, st);
  if (rc != STA_OK) return rc;
  // 16-bit inputs with plain votes score pass 2 with the fp6 correction (sta_fp6.h); fp32 inputs
  // keep the three-product scores throughout
  const bool want6 = a->dtype != STA_DTYPE_F32 && a->select_score == STA_SCORE_FREQ && !a->row_counts;
  hipError_t e = launch_rope_frag(a->dtype, a->D, a->q, a->q_head_stride, a->q_tok_stride, a->H, a->N,
                                  L.q_rows_pad, a->q_pos_base, a->pos_scale_a, a->rope_scale_a,
                                  a->inv_freq_a, qfrag, st, want6);
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (q)");
  e = launch_rope_frag(a->dtype, a->D, a->k, a->k_head_stride, a->k_tok_stride, a->Hkv, a->N,
                       L.k_rows_pad, 0, a->pos_scale_a, a->rope_scale_a, a->inv_freq_a, kfrag, st, want6,
                       (float2*)(ws + L.ktrig_off));
  if (e != hipSuccess) return hip_fail(e, "rope pre-kernel (k)");
  if ((rc = mark(a, 1, st)) != STA_OK) return rc;
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
  sa.votes = (uint8_t*)(ws + L.votes_off);
  sa.votes_stride = L.votes_stride;
  sa.row_max = a->row_max;
  sa.row_counts = a->row_counts;
  sa.want_fast6 = want6 ? 1 : 0;
  if (a->select_score != STA_SCORE_FREQ) {
    sa.wvotes = (float*)(ws + L.wv_off);
    e = launch_score_weighted(a->D, a->tile, a->select_score, sa, st);
  } else {
    e = launch_score(a->D, a->tile, sa, st);
  }
  if (e != hipSuccess) return hip_fail(e, "score kernel");
  return STA_OK;
}

int run_gather(const sta_shared_args* a, const Layout& L, hipStream_t st) {
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
  g.nt = L.nt;
  g.k_max = a->k_max;
  g.q_pos_base = a->q_pos_base;
  g.inv_freq = a->inv_freq_c;
  g.rope_scale = a->rope_scale_c;
  g.sm_scale = a->sm_scale;
  g.idx = a->idx;
  g.newpos_k = a->newpos_k;
  g.newpos_q = a->newpos_q;
  g.kept_size = a->kept_size;
  g.out = a->out;
  hipError_t e = launch_gather(a->dtype, a->D, a->tile, g, st);
  if (e != hipSuccess) return hip_fail(e, "gather kernel");
  return STA_OK;
}

// the whole prefill path on `st`, with args->workspace holding at least L.total bytes
int run_shared(const sta_shared_args* args, const Layout& L, hipStream_t st);

int check_shared_call(const sta_shared_args* args) {
  int rc = check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = check_qkv(args, true)) != STA_OK) return rc;
  if (!args->tau || !args->inv_freq_a || !args->inv_freq_c || !args->out)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a, inv_freq_c and out must be non-NULL");
  return check_sets_outputs(args);
}

// ------------------------------------------------------------------------------------------
// Scratch of the allocation-free entry point: a fixed device array in this library's code
// object, one copy per GPU, held until the process ends.  Its name is a host-side handle, not a
// device address: the device address of each GPU's copy comes from hipGetSymbolAddress, taken
// once per device with that device current and kept here.  Every call on one GPU shares that
// GPU's copy, so calls that overlap on one GPU race.  Nothing in it has to start at zero: every
// byte the kernels read is written earlier in the same call.
// ------------------------------------------------------------------------------------------
constexpr size_t kScratchBytes = STA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(STA_ERR_UNSUPPORTED, "device %d above %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p || ((uintptr_t)p & 255u) != 0)
      return fail(STA_ERR_HIP, "scratch of device %d at %p is not 256-byte aligned", dev, p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return STA_OK;
}

}  // namespace

extern "C" {

int sta_abi_version(void) { return 5; }

const char* sta_last_error(void) { return g_last_error.c_str(); }

size_t sta_shared_workspace_size(const sta_shared_args* args) {
  if (check_common(args) != STA_OK) return 0;
  return layout_of(args).total;
}

int sta_shared_attention(const sta_shared_args* args, void* stream) {
  int rc = check_shared_call(args);
  if (rc != STA_OK) return rc;
  const Layout L = layout_of(args);
  if ((rc = check_workspace(args, L)) != STA_OK) return rc;
  return run_shared(args, L, (hipStream_t)stream);
}

int sta_shared_attention_noalloc(const sta_shared_args* args, void* stream) {
  int rc = check_shared_call(args);
  if (rc != STA_OK) return rc;
  const Layout L = layout_of(args);
  if (L.total > kScratchBytes)
    return fail(STA_ERR_WORKSPACE,
                "sta_shared_attention_noalloc: this shape needs %zu bytes of scratch, above the "
                "library's fixed %zu (use sta_shared_attention with a caller workspace)",
                L.total, kScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(&ws)) != STA_OK) return rc;
  sta_shared_args a = *args;   // the same call with the library's scratch as its workspace
  a.workspace = ws;
  a.workspace_bytes = kScratchBytes;
  return run_shared(&a, L, (hipStream_t)stream);
}

}  // extern "C"

namespace {

int run_shared(const sta_shared_args* args, const Layout& L, hipStream_t st) {
  int rc;
  if ((rc = run_kernel_a(args, L, st)) != STA_OK) return rc;
  if ((rc = mark(args, 2, st)) != STA_OK) return rc;
  SelectArgs s = select_args_of(args, L);
  s.votes = (const void*)((char*)args->workspace + L.votes_off);
  s.votes_stride = L.votes_stride;
  hipError_t e;
  if (args->select_score != STA_SCORE_FREQ) {
    s.wvotes = (const float*)((char*)args->workspace + L.wv_off);
    e = launch_select_weighted(s, 1, st);
  } else {
    e = launch_select(s, 1, st);
  }
  if (e != hipSuccess) return hip_fail(e, "select kernel");
  if ((rc = mark(args, 3, st)) != STA_OK) return rc;
  if ((rc = run_gather(args, L, st)) != STA_OK) return rc;
  return mark(args, 4, st);
}

}  // namespace

extern "C" {

int sta_select_vote(const sta_shared_args* args, void* stream) {
  int rc = check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = check_qkv(args, false)) != STA_OK) return rc;
  if (!args->tau || !args->inv_freq_a || !args->votes)
    return fail(STA_ERR_INVALID_ARG, "tau, inv_freq_a and votes must be non-NULL");
  const Layout L = layout_of(args);
  if ((rc = check_workspace(args, L)) != STA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = run_kernel_a(args, L, st)) != STA_OK) return rc;
  const bool wv = args->select_score != STA_SCORE_FREQ && args->wvotes;
  hipError_t e = launch_expand_votes((const uint8_t*)((char*)args->workspace + L.votes_off), L.votes_stride,
                                     args->H, L.nt, args->N, args->tile, args->q_pos_base, args->votes,
                                     wv ? (const float*)((char*)args->workspace + L.wv_off) : nullptr,
                                     wv ? args->wvotes : nullptr, st);
  if (e != hipSuccess) return hip_fail(e, "vote expansion");
  return STA_OK;
}

int sta_build_sets(const sta_shared_args* args, const int32_t* votes, int32_t num_tiles, void* stream) {
  int rc = check_common(args);
  if (rc != STA_OK) return rc;
  if (!votes) return fail(STA_ERR_INVALID_ARG, "votes is NULL");
  if (num_tiles < 1) return fail(STA_ERR_INVALID_ARG, "num_tiles=%d must be >= 1", num_tiles);
  if ((rc = check_sets_outputs(args)) != STA_OK) return rc;
  Layout L = layout_of(args);
  L.nt = num_tiles;
  SelectArgs s = select_args_of(args, L);
  s.votes = votes;
  s.votes_stride = args->N;
  s.votes_dense = 1;
  s.votes_out = nullptr;
  hipError_t e = launch_select(s, 4, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "select kernel");
  return STA_OK;
}

int sta_build_sets_weighted(const sta_shared_args* args, const int32_t* votes, const float* wvotes,
                            int32_t num_tiles, void* stream) {
  int rc = check_common(args);
  if (rc != STA_OK) return rc;
  if (!votes || !wvotes) return fail(STA_ERR_INVALID_ARG, "votes and wvotes must be non-NULL");
  if (num_tiles < 1) return fail(STA_ERR_INVALID_ARG, "num_tiles=%d must be >= 1", num_tiles);
  if (args->tile > 256) return fail(STA_ERR_UNSUPPORTED, "tile %d above 256", args->tile);
  if ((rc = check_sets_outputs(args)) != STA_OK) return rc;
  if (select_w_lds_bytes(args->N, args->k_max, true) > 160 * 1024)
    return fail(STA_ERR_UNSUPPORTED,
                "weighted ranking with k_max=%d needs more than 160 KB of LDS for selection", args->k_max);
  Layout L = layout_of(args);
  L.nt = num_tiles;
  SelectArgs s = select_args_of(args, L);
  s.votes = votes;
  s.wvotes = wvotes;
  s.votes_stride = args->N;
  s.votes_dense = 1;
  s.votes_out = nullptr;
  s.wvotes_out = nullptr;
  hipError_t e = launch_select_weighted(s, 4, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "weighted select kernel");
  return STA_OK;
}

int sta_gather_attention(const sta_shared_args* args, void* stream) {
  int rc = check_common(args);
  if (rc != STA_OK) return rc;
  if ((rc = check_qkv(args, true)) != STA_OK) return rc;
  if (!args->inv_freq_c || !args->out || !args->idx || !args->newpos_k || !args->newpos_q)
    return fail(STA_ERR_INVALID_ARG, "inv_freq_c, out, idx, newpos_k and newpos_q must be non-NULL");
  const Layout L = layout_of(args);
  return run_gather(args, L, (hipStream_t)stream);
}

}  // extern "C"
