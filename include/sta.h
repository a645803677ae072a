/*
 * sta.h -- C ABI of libsta_hip.so: exact-max shared-selection thresholded attention (prefill)
 * on AMD Instinct MI355X (gfx950).
 *
 * Plain C: device pointers, sizes and a HIP stream handle (passed as void*).  No framework
 * types.  Every entry point is asynchronous on `stream`, performs no host synchronisation and no
 * device allocation: the caller owns every output and passes one workspace buffer whose size
 * comes from sta_shared_workspace_size() (sta_shared_attention_noalloc uses a fixed array inside
 * the library instead).  Calls that share a workspace must not overlap.
 *
 * Geometry.  Kernel A (the two score passes) rotates queries and keys with the a-triple
 * (inv_freq_a, pos_scale_a, rope_scale_a); the reposition and the gather-attention use the
 * c-triple.  PI_exact and YaRN_exact pass the same triple twice; the hybrid file passes two.
 *
 * Tensor layout.  q is (H, N, D), k and v are (Hkv, N, D) with H % Hkv == 0 (kv head = h / (H /
 * Hkv), which is what repeat_kv materialises in the reference).  Element strides per head and
 * per token; the head_dim stride is 1; rows must be 16-byte aligned.  out is (H, N, D)
 * contiguous in the input dtype.  Supported: D in {64, 128}, tile in {32, 64}.
 *
 * Return value: STA_OK or a negative STA_ERR_*; sta_last_error() describes the last failure on
 * the calling thread.
 */
#ifndef STA_H_
#define STA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STA_OK 0
#define STA_ERR_INVALID_ARG (-1)
#define STA_ERR_UNSUPPORTED (-2)
#define STA_ERR_HIP (-3)
#define STA_ERR_WORKSPACE (-4)

#define STA_DTYPE_F32 0
#define STA_DTYPE_BF16 1
#define STA_DTYPE_F16 2

/* key ranking (select_score): frequency, or a weighted vote with frequency as a 1e-6 tiebreak */
#define STA_SCORE_FREQ 0    /* rank by votes */
#define STA_SCORE_MARGIN 1  /* by the summed margin fl(s - fl(m - tau)) + 1e-6 votes */
#define STA_SCORE_EXPMASS 2 /* by the summed exp(fl(s - m)) + 1e-6 votes */

typedef struct sta_shared_args {
  /* inputs */
  const void* q;
  const void* k;
  const void* v;
  int64_t q_head_stride, q_tok_stride;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype;           /* STA_DTYPE_* of q, k, v and out */
  int32_t H, Hkv, N, D;
  const float* tau;        /* (H,) threshold below the exact row max */
  const float* inv_freq_a; /* (D/2,) Kernel A geometry */
  float pos_scale_a, rope_scale_a;
  const float* inv_freq_c; /* (D/2,) reposition + attend geometry */
  float pos_scale_c, rope_scale_c;
  float sm_scale;
  int32_t start_pct;       /* max(0, int(round(pct))) with round-half-even, as the reference */
  int32_t n_global, n_local, tile, k_max, q_pos_base, measure;
  /* outputs (device) */
  void* out;               /* (H, N, D) */
  int32_t* idx;            /* (H, nt, k_max) ascending kept key positions, sentinel N */
  float* newpos_k;         /* (H, nt, k_max) repositioned key positions, 0 at sentinels */
  float* newpos_q;         /* (H, nt, tile) repositioned query positions */
  int32_t* shared_size;    /* (H, nt) |top-X% voted set| */
  int32_t* kept_size;      /* (H, nt) |voted set U forced global/local| before truncation */
  int32_t* chosen;         /* (H, nt) pct step that fit k_max, 0 if none */
  uint8_t* orig_overflow;  /* (H, nt) the requested pct exceeded k_max */
  int32_t* kpct_meas;      /* (H, nt) chosen, refined in 1% steps when measure != 0 */
  uint8_t* overflow20;     /* (H, nt) still over k_max at the floor pct */
  /* optional outputs (NULL to skip) */
  int32_t* votes;          /* (H, nt, N) per-tile key occurrence counts */
  int32_t* row_counts;     /* (H, N) kept keys per query (Kernel A's RowCounts) */
  float* row_max;          /* (H, N) exact row max m of every query */
  /* scratch */
  void* workspace;
  size_t workspace_bytes;
  /* optional instrumentation: NULL, or 5 hipEvent_t handles that sta_shared_attention records
   * on `stream` before the RoPE pre-kernels, before the score kernel, before selection, before
   * the gather and after it (stage durations without a host sync) */
  void* const* stage_events;
  /* ranking of the top-X% cut (added in ABI version 2) */
  int32_t select_score;    /* STA_SCORE_*: the reference's select_score (exact_2.py:450) */
  float* wvotes;           /* optional output (H, nt, N): Kernel A's weighted votes (WMODE 1 / 2);
                            * NULL to skip; ignored for STA_SCORE_FREQ */
} sta_shared_args;

/* ABI version of this header (bumped on any layout change of an argument struct): 5.
 * 2: sta_shared_args.select_score; 3: the rule fields of sta_decode_args and config 4's fields of
 * sta_dca_args; 4: sta_dca_args.mscale, sta_dca_rotate_keys and sta_dca_decode; 5: the chunked
 * entry points and sta_pqstream_args.bits. */
int sta_abi_version(void);

/* Description of the last error returned on the calling thread ("" if none). */
const char* sta_last_error(void);

/* Bytes of device workspace the entry points below need for these arguments (shape fields). */
size_t sta_shared_workspace_size(const sta_shared_args* args);

/* The whole prefill path: RoPE remap, pass 1 (exact row max), pass 2 (threshold + votes),
 * LDS selection (top-X% with the 30->25->20 fallback under k_max, compaction, reposition) and
 * the sparse gather-attention.
 * Replaces shared_pi_attention, shared_selection_triton_exact_2.py:432-486 (also
 * shared_selection_triton_exact.py:376-423, shared_selection_triton_YaRN_exact.py:442-496 and,
 * with two geometries, shared_selection_triton_hybrid_exact.py:450-510). */
int sta_shared_attention(const sta_shared_args* args, void* stream);

/* Bytes of the fixed scratch array behind sta_shared_attention_noalloc (64 MiB per GPU). */
#define STA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* sta_shared_attention without a caller workspace and without any device allocation: the
 * workspace is a fixed device array of STA_NOALLOC_SCRATCH_BYTES inside the library, one copy
 * per GPU, held until the process ends.  args->workspace / workspace_bytes are ignored; the
 * caller still passes every input and output.  Shapes whose workspace
 * (sta_shared_workspace_size) exceeds STA_NOALLOC_SCRATCH_BYTES return STA_ERR_WORKSPACE.
 * Every call on one GPU shares that GPU's array (it keeps the last call's contents), so calls
 * that overlap on one GPU race: serialise them on one stream.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int sta_shared_attention_noalloc(const sta_shared_args* args, void* stream);

/* Kernel A alone: writes votes (required), row_counts, row_max and, for a weighted
 * select_score, wvotes (optional).
 * Replaces the _select_vote_kernel launch, shared_selection_triton_exact_2.py:50-140, 454-465. */
int sta_select_vote(const sta_shared_args* args, void* stream);

/* _build_sets alone (freq ranking) from int32 votes (H, num_tiles, N) with values in [0, 255]
 * (a tile's vote count is at most its tile size; the votes are staged as bytes and values outside
 * that range are not detected: they wrap modulo 256, so the caller must keep them in range);
 * writes idx, newpos_k, newpos_q and the six statistics, all with num_tiles tiles (the
 * reference takes the tile count from the votes tensor, not from N).  Uses pos_scale_c,
 * n_global, n_local, start_pct, tile, k_max, q_pos_base, measure.
 * Replaces _build_sets, shared_selection_triton_exact_2.py:277-426. */
int sta_build_sets(const sta_shared_args* args, const int32_t* votes, int32_t num_tiles, void* stream);

/* _build_sets ranked by weighted votes (select_score "margin" / "expmass"): as sta_build_sets,
 * with the fp32 weighted votes wvotes (H, num_tiles, N) beside the int32 votes; the ranking
 * value is fl(wvotes + fl(1e-6 votes)) and the union size and budgets stay frequency-based.
 * Replaces _build_sets(..., wvotes=..., select_score=...), exact_2.py:277-426 (:299-302). */
int sta_build_sets_weighted(const sta_shared_args* args, const int32_t* votes, const float* wvotes,
                            int32_t num_tiles, void* stream);

/* Kernel C alone: gather + repositioned attention from idx / newpos_k / newpos_q under the
 * c-geometry.  kept_size, when non-NULL, bounds the slots swept; otherwise all k_max slots are.
 * Replaces the _gather_attn_kernel launch, shared_selection_triton_exact_2.py:146-225, 471-485. */
int sta_gather_attention(const sta_shared_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Per-query variant, PQ Union: every query keeps its own threshold passers; the tile's union  */
/* (plus forced global / local keys) is gathered once and a per-slot bitmask selects, for each */
/* query, the keys it attends.  Positions are dense ranks over the kept set, attended under    */
/* base RoPE (inv_freq_c, rope scale 1).  tile must be 32 (one bit per query in an int32).     */
/* ------------------------------------------------------------------------------------------ */

typedef struct sta_pq_args {
  /* inputs (layout rules as sta_shared_args) */
  const void* q;
  const void* k;
  const void* v;
  int64_t q_head_stride, q_tok_stride;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype;
  int32_t H, Hkv, N, D;
  const float* tau;         /* (H,) */
  const float* inv_freq_a;  /* (D/2,) selection geometry */
  float pos_scale_a, rope_scale_a;
  const float* inv_freq_c;  /* (D/2,) attend geometry (base RoPE at dense ranks, scale 1) */
  float sm_scale;
  int32_t n_global, n_local, tile, k_max, q_pos_base;
  int32_t select_score;     /* STA_SCORE_*: ranking when |union U forced| > k_max */
  /* outputs (device) */
  void* out;                /* (H, N, D) */
  int32_t* idx;             /* (H, nt, k_max) ascending kept keys, sentinel N */
  float* newpos_k;          /* (H, nt, k_max) dense rank of each slot, 0 at sentinels */
  float* newpos_q;          /* (H, nt, tile) dense rank of each query's own position */
  int32_t* mask;            /* (H, nt, k_max) per-slot query bits, forced keys -1, sentinels 0 */
  int32_t* usize;           /* (H, nt) |union| before forced keys */
  int32_t* kept_size;       /* (H, nt) |kept| after any truncation */
  uint8_t* overflow;        /* (H, nt) the union with forced keys exceeded k_max */
  /* optional outputs (NULL to skip) */
  int32_t* votes;           /* (H, nt, N) */
  int32_t* bits;            /* (H, nt, N) bit i = keep(query i of the tile, key) */
  float* wvotes;            /* (H, nt, N) weighted votes (zero for STA_SCORE_FREQ) */
  int32_t* row_counts;      /* (H, N) */
  float* row_max;           /* (H, N) */
  void* workspace;
  size_t workspace_bytes;
  void* const* stage_events; /* NULL or 5 hipEvent_t, as for sta_shared_args */
} sta_pq_args;

/* Bytes of device workspace the PQ entry points need for these arguments. */
size_t sta_pq_workspace_size(const sta_pq_args* args);

/* The whole PQ Union prefill.  Replaces shared_pq_attention,
 * shared_selection_triton_perquery.py:459-525. */
int sta_pq_attention(const sta_pq_args* args, void* stream);

/* PQ Kernel A alone: writes votes, bits and wvotes (required) and row_counts / row_max
 * (optional).  Replaces the _select_bits_kernel launch, perquery.py:119-218, 495-508. */
int sta_pq_select_bits(const sta_pq_args* args, void* stream);

/* _build_sets_pq alone from dense (H, num_tiles, N) votes, bits and wvotes (wvotes may be NULL
 * for STA_SCORE_FREQ); writes idx, newpos_k, newpos_q, mask, usize, kept_size and overflow.
 * Replaces _build_sets_pq, perquery.py:363-453. */
int sta_pq_build_sets(const sta_pq_args* args, const int32_t* votes, const int32_t* bits,
                      const float* wvotes, int32_t num_tiles, void* stream);

/* PQ Kernel C alone: gather + dense-rank attention with the per-slot query bitmask.
 * Replaces the _gather_attn_pq_kernel launch, perquery.py:226-312, 511-524. */
int sta_pq_gather_attention(const sta_pq_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Chunk-granular selection ("chunk_exact"): keys grouped into fixed chunks of chunk_size; per   */
/* tile, the forced global / local chunks plus the n_chunk visible chunks of largest value (the */
/* sum, or the mean over its threshold passers, of the passers' rank values: weighted votes for */
/* STA_SCORE_MARGIN / EXPMASS, votes for FREQ; equal values in ascending chunk order) are kept; */
/* their keys up to the tile's last query are attended by every query of the tile (pooled) at   */
/* dense ranks under base RoPE.  At most (forced + n_chunk) chunks: the budget is exact.  The   */
/* prefill runs on sta_pq_args (tile 32): PQ Kernel A, the chunk selection, PQ Kernel C with a  */
/* pooled mask (every valid slot -1).                                                           */
/* ------------------------------------------------------------------------------------------ */
#define STA_CHUNK_SUM 0
#define STA_CHUNK_MEAN 1

typedef struct sta_chunk_params {
  int32_t chunk_size;       /* C: keys per chunk (>= 1) */
  int32_t n_chunk;          /* chunks selected beyond the forced ones (>= 1) */
  int32_t chunk_agg;        /* STA_CHUNK_SUM or STA_CHUNK_MEAN */
  int32_t* passers_kept;    /* optional (H, nt) at prefill, (H, Q) at decode: threshold passers
                               among the kept keys (the measurement counter, chunked.py:205-208) */
} sta_chunk_params;

/* The whole chunked prefill.  Replaces shared_chunk_attention,
 * shared_selection_triton_chunked.py:249-322; requires min(nC, forced + n_chunk) * chunk_size <=
 * k_max (:270-278), forced = ceil(n_global / C) + ceil((n_local + tile - 1) / C) + 1 chunks.
 * args->overflow may be NULL (a chunked tile never overflows). */
int sta_chunk_attention(const sta_pq_args* args, const sta_chunk_params* chunk, void* stream);

/* _build_sets_chunk alone from dense (H, num_tiles, N) votes and weighted votes (NULL for
 * STA_SCORE_FREQ); writes idx, newpos_k, newpos_q, mask (pooled), usize, kept_size.  Replaces
 * _build_sets_chunk, shared_selection_triton_chunked.py:149-243.  No workspace. */
int sta_chunk_build_sets(const sta_pq_args* args, const sta_chunk_params* chunk, const int32_t* votes,
                         const float* wvotes, int32_t num_tiles, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Per-query variant, PQ Stream: every query keeps its own threshold passers (plus forced      */
/* global / local keys) and attends them in one sweep over aligned key blocks, newest first;   */
/* key positions stream: npk = -(d + hi_t - j), d advancing per block by the largest per-query */
/* kept count (or the block's slot count).  No index sets, no k_max.  tile must be 32.          */
/* ------------------------------------------------------------------------------------------ */
#define STA_ADV_MAX 0   /* d += max_i c_i */
#define STA_ADV_FULL 1  /* d += slots the block occupies (native RoPE distances) */

typedef struct sta_pqstream_args {
  const void* q;
  const void* k;
  const void* v;
  int64_t q_head_stride, q_tok_stride;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype;
  int32_t H, Hkv, N, D;
  const float* tau;         /* (H,) */
  const float* inv_freq_a;  /* (D/2,) selection geometry */
  float pos_scale_a, rope_scale_a;
  const float* inv_freq_c;  /* (D/2,) attend geometry (base RoPE, scale 1) */
  float sm_scale;           /* finite and > 0 */
  int32_t n_global, n_local, tile, block_n, pos_advance, use_skip, q_pos_base;
  /* outputs (device) */
  void* out;                /* (H, N, D) */
  float* span;              /* (H, nt) final base d of each tile */
  int32_t* kept;            /* (H, N) keys each query attended */
  float* blocks;            /* (H, nt) key blocks of each tile */
  float* skipped;           /* (H, nt) blocks no query kept a key of */
  /* optional outputs (NULL to skip) */
  float* row_max;           /* (H, N) exact row max under the selection geometry */
  void* workspace;
  size_t workspace_bytes;
  void* const* stage_events; /* NULL or 5 hipEvent_t: before RoPE, before the score passes,
                                before the attend pre-rotation, before the sweep, after it */
  /* ABI 5: optional (H, nt, N) int32 threshold keep bits s >= m - tau (bit i = row i of the
   * tile, causal, rows < N; forced keys not included), as the sweep applied them.  Only keys up
   * to each tile's last query are written: pass zeroed memory. */
  int32_t* bits;
  /* ABI 5: STA_STREAM_AUTO (0): the separate keep-bit pass while its buffer, H * ceil(N / 32) *
   * N * 4 bytes, stays within 4 GiB, the fused sweep beyond; STA_STREAM_FUSED (1): always the
   * fused sweep (error where none exists: fp32 inputs with block_n 64); STA_STREAM_UNFUSED (2). */
  int32_t fused;
} sta_pqstream_args;

#define STA_STREAM_AUTO 0
#define STA_STREAM_FUSED 1
#define STA_STREAM_UNFUSED 2

/* Bytes of device workspace sta_pqstream_attention needs for these arguments. */
size_t sta_pqstream_workspace_size(const sta_pqstream_args* args);

/* The PQ Stream prefill.  Replaces pqstream_attention and its fused _pqstream_kernel,
 * pqstream_kernel.py:174-368, 498-564.  block_n in {32, 64}; q_pos_base must be 0 (:512).
 * Pass 1 (each query's exact row max) runs first.  Fused (sta_pqstream_args.fused), the sweep
 * then computes each block's keep bits itself, as the reference's fused kernel does, with no
 * keep-bit buffer; unfused, pass 2 writes one keep bit per (query, key) and the sweep reads them
 * -- faster at moderate N, but the buffer grows as H N^2 / 8 bytes. */
int sta_pqstream_attention(const sta_pqstream_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* DCA (dual chunk attention) prefill: dense causal attention with chunk-remapped RoPE         */
/* positions.  Keys at j mod L (L = chunk_size - local_window); a query i scores its own chunk */
/* at i mod L, the previous chunk at min(i mod L + L, chunk_size) and older chunks at          */
/* min(2L - 1, chunk_size); tables cos/sin(t * inv_freq) * mscale in the model dtype, mscale = */
/* 0.05 ln(N / pretrain_len) + 1 above pretrain_len.  L must be a multiple of 64.               */
/* ------------------------------------------------------------------------------------------ */
typedef struct sta_dca_args {
  const void* q;            /* (H, N, D) raw, before any rotation */
  const void* k;            /* (Hkv, N, D) raw */
  const void* v;            /* (Hkv, N, D) */
  int64_t q_head_stride, q_tok_stride;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype;
  int32_t H, Hkv, N, D;
  const float* inv_freq;    /* (D/2,) base RoPE frequencies */
  int32_t chunk_size, pretrain_len, local_window;
  float scale;              /* softmax scale (the module's scaling, 1/sqrt(D) for Llama) */
  void* out;                /* (H, N, D) */
  void* workspace;
  size_t workspace_bytes;
  void* const* stage_events; /* NULL or hipEvent_t: dense, 3 (before the rotations, before the
                                sweep, after); with select, 5 (before the rotations, the votes,
                                the selection and the attention, after) */
  /* ABI 3: config 4 -- exact-max selection over the inter-chunk keys (select = 1).  Each 64-query
   * tile of DCA chunk c >= 2 scores its inter keys [0, (c - 1) L) at DCA's inter positions
   * (dca_kernel.py:481-487), takes the exact row max, votes s >= m - tau and selects among them by
   * _build_sets (shared_selection_triton_exact_2.py:277-426) applied to that key range: top
   * start_pct% with the 25 / 20% fallback, tie-inclusive cut, the global keys [0, n_global)
   * forced, k_max cap, unresolved tiles truncated to their k_max smallest keys.  The query then
   * attends the selected inter keys (inter position) plus every key of its own and the previous
   * chunk densely (intra / succ positions), in one softmax.  No repositioning: DCA's positions
   * already stay inside the pretraining window.  With tau = inf, start_pct = 100 and k_max >= N
   * it is the dense DCA attention. */
  int32_t select;           /* 0: dense DCA (the fields below are ignored); 1: config 4 */
  const float* tau;         /* (H,) */
  int32_t start_pct;        /* max(0, round(pct)) */
  int32_t k_max, n_global, measure;
  int32_t* idx;             /* (H, nt, k_max), nt = ceil(N / 64): selected inter keys ascending,
                               sentinel = the tile's inter key count */
  int32_t* shared_size;     /* (H, nt) statistics of the selection, as sta_shared_args */
  int32_t* kept_size;
  int32_t* chosen;
  uint8_t* orig_overflow;
  int32_t* kpct_meas;
  uint8_t* overflow20;
  int32_t* votes;           /* optional (H, nt, N) dense int32 votes (0 past a tile's inter keys) */
  float* row_max;           /* optional (H, N) exact max over the inter keys, -inf without any */
  /* ABI 4: the table factor.  > 0: use it -- a patched model's rotary keeps the factor of the
   * length its tables were last built for (dca_kernel.py:174-231: rebuilt only when a call's
   * length exceeds the last build's length + 512); 0: get_mscale(N / pretrain_len). */
  float mscale;
} sta_dca_args;

/* Bytes of device workspace sta_dca_attention needs for these arguments. */
size_t sta_dca_workspace_size(const sta_dca_args* args);

/* The DCA prefill attention core.  Replaces the prefill branch of dca_forward with its position
 * tables and the log-sum-exp merge of its three attention blocks, dca_kernel.py:166-231,
 * 278-366, 372-489 (the module the reference installs with install_dca_forward, :660-663).
 * With select = 1, config 4: DCA positions with exact-max selection over the inter-chunk keys
 * (no reference combines them; the rule is described at sta_dca_args.select). */
int sta_dca_attention(const sta_dca_args* args, void* stream);

/* Keys of N new tokens at positions pos0 .. pos0 + N - 1, rotated at (pos mod L) with the key
 * table for the KV cache: the cache of a DCA model holds rotated keys.  Replaces
 * k = apply_rotary_pos_emb(k, k_cos, k_sin, position_ids) of dca_forward (dca_kernel.py:434-435)
 * with the cyclic key table of ChunkLlamaRotaryEmbedding (:187-190, 198-206). */
typedef struct sta_dca_rotate_args {
  const void* x;            /* (heads, N, D) raw keys */
  int64_t x_head_stride, x_tok_stride;
  void* out;                /* (heads, N, D) rotated keys in the model dtype */
  int64_t out_head_stride, out_tok_stride;
  int32_t dtype, heads, N, D;
  int32_t pos0;             /* absolute position of row 0 */
  const float* inv_freq;    /* (D/2,) */
  int32_t chunk_size, local_window;
  float mscale;             /* the table factor (> 0) */
} sta_dca_rotate_args;

int sta_dca_rotate_keys(const sta_dca_rotate_args* args, void* stream);

/* DCA at decode: the new token's query at position M - 1 over a cache of M rotated keys.  The
 * query is rotated three ways (intra at (M-1) mod L, succ at min((M-1) mod L + L, chunk_size),
 * inter at min(2L - 1, chunk_size)) and scores the keys [0, inter_end) inter, [inter_end,
 * chunk_start) succ, [chunk_start, M) intra, chunk_start = floor((M-1) / L) L, inter_end =
 * max(0, chunk_start - L); one softmax.  The reference's model-dtype matmuls are kept: scores
 * rnd(rnd(q.k) * scale), weights rnd(softmax in fp32), output rnd(P.V) with rnd the rounding to
 * the model dtype.  Replaces the decode branch of dca_forward, dca_kernel.py:491-522.  Any
 * L = chunk_size - local_window >= 1; H / Hkv <= 16. */
typedef struct sta_dca_decode_args {
  const void* q;            /* (H, D) raw query of the new token */
  int64_t q_head_stride;
  const void* k;            /* (Hkv, M, D) cached keys, rotated (sta_dca_rotate_keys) */
  int64_t k_head_stride, k_tok_stride;
  const void* v;            /* (Hkv, M, D) */
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype, H, Hkv, M, D;
  const float* inv_freq;    /* (D/2,) */
  int32_t chunk_size, local_window;
  float mscale;             /* the table factor (> 0) */
  float scale;              /* softmax scale */
  void* out;                /* (H, D) model dtype */
  void* workspace;
  size_t workspace_bytes;
} sta_dca_decode_args;

/* Bytes of device workspace sta_dca_decode needs for these arguments (0 if they are invalid). */
size_t sta_dca_decode_workspace_size(const sta_dca_decode_args* args);

int sta_dca_decode(const sta_dca_decode_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Decode: each query selects its own key set over the KV cache and attends it.  A batch of Q   */
/* queries shares one cache of M raw (unrotated) keys; query i sits at position q_pos0 + i and  */
/* sees the keys [0, m_i), m_i = M - (Q - 1 - i): the cache prefix K[:, :P + 1] of the         */
/* reference's per-token loop when q_pos0 + Q == M.  Q = 1 is one call of the reference on M   */
/* keys at q_pos = q_pos0.  Selection: keep s >= max - tau, the top pct_decode% of those by    */
/* score when pct_decode < 100, plus the forced keys [0, n_global) U [q_pos - n_local + 1,     */
/* q_pos]; above k_max the forced keys and the best-scored others (tie-inclusive); positions   */
/* repositioned as in the prefill; idx ascending, truncated to k_max, sentinel m_i.  Scores   */
/* under the a-triple, reposition with pos_scale_c, attend under (inv_freq_c, rope_scale_c):   */
/* PI_exact / exact / YaRN_exact pass one geometry twice, the hybrid file two.                 */
/* ------------------------------------------------------------------------------------------ */
/* Per-query selection rules of the decode entry points.
 * STA_RULE_SHARED: _decode_build_sets of the shared files (shared_selection_triton_exact_2.py:
 *   527-604): threshold passers, optional top-pct_decode%, forced global / local / self keys, the
 *   k_max cap by score with a tie-inclusive cut, positions by the fp32 reposition recurrence.
 * STA_RULE_PQ: _decode_build_sets_pq of the per-query file (shared_selection_triton_perquery.py:
 *   651-720): every passer (pct_decode ignored), the forced keys, above k_max the forced keys plus
 *   the top-(k_max - n_forced) others by score with an exact budget (equal scores at the cut
 *   taken in ascending key order), positions = dense ranks over the final set (pos_scale_c
 *   unused); attend with rope_scale_c = 1 and inv_freq_c = the base frequencies, as the
 *   reference's _decode_attend_*_pq do.  Run with Q = M, q_pos0 = 0 it is the per-query prefill
 *   (prefill_mode="perquery", perquery.py:905-924). */
#define STA_RULE_SHARED 0
#define STA_RULE_PQ 1
/* STA_RULE_STREAM: _decode_build_sets_pqs of PQ Stream (pqstream_kernel.py:695-797): every passer
 *   and forced key (no cap: give k_max >= M, the reference's buffer rounds M up to 1024), at
 *   streamed positions -- blocks of block_n keys aligned at 0 walked from the query backwards, key
 *   j of block b at newpos = -(kept keys after b + min(q_pos, end of b) - j), newpos_q = 0; attend
 *   with rope_scale_c = 1 and the base inv_freq_c (_decode_attend_torch / _triton, :800-850). */
#define STA_RULE_STREAM 2

typedef struct sta_decode_args {
  const void* q;            /* (H, Q, D) raw queries */
  const void* k;            /* (Hkv, M, D) raw cache */
  const void* v;            /* (Hkv, M, D) */
  int64_t q_head_stride, q_tok_stride;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int32_t dtype;
  int32_t H, Hkv, Q, M, D;
  const float* tau;         /* (H,) */
  const float* inv_freq_a;  /* (D/2,) scores (selection geometry) */
  float pos_scale_a, rope_scale_a;
  float pos_scale_c;        /* reposition: cpos = key * pos_scale_c */
  const float* inv_freq_c;  /* (D/2,) attend geometry */
  float rope_scale_c, sm_scale;
  int32_t q_pos0;           /* position of query 0; q_pos0 + Q <= M (any q_pos0 >= 0 for the
                               scores alone) */
  int32_t n_global, n_local, k_max;   /* k_max <= 65536 */
  double pct_decode;        /* the reference's pct_decode (100 = keep every passer) */
  int32_t causal;           /* attend: 0 masks sentinel slots only (_decode_attend_torch); 1 also
                               slots past the query's position (Kernel C, _decode_attend_kernelC) */
  /* outputs (device) */
  void* out;                /* (H, Q, D) contiguous, input dtype */
  int32_t* idx;             /* (H, Q, k_max) ascending kept positions, sentinel m_i */
  float* newpos_k;          /* (H, Q, k_max) repositioned key positions, 0 at sentinels; may be
                               NULL under STA_RULE_PQ (selection and attend: the positions are
                               then the slot indices, the rule's dense ranks) */
  float* newpos_q;          /* (H, Q) repositioned query positions */
  /* optional outputs (NULL to skip) */
  int32_t* set_size;        /* (H, Q) |selected set| before the truncation to k_max */
  float* scores;            /* (H, Q, M) per-key scores; entries past m_i are not written */
  void* workspace;
  size_t workspace_bytes;
  void* const* stage_events; /* NULL or 4 hipEvent_t: before the scores, before the selection,
                                before the attend, after it */
  /* ABI 3: the selection rule, its per-query counters and PQ Stream's position blocks */
  int32_t rule;             /* STA_RULE_SHARED, STA_RULE_PQ or STA_RULE_STREAM */
  int32_t* usize;           /* (H, Q) or NULL: STA_RULE_PQ, |threshold passers| before the forced keys */
  uint8_t* overflow;        /* (H, Q) or NULL: STA_RULE_PQ, 1 where passers U forced exceed k_max */
  int32_t block_n;          /* STA_RULE_STREAM: keys per position block */
} sta_decode_args;

/* Bytes of device workspace the decode entry points need for these arguments. */
size_t sta_decode_workspace_size(const sta_decode_args* args);

/* The chunk rule at decode from given scores (H, Q, M) fp32: per query, keep = s >= max - tau,
 * chunk values over the query's keys (exp(s - max) of the kept keys, or 1 for STA_SCORE_FREQ;
 * summed or averaged), the forced global chunks and the chunks of the local window, the n_chunk
 * visible others of largest value, then the chunks' keys up to the query and the query itself
 * at dense ranks into idx / newpos_k / newpos_q / set_size (kept count), and, when
 * args->usize is non-NULL, each query's threshold passers into it.  args->rule and
 * args->pct_decode are ignored.  Replaces _decode_build_sets_chunk,
 * shared_selection_triton_chunked.py:411-489; attend with sta_decode_attend (base RoPE at the
 * ranks, rope_scale_c 1). */
int sta_decode_build_sets_chunk(const sta_decode_args* args, const sta_chunk_params* chunk, int32_t select_score,
                                const float* scores, void* stream);

/* Per-key scores of every query under (inv_freq, pos_scale, rope_scale) into `scores`
 * (H, Q, M) fp32 (row (h, i) written for keys < m_i).
 * Replaces _decode_scores_kernel / _decode_select_kernel, shared_selection_triton_exact_2.py:
 * 235-271, 505-525. */
int sta_decode_scores(const sta_decode_args* args, float* scores, void* stream);

/* Selection from given scores (H, Q, M): writes idx, newpos_k, newpos_q (and set_size; usize and
 * overflow under STA_RULE_PQ).
 * Replaces _decode_build_sets, shared_selection_triton_exact_2.py:527-604 (STA_RULE_SHARED), and
 * _decode_build_sets_pq, shared_selection_triton_perquery.py:651-720 (STA_RULE_PQ). */
int sta_decode_build_sets(const sta_decode_args* args, const float* scores, void* stream);

/* Attend over idx / newpos_k / newpos_q (set_size, when non-NULL, bounds the slots swept).
 * Replaces _decode_attend_torch (causal = 0) and _decode_attend_kernelC (causal = 1),
 * shared_selection_triton_exact_2.py:608-655; with the dense ranks of STA_RULE_PQ and
 * rope_scale_c = 1, _decode_attend_torch_pq / _decode_attend_kernelC_pq,
 * shared_selection_triton_perquery.py:723-778. */
int sta_decode_attend(const sta_decode_args* args, void* stream);

/* Scores, selection and attend in one call: the body of the decode branch of spi_forward,
 * shared_selection_triton_exact_2.py:734-762 (perquery.py:893-924 under STA_RULE_PQ), for all
 * Q queries at once. */
int sta_decode_attention(const sta_decode_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STA_H_ */
