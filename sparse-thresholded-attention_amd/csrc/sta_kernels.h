// sta_kernels.h -- internal argument blocks and launchers of the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "sta_device.h"
#include "sta_fp6.h"

namespace sta {

// Workspace region of the selection-geometry fragments of `heads` x `rows_pad` rows: the
// fragments (hi/lo bf16, 4 bytes per element), then per row (||hi||, ||lo||), then per head the
// maxima of those two norms over its rows -- all three written by the RoPE pre-kernel -- then,
// for the query side, the screened pass 1's results: each row's exact raw maximum and one
// fallback flag per 256-row workgroup.  After them (256-byte aligned) the fp6 correction
// operands of the pass-2 kernel that scores with one bf16 product plus an fp6 correction
// (sta_fp6.h): the e2m3 planes of each row's [hi | x - hi] vector, one E8M0 scale per 32
// elements, per row the norms of the two halves' quantisation errors, and their per-head maxima.
inline size_t frag_a256(size_t x) { return (x + 255) & ~(size_t)255; }
inline size_t frag_base_bytes(int heads, int rows_pad, int D) {
  return (size_t)heads * rows_pad * D * 4 + (size_t)heads * rows_pad * 8 + (size_t)heads * 8 +
         (size_t)heads * rows_pad * 4 + (size_t)heads * (rows_pad / 256 + 1) * 4;
}
// fp6 planes: per (head, 32-row block) D/32 units of 3 planes x 64 lanes x 8 bytes (1.5 D bytes
// per row); scales: per (head, 32-row block) 64 lane dwords
inline size_t frag6_plane_bytes(int heads, int rows_pad, int D) { return (size_t)heads * rows_pad * D * 3 / 2; }
// with6: the region carries the fp6 operands (only the shared path's pass 2 reads them)
inline size_t frag_region_bytes(int heads, int rows_pad, int D, bool with6 = false) {
  if (!with6) return frag_base_bytes(heads, rows_pad, D);
  return frag_a256(frag_base_bytes(heads, rows_pad, D)) + frag_a256(frag6_plane_bytes(heads, rows_pad, D)) +
         (size_t)heads * rows_pad * 8 + (size_t)heads * rows_pad * 8 + (size_t)heads * 8;
}
inline uint64_t* frag6_planes(const u32x4* frag, int heads, int rows_pad, int D) {
  return (uint64_t*)((char*)frag + frag_a256(frag_base_bytes(heads, rows_pad, D)));
}
inline uint32_t* frag6_scales(const u32x4* frag, int heads, int rows_pad, int D) {
  return (uint32_t*)((char*)frag6_planes(frag, heads, rows_pad, D) + frag_a256(frag6_plane_bytes(heads, rows_pad, D)));
}
inline float2* frag6_dnorms(const u32x4* frag, int heads, int rows_pad, int D) {
  return (float2*)(frag6_scales(frag, heads, rows_pad, D) + (size_t)heads * rows_pad * 2);
}
inline float2* frag6_dnorm_max(const u32x4* frag, int heads, int rows_pad, int D) {
  return frag6_dnorms(frag, heads, rows_pad, D) + (size_t)heads * rows_pad;
}
inline float2* frag_norms(const u32x4* frag, int heads, int rows_pad, int D) {
  return (float2*)((char*)frag + (size_t)heads * rows_pad * D * 4);
}
inline float2* frag_norm_max(const u32x4* frag, int heads, int rows_pad, int D) {
  return frag_norms(frag, heads, rows_pad, D) + (size_t)heads * rows_pad;
}
inline float* frag_rowmax(const u32x4* frag, int heads, int rows_pad, int D) {
  return (float*)(frag_norm_max(frag, heads, rows_pad, D) + heads);
}
inline int* frag_flags(const u32x4* frag, int heads, int rows_pad, int D) {
  return (int*)(frag_rowmax(frag, heads, rows_pad, D) + (size_t)heads * rows_pad);
}

struct ScoreArgs {
  const u32x4* qfrag;     // selection-geometry Q fragments (hi/lo), rows padded to nt*tile
  const u32x4* kfrag;     // selection-geometry K fragments (hi/lo), rows padded to k_rows_pad
  const float2* qnorm;    // (H, q_rows_pad) (||q_hi||, ||q_lo||) of every fragment row
  const float2* knorm_max;// (Hkv,) maxima of (||k_hi||, ||k_lo||) over the head's rows
  int H, Hkv, N, nt;
  int q_rows_pad, k_rows_pad;
  int q_pos_base;
  const float* tau;       // (H,)
  float sm_scale;
  uint8_t* votes;         // (H, nt, votes_stride): keys < min(N, hi_t) written
  int64_t votes_stride;
  uint32_t* bits;         // per-query variant: (H, nt, votes_stride) keep bits, bit i = row i
  float* wvotes;          // (H, nt, votes_stride) margin / expmass votes (per-query or shared)
  float* row_max;         // (H, N) or null
  int32_t* row_counts;    // (H, N) or null
  int ib;                 // set by the launcher: block-index bits of the screened pass 1, 0 = off
  int exact_pass1;        // 1: always run the three-product pass 1 sweep
  int screened;           // set by the launcher: the screen kernel ran before the pass-2 kernel
  float* srmax;           // (H, q_rows_pad) the screen's exact raw row maxima
  int* sflags;            // (H, ngroups) the screen's fallback flags
  float* xthr;            // thresholds-only instance: (H, q_rows_pad) each row's x0 (+inf: no row)
  // pass 2 with one bf16 product plus an fp6 correction (plain votes only, sta_score6.hip)
  int want_fast6;         // caller: the fragments carry the fp6 operands (16-bit inputs)
  int fast6;              // set by the launcher: the fp6 pass-2 kernel runs before the
                          // three-product one, which then skips the workgroups it served
  const float2* qnorm_max;// (H,) maxima of (||q_hi||, ||q_lo||)
  const uint64_t* q6;     // fp6 planes / scales / error norms of the Q and K fragments
  const uint32_t* q6sc;
  const float2* q6dn;     // (H, q_rows_pad) per row
  const float2* q6dmax;   // (H,)
  const uint64_t* k6;
  const uint32_t* k6sc;
  const float2* k6dmax;   // (Hkv,)
  // The screened pass 1 scores its candidate keys from the raw K rows and the K rotation's
  // (cos, sin) table (key-major: a few cache lines per key) when ktrig is set, else from the K
  // fragments.  kraw: the K input as the rope pre-kernel read it (dtype kraw_dt, strides in elements).
  const float2* ktrig;    // (k_rows_pad, D/2) scaled (cos, sin) of every key row, or null
  const void* kraw;
  int64_t kraw_hs, kraw_ts;
  int kraw_dt;
};

struct SelectArgs {
  const void* votes;      // uint8 or int32 (H, nt, votes_stride), values in [0, 255]
  int64_t votes_stride;
  int votes_dense;        // 1: all N votes are valid; 0: keys < min(N, tile end) are valid
  int H, nt, N, T, k_max, q_pos_base, n_global, n_local;
  float pos_scale;
  int nsteps;
  int steps[3];
  int64_t K_ord;
  int start_pct, measure;
  int32_t* idx;
  float* newpos_k;
  float* newpos_q;
  int32_t* shared_size;
  int32_t* kept_size;
  int32_t* chosen;
  uint8_t* orig_overflow;
  int32_t* kpct_meas;
  uint8_t* overflow20;
  int32_t* votes_out;     // optional dense int32 copy (H, nt, N)
  const float* wvotes;    // weighted ranking: (H, nt, votes_stride) margin / expmass votes
  float* wvotes_out;      // optional dense fp32 copy (H, nt, N) of the weighted votes
  int dca_L;              // > 0: DCA inter-key selection -- tile t of chunk c = tstart / dca_L
                          // selects among its inter keys [0, max(0, (c - 1) dca_L)) as if they
                          // were the whole key axis (N and K_ord per tile; the local window then
                          // falls outside it); 0: the shared selection over [0, N)
  int stage_slots;        // set by the launcher: the kept slots are gathered in LDS and written
                          // coalesced (short rows), or written straight from the compaction
};

struct GatherArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t q_head_stride, q_tok_stride, k_head_stride, k_tok_stride, v_head_stride, v_tok_stride;
  int H, Hkv, N, nt, k_max, q_pos_base;
  const float* inv_freq;
  float rope_scale, sm_scale;
  const int32_t* idx;
  const float* newpos_k;
  const float* newpos_q;
  const int32_t* kept_size;  // (H, nt) or null (then every k_max slot is swept)
  const int32_t* mask;       // (H, nt, k_max) per-slot query bits (tile 32) or null
  void* out;                 // (H, N, D) contiguous
};

// per-query (PQ Union) set construction: shared_selection_triton_perquery.py:363-453
struct PqSelectArgs {
  const uint32_t* bits;   // (H, nt, stride) keep bits
  const float* wvotes;    // (H, nt, stride) weighted votes, or null (rank by votes)
  const int32_t* votes;   // (H, nt, stride) votes, or null (popcount of the bits)
  int64_t stride;
  int dense;              // 1: all N keys valid; 0: keys >= min(N, tile end) read as zero
  int H, nt, N, T, k_max, q_pos_base, n_global, n_local;
  int32_t* idx;
  float* newpos_k;
  float* newpos_q;
  int32_t* mask;
  int32_t* usize;
  int32_t* kept_size;
  uint8_t* overflow;
};

// chunk-granular set construction: shared_selection_triton_chunked.py:149-243, 411-489
struct ChunkSelectArgs {
  const uint32_t* bits;   // (H, nt, stride) compact keep bits (votes = popcount), or null
  const int32_t* votes;   // (H, nt, stride) votes, or null
  const float* wvotes;    // (H, nt, stride) weighted votes, or null (rank by votes)
  int64_t stride;
  int dense;              // 1: all N keys valid; 0: keys >= min(N, tile end) read as zero
  int H, nt, N, T, k_max, q_pos_base, n_global, n_local, C, n_chunk, mean;
  int32_t* idx;
  float* newpos_k;
  float* newpos_q;
  int32_t* mask;          // or null
  int32_t* usize;
  int32_t* kept_size;
  uint8_t* overflow;      // or null (always 0)
  int32_t* passers_kept;  // or null
};
struct ChunkDecodeArgs {
  const float* scores;    // (H, Q, M)
  const float* tau;       // (H,)
  int H, Q, M, q_pos0, k_max, n_global, n_local, C, n_chunk, weighted, mean;
  int32_t* idx;           // (H, Q, k_max), sentinel m_i
  float* newpos_k;
  float* newpos_q;        // (H, Q)
  int32_t* kept_size;     // (H, Q)
  int32_t* passers_kept;  // or null
  int32_t* usize;         // or null: (H, Q) threshold passers of the query
};
size_t chunk_select_lds_bytes(int n_keys, int C);
hipError_t launch_chunk_select(const ChunkSelectArgs& a, hipStream_t st);
hipError_t launch_chunk_decode_select(const ChunkDecodeArgs& a, hipStream_t st);

// PQ Stream attend sweep: pqstream_kernel.py:174-368
struct StreamArgs {
  const void* q;
  int64_t q_head_stride, q_tok_stride;
  const uint16_t* ktil;     // (Hkv, Npad, P, D) keys rotated at their absolute positions
  const void* v;
  int64_t v_head_stride, v_tok_stride;
  const uint32_t* bits;     // unfused sweep: (H, nt, bits_stride) threshold keep bits, bit i = row i
  int64_t bits_stride;
  // fused sweep: the keep bits are computed in the sweep from the selection-geometry fragments
  const u32x4* qfrag;       // (H, q_rows_pad) Q fragments (hi / lo), score-kernel layout
  const u32x4* kfrag;       // (Hkv, k_rows_pad) K fragments
  int q_rows_pad, k_rows_pad;
  const float* xthr;        // (H, q_rows_pad) keep threshold on the raw dot, +inf past N
  uint32_t* bits_out;       // optional (H, nt, bits_stride): the threshold bits the sweep computed
  const float* inv_freq;    // attend geometry (base RoPE)
  float sm_scale;
  int H, Hkv, N, nt, Npad, n_global, n_local, adv_full, use_skip;
  void* out;                // (H, N, D)
  float* span;              // (H, nt)
  int32_t* kept;            // (H, N)
  float* blocks;            // (H, nt)
  float* skipped;           // (H, nt)
};

// DCA attention sweep: dca_kernel.py:372-489
struct DcaArgs {
  const uint16_t* qrot;     // (3, H, Npad, P, D) queries in their intra / succ / inter positions
  const uint16_t* krot;     // (Hkv, Npad, P, D) keys at j mod L
  const void* v;
  int64_t v_head_stride, v_tok_stride;
  int H, Hkv, N, Npad, L;
  float scale;
  void* out;                // (H, N, D)
  // config 4 (selected inter keys + dense local keys); state == null: dense DCA
  const int32_t* idx;       // (H, nt64, k_max) each 64-query tile's selected inter keys
  const int32_t* kept_size; // (H, nt64) its selected count (slots past min(kept, k_max) unused)
  int k_max, nt64;
  float* state;             // (H, Npad, D + 4) per row: unnormalised o (D), running max, sum
};

// config 4's selection over DCA's inter-chunk keys (sta_dca_sel.hip)
struct DcaVoteArgs {
  const uint16_t* qrot;   // (3, H, Npad, P, D) rotated queries; variant 2 = the inter position
  const uint16_t* krot;   // (Hkv, Npad, P, D) rotated keys
  int H, Hkv, N, Npad, L, nt;   // nt: 64-query tiles
  float scale;
  const float* tau;       // (H,)
  float* rmax;            // (H, Npad) raw maxima over the inter keys (pass 0 writes, pass 1 reads)
  float* row_max;         // (H, N) or null: fl(max * scale), -inf where a row has no inter keys
  uint8_t* votes;         // (H, nt, votes_stride): tile t's votes for its inter keys [0, ext_t)
  int64_t votes_stride;
};
hipError_t launch_dca_votes(int dtype, int D, const DcaVoteArgs& a, hipStream_t st);

// DCA key rotation into the cache and DCA decode (sta_dca_dec.hip)
struct DcaRotArgs {
  const void* x;            // (heads, N, D) raw keys
  int64_t x_head_stride, x_tok_stride;
  void* out;                // (heads, N, D) rotated, model dtype
  int64_t out_head_stride, out_tok_stride;
  int heads, N, pos0, L;
  float mscale;
  const float* inv_freq;
};
hipError_t launch_dca_rotate_keys(int dtype, int D, const DcaRotArgs& a, hipStream_t st);

struct DcaDecArgs {
  const void* q;            // (H, D) the new token's raw query, at position M - 1
  int64_t q_head_stride;
  const void* k;            // (Hkv, M, D) cached keys, rotated at j mod L
  int64_t k_head_stride, k_tok_stride;
  const void* v;            // (Hkv, M, D)
  int64_t v_head_stride, v_tok_stride;
  int H, Hkv, M, L, chunk_size, nb;
  float mscale, scale;
  const float* inv_freq;
  void* out;                // (H, D) model dtype
  float* qrot;              // workspace: (H, 3, D) rotated query variants
  float* scores;            // (H, M)
  float* pmax;              // (H, nb) per 256-key block: max score, sum of exp(s - max)
  float* psum;
  float* part;              // (H, nb, D) partial P.V
};
int dca_dec_nblocks(int M);
int dca_dec_max_group();
hipError_t launch_dca_decode(int dtype, int D, const DcaDecArgs& a, hipStream_t st);

// Score rows in 64-row tiles: (H, ceil(Q / 64), ceil(M / SCORE_TW), 64, SCORE_TW) floats, the
// layout the batched score rows kernel writes when only the selection of the same call reads the
// scores.  Key j of query i sits at score_tile_row(...) + (j / SCORE_TW) * 64 * SCORE_TW +
// j % SCORE_TW; rows past Q and keys past M are padding.  A wave's 64 x 32 block of scores then
// lands inside one 32 KB tile, and a row is read in 512-byte pieces.
constexpr int SCORE_TW_LG = 7;
constexpr int SCORE_TW = 1 << SCORE_TW_LG;
__host__ __device__ inline int64_t score_tiles_per_head(int Q, int M) {
  return (int64_t)((Q + 63) / 64) * 64 * (((M + SCORE_TW - 1) / SCORE_TW) * SCORE_TW);
}
__host__ __device__ inline int64_t score_tile_row(int h, int i, int Q, int M) {
  return h * score_tiles_per_head(Q, M) + ((int64_t)(i >> 6) * ((M + SCORE_TW - 1) / SCORE_TW) << (6 + SCORE_TW_LG)) +
         ((i & 63) << SCORE_TW_LG);
}

// decode: Q queries over one cache of M keys, query i at position q_pos0 + i seeing keys
// [0, M - (Q - 1 - i)): shared_selection_triton_exact_2.py:235-271, 505-655
struct DecodeArgs {
  const void* q;          // (H, Q, D) raw
  int64_t q_hs, q_ts;
  const void* k;          // (Hkv, M, D) raw cache
  int64_t k_hs, k_ts;
  const void* v;
  int64_t v_hs, v_ts;
  int H, Hkv, Q, M, q_pos0;
  const float* inv_freq_a;  // selection geometry (scores)
  float pos_scale_a, rope_scale_a;
  float pos_scale_c;        // reposition
  const float* inv_freq_c;  // attend geometry
  float rope_scale_c, sm_scale;
  const float* tau;       // (H,)
  int n_global, n_local, k_max;
  int use_pct;            // pct_decode < 100
  float pct_frac;         // float32(pct_decode / 100)
  float* scores;          // (H, Q, M), or 64 x 32 tiles when score_tiles
  int score_tiles;        // the scores' layout (score_tile_row)
  uint32_t* keys;         // key store of the selection when the cache is too long for LDS
  int32_t* idx;           // (H, Q, k_max)
  float* newpos_k;        // (H, Q, k_max)
  float* newpos_q;        // (H, Q)
  int32_t* set_size;      // (H, Q) or null
  int causal;             // attend also masks slots past the query's position
  float* part;            // (H * Q, nsplit, D + 2) split states of the attend
  const float* qrot;      // (H, Q, D) rotated queries, or null (the score kernel rotates them)
  void* out;              // (H, Q, D)
  int rule;               // 0: _decode_build_sets (shared files); 1: _decode_build_sets_pq;
                          // 2: _decode_build_sets_pqs (PQ Stream, streamed positions)
  int block_n;            // rule 2: the position blocks
  int32_t* usize;         // (H, Q) or null: rule 1, |threshold passers|
  uint8_t* overflow;      // (H, Q) or null: rule 1, passers U forced above k_max
  int dense_ranks;        // rule 1 in one call with its selection: newpos_k[s] == s on every slot
};

// scores of a batch of queries from the RoPE pre-kernel's fragments (matrix cores)
struct RowsArgs {
  const u32x4* qfrag;     // (H, q_rows_pad) query fragments, rows at positions q_pos0 + i
  const u32x4* kfrag;     // (Hkv, k_rows_pad) key fragments, rows at positions 0 ..
  int H, Hkv, Q, M, q_pos0;
  int q_rows_pad, k_rows_pad;   // multiples of 32; k_rows_pad >= M
  float sm_scale;
  float* scores;          // (H, Q, M), or 64 x 32 tiles (score_tile_row) when tiles: row i
                          // written for its keys [0, M - (Q - 1 - i))
  int tiles;
};
hipError_t launch_score_rows(int D, const RowsArgs& a, hipStream_t st);

// qrot: workspace of (H, Q, D) floats, used when a workgroup's query rows outgrow its LDS
hipError_t launch_decode_scores(int dtype, int D, const DecodeArgs& a, float* qrot, hipStream_t st);
// nbend: the PQ Stream rule's block-end counts (decode_bend_words), 0 for the other rules
bool decode_select_in_lds(int M, int nbend);
size_t decode_keys_bytes(int H, int Q, int M, int nbend);
int decode_bend_words(const DecodeArgs& a);
hipError_t launch_decode_select(const DecodeArgs& a, hipStream_t st);
int decode_nsplit(int k_max);
hipError_t launch_decode_attend(int dtype, int D, const DecodeArgs& a, hipStream_t st);

// Whether the fp6 pass-2 kernel (sta_score6.hip) serves workgroup g (wg_rows query rows) of
// head h in the plain pass 2; the three-product kernel then skips it.  It does when the launcher
// enabled it, the screened pass 1 resolved every row of the workgroup (its 256-row workgroups
// raised no fallback flag) and the head's fp6 error estimate stays within the limit.  Both
// kernels evaluate this one function on the same inputs.
__device__ inline bool fast6_serves(const ScoreArgs& a, int h, int g, int D, int wg_rows) {
  if (!a.fast6) return false;
  const int rows_total = a.q_rows_pad;
  constexpr int SG = 256;
  const int ng_s = (rows_total + SG - 1) / SG;
  for (int gs = g * wg_rows / SG; gs < min((g + 1) * wg_rows / SG, ng_s); ++gs)
    if (a.sflags[h * ng_s + gs] != 0) return false;
  const int kvh = h / (a.H / a.Hkv);
  const float2 qn = a.qnorm_max[h], kn = a.knorm_max[kvh], qd = a.q6dmax[h], kd = a.k6dmax[kvh];
  const float sg = fast6_sigma(qn.x, qn.y, qd.x, qd.y, kn.x, kn.y, kd.x, kd.y, a.sm_scale, D);
  return sg <= FAST6_SIGMA_LIMIT;
}

// want6: also write the fp6 correction operands of the fragment region; trig: also write each
// row's scaled (cos, sin) pairs, (rows_pad, D/2) float2 (ScoreArgs::ktrig)
hipError_t launch_rope_frag(int dtype, int D, const void* x, int64_t head_stride, int64_t tok_stride,
                            int heads, int N, int rows_pad, int pos_base, float pos_scale,
                            float rope_scale, const float* inv_freq, u32x4* frag, hipStream_t st,
                            bool want6 = false, float2* trig = nullptr);
// the fp6 pass-2 kernel (plain votes); the launcher of the score passes calls it
hipError_t launch_score6(int D, int tile, const ScoreArgs& a, hipStream_t st);
hipError_t launch_score(int D, int tile, const ScoreArgs& a, hipStream_t st);
hipError_t launch_score_pq(int D, int wmode, const ScoreArgs& a, hipStream_t st);
// the screen + pass 1 only, writing each row's keep threshold to a.xthr (tile 32)
hipError_t launch_score_thresholds(int D, const ScoreArgs& a, hipStream_t st);
// shared selection with weighted votes: wmode 1 margin / 2 expmass, byte votes + fp32 wvotes
hipError_t launch_score_weighted(int D, int tile, int wmode, const ScoreArgs& a, hipStream_t st);
size_t pq_select_lds_bytes(int N, int k_max, bool global_keys);
hipError_t launch_pq_select(const PqSelectArgs& a, hipStream_t st);
hipError_t launch_expand_pq(const uint32_t* bits, const float* wv, int64_t stride, int H, int nt, int N,
                            int T, int q_pos_base, int32_t* votes_out, int32_t* bits_out,
                            float* wv_out, hipStream_t st);
size_t select_lds_bytes(int N, int k_max);
hipError_t launch_select(const SelectArgs& a, int vote_bytes, hipStream_t st);
// _build_sets ranked by weighted votes (select_score margin / expmass)
size_t select_w_lds_bytes(int N, int k_max, bool global_keys);
hipError_t launch_select_weighted(const SelectArgs& a, int vote_bytes, hipStream_t st);
hipError_t launch_expand_votes(const uint8_t* v8, int64_t stride, int H, int nt, int N, int T, int q_pos_base,
                               int32_t* out, const float* wv, float* wv_out, hipStream_t st);
size_t gather_lds_bytes(int dtype, int D, int k_max);
hipError_t launch_abs_rope(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad,
                           const float* inv_freq, uint16_t* out, hipStream_t st);
size_t stream_lds_bytes(int dtype, int D, int BN, bool fused);
bool stream_can_fuse(int dtype, int D, int BN);   // a sweep that computes the keep bits itself exists
// launch_stream runs the fused sweep when a.qfrag is set, else the sweep that reads a.bits
// the remap's (cos, sin) table for positions 0 .. chunk_size, (chunk_size + 1) x D/2 float2
size_t dca_table_bytes(int D, int chunk_size);
hipError_t launch_dca_table(int dtype, int D, const float* inv_freq, float mscale, int chunk_size, float2* table,
                            hipStream_t st);
hipError_t launch_dca_rope(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad,
                           int L, int chunk_size, int is_key, const float2* table, uint16_t* out,
                           hipStream_t st);
size_t dca_lds_bytes(int dtype, int D);
hipError_t launch_dca_attn(int dtype, int D, const DcaArgs& a, hipStream_t st);
hipError_t launch_stream(int dtype, int D, int BN, const StreamArgs& a, hipStream_t st);
hipError_t launch_gather(int dtype, int D, int tile, const GatherArgs& a, hipStream_t st);

}  // namespace sta
