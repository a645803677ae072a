"""CPU oracle for the exact-max shared-selection path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this
module.  The product library never calls it and never falls back to it.

Thin ctypes/numpy wrapper over ``libsta_oracle.so`` (built from ``sta_oracle.c`` by the Makefile
next to it).  Each function names the reference lines it restates:

  select_vote  <- shared_selection_triton_exact_2.py:50-140   (Kernel A, freq mode)
  build_sets   <- shared_selection_triton_exact_2.py:277-426  (_build_sets, freq mode)
  gather_attn  <- shared_selection_triton_exact_2.py:146-225  (Kernel C)
  shared_pi_attention <- shared_selection_triton_exact_2.py:432-486 (composition) and, with two
                         geometries, shared_selection_triton_hybrid_exact.py:450-510
  select_bits  <- shared_selection_triton_perquery.py:119-218 (PQ Union Kernel A)
  build_sets_pq <- shared_selection_triton_perquery.py:363-453 (_build_sets_pq)
  gather_attn_mask <- shared_selection_triton_perquery.py:226-312 (PQ Union Kernel C)
  shared_pq_attention <- shared_selection_triton_perquery.py:459-525 (composition)
  pqstream     <- pqstream_kernel.py:174-368, 498-564 (the fused PQ Stream kernel)
  decode_scores     <- shared_selection_triton_exact_2.py:235-271, 505-525 (_decode_select_kernel)
  decode_build_sets <- shared_selection_triton_exact_2.py:527-604 (_decode_build_sets)
  decode_attend     <- shared_selection_triton_exact_2.py:608-623 (_decode_attend_torch) and, with
                       causal=True, the slot rule of _decode_attend_kernelC (:626-655)
  build_sets_chunk  <- shared_selection_triton_chunked.py:149-243 (_build_sets_chunk)
  decode_build_sets_chunk <- shared_selection_triton_chunked.py:411-489 (_decode_build_sets_chunk)
  dca_rotate_keys / dca_decode <- dca_kernel.py:434-435, 491-522 (the cached keys and decode)

Arrays are numpy.  Half-precision tensors travel as uint16 bit patterns with a dtype code:
0 = fp32, 1 = bf16, 2 = fp16.
"""
import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, BF16, F16 = 0, 1, 2
_DTYPE_CODES = {"float32": F32, "bfloat16": BF16, "float16": F16}


def build():
    """Compile libsta_oracle.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libsta_oracle.so")
        srcs = ["sta_oracle.c", "sta_oracle_pq.c", "sta_oracle_decode.c", "sta_oracle_chunk.c", "sta_oracle_common.h"]
        if not os.path.exists(path) or any(os.path.getmtime(path) < os.path.getmtime(
                os.path.join(_HERE, f)) for f in srcs):
            build()
        _LIB = ctypes.CDLL(path)
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def num_threads():
    return int(lib().oracle_num_threads())


def set_num_threads(n):
    lib().oracle_set_num_threads(ctypes.c_int(int(n)))


# ---------------------------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------------------------
def from_torch(t):
    """torch tensor -> (numpy array, dtype code).  bf16/fp16 become uint16 bit patterns."""
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy(), F32
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16), BF16
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16), F16
    raise TypeError(f"unsupported dtype {t.dtype}")


def to_f32(a, dtype):
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.float32)
    lib().oracle_to_f32(_p(a), _p(out), ctypes.c_size_t(a.size), ctypes.c_int(dtype))
    return out


def round_to_dtype(x, dtype):
    """fp32 array -> dtype storage (RNE); uint16 bit patterns for bf16/fp16."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.float32 if dtype == F32 else np.uint16)
    lib().oracle_round_to_dtype(_p(x), _p(out), ctypes.c_size_t(x.size), ctypes.c_int(dtype))
    return out


# ---------------------------------------------------------------------------------------------
# the three stages
# ---------------------------------------------------------------------------------------------
def rope_rotate(x, dtype, posf, inv_freq, rope_scale):
    """Rotate rows of x (rows, D) at fp32 angle bases posf (rows,)."""
    x = np.ascontiguousarray(x)
    rows, D = x.shape
    out = np.empty((rows, D), np.float32)
    lib().oracle_rope_rotate(_p(x), ctypes.c_int(dtype), ctypes.c_int(rows), ctypes.c_int(D),
                             _p(_c(posf, np.float32)), _p(_c(inv_freq, np.float32)),
                             ctypes.c_float(rope_scale), _p(out))
    return out


def select_vote(q, k, dtype, tau, inv_freq, pos_scale, rope_scale, sm_scale, tile, q_pos_base=0,
                band_eps=1e-3, want_band=False, want_keep=False, wmode=0):
    """Kernel A (exact_2.py:50-140).  q (H,N,D), k (Hkv,N,D).  Returns a dict with
    votes (H,nt,N) int32, row_counts (H,N) int32, row_max (H,N) fp32 and optionally
    band (H,nt,N) int32, keep (H,N,N) uint8 and, for wmode 1 (margin) / 2 (expmass), the
    weighted votes wvotes (H,nt,N) fp32 (exact_2.py:126-138)."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    H, N, D = q.shape
    Hkv = k.shape[0]
    nt = (N + tile - 1) // tile
    votes = np.empty((H, nt, N), np.int32)
    row_counts = np.empty((H, N), np.int32)
    row_max = np.empty((H, N), np.float32)
    band = np.empty((H, nt, N), np.int32) if want_band else None
    band_rows = np.empty((H, N), np.int32) if want_band else None
    keep = np.empty((H, N, N), np.uint8) if want_keep else None
    wvotes = np.empty((H, nt, N), np.float32) if wmode else None
    lib().oracle_select_vote(
        _p(q), _p(k), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv), ctypes.c_int(N),
        ctypes.c_int(D), _p(_c(tau, np.float32)), _p(_c(inv_freq, np.float32)),
        ctypes.c_float(pos_scale), ctypes.c_float(rope_scale), ctypes.c_float(sm_scale),
        ctypes.c_int(tile), ctypes.c_int(q_pos_base), _p(votes), _p(row_counts), _p(row_max),
        _p(band), _p(band_rows), ctypes.c_float(band_eps), _p(keep), ctypes.c_int(wmode), _p(wvotes))
    out = {"votes": votes, "row_counts": row_counts, "row_max": row_max}
    if wmode:
        out["wvotes"] = wvotes
    if want_band:
        out["band"] = band
        out["band_rows"] = band_rows
    if want_keep:
        out["keep"] = keep
    return out


WMODES = {"freq": 0, "margin": 1, "expmass": 2}


def start_pct_of(pct):
    """start_pct = max(0, int(round(pct))) with Python's round-half-even (exact_2.py:309)."""
    return max(0, int(round(pct)))


def build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
               wvotes=None, want_cut=False):
    """_build_sets (exact_2.py:277-426).  votes (H,nt,N) int; wvotes (H,nt,N) fp32 switches the
    ranking to fl(wvotes + fl(1e-6 votes)) (margin / expmass, exact_2.py:299-302), None ranks by
    votes.  Returns the reference's 9-tuple (idx, newpos_k, newpos_q, shared_size, kept_size,
    chosen, orig_overflow, kpct_meas, overflow20) as numpy arrays; with want_cut a 10th entry,
    the (H, nt) fp32 rank-value cut of the kept step (+inf where only forced keys are kept)."""
    votes = _c(votes, np.int32)
    if wvotes is not None:
        wvotes = _c(wvotes, np.float32)
        assert wvotes.shape == votes.shape
    H, nt, N = votes.shape
    idx = np.empty((H, nt, k_max), np.int32)
    npk = np.empty((H, nt, k_max), np.float32)
    npq = np.empty((H, nt, T), np.float32)
    ss = np.empty((H, nt), np.int32)
    ks = np.empty((H, nt), np.int32)
    ch = np.empty((H, nt), np.int32)
    oo = np.empty((H, nt), np.uint8)
    km = np.empty((H, nt), np.int32)
    o20 = np.empty((H, nt), np.uint8)
    cut = np.empty((H, nt), np.float32) if want_cut else None
    lib().oracle_build_sets(
        _p(votes), ctypes.c_int(H), ctypes.c_int(nt), ctypes.c_int(N), ctypes.c_float(pos_scale),
        ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(start_pct_of(pct)),
        ctypes.c_int(T), ctypes.c_int(k_max), ctypes.c_int(q_pos_base), ctypes.c_int(int(measure)),
        _p(idx), _p(npk), _p(npq), _p(ss), _p(ks), _p(ch), _p(oo), _p(km), _p(o20), _p(wvotes),
        _p(cut))
    res = (idx, npk, npq, ss, ks, ch, oo.astype(bool), km, o20.astype(bool))
    return res + (cut,) if want_cut else res


def gather_attn(q, k, v, dtype, idx, newpos_k, newpos_q, inv_freq, rope_scale, sm_scale, T,
                k_max, block_k=64, q_pos_base=0):
    """Kernel C (exact_2.py:146-225).  Returns the fp32 accumulator (H,N,D) before the final cast."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, N, D = q.shape
    Hkv = k.shape[0]
    out = np.full((H, N, D), np.nan, np.float32)
    lib().oracle_gather_attn(
        _p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
        ctypes.c_int(N), ctypes.c_int(D), _p(_c(inv_freq, np.float32)), ctypes.c_float(rope_scale),
        ctypes.c_float(sm_scale), ctypes.c_int(T), ctypes.c_int(k_max), ctypes.c_int(block_k),
        ctypes.c_int(q_pos_base), _p(_c(idx, np.int32)), _p(_c(newpos_k, np.float32)),
        _p(_c(newpos_q, np.float32)), _p(out))
    return out


def shared_pi_attention(q, k, v, dtype, tau, inv_freq_a, pos_scale_a, rope_scale_a,
                        inv_freq_c=None, pos_scale_c=None, rope_scale_c=None, pct=30.0,
                        sm_scale=None, n_global=32, n_local=32, tile=32, k_max=1024, block_k=64,
                        q_pos_base=0, measure=False, select_score="freq"):
    """Composition of the three stages (exact_2.py:432-486).  With the *_c triple given it is the
    hybrid entry point (hybrid_exact.py:450-510): Kernel A under the a-geometry, _build_sets'
    reposition and Kernel C under the c-geometry.  select_score "margin" / "expmass" ranks by
    Kernel A's weighted votes (exact_2.py:450-453, 467-469).  Returns
    (out_f32, shared_size, kept_size, kpct, overflow, kpct_meas, overflow20, extras)."""
    H, N, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if inv_freq_c is None:
        inv_freq_c, pos_scale_c, rope_scale_c = inv_freq_a, pos_scale_a, rope_scale_a
    wmode = WMODES[select_score]
    a = select_vote(q, k, dtype, tau, inv_freq_a, pos_scale_a, rope_scale_a, sm_scale, tile,
                    q_pos_base, wmode=wmode)
    idx, npk, npq, ss, ks, ch, oo, km, o20 = build_sets(
        a["votes"], pos_scale_c, n_global, n_local, pct, tile, k_max, q_pos_base, measure,
        wvotes=a.get("wvotes"))
    out = gather_attn(q, k, v, dtype, idx, npk, npq, inv_freq_c, rope_scale_c, sm_scale, tile,
                      k_max, block_k, q_pos_base)
    extras = {"votes": a["votes"], "wvotes": a.get("wvotes"), "row_max": a["row_max"],
              "row_counts": a["row_counts"],
              "idx": idx, "newpos_k": npk, "newpos_q": npq}
    return out, ss, ks, ch, oo, km, o20, extras


# ---------------------------------------------------------------------------------------------
# PQ Union (per-query sets through a tile union + bitmask) and PQ Stream
# ---------------------------------------------------------------------------------------------
def select_bits(q, k, dtype, tau, inv_freq, pos_scale, rope_scale, sm_scale, tile=32, q_pos_base=0,
                wmode=2, band_eps=1e-3, want_band=False):
    """PQ Union Kernel A (perquery.py:119-218).  Returns a dict with votes, bits (int32, bit i =
    row i), wvotes (fp32, zeros for wmode 0), row_counts, row_max and optionally band/band_rows."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    H, N, D = q.shape
    Hkv = k.shape[0]
    nt = (N + tile - 1) // tile
    votes = np.empty((H, nt, N), np.int32)
    bits = np.empty((H, nt, N), np.int32)
    wv = np.zeros((H, nt, N), np.float32)
    rc = np.empty((H, N), np.int32)
    rm = np.empty((H, N), np.float32)
    band = np.empty((H, nt, N), np.int32) if want_band else None
    band_rows = np.empty((H, N), np.int32) if want_band else None
    lib().oracle_select_bits(
        _p(q), _p(k), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv), ctypes.c_int(N),
        ctypes.c_int(D), _p(_c(tau, np.float32)), _p(_c(inv_freq, np.float32)),
        ctypes.c_float(pos_scale), ctypes.c_float(rope_scale), ctypes.c_float(sm_scale),
        ctypes.c_int(tile), ctypes.c_int(q_pos_base), ctypes.c_int(wmode), _p(votes), _p(bits),
        _p(wv) if wmode > 0 else None, _p(rc), _p(rm), _p(band), _p(band_rows),
        ctypes.c_float(band_eps))
    out = {"votes": votes, "bits": bits, "wvotes": wv, "row_counts": rc, "row_max": rm}
    if want_band:
        out["band"] = band
        out["band_rows"] = band_rows
    return out


def build_sets_pq(votes, bits, wvotes, n_global, n_local, T, k_max, q_pos_base=0, rank_mode=2):
    """_build_sets_pq (perquery.py:363-453).  rank_mode 0 ranks overflow candidates by votes,
    otherwise by wvotes + 1e-6 votes.  Returns (idx, newpos_k, newpos_q, mask, usize, kept_size,
    overflow) as numpy arrays; equal rank values at the cut are taken in ascending key order."""
    votes = _c(votes, np.int32)
    bits = _c(bits, np.int32)
    H, nt, N = votes.shape
    wv = _c(wvotes, np.float32) if (wvotes is not None and rank_mode != 0) else None
    idx = np.empty((H, nt, k_max), np.int32)
    npk = np.empty((H, nt, k_max), np.float32)
    npq = np.empty((H, nt, T), np.float32)
    mask = np.empty((H, nt, k_max), np.int32)
    us = np.empty((H, nt), np.int32)
    ks = np.empty((H, nt), np.int32)
    ov = np.empty((H, nt), np.uint8)
    lib().oracle_build_sets_pq(
        _p(votes), _p(bits), _p(wv), ctypes.c_int(H), ctypes.c_int(nt), ctypes.c_int(N),
        ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(T), ctypes.c_int(k_max),
        ctypes.c_int(q_pos_base), ctypes.c_int(rank_mode), _p(idx), _p(npk), _p(npq), _p(mask),
        _p(us), _p(ks), _p(ov))
    return idx, npk, npq, mask, us, ks, ov.astype(bool)


def gather_attn_mask(q, k, v, dtype, idx, newpos_k, newpos_q, mask, inv_freq, rope_scale, sm_scale,
                     T, k_max, block_k=64, q_pos_base=0):
    """PQ Union Kernel C (perquery.py:226-312): Kernel C with the per-slot query bitmask."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, N, D = q.shape
    Hkv = k.shape[0]
    out = np.full((H, N, D), np.nan, np.float32)
    lib().oracle_gather_attn_mask(
        _p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
        ctypes.c_int(N), ctypes.c_int(D), _p(_c(inv_freq, np.float32)), ctypes.c_float(rope_scale),
        ctypes.c_float(sm_scale), ctypes.c_int(T), ctypes.c_int(k_max), ctypes.c_int(block_k),
        ctypes.c_int(q_pos_base), _p(_c(idx, np.int32)), _p(_c(newpos_k, np.float32)),
        _p(_c(newpos_q, np.float32)), _p(_c(mask, np.int32)), _p(out))
    return out


def shared_pq_attention(q, k, v, dtype, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0,
                        rope_scale_a=1.0, sm_scale=None, n_global=32, n_local=32, tile=32,
                        k_max=4096, block_k=64, q_pos_base=0, select_score="expmass"):
    """Composition (perquery.py:459-525).  Returns (out_f32, usize, kept_size, overflow, extras)."""
    H, N, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    wmode = WMODES[select_score]
    a = select_bits(q, k, dtype, tau, inv_freq_a, pos_scale_a, rope_scale_a, sm_scale, tile,
                    q_pos_base, wmode)
    idx, npk, npq, mask, us, ks, ov = build_sets_pq(a["votes"], a["bits"], a["wvotes"], n_global,
                                                    n_local, tile, k_max, q_pos_base, wmode)
    out = gather_attn_mask(q, k, v, dtype, idx, npk, npq, mask, inv_freq_c, 1.0, sm_scale, tile,
                           k_max, block_k, q_pos_base)
    extras = dict(a, idx=idx, newpos_k=npk, newpos_q=npq, mask=mask)
    return out, us, ks, ov, extras


# ---------------------------------------------------------------------------------------------
# chunk-granular selection (shared_selection_triton_chunked.py)
# ---------------------------------------------------------------------------------------------
CHUNK_AGG = {"sum": 0, "mean": 1}


def n_forced_chunks(chunk_size, n_global, n_local, tile):
    """Chunks the forced global + local keys can occupy (chunked.py:115-129)."""
    C = chunk_size
    return (n_global + C - 1) // C + (n_local + tile - 1 + C - 1) // C + 1


def derive_n_chunk(k_max, chunk_size, n_global, n_local, tile):
    """Chunks to select so that forced + selected fill k_max (chunked.py:132-146)."""
    assert k_max % chunk_size == 0
    n = k_max // chunk_size - n_forced_chunks(chunk_size, n_global, n_local, tile)
    assert n > 0
    return n


def build_sets_chunk(votes, wvotes, n_global, n_local, T, k_max, chunk_size, n_chunk, q_pos_base=0,
                     select_score="expmass", chunk_agg="sum"):
    """_build_sets_chunk (chunked.py:149-243).  Returns (idx, newpos_k, newpos_q, mask, usize,
    kept_size, passers_kept); equal chunk values are taken in ascending chunk order."""
    votes = _c(votes, np.int32)
    H, nt, N = votes.shape
    weighted = select_score != "freq" and wvotes is not None and wvotes.shape[-1] == N
    wv = _c(wvotes, np.float32) if weighted else None
    idx = np.empty((H, nt, k_max), np.int32)
    npk = np.empty((H, nt, k_max), np.float32)
    npq = np.empty((H, nt, T), np.float32)
    mask = np.empty((H, nt, k_max), np.int32)
    us, ks, pk = (np.empty((H, nt), np.int32) for _ in range(3))
    lib().oracle_build_sets_chunk(
        _p(votes), _p(wv), ctypes.c_int(H), ctypes.c_int(nt), ctypes.c_int(N), ctypes.c_int(T),
        ctypes.c_int(k_max), ctypes.c_int(chunk_size), ctypes.c_int(n_chunk), ctypes.c_int(q_pos_base),
        ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(int(weighted)),
        ctypes.c_int(CHUNK_AGG[chunk_agg]), _p(idx), _p(npk), _p(npq), _p(mask), _p(us), _p(ks), _p(pk))
    return idx, npk, npq, mask, us, ks, pk


def decode_build_sets_chunk(scores, tau, q_pos0, n_global, n_local, k_max, chunk_size, n_chunk,
                            select_score="expmass", chunk_agg="sum"):
    """_decode_build_sets_chunk (chunked.py:411-489) for Q queries (H, Q, M) at q_pos0 + i over
    the keys [0, M - (Q - 1 - i)).  Returns (idx (sentinel m_i), newpos_k, newpos_q, kept_size,
    passers_kept)."""
    scores = _c(scores, np.float32)
    H, Q, M = scores.shape
    idx = np.empty((H, Q, k_max), np.int32)
    npk = np.empty((H, Q, k_max), np.float32)
    npq = np.empty((H, Q), np.float32)
    ks, pk = np.empty((H, Q), np.int32), np.empty((H, Q), np.int32)
    lib().oracle_decode_build_sets_chunk(
        _p(scores), ctypes.c_int(H), ctypes.c_int(Q), ctypes.c_int(M), _p(_c(tau, np.float32)),
        ctypes.c_int(q_pos0), ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(k_max),
        ctypes.c_int(chunk_size), ctypes.c_int(n_chunk), ctypes.c_int(int(select_score != "freq")),
        ctypes.c_int(CHUNK_AGG[chunk_agg]), _p(idx), _p(npk), _p(npq), _p(ks), _p(pk))
    return idx, npk, npq, ks, pk


def shared_chunk_attention(q, k, v, dtype, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                           sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096, chunk_size=16,
                           n_chunk=None, q_pos_base=0, select_score="expmass", chunk_agg="sum"):
    """Composition (chunked.py:249-322): PQ Kernel A, _build_sets_chunk, pooled Kernel C.
    Returns (out_f32, usize, kept_size, extras)."""
    H, N, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if n_chunk is None:
        n_chunk = derive_n_chunk(k_max, chunk_size, n_global, n_local, tile)
    a = select_bits(q, k, dtype, tau, inv_freq_a, pos_scale_a, rope_scale_a, sm_scale, tile, q_pos_base,
                    WMODES[select_score])
    idx, npk, npq, mask, us, ks, pk = build_sets_chunk(a["votes"], a["wvotes"], n_global, n_local, tile, k_max,
                                                       chunk_size, n_chunk, q_pos_base, select_score, chunk_agg)
    out = gather_attn_mask(q, k, v, dtype, idx, npk, npq, mask, inv_freq_c, 1.0, sm_scale, tile, k_max,
                           q_pos_base=q_pos_base)
    return out, us, ks, dict(a, idx=idx, newpos_k=npk, newpos_q=npq, mask=mask, passers_kept=pk)


def pqstream(q, k, v, dtype, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
             sm_scale=None, n_global=32, n_local=32, tile=32, block_n=32, pos_advance="max",
             use_skip=True, band_eps=1e-3, bits_in=None, want_band=True):
    """The fused PQ Stream kernel (pqstream_kernel.py:174-368).  Returns (out_f32, span, kept,
    blocks, skipped, band_rows).  With bits_in (H, nt, N) int32 the threshold decisions are taken
    from those bits (bit i = row i of the tile) instead of being recomputed."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, N, D = q.shape
    Hkv = k.shape[0]
    nt = (N + tile - 1) // tile
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = np.full((H, N, D), np.nan, np.float32)
    span = np.empty((H, nt), np.float32)
    blocks = np.empty((H, nt), np.float32)
    skipped = np.empty((H, nt), np.float32)
    kept = np.empty((H, N), np.int32)
    band_rows = np.empty((H, N), np.int32) if want_band else None
    bits_c = _c(bits_in, np.int32) if bits_in is not None else None
    lib().oracle_pqstream(
        _p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
        ctypes.c_int(N), ctypes.c_int(D), _p(_c(tau, np.float32)), _p(_c(inv_freq_a, np.float32)),
        _p(_c(inv_freq_c, np.float32)), ctypes.c_float(pos_scale_a), ctypes.c_float(rope_scale_a),
        ctypes.c_float(sm_scale), ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(tile),
        ctypes.c_int(block_n), ctypes.c_int(1 if pos_advance == "full" else 0),
        ctypes.c_int(int(use_skip)), _p(bits_c), _p(out), _p(span), _p(kept), _p(blocks),
        _p(skipped), _p(band_rows), ctypes.c_float(band_eps))
    return out, span, kept, blocks, skipped, band_rows


# ---------------------------------------------------------------------------------------------
# DCA (dense attention, dual-chunk positions)
# ---------------------------------------------------------------------------------------------
def dca_mscale(seq_len, pretrain_len):
    """The ChunkLlama attention factor: 0.05 ln(seq_len / c) + 1 above c, else 1
    (dca_kernel.py:163-170; the tables are rebuilt at the prefill length when it exceeds c)."""
    scale = seq_len / pretrain_len
    return 1.0 if scale <= 1 else 0.05 * math.log(scale) + 1.0


def dca_attention(q, k, v, dtype, inv_freq, chunk_size, pretrain_len, local_window, scale=None,
                  rows=None, mscale=None):
    """The prefill branch of dca_forward (dca_kernel.py:372-489) on raw q (H,N,D), k/v (Hkv,N,D).
    Returns out (H, N, D) fp32; with `rows` only those query rows are computed (others NaN).
    mscale: the table factor (default get_mscale(N / pretrain_len))."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, N, D = q.shape
    Hkv = k.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ms = np.float32(dca_mscale(N, pretrain_len) if mscale is None else mscale)
    out = np.full((H, N, D), np.nan, np.float32)
    r = _c(rows, np.int32) if rows is not None else None
    lib().oracle_dca(_p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                     ctypes.c_int(N), ctypes.c_int(D), _p(_c(inv_freq, np.float32)), ctypes.c_int(chunk_size),
                     ctypes.c_int(local_window), ctypes.c_float(ms), ctypes.c_float(scale), _p(r),
                     ctypes.c_int(len(r) if r is not None else 0), _p(out))
    return out


def dca_rotate_keys(k, dtype, inv_freq, chunk_size, local_window, mscale, pos0=0):
    """Raw keys (heads, N, D) at positions pos0.. rotated with the cyclic key table
    (dca_kernel.py:187-190, 434-435) -> (heads, N, D) fp32 holding model-dtype values."""
    k = np.ascontiguousarray(k)
    heads, N, D = k.shape
    out = np.empty((heads, N, D), np.float32)
    lib().oracle_dca_rotate_keys(_p(k), ctypes.c_int(dtype), ctypes.c_int(heads), ctypes.c_int(N), ctypes.c_int(D),
                                 ctypes.c_int(pos0), _p(_c(inv_freq, np.float32)), ctypes.c_int(chunk_size),
                                 ctypes.c_int(local_window), ctypes.c_float(mscale), _p(out))
    return out


def dca_decode(q, krot, v, dtype, inv_freq, chunk_size, local_window, mscale, scale=None):
    """The decode branch of dca_forward (dca_kernel.py:491-522): q (H, D) raw at position M - 1 over
    the rotated cache krot and v (Hkv, M, D), all in the storage of `dtype` -> (H, D) fp32 holding
    model-dtype values."""
    q = np.ascontiguousarray(q)
    krot = np.ascontiguousarray(krot)
    v = np.ascontiguousarray(v)
    H, D = q.shape
    Hkv, M = krot.shape[0], krot.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.empty((H, D), np.float32)
    lib().oracle_dca_decode(_p(q), _p(krot), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                            ctypes.c_int(M), ctypes.c_int(D), _p(_c(inv_freq, np.float32)), ctypes.c_int(chunk_size),
                            ctypes.c_int(local_window), ctypes.c_float(mscale), ctypes.c_float(scale), _p(out))
    return out


# ---------------------------------------------------------------------------------------------
# config 4: DCA positions with exact-max selection over the inter-chunk keys (build-defined
# composition of dca_kernel.py's positions and exact_2.py's Kernel A + _build_sets)
# ---------------------------------------------------------------------------------------------
def dca_inter_votes(q, k, dtype, inv_freq, chunk_size, pretrain_len, local_window, tau, scale=None, T=64,
                    band_eps=1e-3, want_band=False, tiles=None):
    """Votes (H, nt, N) int32 over each 64-query tile's inter keys [0, (c - 1) L), row_max (H, N)
    (-inf without inter keys) and optionally band (H, nt, N).  tiles: evaluate only these tile
    indices (the others keep zero votes and a NaN row max)."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    H, N, D = q.shape
    Hkv = k.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    nt = (N + T - 1) // T
    votes = np.empty((H, nt, N), np.int32)
    rm = np.empty((H, N), np.float32)
    band = np.empty((H, nt, N), np.int32) if want_band else None
    ms = np.float32(dca_mscale(N, pretrain_len))
    tmask = None
    if tiles is not None:
        tmask = np.zeros(nt, np.uint8)
        tmask[np.asarray(tiles, np.int64)] = 1
    lib().oracle_dca_inter_votes(_p(q), _p(k), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                                 ctypes.c_int(N), ctypes.c_int(D), _p(_c(inv_freq, np.float32)),
                                 ctypes.c_int(chunk_size), ctypes.c_int(local_window), ctypes.c_float(ms),
                                 ctypes.c_float(scale), _p(_c(tau, np.float32)), ctypes.c_int(T),
                                 ctypes.c_float(band_eps), _p(votes), _p(rm), _p(band), _p(tmask))
    out = {"votes": votes, "row_max": rm}
    if want_band:
        out["band"] = band
    return out


def dca_build_sets(votes, chunk_size, local_window, n_global, pct, k_max, T=64, measure=False, want_cut=False):
    """_build_sets over each tile's inter keys.  Returns (idx, shared_size, kept_size, chosen,
    orig_overflow, kpct_meas, overflow20[, cut])."""
    votes = _c(votes, np.int32)
    H, nt, N = votes.shape
    idx = np.empty((H, nt, k_max), np.int32)
    ss, ks, ch, km = (np.empty((H, nt), np.int32) for _ in range(4))
    oo, o20 = np.empty((H, nt), np.uint8), np.empty((H, nt), np.uint8)
    cut = np.empty((H, nt), np.float32) if want_cut else None
    lib().oracle_dca_build_sets(_p(votes), ctypes.c_int(H), ctypes.c_int(N), ctypes.c_int(chunk_size),
                                ctypes.c_int(local_window), ctypes.c_int(T), ctypes.c_int(n_global),
                                ctypes.c_int(start_pct_of(pct)), ctypes.c_int(k_max), ctypes.c_int(int(measure)),
                                _p(idx), _p(ss), _p(ks), _p(ch), _p(oo), _p(km), _p(o20), _p(cut))
    res = (idx, ss, ks, ch, oo.astype(bool), km, o20.astype(bool))
    return res + (cut,) if want_cut else res


def dca_select_attn(q, k, v, dtype, inv_freq, chunk_size, pretrain_len, local_window, idx, kept_size, scale=None,
                    T=64, rows=None):
    """Attention given each tile's selected inter keys: out (H, N, D) fp32 (NaN outside `rows`)."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, N, D = q.shape
    Hkv = k.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ms = np.float32(dca_mscale(N, pretrain_len))
    out = np.full((H, N, D), np.nan, np.float32)
    r = _c(rows, np.int32) if rows is not None else None
    idx = _c(idx, np.int32)
    lib().oracle_dca_select_attn(_p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                                 ctypes.c_int(N), ctypes.c_int(D), _p(_c(inv_freq, np.float32)),
                                 ctypes.c_int(chunk_size), ctypes.c_int(local_window), ctypes.c_float(ms),
                                 ctypes.c_float(scale), ctypes.c_int(T), _p(idx), _p(_c(kept_size, np.int32)),
                                 ctypes.c_int(idx.shape[-1]), _p(r), ctypes.c_int(len(r) if r is not None else 0),
                                 _p(out))
    return out


def dca_select_attention(q, k, v, dtype, inv_freq, chunk_size, pretrain_len, local_window, tau, pct=30.0,
                         k_max=2048, n_global=32, scale=None, T=64, measure=False, rows=None):
    """Config 4 composed: inter votes, selection, attention.  Returns (out, sets tuple, votes dict)."""
    a = dca_inter_votes(q, k, dtype, inv_freq, chunk_size, pretrain_len, local_window, tau, scale, T)
    sets = dca_build_sets(a["votes"], chunk_size, local_window, n_global, pct, k_max, T, measure)
    out = dca_select_attn(q, k, v, dtype, inv_freq, chunk_size, pretrain_len, local_window, sets[0], sets[2],
                          scale, T, rows)
    return out, sets, a


# ---------------------------------------------------------------------------------------------
# decode: a batch of Q queries over one cache of M keys; query i at position q_pos0 + i sees the
# keys [0, M - (Q - 1 - i)) (the cache prefix of spi_forward's per-token loop, exact_2.py:743-745)
# ---------------------------------------------------------------------------------------------
def decode_scores(q, k, dtype, inv_freq, pos_scale, rope_scale, sm_scale, q_pos0):
    """q (H,Q,D), k (Hkv,M,D) -> scores (H,Q,M) fp32, NaN past each query's key range."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    H, Q, D = q.shape
    Hkv, M = k.shape[0], k.shape[1]
    out = np.empty((H, Q, M), np.float32)
    lib().oracle_decode_scores(_p(q), _p(k), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                               ctypes.c_int(Q), ctypes.c_int(M), ctypes.c_int(D), _p(_c(inv_freq, np.float32)),
                               ctypes.c_float(pos_scale), ctypes.c_float(rope_scale), ctypes.c_float(sm_scale),
                               ctypes.c_int(q_pos0), _p(out))
    return out


def decode_build_sets(scores, tau, q_pos0, pos_scale, n_global, n_local, k_max, pct_decode=100.0):
    """_decode_build_sets from scores (H,Q,M) -> idx (H,Q,k_max) int32 (sentinel m_i),
    newpos_k (H,Q,k_max), newpos_q (H,Q), set_size (H,Q) (|set| before the k_max truncation)."""
    scores = _c(scores, np.float32)
    H, Q, M = scores.shape
    idx = np.empty((H, Q, k_max), np.int32)
    npk = np.empty((H, Q, k_max), np.float32)
    npq = np.empty((H, Q), np.float32)
    size = np.empty((H, Q), np.int32)
    lib().oracle_decode_build_sets(_p(scores), ctypes.c_int(H), ctypes.c_int(Q), ctypes.c_int(M),
                                   _p(_c(tau, np.float32)), ctypes.c_int(q_pos0), ctypes.c_float(pos_scale),
                                   ctypes.c_int(n_global), ctypes.c_int(n_local), ctypes.c_int(k_max),
                                   ctypes.c_double(pct_decode), _p(idx), _p(npk), _p(npq), _p(size))
    return idx, npk, npq, size


def decode_build_sets_pq(scores, tau, q_pos0, n_global, n_local, k_max):
    """_decode_build_sets_pq (perquery.py:651-720) from scores (H,Q,M) -> idx (H,Q,k_max) int32
    (sentinel m_i), newpos_k (H,Q,k_max) dense ranks, newpos_q (H,Q), set_size (H,Q),
    usize (H,Q) (|keep| before the forced keys) and overflow (H,Q) bool; equal scores at the
    k_max cut are taken in ascending key order."""
    scores = _c(scores, np.float32)
    H, Q, M = scores.shape
    idx = np.empty((H, Q, k_max), np.int32)
    npk = np.empty((H, Q, k_max), np.float32)
    npq = np.empty((H, Q), np.float32)
    size = np.empty((H, Q), np.int32)
    us = np.empty((H, Q), np.int32)
    ov = np.empty((H, Q), np.uint8)
    lib().oracle_decode_build_sets_pq(_p(scores), ctypes.c_int(H), ctypes.c_int(Q), ctypes.c_int(M),
                                      _p(_c(tau, np.float32)), ctypes.c_int(q_pos0), ctypes.c_int(n_global),
                                      ctypes.c_int(n_local), ctypes.c_int(k_max), _p(idx), _p(npk), _p(npq),
                                      _p(size), _p(us), _p(ov))
    return idx, npk, npq, size, us, ov.astype(bool)


def decode_build_sets_pqs(scores, tau, q_pos0, n_global, n_local, block_n, k_max=None):
    """_decode_build_sets_pqs (pqstream_kernel.py:695-797) from scores (H,Q,M) -> idx (H,Q,k_max)
    int32 (sentinel m_i), newpos_k (streamed, -dist), newpos_q (0), set_size, span (H,Q) fp32 and
    skipped (H,Q).  k_max defaults to the reference's buffer, M rounded up to a multiple of 1024."""
    scores = _c(scores, np.float32)
    H, Q, M = scores.shape
    if k_max is None:
        k_max = max(1024, -(-M // 1024) * 1024)
    idx = np.empty((H, Q, k_max), np.int32)
    npk = np.empty((H, Q, k_max), np.float32)
    npq = np.empty((H, Q), np.float32)
    size = np.empty((H, Q), np.int32)
    span = np.empty((H, Q), np.float32)
    skp = np.empty((H, Q), np.int32)
    lib().oracle_decode_build_sets_pqs(_p(scores), ctypes.c_int(H), ctypes.c_int(Q), ctypes.c_int(M),
                                       _p(_c(tau, np.float32)), ctypes.c_int(q_pos0), ctypes.c_int(n_global),
                                       ctypes.c_int(n_local), ctypes.c_int(block_n), ctypes.c_int(k_max), _p(idx),
                                       _p(npk), _p(npq), _p(size), _p(span), _p(skp))
    return idx, npk, npq, size, span, skp


def decode_attend(q, k, v, dtype, inv_freq, rope_scale, sm_scale, q_pos0, idx, newpos_k, newpos_q,
                  causal=False):
    """Attention of each query over its slots -> (H,Q,D) fp32 before the cast to the dtype."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    H, Q, D = q.shape
    Hkv, M = k.shape[0], k.shape[1]
    k_max = idx.shape[-1]
    out = np.empty((H, Q, D), np.float32)
    lib().oracle_decode_attend(_p(q), _p(k), _p(v), ctypes.c_int(dtype), ctypes.c_int(H), ctypes.c_int(Hkv),
                               ctypes.c_int(Q), ctypes.c_int(M), ctypes.c_int(D), _p(_c(inv_freq, np.float32)),
                               ctypes.c_float(rope_scale), ctypes.c_float(sm_scale), ctypes.c_int(q_pos0),
                               ctypes.c_int(k_max), _p(_c(idx, np.int32)), _p(_c(newpos_k, np.float32)),
                               _p(_c(newpos_q, np.float32)), ctypes.c_int(int(bool(causal))), _p(out))
    return out
