"""Drop-in for shared_selection_triton_chunked.py ("chunk_exact"): selection at chunk granularity.

PQ Kernel A (votes and weighted votes per 32-query tile), then _build_sets_chunk: keys grouped
into fixed chunks of chunk_size, each chunk valued by the sum (or the mean) of its threshold
passers' rank values, the forced global / local chunks kept plus the n_chunk visible chunks of
largest value; their keys up to the tile's last query are attended by every query of the tile
(pooled) at dense ranks under base RoPE.  The budget is exact: kept <= (forced + n_chunk) chunks.
Same entry points and signatures as the reference (n_forced_chunks, derive_n_chunk,
_build_sets_chunk, shared_chunk_attention, _decode_build_sets_chunk, install_shared_pi_forward,
get_chunk_stats / reset_chunk_stats; chunked.py:64-643); the work runs in the gfx950 HIP kernels of
libsta_hip.so (no Triton, no fallback).  `block_n` / `block_k` are the reference's Triton tile
knobs and are accepted and ignored.

Differences by design: equal chunk values are taken in ascending chunk order (the reference leaves
that to torch.topk, whose order among equal values is unspecified); the forced-chunk mask follows
the rule the reference's own golden, chunk_attention_torch (:368-376), states -- the module the
reference imports it from (chunk_recall_core) is not part of the reference tree; the golden
itself, a CPU torch restatement, is not part of this package.
"""
import math

import torch

import _sta_native as native
from _counters import PhaseCounters, ratio
from _torch_golden import _rope_rotate, chunk_attention_torch  # noqa: F401  (torch helper and golden)
from _sta_native import derive_n_chunk, n_forced_chunks  # noqa: F401  (the reference's budget helpers)

# measurement-only chunk-quality counters per phase (get_chunk_stats keys, chunked.py:64-110):
# passers inside kept chunks, passers visible, slots gathered
_CHUNK_STATS = {p: PhaseCounters(sums=("cap", "tot", "slots")) for p in ("prefill", "decode")}


def reset_chunk_stats():
    for c in _CHUNK_STATS.values():
        c.clear()


def _phase(c):
    n, s, _ = c.read()
    cells = n["cells"]
    return {"cells": cells, "recall_count": ratio(s["cap"], s["tot"]), "utilisation": ratio(s["cap"], s["slots"]),
            "slots_per_cell": ratio(s["slots"], cells)}


def get_chunk_stats():
    """Per phase: recall_count = kept passers / visible passers, utilisation = kept passers /
    gathered slots, slots_per_cell (one host sync here, none during the run)."""
    return {p: _phase(c) for p, c in _CHUNK_STATS.items()}


def _stat_acc(cap, tot, slots, phase):
    _CHUNK_STATS[phase].add({"cells": slots.numel()},
                            (cap.sum(dtype=torch.float64), tot.sum(dtype=torch.float64),
                             slots.sum(dtype=torch.float64)))


def _build_sets_chunk(votes, wvotes, n_global, n_local, T, k_max, chunk_size, n_chunk, q_pos_base=0,
                      select_score="expmass", chunk_agg="sum", measure=False):
    """votes (H,nt,N) int, wvotes (H,nt,N) fp32 -> (idx, newpos_k, newpos_q, mask, usize,
    kept_size).  shared_selection_triton_chunked.py:149-243."""
    assert chunk_agg in native.CHUNK_AGG, f"chunk_agg must be sum|mean, got {chunk_agg!r}"
    res, pk = native.chunk_build_sets(votes, wvotes, n_global, n_local, T, k_max, chunk_size, n_chunk, q_pos_base,
                                      select_score, chunk_agg)
    if measure:
        _stat_acc(pk, res[4], res[5], "prefill")
    return res


def shared_chunk_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                           sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096, chunk_size=16,
                           n_chunk=None, block_n=64, block_k=64, q_pos_base=0, select_score="expmass",
                           chunk_agg="sum", measure=False):
    """q,k,v: (1,H,N,D) raw (k, v may carry H/g heads).  Kernel A selects under the a-geometry,
    the pooled Kernel C attends under base RoPE at dense ranks.  Returns (out, usize, kept_size).
    shared_selection_triton_chunked.py:249-322."""
    Z, H, N, D = q.shape
    assert Z == 1
    assert tile == 32, "the chunked kernel runs PQ Kernel A: tile must be 32"
    assert chunk_agg in native.CHUNK_AGG, f"chunk_agg must be sum|mean, got {chunk_agg!r}"
    if n_chunk is None:
        n_chunk = derive_n_chunk(k_max, chunk_size, n_global, n_local, tile)
    nf = n_forced_chunks(chunk_size, n_global, n_local, tile)
    nC_total = (N + chunk_size - 1) // chunk_size
    bound = min(nC_total, nf + n_chunk) * chunk_size
    assert bound <= k_max, (
        f"budget overflow: min(nC={nC_total}, {nf} forced + {n_chunk} selected) * {chunk_size} = "
        f"{bound} > k_max={k_max}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    r = native.chunk_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale, n_global,
                               n_local, tile, k_max, chunk_size, n_chunk, q_pos_base, select_score, chunk_agg)
    if measure:
        _stat_acc(r["passers_kept"], r["usize"], r["kept_size"], "prefill")
    return r["out"].unsqueeze(0), r["usize"], r["kept_size"]


def _decode_build_sets_chunk(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, n_global, n_local,
                             k_max, chunk_size, n_chunk, scores=None, select_score="expmass", chunk_agg="sum",
                             measure=False):
    """Chunk selection for one query.  q:(H,D), K:(H,M,D) (or Hkv heads), M = q_pos + 1.  Returns
    idx (H,k_max) long (sentinel M), newpos_k (H,k_max) fp32, newpos_q (H,) fp32.
    shared_selection_triton_chunked.py:411-489."""
    from _decode import _tau_of
    H, M = q.shape[0], K.shape[-2]
    plan = native.DecodePlan(q, K, None, _tau_of(tau, H), inv_freq_a, int(q_pos), pos_scale_a, rope_scale_a,
                             sm_scale, n_global, n_local, k_max, 100.0)
    if scores is None:
        s = plan.scores(torch.empty((H, 1, M), dtype=torch.float32, device=q.device))
    else:
        s = scores.to(device=q.device, dtype=torch.float32).reshape(H, 1, M).contiguous()
    pk = torch.empty((H, 1), dtype=torch.int32, device=q.device)
    us = torch.empty((H, 1), dtype=torch.int32, device=q.device)
    r = plan.build_sets_chunk(s, chunk_size, n_chunk, select_score, chunk_agg, passers_kept=pk, usize=us)
    if measure:
        _stat_acc(pk, us, r["set_size"], "decode")
    return r["idx"][:, 0].long(), r["newpos_k"][:, 0], r["newpos_q"][:, 0]


def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32, tile=32, k_max=4096,
                              block_n=32, block_k=32, max_len=None, pct_decode=100.0, decode_backend="triton",
                              select_backend="triton", prefill_mode="shared", measure=False,
                              select_score="expmass", select_geom="pi", apply_mscale=True, chunk_size=16,
                              n_chunk=None, chunk_agg="sum"):
    """Patch LlamaAttention.forward to route prefill and decode through the chunked kernels.
    select_geom / apply_mscale / select_score as for the per-query kernel; pct / pct_decode are
    accepted and ignored (the budget is n_chunk).  Each attention module needs ``tau_head_vec``
    (H,) set by the caller.  shared_selection_triton_chunked.py:495-643."""
    from _install import install_chunked
    assert select_geom in ("pi", "yarn"), f"select_geom must be pi|yarn, got {select_geom!r}"
    assert chunk_agg in ("sum", "mean"), f"chunk_agg must be sum|mean, got {chunk_agg!r}"
    if n_chunk is None:
        n_chunk = derive_n_chunk(k_max, chunk_size, n_global, n_local, tile)
    install_chunked(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, k_max, max_len,
                    decode_backend, prefill_mode, select_score, measure, chunk_size, n_chunk, chunk_agg)
