"""Drop-in for shared_selection_triton_perquery.py (PQ Union): per-query key sets through the
tile's union, dense-rank positions and a per-slot query bitmask.

Same prefill entry points and signatures as the reference (shared_pq_attention,
perquery.py:459-525; _build_sets_pq, perquery.py:363-453) and the same measurement-only overflow
counters (get_overflow_stats / reset_overflow_stats, perquery.py:52-112).  The work runs in the
gfx950 HIP kernels of libsta_hip.so (no Triton, no fallback).  `block_n` / `block_k` are the
reference's Triton tile knobs and are accepted and ignored.

One documented difference: when the union overflows k_max, keys whose rank value ties at the cut
are taken in ascending key order; the reference leaves that choice to torch.topk, whose order
among equal values is unspecified.
"""
import math

import torch

import _sta_native as native
from _counters import PhaseCounters, ratio


# measurement-only statistics per phase (the reference's get_overflow_stats keys,
# perquery.py:52-112): a prefill cell is a (head, 32-query tile), a decode cell a (head, query)
_OVF_STATS = {p: PhaseCounters(sums=("overflow", "union"), maxes=("union",)) for p in ("prefill", "decode")}


def reset_overflow_stats():
    """Zero the cumulative overflow / union counters."""
    for c in _OVF_STATS.values():
        c.clear()


def _summary(c):
    n, s, m = c.read()
    cells, ovf = n["cells"], int(s["overflow"])
    return {"total_cells": cells, "overflow_cells": ovf, "overflow_frac": ratio(ovf, cells),
            "union_mean": ratio(s["union"], cells), "union_max": int(m["union"])}


def get_overflow_stats():
    """Cumulative since the last reset, per phase (one host sync here, none during the run)."""
    return {p: _summary(c) for p, c in _OVF_STATS.items()}


def _record(overflow, usize, phase="prefill"):
    """overflow (H, n) bool, usize (H, n) int32, on the device."""
    _OVF_STATS[phase].add({"cells": overflow.numel()},
                          (overflow.sum(dtype=torch.float64), usize.sum(dtype=torch.float64)),
                          (usize.max(),))


def _build_sets_pq(votes, bits, wvotes, n_global, n_local, T, k_max, q_pos_base=0,
                   select_score="expmass"):
    """votes / bits (H,nt,N) int32, wvotes (H,nt,N) fp32 (or a dummy) -> (idx, newpos_k,
    newpos_q, mask, usize, kept_size, overflow).  shared_selection_triton_perquery.py:363-453."""
    res = native.pq_build_sets(votes, bits, wvotes, n_global, n_local, T, k_max, q_pos_base, select_score)
    _record(res[6], res[4])
    return res


def shared_pq_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                        sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096,
                        block_n=64, block_k=64, q_pos_base=0, select_score="expmass"):
    """q,k,v: (1,H,N,D) raw (k, v may carry H/g heads for GQA).  Selection under the
    a-geometry, attention under base RoPE (inv_freq_c, scale 1) at dense ranks.  Returns
    (out, usize, kept_size, overflow).  shared_selection_triton_perquery.py:459-525."""
    Z, H, N, D = q.shape
    assert Z == 1
    assert tile == 32, "pq_exact packs per-query keep bits into int32 -> tile must be 32"
    assert n_global + n_local + tile - 1 <= k_max, (
        f"forced set (n_global={n_global} + n_local={n_local} + tile-1={tile - 1} = "
        f"{n_global + n_local + tile - 1}) exceeds k_max={k_max}: forced keys would be dropped")
    if select_score not in native.SCORES:
        raise KeyError(select_score)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    r = native.pq_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale,
                            n_global, n_local, tile, k_max, q_pos_base, select_score)
    _record(r["overflow"], r["usize"])
    return r["out"].unsqueeze(0), r["usize"], r["kept_size"], r["overflow"]
