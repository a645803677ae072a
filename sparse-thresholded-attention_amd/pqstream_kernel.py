"""Drop-in for pqstream_kernel.py (PQ Stream): per-query keep sets with streamed tile positions.

Same prefill entry point and signature as the reference (pqstream_attention,
pqstream_kernel.py:498-564) and the same measurement-only span / kept / skip counters
(get_overflow_stats, reset_overflow_stats, reset_span_stats; pqstream_kernel.py:88-150).  The
work runs in the gfx950 HIP kernels of libsta_hip.so (no Triton, no fallback).  `num_warps` is
the reference's Triton knob and is accepted and ignored; block_n must be 32 or 64.
"""
import math

import torch

import _sta_native as native
from _counters import PhaseCounters, ratio

ADV_MAX = 0
ADV_FULL = 1
_ADV = {"max": ADV_MAX, "full": ADV_FULL}


# measurement-only statistics per phase (the reference's get_overflow_stats keys,
# pqstream_kernel.py:85-150): a cell is a (head, tile), a row is one query
_STATS = {p: PhaseCounters(sums=("span", "kept", "blocks", "skipped"), maxes=("span",),
                           counts=("cells", "rows")) for p in ("prefill", "decode")}


def reset_overflow_stats():
    """Zero the cumulative span / kept / skip counters."""
    for c in _STATS.values():
        c.clear()


reset_span_stats = reset_overflow_stats


def _summary(c):
    n, s, m = c.read()
    blocks, skipped = int(s["blocks"]), int(s["skipped"])
    # PQ Stream has no k_max: the two overflow fields are always 0 (kept for pq_exact callers)
    return {"total_cells": n["cells"], "span_mean": ratio(s["span"], n["cells"]), "span_max": m["span"],
            "kept_mean": ratio(s["kept"], n["rows"]), "blocks": blocks, "skipped": skipped,
            "skip_frac": ratio(skipped, blocks), "overflow_cells": 0, "overflow_frac": 0.0}


def get_overflow_stats():
    """Cumulative since the last reset, per phase (one host sync here, none during the run)."""
    return {p: _summary(c) for p, c in _STATS.items()}


def _record(span, kept, blocks, skipped, phase="prefill"):
    """span (H,nt) fp32, kept (H,N) int32, blocks / skipped (H,nt) int32, all on the device."""
    _STATS[phase].add({"cells": span.numel(), "rows": kept.numel()},
                      (span.sum(dtype=torch.float64), kept.sum(dtype=torch.float64),
                       blocks.sum(dtype=torch.float64), skipped.sum(dtype=torch.float64)),
                      (span.max(),))


def pqstream_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                       sm_scale=None, n_global=32, n_local=32, tile=32, block_n=32,
                       pos_advance="max", q_pos_base=0, use_skip=True, num_warps=None):
    """q,k,v: (1,H,N,D) raw (k, v may carry H/g heads for GQA).  Selection under the a-geometry,
    attention under base RoPE (inv_freq_c) at the streamed positions.  Returns (out, span, kept,
    blocks, skipped).  pqstream_kernel.py:498-564."""
    Z, H, N, D = q.shape
    assert Z == 1
    assert tile == 32, "BLOCK_M is fixed at 32 by the tile convention"
    assert q_pos_base == 0, f"pqstream prefill expects q_pos_base == 0, got {q_pos_base}"
    assert block_n >= tile - 1, f"block_n={block_n} < tile-1={tile - 1}: the tau=inf oracle would not hold"
    if pos_advance not in _ADV:
        raise KeyError(pos_advance)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    r = native.pqstream_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale,
                                  n_global, n_local, tile, block_n, pos_advance, q_pos_base, use_skip)
    _record(r["span"], r["kept"], r["blocks"], r["skipped"], phase="prefill")
    return r["out"].unsqueeze(0), r["span"], r["kept"], r["blocks"], r["skipped"]
