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

ADV_MAX = 0
ADV_FULL = 1
_ADV = {"max": ADV_MAX, "full": ADV_FULL}


def _fresh():
    return {"cells": 0, "span_sum": None, "span_max": None,
            "kept_sum": None, "rows": 0, "blocks": None, "skipped": None}


_STATS = {"prefill": _fresh(), "decode": _fresh()}


def reset_overflow_stats():
    """Zero the cumulative span / kept / skip counters."""
    _STATS["prefill"] = _fresh()
    _STATS["decode"] = _fresh()


reset_span_stats = reset_overflow_stats


def _phase_stats(d):
    tot = d["cells"]
    ssum = float(d["span_sum"].item()) if d["span_sum"] is not None else 0.0
    smax = float(d["span_max"].item()) if d["span_max"] is not None else 0.0
    ksum = float(d["kept_sum"].item()) if d["kept_sum"] is not None else 0.0
    blk = int(d["blocks"].item()) if d["blocks"] is not None else 0
    skp = int(d["skipped"].item()) if d["skipped"] is not None else 0
    return {"total_cells": tot, "span_mean": (ssum / tot) if tot else 0.0, "span_max": smax,
            "kept_mean": (ksum / d["rows"]) if d["rows"] else 0.0, "blocks": blk, "skipped": skp,
            "skip_frac": (skp / blk) if blk else 0.0, "overflow_cells": 0, "overflow_frac": 0.0}


def get_overflow_stats():
    """Cumulative since the last reset, per phase (one host sync here, none during the run)."""
    return {"prefill": _phase_stats(_STATS["prefill"]), "decode": _phase_stats(_STATS["decode"])}


def _acc(dst, key, val, reduce="sum"):
    if dst[key] is None:
        dst[key] = val
    elif reduce == "max":
        dst[key] = torch.maximum(dst[key], val)
    else:
        dst[key] = dst[key] + val


def _stats_accumulate(span, kept, blocks, skipped, phase="prefill"):
    """Measurement only, on the device (pqstream_kernel.py:138-150)."""
    d = _STATS[phase]
    d["cells"] += span.numel()
    d["rows"] += kept.numel()
    _acc(d, "span_sum", span.double().sum())
    _acc(d, "span_max", span.max(), reduce="max")
    _acc(d, "kept_sum", kept.double().sum())
    _acc(d, "blocks", blocks.long().sum())
    _acc(d, "skipped", skipped.long().sum())


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
    _stats_accumulate(r["span"], r["kept"], r["blocks"], r["skipped"], phase="prefill")
    return r["out"].unsqueeze(0), r["span"], r["kept"], r["blocks"], r["skipped"]
