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
from _torch_golden import _rope_rotate, pqstream_attention_torch  # noqa: F401  (torch helper and golden)

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


# ---------------------------------------------------------------------------------------------
# decode (one query per call) and model integration: pqstream_kernel.py:673-998
# ---------------------------------------------------------------------------------------------
def _kbuf(M):
    """The reference's slot buffer: M rounded up to a multiple of 1024, at least 1024 (:758-767)."""
    return max(1024, -(-M // 1024) * 1024)


def _decode_scores_kernel(q, K, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, block_n=64):
    """Per-key scores (H,M) for one query.  q:(H,D), K:(H,M,D) (or Hkv heads).  block_n is the
    reference's Triton knob, accepted and ignored.  pqstream_kernel.py:673-692."""
    from _decode import decode_scores
    return decode_scores(q, K, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale)


def _record_decode(idx, newpos_k, size, m, block_n):
    """The decode counters of a batch of queries (pqstream_kernel.py:786-791): per query the
    largest streamed distance among its kept keys, its kept count, its block count ceil(m / block_n)
    and the blocks without a kept key.  idx / newpos_k (H, Q, S) with the sentinel m, size (H, Q),
    m (Q,) the key count each query sees."""
    m = torch.as_tensor(m, device=idx.device).reshape(1, -1, 1)
    idx = idx.long()
    valid = idx < m
    span = torch.where(valid, -newpos_k, torch.zeros_like(newpos_k)).amax(-1)
    blk = torch.div(idx, block_n, rounding_mode="floor")
    first = torch.ones_like(valid)
    first[..., 1:] = blk[..., 1:] != blk[..., :-1]
    nb = torch.div(m[..., 0] + block_n - 1, block_n, rounding_mode="floor").expand_as(span)
    used = (first & valid).sum(-1)
    _record(span, size, nb.float(), (nb - used).float(), phase="decode")


def _decode_build_sets_pqs(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale,
                           n_global, n_local, block_n, scores=None, block_k=32):
    """Per-query selection with streamed positions for one query: every threshold passer plus the
    forced global / local / self keys (no cap), blocks of block_n keys walked from the query
    backwards.  Returns idx (H,kbuf) long (sentinel M), newpos_k (H,kbuf) fp32, newpos_q (H,)
    fp32 zeros, with kbuf = M rounded up to 1024; records the decode counters.
    pqstream_kernel.py:695-797."""
    import _sta_native as nat
    from _decode import _tau_of
    H, M = q.shape[0], K.shape[-2]
    kbuf = _kbuf(M)
    assert kbuf % block_k == 0, f"kbuf={kbuf} must be a multiple of block_k={block_k}"
    plan = nat.DecodePlan(q, K, None, _tau_of(tau, H), inv_freq_a, int(q_pos), pos_scale_a, rope_scale_a,
                          sm_scale, n_global, n_local, kbuf, 100.0, rule="stream", block_n=block_n)
    if scores is None:
        s = plan.scores(torch.empty((H, 1, M), dtype=torch.float32, device=q.device))
    else:
        s = scores.to(device=q.device, dtype=torch.float32).reshape(H, 1, M).contiguous()
    r = plan.build_sets(s)
    idx, npk, npq = r["idx"][:, 0].long(), r["newpos_k"][:, 0], r["newpos_q"][:, 0]
    _record_decode(r["idx"], r["newpos_k"], r["set_size"], [M], block_n)
    return idx, npk, npq


def _decode_attend_torch(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, sm_scale):
    """Attend over the selected set under base RoPE (rope_scale 1) at the streamed positions ->
    (H,D) in q.dtype.  pqstream_kernel.py:800-817."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, 1.0, sm_scale)


def _decode_attend_triton(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, sm_scale, q_pos, block_m=16,
                          block_k=32):
    """The same attend with the kernel's slot rule (idx < M and idx <= q_pos) -> (H,D).  block_m /
    block_k are the reference's tile knobs, accepted and ignored.  pqstream_kernel.py:820-850."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, 1.0, sm_scale, q_pos=q_pos)


def install_pqstream_forward(model, context_window=4096, n_global=32, n_local=32, tile=32, block_n=32,
                             block_k=32, max_len=None, decode_backend="torch", select_backend="torch",
                             prefill_mode="stream", select_geom="pi", apply_mscale=True, pos_advance="max",
                             use_skip=True, num_warps=None, pct=None, pct_decode=None, k_max=None,
                             select_score=None, measure=False, **_unused):
    """Patch LlamaAttention.forward to route prefill and decode through the PQ Stream kernels.

    select_geom "pi": base frequencies at positions compressed by the frozen pos_scale = min(1,
    W / L); "yarn": the model's rotary frequencies at raw positions, its attention scaling as the
    selection's rope scale when apply_mscale.  Attention runs under base RoPE at the streamed
    positions.  prefill_mode "stream" (or "shared") runs the streamed prefill, "perquery" lets
    every prompt position select its own set as decode steps do.  pct / pct_decode / k_max /
    select_score / measure are accepted and ignored, as in the reference (PQ Stream has no budget
    and no ranking).  Each attention module needs ``tau_head_vec`` (H,) set by the caller.
    pqstream_kernel.py:834-998."""
    from _install import install_pqstream
    assert select_geom in ("pi", "yarn"), f"select_geom must be pi|yarn, got {select_geom!r}"
    assert pos_advance in _ADV, f"pos_advance must be max|full, got {pos_advance!r}"
    assert block_n >= tile - 1, f"block_n={block_n} must be >= tile-1={tile - 1}"
    if prefill_mode == "shared":
        prefill_mode = "stream"
    install_pqstream(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, block_n, block_k,
                     max_len, decode_backend, prefill_mode, pos_advance, use_skip)


install_shared_pi_forward = install_pqstream_forward
