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
from _torch_golden import _rope_rotate, pq_attention_torch  # noqa: F401  (torch helper and golden)


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


# ---------------------------------------------------------------------------------------------
# decode (one query per call) and the per-query prefill: shared_selection_triton_perquery.py:630-778
# ---------------------------------------------------------------------------------------------
def _decode_scores_kernel(q, K, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, block_n=64):
    """Per-key scores (H,M) for one query.  q:(H,D), K:(H,M,D) (or Hkv heads).  block_n is the
    reference's Triton knob, accepted and ignored.  perquery.py:630-647."""
    from _decode import decode_scores
    return decode_scores(q, K, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale)


def _decode_build_sets_pq(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale,
                          n_global, n_local, k_max, scores=None):
    """Per-query selection with dense-rank positions for one query: threshold passers plus the
    forced global / local / self keys; above k_max the forced keys plus the top-(k_max - n_forced)
    others by score (keys with equal scores at the cut in ascending key order).  Returns idx
    (H,k_max) long (sentinel M), newpos_k (H,k_max) fp32, newpos_q (H,) fp32, and records the
    decode overflow counters.  perquery.py:651-720."""
    assert n_global + n_local <= k_max, (
        f"decode forced set (n_global={n_global} + n_local={n_local}) exceeds k_max={k_max}")
    from _decode import decode_build_sets
    st = {}
    res = decode_build_sets(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, n_global,
                            n_local, k_max, 100.0, scores, rule="pq", stats=st)
    _record(st["overflow"][:, None], st["usize"][:, None], phase="decode")
    return res


def _decode_attend_torch_pq(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, sm_scale):
    """Attend over the selected set under base RoPE (rope_scale 1) at the dense ranks -> (H,D) in
    q.dtype.  perquery.py:723-740."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, 1.0, sm_scale)


def _decode_attend_kernelC_pq(q, K, V, idx, newpos_k, newpos_q, inv_freq_c, sm_scale, k_max, q_pos,
                              block_m=16, block_k=32):
    """The same attend with the PQ Kernel C's slot rule (idx < M and idx <= q_pos) -> (H,D).
    block_m / block_k are the reference's tile knobs, accepted and ignored.  perquery.py:743-778."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx[..., :k_max], newpos_k[..., :k_max], newpos_q, inv_freq_c, 1.0, sm_scale,
                         q_pos=q_pos)


def perquery_prefill_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                               sm_scale=None, n_global=32, n_local=32, k_max=4096):
    """prefill_mode="perquery" (perquery.py:905-924) as one call: every prompt position P selects
    over the keys [0, P] with _decode_build_sets_pq's rule and attends them under base RoPE at the
    dense ranks.  q,k,v: (1,H,N,D) (k, v may carry H/g heads).  Returns (out (1,H,N,D), usize,
    set_size, overflow), the last three (H,N) per query; the overflow counters are recorded under
    the "decode" phase, as the reference's per-token loop records them."""
    Z, H, N, D = q.shape
    assert Z == 1
    assert n_global + n_local <= k_max, (
        f"decode forced set (n_global={n_global} + n_local={n_local}) exceeds k_max={k_max}")
    r = native.perquery_prefill_attention(q, k, v, _tau(tau, H, q.device), inv_freq_a, inv_freq_c, pos_scale_a,
                                          rope_scale_a, sm_scale, n_global, n_local, k_max)
    _record(r["overflow"], r["usize"], phase="decode")
    return r["out"].unsqueeze(0), r["usize"], r["set_size"], r["overflow"]


def _tau(tau, H, dev):
    t = torch.as_tensor(tau, dtype=torch.float32).reshape(-1).to(dev)
    return t.expand(H).contiguous() if t.numel() == 1 else t


# ---------------------------------------------------------------------------------------------
# model integration: shared_selection_triton_perquery.py:784-930
# ---------------------------------------------------------------------------------------------
def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32,
                              tile=32, k_max=4096, block_n=32, block_k=32, max_len=None,
                              pct_decode=100.0, decode_backend="torch", select_backend="torch",
                              prefill_mode="shared", measure=False, select_score="expmass",
                              select_geom="pi", apply_mscale=True):
    """Patch LlamaAttention.forward to route prefill and decode through the per-query kernels.

    select_geom "pi": base frequencies at positions compressed by pos_scale = min(1, W / L), frozen
    at prefill; "yarn": the model's (YaRN-loaded) rotary frequencies at raw positions, with its
    attention scaling as the selection's rope scale when apply_mscale.  Attention always runs
    under base RoPE at dense ranks.  prefill_mode "shared" runs the tile-32 union prefill
    (shared_pq_attention), "perquery" lets every prompt position select its own set, as decode
    steps do.  pct / pct_decode / measure are accepted and ignored, as in the reference;
    decode_backend / select_backend pick the reference's torch or Triton rule, which select and
    attend identically here.  Each attention module needs ``tau_head_vec`` (H,) set by the caller.
    perquery.py:784-930."""
    from _install import install_perquery
    assert select_geom in ("pi", "yarn"), f"select_geom must be pi|yarn, got {select_geom!r}"
    install_perquery(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, k_max, max_len,
                     decode_backend, prefill_mode, select_score, block_n, block_k)
