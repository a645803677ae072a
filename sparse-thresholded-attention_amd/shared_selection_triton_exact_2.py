"""Drop-in for shared_selection_triton_exact_2.py (PI_exact): exact-max shared-selection prefill.

Same entry points and signatures as the reference; the work runs in the gfx950 HIP kernels of
libsta_hip.so (no Triton, no fallback).  `block_n` / `block_k` are the reference's Triton tile
knobs and are accepted and ignored.
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill


def _build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
                wvotes=None, select_score="freq"):
    """votes (H,nt,N) int -> (idx, newpos_k, newpos_q, shared_size, kept_size, chosen,
    orig_overflow, kpct_meas, overflow20).  shared_selection_triton_exact_2.py:277-426."""
    return _device_build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base,
                              measure, wvotes, select_score)


def shared_pi_attention(q, k, v, tau, inv_freq, pos_scale=1.0, pct=30.0, sm_scale=None,
                        rope_scale=1.0, n_global=32, n_local=32, tile=32, k_max=1024,
                        block_n=64, block_k=64, q_pos_base=0, measure=False, select_score="freq"):
    """q,k,v: (1,H,N,D) raw (k, v may carry H/g heads for GQA).  Returns (out, shared_size,
    kept_size, kpct, overflow, kpct_meas, overflow20).  shared_selection_triton_exact_2.py:432-486."""
    return shared_prefill(q, k, v, tau, inv_freq, pos_scale, rope_scale, inv_freq, pos_scale,
                          rope_scale, pct, sm_scale, n_global, n_local, tile, k_max, q_pos_base,
                          measure, select_score)
