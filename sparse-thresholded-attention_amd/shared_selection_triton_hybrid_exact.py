"""Drop-in for shared_selection_triton_hybrid_exact.py: Kernel A selects under one geometry
(YaRN), the reposition and the gather-attention run under another (PI with base RoPE).
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill


def _build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
                wvotes=None, select_score="freq"):
    """shared_selection_triton_hybrid_exact.py:296-444."""
    return _device_build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base,
                              measure, wvotes, select_score)


def shared_pi_attention(q, k, v, tau,
                        inv_freq_a, pos_scale_a, rope_scale_a,
                        inv_freq_c, pos_scale_c, rope_scale_c,
                        pct=30.0, sm_scale=None, n_global=32, n_local=32, tile=32, k_max=1024,
                        block_n=64, block_k=64, q_pos_base=0, measure=False, select_score="freq"):
    """shared_selection_triton_hybrid_exact.py:450-510."""
    return shared_prefill(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c,
                          pos_scale_c, rope_scale_c, pct, sm_scale, n_global, n_local, tile, k_max,
                          q_pos_base, measure, select_score)
