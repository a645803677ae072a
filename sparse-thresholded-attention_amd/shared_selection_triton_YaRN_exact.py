"""Drop-in for shared_selection_triton_YaRN_exact.py: the same kernels under YaRN geometry.

The caller passes the YaRN inv_freq, pos_scale = 1 and rope_scale = mscale
(shared_selection_triton_YaRN_exact.py:681-690, 735-740); nothing else differs from PI_exact.
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill


def _build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
                wvotes=None, select_score="freq"):
    """shared_selection_triton_YaRN_exact.py:288-436."""
    return _device_build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base,
                              measure, wvotes, select_score)


def shared_pi_attention(q, k, v, tau, inv_freq, pos_scale=1.0, pct=30.0, sm_scale=None,
                        rope_scale=1.0, n_global=32, n_local=32, tile=32, k_max=1024,
                        block_n=64, block_k=64, q_pos_base=0, measure=False, select_score="freq"):
    """shared_selection_triton_YaRN_exact.py:442-496."""
    return shared_prefill(q, k, v, tau, inv_freq, pos_scale, rope_scale, inv_freq, pos_scale,
                          rope_scale, pct, sm_scale, n_global, n_local, tile, k_max, q_pos_base,
                          measure, select_score)
