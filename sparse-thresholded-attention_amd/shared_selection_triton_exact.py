"""Drop-in for shared_selection_triton_exact.py (the original exact-max kernel, freq votes).

Its _build_sets sorts where exact_2 uses topk/scatter; in frequency mode both produce the same
sets (shared_selection_triton_exact.py:253-370 vs shared_selection_triton_exact_2.py:277-426), so
both files map onto the same HIP path.
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill
from _torch_golden import _rope_rotate  # noqa: F401  (the reference's torch RoPE helper)


def _build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False):
    """shared_selection_triton_exact.py:254-370."""
    return _device_build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base, measure)


def shared_pi_attention(q, k, v, tau, inv_freq, pos_scale=1.0, pct=30.0, sm_scale=None,
                        rope_scale=1.0, n_global=32, n_local=32, tile=32, k_max=1024,
                        block_n=64, block_k=64, q_pos_base=0, measure=False):
    """shared_selection_triton_exact.py:376-423."""
    return shared_prefill(q, k, v, tau, inv_freq, pos_scale, rope_scale, inv_freq, pos_scale,
                          rope_scale, pct, sm_scale, n_global, n_local, tile, k_max, q_pos_base,
                          measure, "freq")


# ---------------------------------------------------------------------------------------------
# decode (one query per call): shared_selection_triton_exact.py:442-594, the same helpers as
# shared_selection_triton_exact_2.py:505-655
# ---------------------------------------------------------------------------------------------
from shared_selection_triton_exact_2 import (_decode_attend_kernelC, _decode_attend_torch,  # noqa: E402,F401
                                             _decode_build_sets, _decode_scores_kernel)



def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32,
                              tile=32, k_max=1024, block_n=32, block_k=32, max_len=None,
                              pct_decode=100.0, decode_backend="torch", select_backend="torch",
                              prefill_mode="shared", measure=False):
    """shared_selection_triton_exact.py:595-700 (frequency ranking)."""
    from _install import install
    install(model, "pi", pct, context_window, n_global, n_local, tile, k_max, block_n, block_k, max_len,
            pct_decode, decode_backend, select_backend, prefill_mode, measure, "freq")
