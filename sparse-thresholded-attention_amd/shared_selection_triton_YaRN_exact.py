"""Drop-in for shared_selection_triton_YaRN_exact.py: the same kernels under YaRN geometry.

The caller passes the YaRN inv_freq, pos_scale = 1 and rope_scale = mscale
(shared_selection_triton_YaRN_exact.py:681-690, 735-740); nothing else differs from PI_exact.
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill
from _torch_golden import _rope_rotate  # noqa: F401  (the reference's torch RoPE helper)


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


# ---------------------------------------------------------------------------------------------
# decode (one query per call): shared_selection_triton_YaRN_exact.py:515-666, the same helpers as
# shared_selection_triton_exact_2.py:505-655
# ---------------------------------------------------------------------------------------------
from shared_selection_triton_exact_2 import (_decode_attend_kernelC, _decode_attend_torch,  # noqa: E402,F401
                                             _decode_build_sets, _decode_scores_kernel)



def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32,
                              tile=32, k_max=1024, block_n=32, block_k=32, max_len=None,
                              pct_decode=100.0, decode_backend="torch", select_backend="torch",
                              prefill_mode="shared", measure=False, select_score="freq",
                              apply_mscale=True):
    """shared_selection_triton_YaRN_exact.py:668-776: the model must be loaded with YaRN rope
    scaling; its rotary frequencies and attention scaling (mscale) are the geometry, positions stay
    raw (pos_scale 1); apply_mscale=False rotates with scale 1."""
    from _install import install
    mscale = float(getattr(model.model.rotary_emb, "attention_scaling", 1.0))
    if mscale == 1.0:
        print("WARNING [YaRN kernel]: rotary.attention_scaling == 1.0 -- the model does not look "
              "yarn-loaded (mscale should be > 1).  Load it with rope_scaling rope_type='yarn'.", flush=True)
    install(model, "yarn", pct, context_window, n_global, n_local, tile, k_max, block_n, block_k, max_len,
            pct_decode, decode_backend, select_backend, prefill_mode, measure, select_score,
            rope_scale=mscale if apply_mscale else 1.0)
