"""Drop-in for shared_selection_triton_hybrid_exact.py: Kernel A selects under one geometry
(YaRN), the reposition and the gather-attention run under another (PI with base RoPE).
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill
from _torch_golden import _rope_rotate  # noqa: F401  (the reference's torch RoPE helper)


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


# ---------------------------------------------------------------------------------------------
# decode (one query per call): shared_selection_triton_hybrid_exact.py:529-681 -- selection
# under the a-geometry, reposition with pos_scale_c, attend under the geometry its caller passes
# ---------------------------------------------------------------------------------------------
from shared_selection_triton_exact_2 import (_decode_attend_kernelC, _decode_attend_torch,  # noqa: E402,F401
                                             _decode_scores_kernel)


def _decode_build_sets(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, n_global, n_local,
                       k_max, pct_decode, pos_scale_c, scores=None):
    """Per-query selection under (inv_freq_a, pos_scale_a, rope_scale_a) + reposition with
    pos_scale_c: (idx (H,k_max) long, sentinel M; newpos_k (H,k_max); newpos_q (H,)).
    shared_selection_triton_hybrid_exact.py:551-629."""
    from _decode import decode_build_sets
    return decode_build_sets(q, K, tau, inv_freq_a, q_pos, pos_scale_a, rope_scale_a, sm_scale, n_global,
                             n_local, k_max, pct_decode, scores, pos_scale_c=pos_scale_c)



def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32,
                              tile=32, k_max=1024, block_n=32, block_k=32, max_len=None,
                              pct_decode=100.0, decode_backend="torch", select_backend="torch",
                              prefill_mode="shared", measure=False, select_score="freq",
                              apply_mscale=True):
    """shared_selection_triton_hybrid_exact.py:683-811: selection under the model's YaRN rotary
    (raw positions, mscale when apply_mscale), reposition and attend under base RoPE with
    pos_scale_c = min(1, W / L) frozen at prefill."""
    from _install import base_inv_freq_of, install
    rotary = model.model.rotary_emb
    mscale = float(getattr(rotary, "attention_scaling", 1.0))
    if mscale == 1.0:
        print("WARNING [hybrid kernel]: rotary.attention_scaling == 1.0 -- the model does not look "
              "yarn-loaded (mscale should be > 1).  Load it with rope_scaling rope_type='yarn'.", flush=True)
    inv_freq_a = rotary.inv_freq.detach().float()
    inv_freq_c = base_inv_freq_of(model)
    assert inv_freq_c.numel() == inv_freq_a.numel(), \
        f"base/yarn inv_freq length mismatch: {inv_freq_c.numel()} vs {inv_freq_a.numel()}"
    geometry = {"inv_freq_a": inv_freq_a, "rope_scale_a": mscale if apply_mscale else 1.0, "inv_freq_c": inv_freq_c}
    install(model, geometry, pct, context_window, n_global, n_local, tile, k_max, block_n, block_k, max_len,
            pct_decode, decode_backend, select_backend, prefill_mode, measure, select_score)
