"""Drop-in for shared_selection_triton_exact_2.py (PI_exact): exact-max shared-selection prefill.

Same entry points and signatures as the reference; the work runs in the gfx950 HIP kernels of
libsta_hip.so (no Triton, no fallback).  `block_n` / `block_k` are the reference's Triton tile
knobs and are accepted and ignored.
"""
from _shared_prefill import build_sets as _device_build_sets
from _shared_prefill import shared_prefill
from _torch_golden import _rope_rotate  # noqa: F401  (the reference's torch RoPE helper)


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


# ---------------------------------------------------------------------------------------------
# decode (one query per call): shared_selection_triton_exact_2.py:505-655
# ---------------------------------------------------------------------------------------------
def _decode_scores_kernel(q, K, inv_freq, q_pos, pos_scale, rope_scale, sm_scale, block_n=64):
    """Per-key scores (H,M) for one query.  q:(H,D), K:(H,M,D) (or Hkv heads).
    shared_selection_triton_exact_2.py:505-525 (the _decode_select_kernel launch)."""
    from _decode import decode_scores
    return decode_scores(q, K, inv_freq, q_pos, pos_scale, rope_scale, sm_scale)


def _decode_build_sets(q, K, tau, inv_freq, q_pos, pos_scale, rope_scale, sm_scale, n_global, n_local,
                       k_max, pct_decode, scores=None):
    """Per-query selection + PI reposition: (idx (H,k_max) long, sentinel M; newpos_k (H,k_max);
    newpos_q (H,)).  shared_selection_triton_exact_2.py:527-604."""
    from _decode import decode_build_sets
    return decode_build_sets(q, K, tau, inv_freq, q_pos, pos_scale, rope_scale, sm_scale, n_global, n_local,
                             k_max, pct_decode, scores)


def _decode_attend_torch(q, K, V, idx, newpos_k, newpos_q, inv_freq, rope_scale, sm_scale):
    """Attend over the selected set -> (H,D) in q.dtype (slots valid where idx < M).
    shared_selection_triton_exact_2.py:608-623."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx, newpos_k, newpos_q, inv_freq, rope_scale, sm_scale)


def _decode_attend_kernelC(q, K, V, idx, newpos_k, newpos_q, inv_freq, rope_scale, sm_scale, k_max, q_pos,
                           block_m=16, block_k=32):
    """Attend with Kernel C's slot rule (idx < M and idx <= q_pos) -> (H,D).  block_m / block_k are
    the reference's tile knobs, accepted and ignored.  shared_selection_triton_exact_2.py:626-655."""
    from _decode import decode_attend
    return decode_attend(q, K, V, idx[..., :k_max], newpos_k[..., :k_max], newpos_q, inv_freq, rope_scale,
                         sm_scale, q_pos=q_pos)


# ---------------------------------------------------------------------------------------------
# model integration: shared_selection_triton_exact_2.py:658-767
# ---------------------------------------------------------------------------------------------
def install_shared_pi_forward(model, pct=30.0, context_window=4096, n_global=32, n_local=32,
                              tile=32, k_max=1024, block_n=32, block_k=32, max_len=None,
                              pct_decode=100.0, decode_backend="torch", select_backend="torch",
                              prefill_mode="shared", measure=False, select_score="freq"):
    """Patch LlamaAttention.forward to route prefill and decode through the HIP kernels (PI
    geometry: the model's rotary frequencies, positions compressed by pos_scale = min(1, W / L)
    frozen at prefill).  Each attention module needs ``tau_head_vec`` (H,) set by the caller."""
    from _install import install
    install(model, "pi", pct, context_window, n_global, n_local, tile, k_max, block_n, block_k, max_len,
            pct_decode, decode_backend, select_backend, prefill_mode, measure, select_score)
