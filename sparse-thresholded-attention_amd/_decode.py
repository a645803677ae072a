"""Decode entry points: each query selects its own key set over the KV cache and attends it.

The reference's decode helpers (shared_selection_triton_exact_2.py:505-655) take one query per
call; here they run on the HIP kernels of libsta_hip.so (sta_decode_*), and decode_attention
serves a whole batch of queries over one cache in a single call.  No torch or Triton fallback.
"""
import math

import torch

import _sta_native as native


def _tau_of(tau, H):
    t = torch.as_tensor(tau, dtype=torch.float32).reshape(-1)
    return t.expand(H).contiguous() if t.numel() == 1 else t


def decode_scores(q, K, inv_freq, q_pos, pos_scale, rope_scale, sm_scale):
    """Per-key scores (H, M) fp32 of one query q (H, D) over K (H or Hkv, M, D)."""
    H, M = q.shape[0], K.shape[-2]
    plan = native.DecodePlan(q, K, None, torch.zeros(H), inv_freq, int(q_pos), pos_scale, rope_scale,
                             sm_scale, k_max=1)
    out = torch.empty((H, 1, M), dtype=torch.float32, device=q.device)
    return plan.scores(out)[:, 0]


def decode_build_sets(q, K, tau, inv_freq, q_pos, pos_scale, rope_scale, sm_scale, n_global, n_local, k_max,
                      pct_decode, scores=None, pos_scale_c=None, rule="shared", stats=None):
    """(idx (H, k_max) int64 with sentinel M, newpos_k (H, k_max) fp32, newpos_q (H,) fp32).  Scores
    under (inv_freq, pos_scale, rope_scale); reposition with pos_scale_c (default pos_scale).
    rule "pq": the per-query file's rule (dense ranks, exact cap budget); stats, a dict, then
    receives usize and overflow (H,) of the call."""
    H, M = q.shape[0], K.shape[-2]
    plan = native.DecodePlan(q, K, None, _tau_of(tau, H), inv_freq, int(q_pos), pos_scale, rope_scale,
                             sm_scale, n_global, n_local, k_max, pct_decode, pos_scale_c=pos_scale_c, rule=rule)
    if scores is None:
        s = plan.scores(torch.empty((H, 1, M), dtype=torch.float32, device=q.device))
    else:
        s = scores.to(device=q.device, dtype=torch.float32).reshape(H, 1, M).contiguous()
    r = plan.build_sets(s)
    if stats is not None and rule == "pq":
        stats["usize"], stats["overflow"] = r["usize"][:, 0], r["overflow"][:, 0]
    return r["idx"][:, 0].long(), r["newpos_k"][:, 0], r["newpos_q"][:, 0]


def decode_attend(q, K, V, idx, newpos_k, newpos_q, inv_freq, rope_scale, sm_scale, q_pos=None):
    """Attention of one query q (H, D) over its slots -> (H, D) in q.dtype.  q_pos given: Kernel C's
    slot rule (key <= q_pos) on top of the sentinel test."""
    H, M = q.shape[0], K.shape[-2]
    causal = q_pos is not None and int(q_pos) < M - 1
    q0 = int(q_pos) if causal else M - 1
    k_max = idx.shape[-1]
    plan = native.DecodePlan(q, K, V, torch.zeros(H), inv_freq, q0, 1.0, rope_scale, sm_scale, k_max=k_max,
                             causal=causal)
    dev = q.device
    idx32 = idx.to(device=dev).clamp(min=-1, max=M).to(torch.int32).reshape(H, 1, k_max).contiguous()
    npk = newpos_k.to(device=dev, dtype=torch.float32).reshape(H, 1, k_max).contiguous()
    npq = newpos_q.to(device=dev, dtype=torch.float32).reshape(H, 1).contiguous()
    return plan.attend(idx32, npk, npq)[:, 0]


def decode_attention(q, k, v, tau, inv_freq, q_pos0, pos_scale=1.0, rope_scale=1.0, sm_scale=None, n_global=32,
                     n_local=32, k_max=1024, pct_decode=100.0, causal=False, inv_freq_c=None, pos_scale_c=None,
                     rope_scale_c=None, rule="shared", stats=None, block_n=32):
    """Q queries q (1, H, Q, D) or (H, Q, D) at positions q_pos0 .. q_pos0 + Q - 1 over the cache
    k, v (1, Hkv, M, D) with q_pos0 + Q <= M; query i sees the keys [0, M - (Q - 1 - i)).
    Returns out (H, Q, D) in q.dtype -- the decode branch of spi_forward (exact_2.py:734-762)
    for all Q queries in one call; rule "pq" is the per-query file's (perquery.py:893-924), whose
    usize / overflow (H, Q) land in `stats` when given.  The *_c triple (default: the selection
    geometry) repositions and attends, as the hybrid file's decode does (hybrid_exact.py:551-633,
    776-800)."""
    qh = q[0] if q.dim() == 4 else q
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(qh.shape[-1])
    r = native.decode_attention(qh, k, v, _tau_of(tau, qh.shape[0]), inv_freq, q_pos0, pos_scale, rope_scale,
                                sm_scale, n_global, n_local, k_max, pct_decode, causal, inv_freq_c=inv_freq_c,
                                pos_scale_c=pos_scale_c, rope_scale_c=rope_scale_c, rule=rule, block_n=block_n)
    if stats is not None and rule == "pq":
        stats["usize"], stats["overflow"] = r["usize"], r["overflow"]
    if stats is not None and rule == "stream":
        stats.update(idx=r["idx"], newpos_k=r["newpos_k"], set_size=r["set_size"])
    return r["out"]
