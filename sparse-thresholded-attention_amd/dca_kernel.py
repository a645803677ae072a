"""Drop-in for the attention core of dca_kernel.py (dual chunk attention, DCA).

The reference installs DCA by monkey-patching a Llama model (install_dca_forward,
dca_kernel.py:660-663); its attention core is the prefill branch of dca_forward
(:372-489): keys rotated at j mod L, queries at their intra / succ / inter chunk positions, three
attention blocks merged by log-sum-exp.  dca_prefill_attention runs that core on raw q, k, v in
the gfx950 HIP kernels of libsta_hip.so (no flash_attn, no fallback); get_mscale is the
reference's attention factor.  The model patching itself (install / patch / unpatch) is not part
of this package.
"""
import math

import torch

import _sta_native as native


def get_mscale(scale: float = 1.0) -> float:
    """ChunkLlama's length factor, 0.05 ln(scale) + 1 above 1 (dca_kernel.py:163-170)."""
    if scale <= 1:
        return 1.0
    return 0.05 * math.log(scale) + 1.0


def base_inv_freq(dim, base=10000):
    """1 / base^(arange(0, dim, 2) / dim) in fp32, as ChunkLlamaRotaryEmbedding builds it (:176)."""
    return 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))


def dca_prefill_attention(q, k, v, chunk_size, pretrain_len, local_window, inv_freq=None, base=10000,
                          scale=None):
    """q (1,H,N,D), k / v (1,Hkv,N,D) raw (before RoPE), in the model dtype.  Returns the
    attention output (1,H,N,D) of dca_forward's prefill branch (dca_kernel.py:372-489) before
    o_proj.  chunk_size - local_window must be a multiple of 64."""
    Z, H, N, D = q.shape
    assert Z == 1
    assert 0 < local_window < chunk_size, f"need 0 < w({local_window}) < s({chunk_size})"
    if inv_freq is None:
        inv_freq = base_inv_freq(D, base)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = native.dca_attention(q, k, v, inv_freq, chunk_size, pretrain_len, local_window, scale)
    return out.unsqueeze(0)
