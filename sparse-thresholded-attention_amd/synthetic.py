"""Seeded synthetic inputs and rotary geometries of the benchmark configurations.

Inputs: Q, K, V ~ N(0, 1) from torch.Generator('cpu').manual_seed(seed) in fp32; a unit vector
u_h per KV head; a fraction `frac` of key positions (chosen by the same generator) gets +3 u_h
and every query of head h gets +1 u_{h // group}; then a cast to the config dtype.

Geometries (all fp32, as the reference's entry points receive them):
  base RoPE    inv_freq = 1 / theta^(arange(0, D, 2) / D)      (hybrid_exact.py:717)
  PI           pos_scale = min(1, W / L)                        (exact_2.py:712-716)
  YaRN         NTK-by-parts inv_freq and attention factor 0.1 ln(s) + 1 (YaRN, arXiv:2309.00071),
               pos_scale = 1 (YaRN_exact.py:681-690, 735-740)
"""
import math
from dataclasses import dataclass

import torch


def base_inv_freq(D, theta):
    return 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))


def pi_pos_scale(window, length):
    return min(1.0, window / float(length))


def yarn_inv_freq(D, theta, factor, original_max, beta_fast=32.0, beta_slow=1.0):
    """NTK-by-parts YaRN frequencies and attention factor (truncated correction range), in the
    fp32 operation order of transformers' yarn initialiser."""
    def corr_dim(rot):
        return (D * math.log(original_max / (rot * 2 * math.pi))) / (2 * math.log(theta))

    low = max(math.floor(corr_dim(beta_fast)), 0)
    high = min(math.ceil(corr_dim(beta_slow)), D - 1)
    if low == high:
        high += 0.001
    pos_freqs = theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D)
    extra = 1.0 / pos_freqs
    inter = 1.0 / (factor * pos_freqs)
    ramp = torch.clamp((torch.arange(D // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
    extra_factor = 1 - ramp
    inv_freq = inter * (1 - extra_factor) + extra * extra_factor
    mscale = 1.0 if factor <= 1 else 0.1 * math.log(factor) + 1.0
    return inv_freq, mscale


def planted_inputs(seed, H, Hkv, N, D, frac, dtype, device="cpu"):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(1, H, N, D, generator=g)
    k = torch.randn(1, Hkv, N, D, generator=g)
    v = torch.randn(1, Hkv, N, D, generator=g)
    u = torch.nn.functional.normalize(torch.randn(Hkv, D, generator=g), dim=-1)
    planted = torch.randperm(N, generator=g)[:max(1, round(frac * N))]
    k[0][:, planted] += 3.0 * u[:, None, :]
    grp = H // Hkv
    q[0] += u.repeat_interleave(grp, dim=0)[:, None, :]
    return q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device)


@dataclass
class Config:
    name: str
    H: int
    Hkv: int
    N: int
    D: int
    dtype: torch.dtype
    tile: int
    tau: float
    frac: float
    theta: float
    pos_scale: float
    rope_scale: float = 1.0
    yarn: tuple = None          # (factor, original_max, beta_fast, beta_slow)
    pct: float = 30.0
    k_max: int = 2048
    n_global: int = 32
    n_local: int = 32
    variant: str = "shared"     # "shared" (tile-shared sets), "pq" (PQ Union), "perquery" (own sets
                                # per query, capped by score), "pqstream", "dca" (dense DCA),
                                # "dca_select" (DCA + selection over the inter-chunk keys)
    select_score: str = "freq"  # key ranking: votes, or margin / expmass weighted votes
    dca: tuple = None           # (chunk_size, pretrain_len, local_window) of the DCA variant
    decode_q: int = 1           # decode variant: queries per step (the last decode_q positions)
    pct_decode: float = 100.0   # decode variant: top-% of the threshold passers kept

    def geometry(self):
        """(inv_freq, pos_scale, rope_scale) of the selection + attend geometry."""
        if self.yarn is not None:
            f, orig, bf, bs = self.yarn
            invf, msc = yarn_inv_freq(self.D, self.theta, f, orig, bf, bs)
            return invf, 1.0, msc
        return base_inv_freq(self.D, self.theta), self.pos_scale, self.rope_scale

    def inputs(self, device="cpu", seed=0):
        return planted_inputs(seed, self.H, self.Hkv, self.N, self.D, self.frac, self.dtype, device)

    def score_flops(self):
        """Algorithmic score-pass flops: 2 passes x 2 D x H x N(N+1)/2 causal pairs."""
        return 2 * 2 * self.D * self.H * self.N * (self.N + 1) // 2


CONFIGS = {
    # 0: plumbing, fp32, PI scale 1.0
    "c0": Config("c0_plumbing_fp32", 8, 8, 2048, 64, torch.float32, 64, 5.0, 0.02, 10000.0, 1.0),
    # 1: PI_exact Llama-2-7B layer, 4096 -> 12288
    "c1": Config("c1_pi_exact_32h_d128_12k_bf16", 32, 32, 12288, 128, torch.bfloat16, 64, 5.0, 0.01,
                 10000.0, pi_pos_scale(4096, 12288)),
    # 1e: config 1 ranked by expmass weighted votes (select_score="expmass", the harness default)
    "c1e": Config("c1e_pi_exact_expmass_32h_d128_12k_bf16", 32, 32, 12288, 128, torch.bfloat16, 64, 5.0, 0.01,
                  10000.0, pi_pos_scale(4096, 12288), select_score="expmass"),
    # 2: YaRN_exact Llama-3-8B GQA layer, factor 4 from 8192
    "c2": Config("c2_yarn_exact_32q8kv_d128_32k_bf16", 32, 8, 32768, 128, torch.bfloat16, 64, 5.0, 0.005,
                 500000.0, 1.0, yarn=(4.0, 8192, 32.0, 1.0)),
    # 3: per-query selection (PQ Union), PI 4096 -> 16384 for selection, base RoPE at dense ranks
    #    for attention, tau 4, tile 32, k_max 2048
    "c3": Config("c3_pq_union_32h_d128_16k_bf16", 32, 32, 16384, 128, torch.bfloat16, 32, 4.0, 0.01,
                 10000.0, pi_pos_scale(4096, 16384), variant="pq", select_score="expmass"),
    # 3q: config 3 as written -- every query keeps its own passers, capped at 2048 keys per query
    #    by score rank (the per-query rule, perquery.py:651-720, run at every prompt position as
    #    prefill_mode="perquery" does), dense-rank positions, base RoPE attention
    "c3q": Config("c3q_pq_perquery_cap_32h_d128_16k_bf16", 32, 32, 16384, 128, torch.bfloat16, 32, 4.0, 0.01,
                  10000.0, pi_pos_scale(4096, 16384), variant="perquery"),
    # 3s: the same shape through PQ Stream (per-query keep, streamed positions, no k_max), BN 32
    "c3s": Config("c3s_pq_stream_32h_d128_16k_bf16", 32, 32, 16384, 128, torch.bfloat16, 32, 4.0, 0.01,
                  10000.0, pi_pos_scale(4096, 16384), variant="pqstream"),
    # decode at config 1's shape: one new query per head over a 12288-key cache (PI 4096 -> 12288)
    "c1d": Config("c1d_decode_pi_32h_d128_12k_bf16", 32, 32, 12288, 128, torch.bfloat16, 64, 5.0, 0.01,
                  10000.0, pi_pos_scale(4096, 12288), variant="decode"),
    # decode at config 2's shape: GQA 32q / 8kv over a 32768-key cache, YaRN geometry
    "c2d": Config("c2d_decode_yarn_32q8kv_d128_32k_bf16", 32, 8, 32768, 128, torch.bfloat16, 64, 5.0, 0.005,
                  500000.0, 1.0, yarn=(4.0, 8192, 32.0, 1.0), variant="decode"),
    # 4: dual chunk attention at 64k (chunk 4096, local window 512, pretraining length 4096, so
    #    chunk_len 3584; base RoPE) with exact-max threshold selection (tau 5, tile 64, top 30%,
    #    2048 cap) over each tile's inter-chunk keys and dense attention over its own and the
    #    previous chunk
    "c4": Config("c4_dca_select_32h_d128_64k_bf16", 32, 32, 65536, 128, torch.bfloat16, 64, 5.0, 0.0025,
                 10000.0, 1.0, variant="dca_select", dca=(4096, 4096, 512)),
    # 4d: the same shape through the reference's dense DCA (every causal key, remapped positions)
    "c4d": Config("c4d_dca_dense_32h_d128_64k_bf16", 32, 32, 65536, 128, torch.bfloat16, 64, 5.0, 0.0025,
                  10000.0, 1.0, variant="dca", dca=(4096, 4096, 512)),
}
