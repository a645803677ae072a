"""Torch restatements of the reference modules' pure-torch helpers and goldens.

The reference modules expose slow torch versions of their algorithms next to the kernels (the
"goldens"), plus a few torch helpers, and callers import them by name:
  _rope_rotate              shared_selection_triton_exact_2.py:495-502 (and its twins)
  pq_attention_torch        shared_selection_triton_perquery.py:545-615
  pqstream_attention_torch  pqstream_kernel.py:583-652
  chunk_attention_torch     shared_selection_triton_chunked.py:328-405
  DCA helpers               dca_kernel.py:149-366 (flash_attn_status, ChunkLlamaRotaryEmbedding,
                            _rotate_half, apply_rotary_pos_emb, _fa_block, _merge_lse)
The drop-in modules re-export them under those names.  They are reference-semantics torch code
for small inputs (O(tiles * N^2) memory and time) and work on any device; no entry point of the
drop-ins calls them: prefill, decode and the model patches run the HIP kernels of libsta_hip.so.
"""
import math

import torch

NEG = float("-inf")


def _rope_rotate(x, pos, inv_freq, rope_scale):
    """Half-split (Llama) RoPE of x (..., D) at positions pos (broadcast to x.shape[:-1]): angle
    fl(pos * inv_freq), cos / sin scaled by rope_scale, in fp32 (exact_2.py:495-502)."""
    d2 = x.shape[-1] // 2
    theta = pos.to(torch.float32).unsqueeze(-1) * inv_freq.to(torch.float32)
    c = torch.cos(theta) * rope_scale
    s = torch.sin(theta) * rope_scale
    a, b = x[..., :d2].float(), x[..., d2:].float()
    return torch.cat((a * c - b * s, b * c + a * s), dim=-1)


def _forced_keys(n_keys, row0, tile, n_global, n_local, device):
    """Global keys and the tile's local window (rows row0 .. row0 + tile - 1) among keys 0 ..
    n_keys - 1 (perquery.py:383-384; pqstream_kernel.py:613)."""
    j = torch.arange(n_keys, device=device)
    return (j < n_global) | ((j >= row0 - n_local + 1) & (j <= row0 + tile - 1))


class _Geom:
    """The rotated rows of one call: queries and keys under the selection geometry, computed once
    and sliced per tile."""

    def __init__(self, q, k, inv_freq_a, pos_scale_a, rope_scale_a):
        N = q.shape[2]
        pos = torch.arange(N, device=q.device, dtype=torch.float32) * pos_scale_a
        invf = inv_freq_a.to(q.device).float()
        self.qa = _rope_rotate(q[0], pos, invf, rope_scale_a)          # (H, N, D)
        self.ka = _rope_rotate(k[0], pos, invf, rope_scale_a)

    def scores(self, r0, r1, n_keys, sm_scale):
        """Scaled scores of rows r0 .. r1 - 1 against keys 0 .. n_keys - 1, non-causal pairs -inf,
        and the causal mask (rows, keys)."""
        s = torch.matmul(self.qa[:, r0:r1], self.ka[:, :n_keys].transpose(1, 2)) * sm_scale
        causal = torch.arange(r0, r1, device=s.device)[:, None] >= torch.arange(n_keys, device=s.device)[None, :]
        return s.masked_fill(~causal[None], NEG), causal


def _masked_attend(q_rows, k_rows, v_rows, q_pos, k_pos, inv_freq_c, sm_scale, allowed):
    """softmax over the allowed keys of base-RoPE scores at the given positions, times V."""
    invf = inv_freq_c.to(q_rows.device).float()
    qr = _rope_rotate(q_rows, q_pos, invf, 1.0)
    kr = _rope_rotate(k_rows, k_pos, invf, 1.0)
    sc = torch.matmul(qr, kr.transpose(-1, -2)) * sm_scale
    sc = sc.masked_fill(~allowed, NEG)
    return torch.matmul(torch.softmax(sc, dim=-1), v_rows.float())


def _top_budget(rank_value, eligible, budget):
    """Boolean mask of the `budget` largest rank values among eligible keys (per head, last axis),
    by torch.topk as the reference's goldens take it (perquery.py:401-405), so equal values at the
    cut are taken in topk's own order, as there."""
    n = rank_value.shape[-1]
    rv = torch.where(eligible, rank_value, torch.full_like(rank_value, NEG))
    kk = max(min(budget, n), 1)
    val, pos = rv.topk(kk, dim=-1)
    ok = (torch.arange(kk, device=rv.device) < budget) & (val > NEG)
    return torch.zeros_like(eligible).scatter_(-1, pos, ok)


@torch.no_grad()
def pq_attention_torch(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                       sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096,
                       select_score="expmass"):
    """PQ Union prefill in torch (perquery.py:545-615): per tile the union of every query's
    threshold passers plus the forced keys, cut to k_max by votes (freq) or expmass + 1e-6 votes
    when it overflows, dense ranks over the kept keys; each query attends the kept keys it passes
    itself plus the forced ones.  q, k, v (1, H, N, D); returns (1, H, N, D) in q.dtype."""
    Z, H, N, D = q.shape
    assert Z == 1
    sm = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    dev = q.device
    g = _Geom(q, k, inv_freq_a, pos_scale_a, rope_scale_a)
    tau = tau.to(dev).float().view(H, 1, 1)
    out = torch.zeros((H, N, D), device=dev, dtype=torch.float32)
    for r0 in range(0, N, tile):
        r1 = min(r0 + tile, N)
        s, causal = g.scores(r0, r1, r1, sm)                               # keys 0 .. r1 - 1
        m = s.amax(-1, keepdim=True)
        keep = (s >= m - tau) & causal[None]
        votes = keep.sum(1)
        forced = _forced_keys(r1, r0, tile, n_global, n_local, dev)
        kept = (votes > 0) | forced[None]
        over = kept.sum(-1) > k_max
        if bool(over.any()):
            if select_score == "freq":
                rank = votes.float()
            else:
                rank = torch.where(keep, torch.exp(s - m), torch.zeros_like(s)).sum(1) + 1e-6 * votes.float()
            take = _top_budget(rank, (votes > 0) & ~forced[None], max(k_max - int(forced.sum()), 0))
            kept = torch.where(over[:, None], take | forced[None], kept)
        rank0 = (kept.int().cumsum(-1) - 1).float()
        allowed = ((keep & kept[:, None, :]) | forced[None, None, :]) & causal[None]
        out[:, r0:r1] = _masked_attend(q[0, :, r0:r1], k[0, :, :r1], v[0, :, :r1], rank0[:, r0:r1], rank0,
                                       inv_freq_c, sm, allowed)
    return out.unsqueeze(0).to(q.dtype)


@torch.no_grad()
def pqstream_attention_torch(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0,
                             rope_scale_a=1.0, sm_scale=None, n_global=32, n_local=32,
                             tile=32, block_n=32, pos_advance="max"):
    """PQ Stream prefill in torch (pqstream_kernel.py:583-652): every query keeps its own passers
    plus the forced keys; aligned blocks of block_n keys are walked from the tile's last row
    backwards, key j of a block sits at -(d + hi_t - j) where d is the advance of the blocks
    nearer the queries (the most keys any of the tile's rows keeps in a block, or the block's
    width under pos_advance="full"), and a block nobody keeps is skipped; the queries sit at
    q_pos - P_top.  q, k, v (1, H, N, D); returns (1, H, N, D) in q.dtype."""
    Z, H, N, D = q.shape
    assert Z == 1
    sm = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    dev = q.device
    g = _Geom(q, k, inv_freq_a, pos_scale_a, rope_scale_a)
    tau = tau.to(dev).float().view(H, 1, 1)
    out = torch.zeros((H, N, D), device=dev, dtype=torch.float32)
    for r0 in range(0, N, tile):
        r1 = min(r0 + tile, N)
        top = min(r0 + tile - 1, N - 1)                                      # P_top
        nk = top + 1
        s, causal = g.scores(r0, r1, nk, sm)
        m = s.amax(-1, keepdim=True)
        forced = _forced_keys(nk, r0, tile, n_global, n_local, dev)
        keep = ((s >= m - tau) | forced[None, None, :]) & causal[None]
        npk = torch.zeros((H, nk), device=dev)
        used = torch.zeros((H, nk), dtype=torch.bool, device=dev)
        d = torch.zeros(H, device=dev)
        for b0 in range(((nk - 1) // block_n) * block_n, -1, -block_n):     # nearest block first
            b1 = min(b0 + block_n, nk)
            hb = min(top, b0 + block_n - 1)
            if pos_advance == "full":
                adv = torch.full((H,), float(hb - b0 + 1), device=dev)
            else:
                adv = keep[:, :, b0:b1].sum(-1).amax(-1).float()             # (H,)
            live = adv > 0
            off = (hb - torch.arange(b0, b1, device=dev)).float()
            npk[:, b0:b1] = torch.where(live[:, None], -(d[:, None] + off[None]), npk[:, b0:b1])
            used[:, b0:b1] = live[:, None]
            d = d + torch.where(live, adv, torch.zeros_like(adv))
        qp = (torch.arange(r0, r1, device=dev) - top).float().expand(H, r1 - r0)
        out[:, r0:r1] = _masked_attend(q[0, :, r0:r1], k[0, :, :nk], v[0, :, :nk], qp, npk, inv_freq_c, sm,
                                       keep & used[:, None, :])
    return out.unsqueeze(0).to(q.dtype)


@torch.no_grad()
def chunk_attention_torch(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                          sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096,
                          chunk_size=16, n_chunk=None, select_score="expmass", chunk_agg="sum"):
    """Chunk-granular prefill in torch (chunked.py:328-405): the tile's per-key votes or expmass
    (over keys some row passes) summed per absolute chunk of chunk_size keys (or averaged over the
    chunk's passed keys under chunk_agg="mean"); the forced chunks (global keys, the tile's local
    window) plus the n_chunk best visible others are kept, trimmed at the tile's last row; dense
    ranks; every row attends all kept causal keys.  q, k, v (1, H, N, D); returns (1, H, N, D)."""
    from _sta_native import derive_n_chunk
    Z, H, N, D = q.shape
    assert Z == 1
    C = chunk_size
    if n_chunk is None:
        n_chunk = derive_n_chunk(k_max, C, n_global, n_local, tile)
    sm = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    dev = q.device
    g = _Geom(q, k, inv_freq_a, pos_scale_a, rope_scale_a)
    tau = tau.to(dev).float().view(H, 1, 1)
    nC = (N + C - 1) // C
    cidx = torch.arange(nC, device=dev)
    out = torch.zeros((H, N, D), device=dev, dtype=torch.float32)
    for r0 in range(0, N, tile):
        r1 = min(r0 + tile, N)
        s, causal = g.scores(r0, r1, r1, sm)
        m = s.amax(-1, keepdim=True)
        keep = (s >= m - tau) & causal[None]
        votes = keep.sum(1)
        passed = votes > 0
        if select_score == "freq":
            val = votes.float()
        else:
            val = torch.where(keep, torch.exp(s - m), torch.zeros_like(s)).sum(1)
        val = torch.where(passed, val, torch.zeros_like(val))
        per_chunk = torch.zeros((H, nC * C), device=dev)
        per_chunk[:, :r1] = val
        mass = per_chunk.view(H, nC, C).sum(-1)
        if chunk_agg == "mean":
            cnt = torch.zeros((H, nC * C), device=dev)
            cnt[:, :r1] = passed.float()
            mass = mass / cnt.view(H, nC, C).sum(-1).clamp(min=1)
        last = r1 - 1
        visible = cidx * C <= last
        forced_c = ((cidx < (n_global + C - 1) // C)
                    | ((cidx >= max(0, r0 - n_local + 1) // C) & (cidx <= last // C))) & visible
        take = _top_budget(mass, (visible & ~forced_c)[None].expand(H, nC), min(n_chunk, nC))
        kept_c = take | forced_c[None]
        kept = kept_c.repeat_interleave(C, dim=1)[:, :r1] & (torch.arange(r1, device=dev) <= last)[None]
        rank0 = (kept.int().cumsum(-1) - 1).float()
        out[:, r0:r1] = _masked_attend(q[0, :, r0:r1], k[0, :, :r1], v[0, :, :r1], rank0[:, r0:r1], rank0,
                                       inv_freq_c, sm, kept[:, None, :] & causal[None])
    return out.unsqueeze(0).to(q.dtype)


# ---------------------------------------------------------------------------------------------
# DCA helpers (dca_kernel.py:149-366)
# ---------------------------------------------------------------------------------------------
def flash_attn_status() -> str:
    """Which attention path the DCA forward takes (dca_kernel.py:149-159): here always the HIP
    kernels; flash_attn is neither used nor needed."""
    return "HIP kernels of libsta_hip.so (gfx950); flash_attn is not used"


def _rotate_half(x):
    d2 = x.shape[-1] // 2
    return torch.cat((-x[..., d2:], x[..., :d2]), dim=-1)


def apply_rotary_pos_emb(x, cos, sin, position_ids):
    """Table RoPE (dca_kernel.py:278-287): x (b, heads, seq, dim) rotated with the rows
    `position_ids` (b, seq) of the (rows, dim) cos / sin tables."""
    cos = cos.reshape(-1, cos.shape[-1]).to(position_ids.device)[position_ids].unsqueeze(1)
    sin = sin.reshape(-1, sin.shape[-1]).to(position_ids.device)[position_ids].unsqueeze(1)
    return x * cos + _rotate_half(x) * sin


class ChunkLlamaRotaryEmbedding(torch.nn.Module):
    """The six DCA cos / sin tables (dca_kernel.py:176-270), in torch: queries at their in-chunk
    offsets 0 .. L-1 (L = chunk_size - local_window), succ / inter queries at L .. 2L-1 clamped to
    chunk_size, keys at j mod L; every table times the length factor get_mscale(seq_len /
    max_position_embeddings), fixed when a call's length first exceeds the tables' length (which
    then grows to that length + 512).  forward(x, seq_len) returns (q_cos, q_sin, qc_cos, qc_sin,
    k_cos, k_sin) in x's dtype, sliced to seq_len rows.  chunk_size / local_window default to the
    values of the last patch_model_with_dca call."""

    def __init__(self, dim, max_position_embeddings=4096, base=10000, scaling_factor=1.0, device=None,
                 chunk_size=None, local_window=None):
        super().__init__()
        import dca_kernel as dk
        self.chunk_size = chunk_size if chunk_size is not None else dk._DCA_CHUNK_SIZE
        self.local_window = local_window if local_window is not None else dk._DCA_LOCAL_WINDOW
        if self.chunk_size is None or self.local_window is None:
            raise ValueError("chunk_size and local_window are needed (or a patch_model_with_dca call first)")
        self.dim = dim
        self.base = base
        self.scaling_factor = scaling_factor
        self.max_position_embeddings = max_position_embeddings
        self.max_seq_len = max_position_embeddings
        self._build(max_position_embeddings, device)

    def _build(self, seq_len, device):
        from dca_kernel import _MAX_NEW_TOKENS, get_mscale
        f = get_mscale(seq_len / self.max_position_embeddings)
        invf = 1.0 / (self.base ** (torch.arange(0, self.dim, 2).float().to(device) / self.dim))
        self.register_buffer("inv_freq", invf, persistent=False)
        L, sf = self.chunk_size - self.local_window, self.scaling_factor
        r = torch.arange(L, device=device, dtype=torch.float32)
        rows = {"q": r / sf,
                "qc": (r + L).clamp(max=self.chunk_size) / sf,
                "k": torch.arange(seq_len + _MAX_NEW_TOKENS, device=device, dtype=torch.float32) % L / sf}
        for name, t in rows.items():
            ang = torch.outer(t, invf).repeat(1, 2)
            self.register_buffer(f"{name}_cos_cached", ang.cos() * f, persistent=False)
            self.register_buffer(f"{name}_sin_cached", ang.sin() * f, persistent=False)
        self._last_mscale = float(f)

    def forward(self, x, seq_len=None):
        n = self.max_seq_len if seq_len is None else seq_len
        if n > self.max_seq_len:
            from dca_kernel import _MAX_NEW_TOKENS
            self._build(n, self.inv_freq.device)
            self.max_seq_len = n + _MAX_NEW_TOKENS
        names = ("q_cos", "q_sin", "qc_cos", "qc_sin", "k_cos", "k_sin")
        return tuple(getattr(self, f"{t}_cached")[:n].to(x.dtype) for t in names)


def _fa_block(q, k, v, causal, softmax_scale):
    """One attention block in fp32 -> (out (b, H, Lq, D) in q.dtype, lse (b, H, Lq)), the
    reference's non-flash path (dca_kernel.py:292-349); no keys: zeros and -inf."""
    b, H, Lq, D = q.shape
    Lk = k.shape[2]
    if Lk == 0:
        return torch.zeros_like(q), torch.full((b, H, Lq), NEG, device=q.device)
    sc = torch.matmul(q.float(), k.float().transpose(-1, -2)) * softmax_scale
    if causal and Lq > 1:
        sc = sc.masked_fill(torch.ones(Lq, Lk, dtype=torch.bool, device=q.device).triu(1), NEG)
    return torch.matmul(torch.softmax(sc, dim=-1), v.float()).to(q.dtype), torch.logsumexp(sc, dim=-1)


def _merge_lse(blocks):
    """Blocks (out, lse) merged by their log-sum-exp weights, in fp32 (dca_kernel.py:352-366):
    one softmax over the concatenated scores."""
    if len(blocks) == 1:
        return blocks[0][0]
    lse = torch.stack([l.float() for _, l in blocks])
    w = torch.softmax(lse, dim=0)
    return sum(o.float() * w[i].unsqueeze(-1) for i, (o, _) in enumerate(blocks)).to(blocks[0][0].dtype)
