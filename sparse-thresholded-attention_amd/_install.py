"""Model integration: route a Llama model's attention through the HIP kernels.

The reference patches ``LlamaAttention.forward`` (shared_selection_triton_exact_2.py:658-767,
shared_selection_triton_exact.py:595-700, shared_selection_triton_YaRN_exact.py:668-776,
shared_selection_triton_hybrid_exact.py:683-811).  The patched forward here keeps its contract:

* the KV cache holds the raw (unrotated) K and V -- the kernels rotate internally;
* pos_scale = min(1, context_window / L) is frozen at prefill (L = max_len, else the prefill
  length) and reused by every decode step;
* a prefill (empty cache) with prefill_mode "shared" runs the shared-selection prefill and keeps
  its statistics on the module (spi_last_shared, spi_last_kept, spi_last_kpct, ...);
* every other call -- decode steps, and prefill with prefill_mode "perquery" -- lets each query
  select its own set over the cache prefix up to its position.

Differences by design: K and V keep their kv heads (grouped-query attention runs natively instead
of through repeat_kv); the per-query path serves all of a call's queries in batches of up to
``PER_QUERY_BATCH`` through one launch sequence each, instead of a Python loop per token; the
decode backends ("torch" / "triton") select between the reference's two attend rules, which agree
whenever a query's position is the last key it sees, as in the model.
"""

import torch

from _decode import decode_attention
from _shared_prefill import shared_prefill

PER_QUERY_BATCH = 256          # queries per per-query launch: bounds the (H, Q, M) score buffer


# ---------------------------------------------------------------------------------------------
# what every patched forward does around its kernels
# ---------------------------------------------------------------------------------------------
def _cached_length(cache, layer_idx):
    """Tokens already in the layer's cache: a transformers Cache (get_seq_length, with or without
    the layer argument) or a legacy tuple of (k, v) per layer."""
    if cache is None:
        return 0
    if hasattr(cache, "get_seq_length"):
        try:
            return int(cache.get_seq_length(layer_idx))
        except TypeError:
            return int(cache.get_seq_length())
    return 0 if hasattr(cache, "update") else int(cache[layer_idx][0].shape[2])


def _cache_append(cache, k, v, layer_idx):
    """The layer's keys / values with this call's appended (the cache keeps them)."""
    if cache is None:
        return k, v
    if hasattr(cache, "update"):
        return cache.update(k, v, layer_idx)
    pk, pv = cache[layer_idx]
    return torch.cat([pk, k], dim=2), torch.cat([pv, v], dim=2)


class _AttnCall:
    """One attention call's projections: q (1, H, N, D), the new raw keys / values k_new, v_new
    (1, Hkv, N, D), the cache's keys / values after the append, k, v (1, Hkv, past + N, D) -- the
    cache stores keys_for_cache(k_new) -- and past, the tokens cached before the call."""

    def __init__(self, module, hidden_states, past_key_values, kwargs, layer_idx, keys_for_cache=None):
        B, N, _ = hidden_states.shape
        assert B == 1, "batch size must be 1 (the kernels take one sequence, as the reference's)"
        shape = (B, N, -1, module.head_dim)
        self.N = N
        self.q, self.k_new, self.v_new = (proj(hidden_states).view(shape).transpose(1, 2)
                                          for proj in (module.q_proj, module.k_proj, module.v_proj))
        # transformers passes the cache as past_key_values, or (older paths) past_key_value
        cache = past_key_values if past_key_values is not None else kwargs.get("past_key_value", None)
        self.past = _cached_length(cache, layer_idx)
        stored = keys_for_cache(self.k_new, self.past) if keys_for_cache is not None else self.k_new
        self.k, self.v = _cache_append(cache, stored, self.v_new, layer_idx)

    def batches(self):
        """(c0, c1, M): the call's queries [c0, c1) in launches of PER_QUERY_BATCH, each over the
        cache prefix [0, M) that its last query sees."""
        for c0 in range(0, self.N, PER_QUERY_BATCH):
            c1 = min(self.N, c0 + PER_QUERY_BATCH)
            yield c0, c1, self.past + c1


def _frozen_pos_scale(geom, context_window, max_len, N):
    """The selection's position scale, fixed at prefill: raw positions under "yarn", else
    min(1, W / L) with L = max_len or the prefill length."""
    if geom == "yarn":
        return 1.0
    return min(1.0, context_window / float(max_len if max_len is not None else N))


def _out_proj(module, out, N):
    """o_proj of the attention output (1, H, N, D)."""
    return module.o_proj(out.transpose(1, 2).reshape(1, N, -1).contiguous())


def base_inv_freq_of(model):
    """theta^(-2i/D) from the model config (the hybrid file's Kernel C frequencies,
    hybrid_exact.py:712-726)."""
    cfg = model.config
    head_dim = getattr(cfg, "head_dim", None) or (cfg.hidden_size // cfg.num_attention_heads)
    theta = 10000.0
    rp = getattr(cfg, "rope_parameters", None) or getattr(cfg, "rope_scaling", None)
    if isinstance(rp, dict) and rp.get("rope_theta"):
        theta = float(rp["rope_theta"])
    elif getattr(cfg, "rope_theta", None):
        theta = float(cfg.rope_theta)
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def install(model, geometry, pct=30.0, context_window=4096, n_global=32, n_local=32, tile=32, k_max=1024,
            block_n=32, block_k=32, max_len=None, pct_decode=100.0, decode_backend="torch",
            select_backend="torch", prefill_mode="shared", measure=False, select_score="freq", rope_scale=None):
    """geometry: "pi" (rotary frequencies, positions compressed by the frozen pos_scale), "yarn"
    (rotary frequencies as loaded, raw positions) or a dict for "hybrid" {"inv_freq_a",
    "rope_scale_a", "inv_freq_c"} (selection under a raw-position geometry, reposition and attend
    under base RoPE with the frozen pos_scale).  rope_scale: the rotation scale of "pi" / "yarn"
    (default: the rotary embedding's attention_scaling)."""
    import transformers.models.llama.modeling_llama as ml
    rotary = model.model.rotary_emb
    inv_freq = rotary.inv_freq.detach().float()
    if rope_scale is None:
        rope_scale = float(getattr(rotary, "attention_scaling", 1.0))
    for li, layer in enumerate(model.model.layers):
        sa = layer.self_attn
        dev = sa.q_proj.weight.device
        if isinstance(geometry, dict):
            sa.spi_geometry = "hybrid"
            sa.spi_inv_freq_a = geometry["inv_freq_a"].to(dev)
            sa.spi_rope_scale_a = float(geometry["rope_scale_a"])
            sa.spi_inv_freq_c = geometry["inv_freq_c"].to(dev)
            sa.spi_rope_scale_c = 1.0
            sa.spi_pos_scale_c = None
        else:
            sa.spi_geometry = geometry
            sa.spi_inv_freq = inv_freq.to(dev)
            sa.spi_rope_scale = float(rope_scale)
        sa.spi_pct = pct
        sa.spi_W = context_window
        sa.spi_ng = n_global
        sa.spi_nl = n_local
        sa.spi_tile = tile
        sa.spi_kmax = k_max
        sa.spi_block_n = block_n
        sa.spi_block_k = block_k
        sa.spi_layer_idx = getattr(sa, "layer_idx", li)
        sa.spi_max_len = max_len
        sa.spi_pos_scale = None
        sa.spi_pct_decode = pct_decode
        sa.spi_decode_backend = decode_backend
        sa.spi_select_backend = select_backend
        sa.spi_prefill_mode = prefill_mode
        sa.spi_measure = measure
        sa.spi_select_score = select_score
    ml.LlamaAttention.forward = spi_forward


def _geometry(self, pos_frozen):
    """(inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c, rope_scale_c)."""
    if self.spi_geometry == "hybrid":
        return (self.spi_inv_freq_a, 1.0, self.spi_rope_scale_a, self.spi_inv_freq_c, pos_frozen,
                self.spi_rope_scale_c)
    ps = 1.0 if self.spi_geometry == "yarn" else pos_frozen
    return self.spi_inv_freq, ps, self.spi_rope_scale, self.spi_inv_freq, ps, self.spi_rope_scale


def spi_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                **kwargs):
    c = _AttnCall(self, hidden_states, past_key_values, kwargs, self.spi_layer_idx)
    # pos_scale frozen at prefill from max_len (or the prefill length), reused at decode
    if c.past == 0:
        frozen = _frozen_pos_scale("pi", self.spi_W, self.spi_max_len, c.N)
        if self.spi_geometry == "hybrid":
            self.spi_pos_scale_c = frozen
        else:
            self.spi_pos_scale = frozen
    frozen = self.spi_pos_scale_c if self.spi_geometry == "hybrid" else self.spi_pos_scale
    ifa, psa, rsa, ifc, psc, rsc = _geometry(self, frozen)

    if c.past == 0 and self.spi_prefill_mode == "shared":
        out, shared_size, kept_size, kpct, overflow, kpct_meas, overflow20 = shared_prefill(
            c.q, c.k, c.v, self.tau_head_vec, ifa, psa, rsa, ifc, psc, rsc, self.spi_pct, self.scaling, self.spi_ng,
            self.spi_nl, self.spi_tile, self.spi_kmax, c.past, self.spi_measure, self.spi_select_score)
        self.spi_last_shared = shared_size.detach()
        self.spi_last_kept = kept_size.detach()
        self.spi_last_kpct = kpct.detach()
        self.spi_last_overflow = overflow.detach()
        self.spi_last_kpct_meas = kpct_meas.detach()
        self.spi_last_overflow20 = overflow20.detach()
    else:
        # each query at position past + i over the keys [0, past + i]
        causal = self.spi_decode_backend == "triton"
        out = torch.cat([decode_attention(
            c.q[0, :, c0:c1, :], c.k[:, :, :M, :], c.v[:, :, :M, :], self.tau_head_vec, ifa, c.past + c0, psa, rsa,
            self.scaling, self.spi_ng, self.spi_nl, self.spi_kmax, self.spi_pct_decode, causal,
            inv_freq_c=ifc, pos_scale_c=psc, rope_scale_c=rsc) for c0, c1, M in c.batches()], dim=1).unsqueeze(0)
    return _out_proj(self, out, c.N), None


# ---------------------------------------------------------------------------------------------
# the per-query file's model integration (shared_selection_triton_perquery.py:784-930)
# ---------------------------------------------------------------------------------------------
def install_perquery(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, k_max,
                     max_len, decode_backend, prefill_mode, select_score, block_n=32, block_k=32):
    """Selection under select_geom ("pi": base frequencies, compressed positions; "yarn": the
    rotary frequencies as loaded, raw positions, attention scaling as the rope scale when
    apply_mscale); attention under base RoPE at dense ranks, scale 1 (perquery.py:800-852)."""
    import transformers.models.llama.modeling_llama as ml
    rotary = model.model.rotary_emb
    inv_freq_rot = rotary.inv_freq.detach().float()
    attn_scaling = float(getattr(rotary, "attention_scaling", 1.0))
    inv_freq_base = base_inv_freq_of(model)
    if select_geom == "yarn":
        inv_freq_a, rope_scale_a = inv_freq_rot, (attn_scaling if apply_mscale else 1.0)
    else:
        inv_freq_a, rope_scale_a = inv_freq_base, 1.0
    assert inv_freq_base.numel() == inv_freq_a.numel(), \
        f"inv_freq length mismatch: {inv_freq_base.numel()} vs {inv_freq_a.numel()}"
    for li, layer in enumerate(model.model.layers):
        sa = layer.self_attn
        dev = sa.q_proj.weight.device
        sa.spi_inv_freq_a = inv_freq_a.to(dev)
        sa.spi_rope_scale_a = rope_scale_a
        sa.spi_inv_freq_c = inv_freq_base.to(dev)
        sa.spi_geom = select_geom
        sa.spi_W = context_window
        sa.spi_ng = n_global
        sa.spi_nl = n_local
        sa.spi_tile = tile
        sa.spi_kmax = k_max
        sa.spi_block_n = block_n
        sa.spi_block_k = block_k
        sa.spi_layer_idx = getattr(sa, "layer_idx", li)
        sa.spi_max_len = max_len
        sa.spi_pos_scale_a = None
        sa.spi_select_score = select_score
        sa.spi_decode_backend = decode_backend
        sa.spi_prefill_mode = prefill_mode
    ml.LlamaAttention.forward = pq_forward


def pq_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
               **kwargs):
    import shared_selection_triton_perquery as pqm
    c = _AttnCall(self, hidden_states, past_key_values, kwargs, self.spi_layer_idx)
    if c.past == 0:   # the selection's pos_scale, frozen at prefill
        self.spi_pos_scale_a = _frozen_pos_scale(self.spi_geom, self.spi_W, self.spi_max_len, c.N)
    if c.past == 0 and self.spi_prefill_mode == "shared":
        out, usize, kept_size, overflow = pqm.shared_pq_attention(
            c.q, c.k, c.v, self.tau_head_vec, self.spi_inv_freq_a, self.spi_inv_freq_c,
            pos_scale_a=self.spi_pos_scale_a, rope_scale_a=self.spi_rope_scale_a, sm_scale=self.scaling,
            n_global=self.spi_ng, n_local=self.spi_nl, tile=self.spi_tile, k_max=self.spi_kmax,
            q_pos_base=c.past, select_score=self.spi_select_score)
        self.spi_last_usize = usize.detach()
        self.spi_last_kept = kept_size.detach()
        self.spi_last_overflow = overflow.detach()
    else:
        # each query at position past + i over the keys [0, past + i], per-query rule
        causal = self.spi_decode_backend == "triton"
        outs = []
        for c0, c1, M in c.batches():
            st = {}
            outs.append(decode_attention(
                c.q[0, :, c0:c1, :], c.k[:, :, :M, :], c.v[:, :, :M, :], self.tau_head_vec, self.spi_inv_freq_a,
                c.past + c0, self.spi_pos_scale_a, self.spi_rope_scale_a, self.scaling, self.spi_ng, self.spi_nl,
                self.spi_kmax, 100.0, causal, inv_freq_c=self.spi_inv_freq_c, pos_scale_c=1.0, rope_scale_c=1.0,
                rule="pq", stats=st))
            pqm._record(st["overflow"], st["usize"], phase="decode")
        out = torch.cat(outs, dim=1).unsqueeze(0)
    return _out_proj(self, out, c.N), None


# ---------------------------------------------------------------------------------------------
# the PQ Stream file's model integration (pqstream_kernel.py:834-998)
# ---------------------------------------------------------------------------------------------
def install_pqstream(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, block_n, block_k,
                     max_len, decode_backend, prefill_mode, pos_advance, use_skip):
    """Selection under select_geom ("pi": base frequencies at positions compressed by the frozen
    pos_scale; "yarn": the rotary frequencies as loaded at raw positions, the attention scaling
    as the rope scale when apply_mscale); attention under base RoPE at the streamed positions
    (pqstream_kernel.py:856-917)."""
    import transformers.models.llama.modeling_llama as ml
    rotary = model.model.rotary_emb
    inv_freq_rot = rotary.inv_freq.detach().float()
    attn_scaling = float(getattr(rotary, "attention_scaling", 1.0))
    inv_freq_base = base_inv_freq_of(model)
    if select_geom == "yarn":
        inv_freq_a, rope_scale_a = inv_freq_rot, (attn_scaling if apply_mscale else 1.0)
    else:
        inv_freq_a, rope_scale_a = inv_freq_base, 1.0
    assert inv_freq_base.numel() == inv_freq_a.numel(), \
        f"inv_freq length mismatch: {inv_freq_base.numel()} vs {inv_freq_a.numel()}"
    for li, layer in enumerate(model.model.layers):
        sa = layer.self_attn
        dev = sa.q_proj.weight.device
        sa.pqs_inv_freq_a = inv_freq_a.to(dev)
        sa.pqs_rope_scale_a = rope_scale_a
        sa.pqs_inv_freq_c = inv_freq_base.to(dev)
        sa.pqs_geom = select_geom
        sa.pqs_W = context_window
        sa.pqs_ng = n_global
        sa.pqs_nl = n_local
        sa.pqs_tile = tile
        sa.pqs_block_n = block_n
        sa.pqs_block_k = block_k
        sa.pqs_layer_idx = getattr(sa, "layer_idx", li)
        sa.pqs_max_len = max_len
        sa.pqs_pos_scale_a = None
        sa.pqs_advance = pos_advance
        sa.pqs_use_skip = bool(use_skip)
        sa.pqs_decode_backend = decode_backend
        sa.pqs_prefill_mode = prefill_mode
    ml.LlamaAttention.forward = pqs_forward


def pqs_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                **kwargs):
    import pqstream_kernel as pqs
    c = _AttnCall(self, hidden_states, past_key_values, kwargs, self.pqs_layer_idx)
    if c.past == 0:
        self.pqs_pos_scale_a = _frozen_pos_scale(self.pqs_geom, self.pqs_W, self.pqs_max_len, c.N)
    if c.past == 0 and self.pqs_prefill_mode == "stream":
        out, span, kept, blocks, skipped = pqs.pqstream_attention(
            c.q, c.k, c.v, self.tau_head_vec, self.pqs_inv_freq_a, self.pqs_inv_freq_c,
            pos_scale_a=self.pqs_pos_scale_a, rope_scale_a=self.pqs_rope_scale_a, sm_scale=self.scaling,
            n_global=self.pqs_ng, n_local=self.pqs_nl, tile=self.pqs_tile, block_n=self.pqs_block_n,
            pos_advance=self.pqs_advance, q_pos_base=c.past, use_skip=self.pqs_use_skip)
        self.pqs_last_span = span.detach()
        self.pqs_last_kept = kept.detach()
        self.pqs_last_skipped = skipped.detach()
    else:
        # each query at position past + i over the keys [0, past + i], the stream rule; the slot
        # buffer is the batch's cache length rounded up to 1024
        causal = self.pqs_decode_backend == "triton"
        outs = []
        for c0, c1, M in c.batches():
            st = {}
            outs.append(decode_attention(
                c.q[0, :, c0:c1, :], c.k[:, :, :M, :], c.v[:, :, :M, :], self.tau_head_vec, self.pqs_inv_freq_a,
                c.past + c0, self.pqs_pos_scale_a, self.pqs_rope_scale_a, self.scaling, self.pqs_ng,
                self.pqs_nl, pqs._kbuf(M), 100.0, causal, inv_freq_c=self.pqs_inv_freq_c, pos_scale_c=1.0,
                rope_scale_c=1.0, rule="stream", stats=st, block_n=self.pqs_block_n))
            m = torch.arange(c.past + c0 + 1, M + 1, device=c.q.device)
            pqs._record_decode(st["idx"], st["newpos_k"], st["set_size"], m, self.pqs_block_n)
        out = torch.cat(outs, dim=1).unsqueeze(0)
    return _out_proj(self, out, c.N), None


# ---------------------------------------------------------------------------------------------
# the chunked file's model integration (shared_selection_triton_chunked.py:495-643)
# ---------------------------------------------------------------------------------------------
def install_chunked(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, k_max, max_len,
                    decode_backend, prefill_mode, select_score, measure, chunk_size, n_chunk, chunk_agg):
    """The per-query file's geometry (selection under select_geom, attention under base RoPE at
    dense ranks, scale 1) with chunk selection at prefill and decode."""
    install_perquery(model, select_geom, apply_mscale, context_window, n_global, n_local, tile, k_max, max_len,
                     decode_backend, prefill_mode, select_score)
    import transformers.models.llama.modeling_llama as ml
    for layer in model.model.layers:
        sa = layer.self_attn
        sa.spi_chunk_size = chunk_size
        sa.spi_n_chunk = n_chunk
        sa.spi_chunk_agg = chunk_agg
        sa.spi_measure = measure
    ml.LlamaAttention.forward = chunk_forward


def chunk_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                  **kwargs):
    import shared_selection_triton_chunked as chm
    import _sta_native as native
    c = _AttnCall(self, hidden_states, past_key_values, kwargs, self.spi_layer_idx)
    if c.past == 0:
        self.spi_pos_scale_a = _frozen_pos_scale(self.spi_geom, self.spi_W, self.spi_max_len, c.N)
    if c.past == 0 and self.spi_prefill_mode == "shared":
        out, usize, kept_size = chm.shared_chunk_attention(
            c.q, c.k, c.v, self.tau_head_vec, self.spi_inv_freq_a, self.spi_inv_freq_c,
            pos_scale_a=self.spi_pos_scale_a, rope_scale_a=self.spi_rope_scale_a, sm_scale=self.scaling,
            n_global=self.spi_ng, n_local=self.spi_nl, tile=self.spi_tile, k_max=self.spi_kmax,
            chunk_size=self.spi_chunk_size, n_chunk=self.spi_n_chunk, q_pos_base=c.past,
            select_score=self.spi_select_score, chunk_agg=self.spi_chunk_agg, measure=self.spi_measure)
        self.spi_last_usize = usize.detach()
        self.spi_last_kept = kept_size.detach()
    else:
        # each query at position past + i over the keys [0, past + i], chunk rule
        causal = self.spi_decode_backend == "triton"
        outs = []
        H = c.q.shape[1]
        for c0, c1, M in c.batches():
            plan = native.DecodePlan(c.q[0, :, c0:c1, :], c.k[:, :, :M, :], c.v[:, :, :M, :], self.tau_head_vec,
                                     self.spi_inv_freq_a, c.past + c0, self.spi_pos_scale_a, self.spi_rope_scale_a,
                                     self.scaling, self.spi_ng, self.spi_nl, self.spi_kmax, 100.0, causal,
                                     inv_freq_c=self.spi_inv_freq_c, pos_scale_c=1.0, rope_scale_c=1.0)
            s = plan.scores(torch.empty((H, c1 - c0, M), dtype=torch.float32, device=c.q.device))
            pk = torch.empty((H, c1 - c0), dtype=torch.int32, device=c.q.device)
            us = torch.empty((H, c1 - c0), dtype=torch.int32, device=c.q.device)
            r = plan.build_sets_chunk(s, self.spi_chunk_size, self.spi_n_chunk, self.spi_select_score,
                                      self.spi_chunk_agg, passers_kept=pk, usize=us)
            outs.append(plan.attend(r["idx"], r["newpos_k"], r["newpos_q"], r["set_size"]).clone())
            if self.spi_measure:
                chm._stat_acc(pk, us, r["set_size"], "decode")
        out = torch.cat(outs, dim=1).unsqueeze(0)
    return _out_proj(self, out, c.N), None
