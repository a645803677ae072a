"""Drop-in for dca_kernel.py (dual chunk attention, DCA).

The reference installs DCA by monkey-patching a Llama model (patch_model_with_dca, unpatch_model,
install_dca_forward, dca_kernel.py:541-663) with a forward (:372-525) whose prefill branch rotates
keys at j mod L and queries at their intra / succ / inter chunk positions and merges three
attention blocks by log-sum-exp, and whose decode branch scores the new token's query against the
cache of rotated keys with one softmax.  Here both branches run in the gfx950 HIP kernels of
libsta_hip.so (no flash_attn, no fallback): sta_dca_attention (prefill), sta_dca_rotate_keys (the
new keys into the cache) and sta_dca_decode (one token).

Per-module table state (DcaRotaryState) follows ChunkLlamaRotaryEmbedding (:166-275): the factor
get_mscale(len / pretrain_len) is fixed when a call's length first exceeds the tables' length,
which then grows to that length + 512; shorter calls keep the last factor, and keys already in the
cache keep the factor they were rotated with.  The kernels compute the table entries on the fly
instead of storing the six tables.
"""
import math

import torch

import _sta_native as native

_MAX_NEW_TOKENS = 512            # table headroom for generation (dca_kernel.py:161)
_ATTN_CLASSES = ("LlamaAttention", "LlamaFlashAttention2", "LlamaSdpaAttention")


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


# ---------------------------------------------------------------------------------------------
# model integration (dca_kernel.py:372-663)
# ---------------------------------------------------------------------------------------------
class DcaRotaryState(torch.nn.Module):
    """The state of ChunkLlamaRotaryEmbedding (dca_kernel.py:166-275) that the kernels need: the
    frequencies 1 / base^(2i / dim) (fp32, built on the CPU) and the table factor.  Built with the
    tables' length at max_position_embeddings (the pretraining length) and factor 1; advance(n)
    rebuilds as the reference's forward does: a call of length n > max_seq_len takes the factor
    get_mscale(n / max_position_embeddings) and max_seq_len = n + 512."""

    def __init__(self, dim, max_position_embeddings=4096, base=10000, scaling_factor=1.0, device=None):
        super().__init__()
        if scaling_factor != 1.0:
            raise NotImplementedError("the DCA kernels take position tables with scaling_factor 1")
        self.dim = dim
        self.base = base
        self.max_position_embeddings = max_position_embeddings
        self.max_seq_len = max_position_embeddings
        self.scaling_factor = scaling_factor
        self.register_buffer("inv_freq", base_inv_freq(dim, base).to(device), persistent=False)
        self._last_mscale = get_mscale(1.0)

    def advance(self, seq_len):
        """The table factor for a call whose cache will hold seq_len tokens."""
        if seq_len > self.max_seq_len:
            self._last_mscale = get_mscale(seq_len / self.max_position_embeddings)
            self.max_seq_len = seq_len + _MAX_NEW_TOKENS
        return self._last_mscale


def _cache_length(cache, layer_idx):
    if cache is None:
        return 0
    if hasattr(cache, "get_seq_length"):
        try:
            return int(cache.get_seq_length(layer_idx))
        except TypeError:
            return int(cache.get_seq_length())
    if not hasattr(cache, "update"):
        return int(cache[layer_idx][0].shape[2])
    return 0


def _make_dca_forward(chunk_size, pretrain_len, local_window):
    """The patched LlamaAttention.forward (dca_kernel.py:372-525).  Prefill (an empty cache, any
    number of tokens) runs sta_dca_attention over the call's tokens; decode (one token on a warm
    cache) runs sta_dca_decode over the whole cache.  The cache receives keys rotated at
    (pos mod L), as the reference's does.  A warm cache with more than one token raises, as the
    reference's assertion does (:424-427)."""
    s, c, w = chunk_size, pretrain_len, local_window

    def dca_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                    **kwargs):
        bsz, q_len, _ = hidden_states.shape
        assert bsz == 1, "batch size must be 1 (the kernels take one sequence, as the reference's)"
        if past_key_values is None:
            past_key_values = kwargs.get("past_key_value", None)
        D = self.head_dim
        H = getattr(self, "num_heads", None) or self.config.num_attention_heads
        H_kv = getattr(self, "num_key_value_heads", None) or self.config.num_key_value_heads
        scale = float(getattr(self, "scaling", None) or (1.0 / math.sqrt(D)))
        q = self.q_proj(hidden_states).view(bsz, q_len, H, D).transpose(1, 2)
        k = self.k_proj(hidden_states).view(bsz, q_len, H_kv, D).transpose(1, 2)
        v = self.v_proj(hidden_states).view(bsz, q_len, H_kv, D).transpose(1, 2)

        start_pos = _cache_length(past_key_values, self.layer_idx)
        assert start_pos == 0 or q_len == 1, (
            f"dca_forward: chunked prefill is unsupported (start_pos={start_pos}, q_len={q_len}). "
            f"Prefill must be a single pass over an empty cache; decode must be one token.")
        rot = self.rotary_emb
        mscale = rot.advance(start_pos + q_len)
        inv_freq = rot.inv_freq

        k_rot = native.dca_rotate_keys(k, start_pos, inv_freq, s, w, mscale).unsqueeze(0)
        k_all, v_all = k_rot, v
        if past_key_values is not None:
            if hasattr(past_key_values, "update"):
                k_all, v_all = past_key_values.update(k_rot, v, self.layer_idx)
            else:
                past_k, past_v = past_key_values[self.layer_idx]
                k_all, v_all = torch.cat([past_k, k_rot], dim=2), torch.cat([past_v, v], dim=2)

        if q_len > 1:
            out = native.dca_attention(q, k, v, inv_freq, s, c, w, scale, mscale=mscale)        # (H, N, D)
        else:
            out = native.dca_decode(q, k_all, v_all, inv_freq, s, w, mscale, scale)[:, None]   # (H, 1, D)
        attn_out = out.transpose(0, 1).reshape(bsz, q_len, H * D)
        return self.o_proj(attn_out), None

    return dca_forward


def _is_patchable_llama(module):
    """An attention module with the projections and indices the forward reads (:530-535)."""
    required = ("q_proj", "k_proj", "v_proj", "o_proj", "head_dim", "layer_idx")
    if not all(hasattr(module, a) for a in required):
        return False
    return hasattr(module, "num_heads") or (
        hasattr(module, "config") and hasattr(module.config, "num_attention_heads"))


def patch_model_with_dca(model, chunk_size, pretrain_len, local_window):
    """Patch LlamaAttention.forward (class level) with the DCA forward and give every patchable
    attention module its own table state.  Returns the `originals` dict for unpatch_model; raises
    RuntimeError, with the classes restored, when no attention module was patchable.
    dca_kernel.py:538-615.

    The table frequencies use base = int(the module's old rotary's base, else the config's
    rope_theta attribute, else 10000), as the reference reads it.  The transformers module's
    rotary classes are left in place (the reference swaps them for ChunkLlamaRotaryEmbedding,
    which only the patched forward reads)."""
    import transformers.models.llama.modeling_llama as ml
    assert 0 < local_window < chunk_size, f"need 0 < w({local_window}) < s({chunk_size})"
    assert chunk_size < pretrain_len, f"need s({chunk_size}) < c({pretrain_len})"
    fwd = _make_dca_forward(chunk_size, pretrain_len, local_window)
    originals = {}
    for name in _ATTN_CLASSES:
        cls = getattr(ml, name, None)
        if cls is not None:
            originals[name] = cls.forward
            cls.forward = fwd
    rotary_originals = {}
    n_patched = 0
    for mod_name, m in model.named_modules():
        if not _is_patchable_llama(m):
            continue
        n_patched += 1
        old = getattr(m, "rotary_emb", None)
        rotary_originals[mod_name] = old
        base = int(getattr(old, "base", None) or getattr(m.config, "rope_theta", 10_000))
        dev = m.q_proj.weight.device
        m.rotary_emb = DcaRotaryState(m.head_dim, max_position_embeddings=pretrain_len, base=base,
                                      device=None if dev.type == "meta" else dev)
    if n_patched == 0:
        for name in _ATTN_CLASSES:
            if name in originals:
                getattr(ml, name).forward = originals[name]
        raise RuntimeError(
            "patch_model_with_dca patched 0 attention layers -- the model would have run dense. "
            "Its attention modules must expose q_proj/k_proj/v_proj/o_proj/head_dim/layer_idx.")
    originals["_model"] = model
    originals["_rotary_emb_originals"] = rotary_originals
    originals["_n_patched"] = n_patched
    print(f"  [DCA] {n_patched} attention layers on the HIP DCA kernels (s={chunk_size}, c={pretrain_len}, "
          f"w={local_window}, chunk_len={chunk_size - local_window})", flush=True)
    return originals


def unpatch_model(originals):
    """Restore the forwards and the modules' rotary attributes saved by patch_model_with_dca
    (:618-653)."""
    try:
        import transformers.models.llama.modeling_llama as ml
    except ImportError:
        return
    n_fwd = 0
    for name in _ATTN_CLASSES:
        if name in originals:
            cls = getattr(ml, name, None)
            if cls is not None:
                cls.forward = originals[name]
                n_fwd += 1
    model = originals.get("_model")
    saved = originals.get("_rotary_emb_originals", {})
    if model is not None and saved:
        for mod_name, m in model.named_modules():
            if mod_name in saved:
                if saved[mod_name] is None:
                    if hasattr(m, "rotary_emb"):
                        delattr(m, "rotary_emb")
                else:
                    m.rotary_emb = saved[mod_name]
    print(f"  [DCA] restored {n_fwd} attention class(es) and rotary attributes", flush=True)


def install_dca_forward(model, chunk_size=3072, context_window=4096, local_window=512):
    """patch_model_with_dca under the install_* naming of the other kernels (:656-663)."""
    return patch_model_with_dca(model, chunk_size, context_window, local_window)
