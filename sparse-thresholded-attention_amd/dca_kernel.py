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
from _install import _AttnCall, _out_proj
from _torch_golden import (ChunkLlamaRotaryEmbedding, _fa_block, _merge_lse, _rotate_half,  # noqa: F401
                           apply_rotary_pos_emb, flash_attn_status)

_MAX_NEW_TOKENS = 512            # table headroom for generation (dca_kernel.py:161)
# the chunking of the last patch_model_with_dca call, the defaults of ChunkLlamaRotaryEmbedding
_DCA_CHUNK_SIZE = None
_DCA_LOCAL_WINDOW = None
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


def _make_dca_forward(chunk_size, pretrain_len, local_window):
    """The patched LlamaAttention.forward (dca_kernel.py:372-525).  Prefill (an empty cache, any
    number of tokens) runs sta_dca_attention over the call's tokens; decode (one token on a warm
    cache) runs sta_dca_decode over the whole cache.  The cache receives keys rotated at
    (pos mod L), as the reference's does.  A warm cache with more than one token raises, as the
    reference's assertion does (:424-427)."""
    s, c, w = chunk_size, pretrain_len, local_window

    def dca_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                    **kwargs):
        # the table factor of this call is fixed before its keys are rotated into the cache
        state = {}

        def rotated(k_new, past):
            state["mscale"] = self.rotary_emb.advance(past + k_new.shape[2])
            return native.dca_rotate_keys(k_new, past, self.rotary_emb.inv_freq, s, w, state["mscale"]).unsqueeze(0)

        call = _AttnCall(self, hidden_states, past_key_values, kwargs, self.layer_idx, keys_for_cache=rotated)
        assert call.past == 0 or call.N == 1, (
            f"dca_forward: chunked prefill is unsupported (start_pos={call.past}, q_len={call.N}). "
            f"Prefill must be a single pass over an empty cache; decode must be one token.")
        scale = float(getattr(self, "scaling", None) or (1.0 / math.sqrt(self.head_dim)))
        inv_freq, mscale = self.rotary_emb.inv_freq, state["mscale"]
        if call.N > 1:   # prefill: the call's raw keys, rotated inside the kernels
            out = native.dca_attention(call.q, call.k_new, call.v_new, inv_freq, s, c, w, scale, mscale=mscale)
        else:            # decode: the cached rotated keys
            out = native.dca_decode(call.q, call.k, call.v, inv_freq, s, w, mscale, scale)[:, None]
        return _out_proj(self, out.unsqueeze(0), call.N), None

    return dca_forward


class DcaPatch:
    """What patch_model_with_dca changed, so that unpatch_model can undo exactly that: for each
    attention class, the forward its own namespace held before the patch (or none: it inherited
    one), and for each module that now runs the DCA forward, whether it had a rotary_emb
    attribute and which."""

    _NONE = object()

    def __init__(self, model):
        self.model = model
        self._class_forwards = []      # (class, own forward or _NONE)
        self._rotaries = []            # (module, previous rotary_emb or _NONE)

    @property
    def n_layers(self):
        return len(self._rotaries)

    def replace_forward(self, cls, fwd):
        self._class_forwards.append((cls, cls.__dict__.get("forward", self._NONE)))
        cls.forward = fwd

    def give_state(self, module, state):
        self._rotaries.append((module, getattr(module, "rotary_emb", self._NONE)))
        module.rotary_emb = state

    def restore(self):
        for module, old in reversed(self._rotaries):
            if old is self._NONE:
                if hasattr(module, "rotary_emb"):
                    delattr(module, "rotary_emb")
            else:
                module.rotary_emb = old
        for cls, old in reversed(self._class_forwards):
            if old is self._NONE:
                del cls.forward
            else:
                cls.forward = old
        n = len(self._class_forwards)
        self._class_forwards, self._rotaries = [], []
        return n


def _needs_dca_state(module, fwd):
    """A module whose class (or a base) now resolves forward to the DCA forward; that forward reads
    its projections, head_dim, layer_idx and head counts."""
    return getattr(type(module), "forward", None) is fwd


def patch_model_with_dca(model, chunk_size, pretrain_len, local_window):
    """Patch the Llama attention classes' forward with the DCA forward and give every module that
    runs it a table state of its own.  Returns the DcaPatch record that unpatch_model takes; raises
    RuntimeError, with everything restored, when no module of the model runs the DCA forward.
    dca_kernel.py:538-615.

    The table frequencies use base = int(the module's old rotary's base, else the config's
    rope_theta attribute, else 10000), as the reference reads it.  The transformers module's
    rotary classes are left in place (the reference swaps them for ChunkLlamaRotaryEmbedding,
    which only the patched forward reads)."""
    import transformers.models.llama.modeling_llama as ml
    assert 0 < local_window < chunk_size, f"need 0 < w({local_window}) < s({chunk_size})"
    assert chunk_size < pretrain_len, f"need s({chunk_size}) < c({pretrain_len})"
    global _DCA_CHUNK_SIZE, _DCA_LOCAL_WINDOW
    _DCA_CHUNK_SIZE, _DCA_LOCAL_WINDOW = chunk_size, local_window
    fwd = _make_dca_forward(chunk_size, pretrain_len, local_window)
    patch = DcaPatch(model)
    for cls in {getattr(ml, name) for name in _ATTN_CLASSES if hasattr(ml, name)}:
        patch.replace_forward(cls, fwd)
    for m in model.modules():
        if not _needs_dca_state(m, fwd):
            continue
        old = getattr(m, "rotary_emb", None)
        base = int(getattr(old, "base", None) or getattr(m.config, "rope_theta", 10_000))
        dev = m.q_proj.weight.device
        patch.give_state(m, DcaRotaryState(m.head_dim, max_position_embeddings=pretrain_len, base=base,
                                           device=None if dev.type == "meta" else dev))
    if patch.n_layers == 0:
        patch.restore()
        raise RuntimeError(
            "patch_model_with_dca patched 0 attention layers -- the model would have run dense. "
            "Its attention modules must expose q_proj/k_proj/v_proj/o_proj/head_dim/layer_idx.")
    print(f"  [DCA] {patch.n_layers} attention layers on the HIP DCA kernels (s={chunk_size}, c={pretrain_len}, "
          f"w={local_window}, chunk_len={chunk_size - local_window})", flush=True)
    return patch


def unpatch_model(originals):
    """Undo patch_model_with_dca: its DcaPatch record restores the attention classes' forwards and
    every patched module's rotary attribute (:618-653)."""
    n = originals.restore()
    print(f"  [DCA] restored {n} attention class(es) and the modules' rotary attributes", flush=True)


def install_dca_forward(model, chunk_size=3072, context_window=4096, local_window=512):
    """patch_model_with_dca under the install_* naming of the other kernels (:656-663)."""
    return patch_model_with_dca(model, chunk_size, context_window, local_window)
