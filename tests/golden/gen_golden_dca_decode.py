#!/usr/bin/env python3
"""Write the golden vectors of DCA with a KV cache: prefill, then decode steps.

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    python tests/golden/gen_golden_dca_decode.py

Executed from the reference (dca_kernel.py): the attention forward that _make_dca_forward builds
(:372-525) on a minimal attention module whose projections hand q, k and v through unchanged
and whose output projection is the identity (as tests/golden/gen_golden_dca.py does), with the
module's own ChunkLlamaRotaryEmbedding (:166-275) and a transformers DynamicCache: one prefill
call over N tokens, then T decode calls of one token each.  Recorded per case: the inputs, the
prefill output, every decode output, the cache's rotated keys after the last call and the
rotary's table factor at every call.  Cases cover the three position types at decode, a decode
that crosses a chunk boundary, a decode that outgrows the table (the factor changes mid-way and
the earlier cached keys keep the old one), GQA, head_dim 128, and fp32 / bf16 / fp16 models.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from gen_golden import planted_inputs  # noqa: E402
from gen_golden_dca import REF, _Core  # noqa: E402


def _import_reference():
    sys.path.insert(0, REF)
    import dca_kernel as dca  # noqa: E402
    return dca


CASES = [
    # chunk_size s, pretrain c, local w -> L = s - w; N prefill tokens, T decode steps
    dict(name="fp32_gqa_cross_chunk", H=2, Hkv=1, N=318, T=5, D=64, s=96, c=128, w=32, dtype=torch.float32, seed=81),
    dict(name="bf16_outgrows_table", H=2, Hkv=2, N=120, T=80, D=64, s=160, c=192, w=32, dtype=torch.bfloat16,
         seed=82),
    dict(name="bf16_d128_gqa", H=4, Hkv=2, N=330, T=4, D=128, s=96, c=256, w=32, dtype=torch.bfloat16, seed=83),
    dict(name="fp16_short", H=2, Hkv=1, N=200, T=3, D=64, s=96, c=128, w=32, dtype=torch.float16, seed=84),
]


def _store(t, dtype):
    if dtype == torch.float32:
        return t.numpy()
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def gen(dca):
    from transformers import DynamicCache
    arrays = {}
    with torch.no_grad():
        for i, c in enumerate(CASES):
            dca._DCA_CHUNK_SIZE, dca._DCA_LOCAL_WINDOW = c["s"], c["w"]
            H, Hkv, N, T, D, dt = c["H"], c["Hkv"], c["N"], c["T"], c["D"], c["dtype"]
            core = _Core(dca, H, Hkv, D, c["c"], dt)
            q, k, v = planted_inputs(c["seed"], H, Hkv, N + T, D, 0.02, dt)
            hidden = torch.cat([q[0].transpose(0, 1).reshape(N + T, -1), k[0].transpose(0, 1).reshape(N + T, -1),
                                v[0].transpose(0, 1).reshape(N + T, -1)], dim=-1)[None]
            fwd = dca._make_dca_forward(c["s"], c["c"], c["w"])
            cache = DynamicCache()
            outs, mscales = [], []
            out, _ = fwd(core, hidden[:, :N], None, None, cache)
            outs.append(out[0].reshape(N, H, D).transpose(0, 1))
            mscales.append(core.rotary_emb._last_mscale)
            for t in range(T):
                out, _ = fwd(core, hidden[:, N + t:N + t + 1], None, None, cache)
                outs.append(out[0].reshape(1, H, D).transpose(0, 1))
                mscales.append(core.rotary_emb._last_mscale)
            layer = cache.layers[0]
            p = f"c{i}_"
            arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = _store(q[0], dt), _store(k[0], dt), _store(v[0], dt)
            arrays[p + "out"] = torch.cat(outs, dim=1).float().numpy()          # (H, N + T, D)
            arrays[p + "krot"] = _store(layer.keys[0], dt)                      # (Hkv, N + T, D)
            arrays[p + "mscale"] = np.array(mscales, np.float64)
            arrays[p + "params"] = np.array([c["s"], c["c"], c["w"], N, T,
                                             {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dt]], np.int64)
            print(f"dca decode case {i} {c['name']}: L={c['s'] - c['w']} mscale {mscales[0]:.6f} -> "
                  f"{mscales[-1]:.6f}", flush=True)
    arrays["ncases"] = np.array(len(CASES))
    np.savez_compressed(os.path.join(HERE, "dca_decode_golden.npz"), **arrays)


MODEL = dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=64, max_position_embeddings=8192, attn_implementation="eager")


def model_of(seed):
    """The random-weight GQA Llama both sides build (CPU init with this seed, fp32)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    return LlamaForCausalLM(LlamaConfig(**MODEL)).eval()


def gen_model(dca):
    """patch_model_with_dca on a small Llama: greedy prefill + decode through the patched model,
    past the first chunks and above the pretraining length (factor > 1)."""
    from transformers import DynamicCache
    s, c, w, N, T, seed = 96, 128, 32, 300, 6, 91
    model = model_of(seed)
    g = torch.Generator().manual_seed(92)
    ids = torch.randint(0, MODEL["vocab_size"], (1, N), generator=g)
    originals = dca.patch_model_with_dca(model, s, c, w)
    logits, toks = [], []
    with torch.no_grad():
        cache = DynamicCache()
        out = model(ids, past_key_values=cache, use_cache=True).logits[0]
        prefill = out.numpy()
        nxt = int(out[-1].argmax())
        logits.append(out[-1].numpy())
        for _ in range(T):
            toks.append(nxt)
            out = model(torch.tensor([[nxt]]), past_key_values=cache, use_cache=True).logits[0, -1]
            logits.append(out.numpy())
            nxt = int(out.argmax())
    dca.unpatch_model(originals)
    np.savez_compressed(os.path.join(HERE, "dca_model_golden.npz"), ids=ids.numpy(), prefill_logits=prefill,
                        step_logits=np.stack(logits), tokens=np.array(toks, np.int64),
                        params=np.array([s, c, w, N, T, seed], np.int64))
    print(f"dca model: tokens {toks}", flush=True)


if __name__ == "__main__":
    torch.set_num_threads(8)
    ref = _import_reference()
    gen(ref)
    gen_model(ref)
