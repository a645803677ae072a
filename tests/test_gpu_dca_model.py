"""DCA with a KV cache on the GPU: the key rotation into the cache (sta_dca_rotate_keys), decode
(sta_dca_decode) and the model drop-ins (patch_model_with_dca / unpatch_model /
install_dca_forward, dca_kernel.py:372-663).

  * rotated keys: bit for bit the oracle's (the same correctly rounded tables and model-dtype
    rounding sequence), any dtype, strided input, a position offset;
  * decode: the oracle's restatement of the reference's model-dtype matmuls and fp32 softmax
    within one unit of the output dtype's last place (the fp32 sum of exponentials is reduced
    in a different order), fp32 within 5e-5; every chunk position (inside chunk 0, 1, 2 and
    later), GQA;
  * the reference's own forward with a DynamicCache (tests/golden/dca_decode_golden.npz):
    prefill and every decode output, the cache's rotated keys and the table factor, including a
    decode that outgrows the table;
  * a patched small Llama (tests/golden/dca_model_golden.npz): prefill logits, every greedy step's
    logits and the tokens of the reference's patched model; dense known answer inside one chunk
    (the unpatched model's logits); unpatch restores the model; a model with nothing to patch
    raises.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import np_of

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda:0"
TDT = {orc.F32: torch.float32, orc.BF16: torch.bfloat16, orc.F16: torch.float16}


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _restore_forward():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()
    import transformers.models.llama.modeling_llama as ml
    orig = ml.LlamaAttention.forward
    yield
    ml.LlamaAttention.forward = orig


def _inv_freq(D):
    return 1.0 / (10000 ** (torch.arange(0, D, 2).float() / D))


def _from_store(a, dt):
    t = torch.from_numpy(a)
    return t if dt == orc.F32 else t.view(torch.int16).view(TDT[dt])


def ulp_close(got, ref, dt, what, vmax=None, frac=0.05):
    """got against ref for outputs rounded to the dtype.  fp32: within 5e-5 (the fp32 sums over up
    to thousands of keys run in another order than the oracle's sequential ones).  16-bit dtypes: the
    softmax weights are rounded to the dtype after a division by the fp32 sum of exponentials,
    which the GPU reduces in another order than the oracle, so a weight may move by one unit in
    its last place, |dp_j| <= 2^(1-p) p_j (p = 8 / 11 significant bits), and the output by at
    most 2^(1-p) max|v| on top of its own rounding: each element within one unit in its last
    place plus 2^(1-p) vmax (vmax = max |v|; without it, one unit), and at most `frac` of the
    elements differing at all."""
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    if dt == orc.F32:
        err = float(np.max(np.abs(got - ref)))
        assert err <= 5e-5, f"{what}: max err {err:.3e}"
        return err
    mant = 8 if dt == orc.BF16 else 11
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -60))) - (mant - 1))
    bound = ulp * 1.0001 + (0.0 if vmax is None else 2.0 ** (1 - mant) * vmax)
    diff = np.abs(got - ref)
    assert np.all(diff <= bound), f"{what}: {int((diff > bound).sum())} elements beyond the bound"
    f = float((diff > 0).mean())
    assert f <= frac, f"{what}: {f:.3%} of the elements differ"
    return float(diff.max())


@pytest.mark.parametrize("dt", [orc.F32, orc.BF16, orc.F16])
def test_rotate_keys_match_oracle(dt):
    import _sta_native as native
    Hkv, N, D, pos0 = 3, 301, 128, 777
    say(f"dca key rotation dtype {dt} pos0 {pos0}")
    g = torch.Generator().manual_seed(31 + dt)
    k_tok_major = torch.randn(1, N, Hkv, D, generator=g).to(TDT[dt])
    k = k_tok_major.to(DEV).transpose(1, 2)                # (1, Hkv, N, D), token stride Hkv * D
    out = native.dca_rotate_keys(k, pos0, _inv_freq(D), 3072, 512, 1.0380026)
    torch.cuda.synchronize()
    kn, odt = np_of(k[0].contiguous())
    ref = orc.dca_rotate_keys(kn, odt, _inv_freq(D).numpy(), 3072, 512, np.float32(1.0380026), pos0=pos0)
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("dt,D,H,Hkv", [(orc.BF16, 128, 32, 8), (orc.F16, 64, 4, 1), (orc.F32, 128, 8, 8)])
def test_decode_matches_oracle_in_every_chunk_position(dt, D, H, Hkv):
    import _sta_native as native
    s, w = 96, 32                                          # L = 64
    g = torch.Generator().manual_seed(41 + dt)
    for M in (1, 37, 64, 65, 128, 200, 1000, 5000):
        say(f"dca decode dtype {dt} D={D} H={H} Hkv={Hkv} M={M}")
        q = (torch.randn(H, D, generator=g) * 2).to(TDT[dt]).to(DEV)
        k = (torch.randn(Hkv, M, D, generator=g) * 2).to(TDT[dt]).to(DEV)
        v = torch.randn(Hkv, M, D, generator=g).to(TDT[dt]).to(DEV)
        ms = 1.0254
        krot = native.dca_rotate_keys(k, 0, _inv_freq(D), s, w, ms)
        out = native.dca_decode(q, krot, v, _inv_freq(D), s, w, ms)
        torch.cuda.synchronize()
        qn, odt = np_of(q)
        kr, _ = np_of(krot)
        vn, _ = np_of(v)
        ref = orc.dca_decode(qn, kr, vn, odt, _inv_freq(D).numpy(), s, w, np.float32(ms))
        e = ulp_close(out.float().cpu().numpy(), ref, dt, f"decode M={M}", vmax=float(v.float().abs().max()))
        print(f"[result] dca decode dtype {dt} M={M}: max err {e:.2e}", flush=True)


def test_decode_matches_reference_goldens():
    import _sta_native as native
    g = np.load(os.path.join(GOLD, "dca_decode_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        s, c, w, N, T, dt = (int(x) for x in g[p + "params"])
        q, krot, v = (_from_store(g[p + n], dt).to(DEV) for n in ("q", "krot", "v"))
        D = q.shape[-1]
        for t in range(T):
            m = N + t + 1
            say(f"dca decode golden {i} step {t}")
            out = native.dca_decode(q[:, N + t], krot[:, :m], v[:, :m], _inv_freq(D), s, w,
                                    float(np.float32(g[p + "mscale"][1 + t])))
            ulp_close(out.float().cpu().numpy(), g[p + "out"][:, N + t], dt, f"golden {i} step {t}",
                      vmax=float(v[:, :m].float().abs().max()))


class _PassThrough(torch.nn.Module):
    """An attention module whose projections hand q, k and v through unchanged (identity output
    projection), as the golden generator's."""

    def __init__(self, H, Hkv, D, dtype):
        from types import SimpleNamespace
        super().__init__()
        self.head_dim, self.num_heads, self.num_key_value_heads, self.layer_idx = D, H, Hkv, 0
        self.config = SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv)
        self.scaling = D ** -0.5
        width = (H + 2 * Hkv) * D
        eye = torch.eye(width, dtype=dtype)
        self.q_proj = torch.nn.Linear(width, H * D, bias=False, dtype=dtype)
        self.k_proj = torch.nn.Linear(width, Hkv * D, bias=False, dtype=dtype)
        self.v_proj = torch.nn.Linear(width, Hkv * D, bias=False, dtype=dtype)
        self.o_proj = torch.nn.Linear(H * D, H * D, bias=False, dtype=dtype)
        with torch.no_grad():
            self.q_proj.weight.copy_(eye[:H * D])
            self.k_proj.weight.copy_(eye[H * D:(H + Hkv) * D])
            self.v_proj.weight.copy_(eye[(H + Hkv) * D:])
            self.o_proj.weight.copy_(torch.eye(H * D, dtype=dtype))


def test_forward_with_cache_reproduces_reference():
    """The drop-in forward on the reference's pass-through module with a DynamicCache: prefill, T
    decode steps, the cache's rotated keys and the table factor at every call."""
    import dca_kernel as dca
    from transformers import DynamicCache
    g = np.load(os.path.join(GOLD, "dca_decode_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        s, c, w, N, T, dt = (int(x) for x in g[p + "params"])
        q, k, v = (_from_store(g[p + n], dt) for n in ("q", "k", "v"))
        H, Hkv, D = q.shape[0], k.shape[0], q.shape[-1]
        say(f"dca forward golden {i}: H={H} Hkv={Hkv} N={N} T={T} D={D} dtype {dt}")
        core = _PassThrough(H, Hkv, D, TDT[dt]).to(DEV)
        core.rotary_emb = dca.DcaRotaryState(D, max_position_embeddings=c, base=10000, device=DEV)
        hidden = torch.cat([q.transpose(0, 1).reshape(N + T, -1), k.transpose(0, 1).reshape(N + T, -1),
                            v.transpose(0, 1).reshape(N + T, -1)], dim=-1)[None].to(DEV)
        fwd = dca._make_dca_forward(s, c, w)
        cache = DynamicCache()
        with torch.no_grad():
            out, _ = fwd(core, hidden[:, :N], None, None, cache)
            got = [out[0].reshape(N, H, D).transpose(0, 1)]
            ms = [core.rotary_emb._last_mscale]
            for t in range(T):
                out, _ = fwd(core, hidden[:, N + t:N + t + 1], None, None, cache)
                got.append(out[0].reshape(1, H, D).transpose(0, 1))
                ms.append(core.rotary_emb._last_mscale)
        got = torch.cat(got, dim=1).float().cpu().numpy()
        ref = g[p + "out"]
        assert np.array_equal(np.array(ms), g[p + "mscale"]), i
        tol = 1e-4 if dt == orc.F32 else 2e-2
        np.testing.assert_allclose(got[:, :N], ref[:, :N], atol=tol, rtol=tol, err_msg=f"{i} prefill")
        ulp_close(got[:, N:], ref[:, N:], dt, f"golden {i} decode", vmax=float(v.float().abs().max()))
        kc = cache.layers[0].keys[0].float().cpu().numpy()
        kref = _from_store(g[p + "krot"], dt).float().numpy()
        if dt == orc.F32:
            np.testing.assert_allclose(kc, kref, atol=1e-6, rtol=0)
        else:
            assert np.array_equal(kc, kref), f"{i}: cached keys differ"


def _llama(seed):
    import sys
    sys.path.insert(0, GOLD)
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
               num_key_value_heads=2, head_dim=64, max_position_embeddings=8192, attn_implementation="eager")
    torch.manual_seed(seed)
    return LlamaForCausalLM(LlamaConfig(**cfg)).eval().to(DEV)


def _greedy(model, ids, T):
    from transformers import DynamicCache
    cache = DynamicCache()
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True).logits[0]
        prefill = out
        steps, toks = [out[-1]], []
        nxt = int(out[-1].argmax())
        for _ in range(T):
            toks.append(nxt)
            out = model(torch.tensor([[nxt]], device=DEV), past_key_values=cache, use_cache=True).logits[0, -1]
            steps.append(out)
            nxt = int(out.argmax())
    return prefill, torch.stack(steps), toks


def test_patched_llama_reproduces_reference_model():
    import dca_kernel as dca
    gm = np.load(os.path.join(GOLD, "dca_model_golden.npz"), allow_pickle=False)
    s, c, w, N, T, seed = (int(x) for x in gm["params"])
    say(f"patched llama vs reference: s={s} c={c} w={w} N={N} T={T}")
    model = _llama(seed)
    patch = dca.patch_model_with_dca(model, s, c, w)
    assert patch.n_layers == 2
    prefill, steps, toks = _greedy(model, torch.from_numpy(gm["ids"]).to(DEV), T)
    perr = float((prefill.cpu() - torch.from_numpy(gm["prefill_logits"])).abs().max())
    serr = float((steps.cpu() - torch.from_numpy(gm["step_logits"])).abs().max())
    print(f"[result] patched llama: prefill logits err {perr:.2e}, step logits err {serr:.2e}, tokens {toks}",
          flush=True)
    assert perr < 1e-3 and serr < 1e-3
    assert toks == gm["tokens"].tolist()
    dca.unpatch_model(patch)


def test_patched_llama_inside_one_chunk_is_the_dense_model():
    """N + T <= L and N <= pretrain_len: keys at j, queries at i, factor 1 -- plain RoPE."""
    import dca_kernel as dca
    import transformers.models.llama.modeling_llama as ml
    say("patched llama, one chunk: dense known answer")
    model = _llama(7)
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, 256, (1, 200), generator=g).to(DEV)
    ref_prefill, ref_steps, ref_toks = _greedy(model, ids, 6)
    orig = ml.LlamaAttention.forward
    patch = dca.install_dca_forward(model, chunk_size=320, context_window=4096, local_window=64)
    assert ml.LlamaAttention.forward is not orig
    assert all(isinstance(l.self_attn.rotary_emb, dca.DcaRotaryState) for l in model.model.layers)
    prefill, steps, toks = _greedy(model, ids, 6)
    perr = float((prefill - ref_prefill).abs().max())
    serr = float((steps - ref_steps).abs().max())
    print(f"[result] one chunk: prefill logits err {perr:.2e}, step logits err {serr:.2e}", flush=True)
    assert perr < 2e-3 and serr < 2e-3 and toks == ref_toks
    dca.unpatch_model(patch)
    assert ml.LlamaAttention.forward is orig
    assert not any(hasattr(l.self_attn, "rotary_emb") for l in model.model.layers)
    prefill2, _, _ = _greedy(model, ids, 0)
    assert torch.equal(prefill2, ref_prefill)


def test_patch_refuses_a_model_without_llama_attention():
    import dca_kernel as dca
    import transformers.models.llama.modeling_llama as ml
    orig = ml.LlamaAttention.forward
    with pytest.raises(RuntimeError):
        dca.patch_model_with_dca(torch.nn.Sequential(torch.nn.Linear(4, 4)), 96, 128, 32)
    assert ml.LlamaAttention.forward is orig
    with pytest.raises(AssertionError):
        dca.patch_model_with_dca(torch.nn.Linear(4, 4), 96, 64, 32)      # s >= c
