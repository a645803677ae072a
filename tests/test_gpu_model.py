"""Model integration on the GPU: install_shared_pi_forward of the PI_exact, YaRN_exact and hybrid
drop-ins on a small random-weight Llama (transformers' LlamaForCausalLM, fp32, grouped-query
attention), prefill and greedy decode through the patched attention.

  * known answer: with tau = inf, pct = 100 and k_max above the sequence, every key is kept and
    repositioned to itself (pos_scale 1), so the patched model must reproduce the unpatched
    model's logits (dense causal attention with the same RoPE) at prefill and at every decode step,
    and its greedy tokens;
  * the per-query path serves a whole prompt (prefill_mode "perquery") exactly as a prompt one
    token shorter followed by one decode step (each query selects over its own cache prefix);
  * finite thresholds: prefill statistics and decode sets stay within their bounds.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _restore_forward():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import transformers.models.llama.modeling_llama as ml
    orig = ml.LlamaAttention.forward
    yield
    ml.LlamaAttention.forward = orig


def _model(rope=None, seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    kw = {} if rope is None else {"rope_parameters": rope}
    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=8192,
                      attn_implementation="eager", **kw)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).to(DEV, torch.float32).eval()


def _set_tau(model, tau):
    for layer in model.model.layers:
        layer.self_attn.tau_head_vec = torch.full((model.config.num_attention_heads,), tau, device=DEV)


def _prompt(n, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (1, n), generator=g).to(DEV)


def _greedy(model, ids, steps):
    # an explicit all-ones mask: generate() would otherwise mask every prompt token equal to the pad id
    with torch.no_grad():
        r = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=steps, do_sample=False,
                           output_logits=True, return_dict_in_generate=True, pad_token_id=0)
    return r.sequences, torch.stack(r.logits, 0)


YARN = {"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 1024, "rope_theta": 10000.0}


@pytest.mark.parametrize("variant", ["pi", "yarn", "hybrid"])
def test_everything_kept_reproduces_the_dense_model(variant):
    import shared_selection_triton_exact_2 as ex2
    import shared_selection_triton_hybrid_exact as hyb
    import shared_selection_triton_YaRN_exact as yarn
    say(f"dense known answer, {variant}")
    model = _model(YARN if variant in ("yarn", "hybrid") else None)
    # the hybrid attends under base RoPE: its dense reference is the same weights without YaRN
    ref_model = _model(None) if variant == "hybrid" else model
    ids = _prompt(300)
    with torch.no_grad():
        ref_logits = ref_model(ids).logits
    ref_seq, ref_steps = _greedy(ref_model, ids, 6)
    kw = dict(pct=100.0, context_window=8192, n_global=8, n_local=8, tile=64, k_max=1024, pct_decode=100.0)
    {"pi": ex2, "yarn": yarn, "hybrid": hyb}[variant].install_shared_pi_forward(model, **kw)
    _set_tau(model, math.inf)
    with torch.no_grad():
        logits = model(ids).logits
    err = (logits - ref_logits).abs().max().item()
    assert err < 2e-3, f"prefill logits differ by {err:.2e}"
    sa = model.model.layers[0].self_attn
    assert bool((sa.spi_last_kpct == 100).all()) and not bool(sa.spi_last_overflow.any())
    seq, steps = _greedy(model, ids, 6)
    assert torch.equal(seq, ref_seq)
    derr = (steps - ref_steps).abs().max().item()
    assert derr < 2e-3, f"decode logits differ by {derr:.2e}"
    print(f"[result] {variant}: prefill logits max err {err:.2e}, decode {derr:.2e}", flush=True)


def test_per_query_prompt_matches_prefill_plus_one_decode_step():
    import shared_selection_triton_exact_2 as ex2
    say("per-query prefill of N tokens vs N - 1 tokens + one decode step")
    model = _model(None, seed=3)
    ex2.install_shared_pi_forward(model, pct=30.0, context_window=200, n_global=8, n_local=8, tile=32,
                                  k_max=96, max_len=600, prefill_mode="perquery", pct_decode=50.0)
    _set_tau(model, 2.0)
    ids = _prompt(513, seed=5)
    with torch.no_grad():
        full = model(ids).logits[0, -1]
        from transformers import DynamicCache
        cache = DynamicCache(config=model.config)
        model(ids[:, :-1], past_key_values=cache, use_cache=True)
        step = model(ids[:, -1:], past_key_values=cache, use_cache=True).logits[0, -1]
    assert torch.isfinite(full).all()
    err = (full - step).abs().max().item()
    assert err < 1e-4, f"per-query prompt vs decode step differ by {err:.2e}"


def test_finite_threshold_prefill_and_decode():
    import shared_selection_triton_exact_2 as ex2
    say("finite thresholds: shared prefill + greedy decode")
    model = _model(None, seed=7)
    ex2.install_shared_pi_forward(model, pct=30.0, context_window=256, n_global=8, n_local=8, tile=64,
                                  k_max=128, pct_decode=100.0, select_score="expmass")
    _set_tau(model, 3.0)
    ids = _prompt(700, seed=9)
    seq, steps = _greedy(model, ids, 4)
    assert seq.shape == (1, 704) and torch.isfinite(steps).all()
    for layer in model.model.layers:
        sa = layer.self_attn
        assert sa.spi_pos_scale == 256 / 700           # frozen at prefill: min(1, W / N)
        assert int(sa.spi_last_kept.max()) <= 2 * 700
        assert sa.spi_last_kept.shape == (4, 11)      # (heads, tiles)


def test_pqstream_everything_kept_reproduces_the_dense_model():
    """PQ Stream installed with tau = inf: every key kept, each block advances by its full length and
    every key streams to its natural distance, so prefill (the fused kernel) and decode (the stream
    rule) reproduce the dense model under base RoPE."""
    import pqstream_kernel as pqs
    say("pqstream dense known answer")
    model = _model(None, seed=11)
    ids = _prompt(300, seed=12)
    with torch.no_grad():
        ref_logits = model(ids).logits
    ref_seq, ref_steps = _greedy(model, ids, 6)
    pqs.install_pqstream_forward(model, context_window=128, n_global=8, n_local=8, block_n=32)
    _set_tau(model, math.inf)
    pqs.reset_overflow_stats()
    with torch.no_grad():
        logits = model(ids).logits
    err = (logits - ref_logits).abs().max().item()
    assert err < 2e-3, f"prefill logits differ by {err:.2e}"
    seq, steps = _greedy(model, ids, 6)
    assert torch.equal(seq, ref_seq)
    derr = (steps - ref_steps).abs().max().item()
    assert derr < 2e-3, f"decode logits differ by {derr:.2e}"
    st = pqs.get_overflow_stats()
    assert st["decode"]["total_cells"] > 0 and st["decode"]["skip_frac"] == 0.0
    print(f"[result] pqstream: prefill logits max err {err:.2e}, decode {derr:.2e}, decode span max "
          f"{st['decode']['span_max']:.0f}", flush=True)


def test_pqstream_per_query_prompt_matches_prefill_plus_one_decode_step():
    import pqstream_kernel as pqs
    say("pqstream per-query prefill of N tokens vs N - 1 tokens + one decode step")
    model = _model(None, seed=13)
    pqs.install_pqstream_forward(model, context_window=200, n_global=8, n_local=8, block_n=32, max_len=600,
                                 prefill_mode="perquery")
    _set_tau(model, 2.0)
    ids = _prompt(513, seed=14)
    with torch.no_grad():
        full = model(ids).logits[0, -1]
        from transformers import DynamicCache
        cache = DynamicCache(config=model.config)
        model(ids[:, :-1], past_key_values=cache, use_cache=True)
        step = model(ids[:, -1:], past_key_values=cache, use_cache=True).logits[0, -1]
    assert torch.isfinite(full).all()
    err = (full - step).abs().max().item()
    assert err < 1e-4, f"per-query prompt vs decode step differ by {err:.2e}"


@pytest.mark.parametrize("prefill_mode", ["shared", "perquery"])
def test_perquery_everything_kept_reproduces_the_dense_model(prefill_mode):
    """The perquery module installed with tau = inf and k_max above the sequence: every key passes,
    no cap applies and the dense ranks are the natural positions, so the PQ Union prefill
    (prefill_mode "shared"), the per-query prefill ("perquery") and the per-query decode reproduce
    the dense model under base RoPE."""
    import shared_selection_triton_perquery as spq
    say(f"perquery module dense known answer, prefill_mode {prefill_mode}")
    model = _model(None, seed=15)
    ids = _prompt(300, seed=16)
    with torch.no_grad():
        ref_logits = model(ids).logits
    ref_seq, ref_steps = _greedy(model, ids, 6)
    spq.install_shared_pi_forward(model, context_window=128, n_global=8, n_local=8, tile=32, k_max=1024,
                                  prefill_mode=prefill_mode, select_score="expmass")
    _set_tau(model, math.inf)
    spq.reset_overflow_stats()
    with torch.no_grad():
        logits = model(ids).logits
    err = (logits - ref_logits).abs().max().item()
    assert err < 2e-3, f"prefill logits differ by {err:.2e}"
    seq, steps = _greedy(model, ids, 6)
    assert torch.equal(seq, ref_seq)
    derr = (steps - ref_steps).abs().max().item()
    assert derr < 2e-3, f"decode logits differ by {derr:.2e}"
    st = spq.get_overflow_stats()
    assert st["decode"]["overflow_frac"] == 0.0
    print(f"[result] perquery {prefill_mode}: prefill logits max err {err:.2e}, decode {derr:.2e}", flush=True)


def test_perquery_module_prompt_matches_prefill_plus_one_decode_step():
    """Finite tau and a cap below the union: the per-query prefill of N tokens gives the last
    position the same logits as N - 1 tokens followed by one decode step."""
    import shared_selection_triton_perquery as spq
    say("perquery module: per-query prefill of N tokens vs N - 1 tokens + one decode step")
    model = _model(None, seed=17)
    spq.install_shared_pi_forward(model, context_window=200, n_global=8, n_local=8, tile=32, k_max=96,
                                  max_len=600, prefill_mode="perquery", select_score="expmass")
    _set_tau(model, 2.0)
    ids = _prompt(513, seed=18)
    with torch.no_grad():
        full = model(ids).logits[0, -1]
        from transformers import DynamicCache
        cache = DynamicCache(config=model.config)
        model(ids[:, :-1], past_key_values=cache, use_cache=True)
        step = model(ids[:, -1:], past_key_values=cache, use_cache=True).logits[0, -1]
    assert torch.isfinite(full).all()
    err = (full - step).abs().max().item()
    assert err < 1e-4, f"per-query prompt vs decode step differ by {err:.2e}"
