"""GPU parity of the chunk-granular selection ("chunk_exact", shared_selection_triton_chunked.py).

  1. sets given votes: the oracle's _build_sets_chunk restatement applied to the GPU's votes /
     weighted votes reproduces idx, newpos_k, newpos_q, mask, usize, kept_size and passers_kept
     bit for bit (freq / margin / expmass ranking, sum / mean, a nonzero q_pos_base, ragged
     tiles); the same from dense votes through sta_chunk_build_sets;
  2. composed prefill: the GPU's PQ Kernel A votes against the oracle's within the threshold band;
     the kept chunks against the oracle's own sets, every differing chunk counted and explained
     (a tile whose votes flipped in the band, or a chunk value within 1e-4 of the tile's cut);
  3. output given the GPU's sets: the oracle's pooled Kernel C within 1e-4 (fp32) or 2e-2 abs +
     1e-2 rel (bf16 / fp16);
  4. decode: the chunk rule from given scores bit for bit (freq; weighted ranks equal except at
     chunk values within 1e-5 of the cut, where exp's last bit can order them), the attend given
     the sets; known answers: every chunk selectable is dense causal attention; a model with every
     key kept is the dense model.
"""
import math

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, check_output, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NAMES = ("idx", "newpos_k", "newpos_q", "mask", "usize", "kept_size")


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()
    import transformers.models.llama.modeling_llama as ml
    orig = ml.LlamaAttention.forward
    yield
    ml.LlamaAttention.forward = orig


def _eq(a, b):
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a.astype(np.int64), b.astype(np.int64))


def _random_votes(seed, H, nt, N, T, q_pos_base, freq):
    rng = np.random.default_rng(seed)
    votes = np.zeros((H, nt, N), np.int32)
    wv = np.zeros((H, nt, N), np.float32)
    for t in range(nt):
        hi = min(N, q_pos_base + (t + 1) * T)
        v = rng.integers(0, 5, size=(H, hi)) * (rng.random((H, hi)) < (0.15 if freq else 0.3))
        votes[:, t, :hi] = v
        wv[:, t, :hi] = np.where(v > 0, rng.random((H, hi)).astype(np.float32) * v, 0)
    return votes, wv


@pytest.mark.parametrize("score,agg,qpb,C", [("freq", "sum", 0, 16), ("expmass", "sum", 0, 16),
                                             ("margin", "mean", 64, 32), ("expmass", "mean", 0, 7),
                                             ("freq", "sum", 5, 64)])
def test_chunk_sets_given_votes(score, agg, qpb, C):
    import _sta_native as native
    H, N, T, ng, nl = 3, 2000, 32, 32, 32
    nt = (N + T - 1) // T
    n_chunk = 9
    k_max = (orc.n_forced_chunks(C, ng, nl, T) + n_chunk) * C
    say(f"chunk sets from votes: {score} {agg} q_pos_base={qpb} C={C} k_max={k_max}")
    votes, wv = _random_votes(hash((score, agg, qpb, C)) % 2**31, H, nt, N, T, qpb, score == "freq")
    res, pk = native.chunk_build_sets(torch.from_numpy(votes).to(DEV), torch.from_numpy(wv).to(DEV), ng, nl, T,
                                      k_max, C, n_chunk, qpb, score, agg)
    torch.cuda.synchronize()
    ref = orc.build_sets_chunk(votes, wv, ng, nl, T, k_max, C, n_chunk, qpb, score, agg)
    for name, g, r in zip(NAMES, res, ref[:6]):
        assert _eq(g.cpu().numpy(), r), f"{name} differs from the oracle"
    assert _eq(pk.cpu().numpy(), ref[6])
    print(f"[result] chunk sets {score} {agg} C={C}: kept mean {ref[5].mean():.0f} of k_max {k_max}", flush=True)


def _explain(votes_g, votes_o, wv_g, wv_o, idx_g, idx_o, N, C, n_chunk, score, rel=1e-4):
    """Count differing kept chunks per (head, tile) and check each is explained."""
    H, nt, _ = votes_g.shape
    tiles = chunks = 0
    for h in range(H):
        for t in range(nt):
            a = set((idx_g[h, t][idx_g[h, t] < N] // C).tolist())
            b = set((idx_o[h, t][idx_o[h, t] < N] // C).tolist())
            if a == b:
                continue
            tiles += 1
            chunks += len(a ^ b)
            if not np.array_equal(votes_g[h, t], votes_o[h, t]):
                continue                                      # a band flip in this tile
            vals = _values(votes_g[h, t], wv_g[h, t], N, C, score)
            vo = _values(votes_o[h, t], wv_o[h, t], N, C, score)
            for c in a ^ b:
                cut = min(vals[list(a)]) if a else 0.0
                assert abs(vals[c] - cut) <= rel * max(1.0, abs(cut)) or abs(vals[c] - vo[c]) > 0, \
                    f"head {h} tile {t} chunk {c}: value {vals[c]} far from the cut {cut}"
    return tiles, chunks


def _values(vr, wr, N, C, score):
    nC = (N + C - 1) // C
    x = np.where(vr > 0, wr if score != "freq" else vr, 0).astype(np.float64)
    x = np.pad(x, (0, nC * C - N))
    return x.reshape(nC, C).sum(-1)


@pytest.mark.parametrize("dt,score", [(torch.float32, "expmass"), (torch.bfloat16, "expmass"),
                                      (torch.float16, "freq")])
def test_chunk_prefill_composed(dt, score):
    import _sta_native as native
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, N, D, C = 4, 2, 1500, 128, 16
    ng, nl, k_max = 32, 32, 512
    n_chunk = orc.derive_n_chunk(k_max, C, ng, nl, 32)
    q, k, v = planted_inputs(71, H, Hkv, N, D, 0.02, dt, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    sm = 1.0 / math.sqrt(D)
    say(f"chunk prefill composed {dt} {score}: H={H} Hkv={Hkv} N={N} C={C} n_chunk={n_chunk}")
    r = native.chunk_attention(q, k, v, tau, invf, invf, 0.25, 1.0, sm, ng, nl, 32, k_max, C, n_chunk, 0, score,
                               "sum", want_votes=True)
    torch.cuda.synchronize()
    votes_g, wv_g = r["votes"].cpu().numpy(), r["wvotes"].cpu().numpy()
    # 1. sets given the GPU's votes
    ref = orc.build_sets_chunk(votes_g, wv_g, ng, nl, 32, k_max, C, n_chunk, 0, score, "sum")
    got = {n: r[n].cpu().numpy() for n in NAMES}
    for name, rr in zip(NAMES, ref[:6]):
        assert _eq(got[name], rr), f"{name} differs from the oracle given the GPU's votes"
    assert _eq(r["passers_kept"].cpu().numpy(), ref[6])
    # 2. votes against the oracle's, sets against the oracle's own
    qn, odt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    a = orc.select_bits(qn, kn, odt, tau.cpu().numpy(), invf.cpu().numpy(), 0.25, 1.0, sm, 32, 0,
                        orc.WMODES[score], band_eps=BAND, want_band=True)
    d = np.abs(votes_g.astype(np.int64) - a["votes"])
    assert not np.any(d > a["band"]), "votes differ beyond the band"
    own = orc.build_sets_chunk(a["votes"], a["wvotes"], ng, nl, 32, k_max, C, n_chunk, 0, score, "sum")
    tiles, chunks = _explain(votes_g, a["votes"], wv_g, a["wvotes"], got["idx"], own[0], N, C, n_chunk, score)
    print(f"[sets] chunk prefill {dt} {score}: {tiles} of {H * ((N + 31) // 32)} tiles keep other chunks than the "
          f"oracle's own sets ({chunks} chunks), each explained by a band flip or a cut tie", flush=True)
    # 3. output given the GPU's sets
    out_ref = orc.gather_attn_mask(qn, kn, vn, odt, got["idx"], got["newpos_k"], got["newpos_q"], got["mask"],
                                   invf.cpu().numpy(), 1.0, sm, 32, k_max)
    e = check_output(r["out"].float().cpu().numpy(), out_ref, odt, "chunk prefill")
    print(f"[result] chunk prefill {dt} {score}: max out err {e:.2e}, kept mean {got['kept_size'].mean():.0f}",
          flush=True)


def test_chunk_prefill_every_chunk_is_dense_causal():
    import _sta_native as native
    from synthetic import planted_inputs, base_inv_freq
    H, N, D, C = 2, 700, 64, 16
    q, k, v = planted_inputs(72, H, H, N, D, 0.02, torch.float32, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    nC = (N + C - 1) // C
    k_max = (orc.n_forced_chunks(C, 8, 8, 32) + nC) * C
    say("chunk prefill, every chunk selectable: dense causal attention")
    r = native.chunk_attention(q, k, v, torch.full((H,), 0.5, device=DEV), invf, invf, 1.0, 1.0, None, 8, 8, 32,
                               k_max, C, nC)
    torch.cuda.synchronize()
    qn, kn, vn = (x[0].double().cpu().numpy() for x in (q, k, v))
    invn = invf.double().cpu().numpy()
    pos = np.arange(N)
    ang = pos[:, None] * invn[None]
    c, s = np.cos(ang), np.sin(ang)

    def rot(x):
        h = D // 2
        return np.concatenate([x[:, :h] * c - x[:, h:] * s, x[:, h:] * c + x[:, :h] * s], -1)
    for h in range(H):
        sc = rot(qn[h]) @ rot(kn[h]).T / math.sqrt(D)
        sc = np.where(np.tril(np.ones((N, N), bool)), sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        ref = (p / p.sum(-1, keepdims=True)) @ vn[h]
        err = float(np.abs(r["out"][h].cpu().numpy() - ref).max())
        assert err < 2e-4, f"head {h}: {err:.2e}"


@pytest.mark.parametrize("score,agg,Q", [("freq", "sum", 1), ("expmass", "sum", 70), ("expmass", "mean", 5)])
def test_chunk_decode_sets_and_attend(score, agg, Q):
    import _sta_native as native
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, M, D, C, ng, nl, n_chunk, k_max = 8, 2, 3000, 128, 16, 32, 32, 40, 1024
    q, k, v = planted_inputs(73 + Q, H, Hkv, M, D, 0.02, torch.bfloat16, DEV)
    qq = q[0, :, M - Q:, :].contiguous()
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.linspace(1.0, 4.0, H, device=DEV)
    sm = 1.0 / math.sqrt(D)
    say(f"chunk decode {score} {agg} Q={Q}: H={H} M={M}")
    plan = native.DecodePlan(qq, k[0], v[0], tau, invf, M - Q, 0.25, 1.0, sm, ng, nl, k_max, 100.0,
                             inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0)
    s = plan.scores(torch.empty((H, Q, M), dtype=torch.float32, device=DEV))
    pk = torch.empty((H, Q), dtype=torch.int32, device=DEV)
    us = torch.empty((H, Q), dtype=torch.int32, device=DEV)
    r = plan.build_sets_chunk(s, C, n_chunk, score, agg, passers_kept=pk, usize=us)
    got = {n: r[n].cpu().numpy() for n in ("idx", "newpos_k", "newpos_q", "set_size")}
    out = plan.attend(r["idx"], r["newpos_k"], r["newpos_q"], r["set_size"]).float().cpu().numpy()
    torch.cuda.synchronize()
    sn = s.cpu().numpy()
    valid = np.isfinite(sn)
    ref = orc.decode_build_sets_chunk(np.where(valid, sn, 0).astype(np.float32), tau.cpu().numpy(), M - Q, ng, nl,
                                      k_max, C, n_chunk, score, agg)
    same = np.all(got["idx"] == ref[0], axis=-1) & (got["set_size"] == ref[3])
    if score == "freq":
        assert same.all(), "freq chunk sets differ from the oracle given the GPU's scores"
    else:
        for h, i in np.argwhere(~same):           # only a near-tie at the cut may order differently
            m = M - (Q - 1 - i)
            row = sn[h, i, :m].astype(np.float64)
            mx = row.max()
            w = np.where(row >= np.float32(mx - tau[h].item()), np.exp(row - mx), 0)
            nC = (m + C - 1) // C
            vals = np.pad(w, (0, nC * C - m)).reshape(nC, C).sum(-1)
            a = set((got["idx"][h, i][got["idx"][h, i] < m] // C).tolist())
            b = set((ref[0][h, i][ref[0][h, i] < m] // C).tolist())
            diff = sorted(a ^ b)
            assert len(diff) == 2 and abs(vals[diff[0]] - vals[diff[1]]) <= 1e-5 * max(1.0, vals[diff].max()), \
                f"head {h} query {i}: chunks {diff} differ beyond a near-tie"
        print(f"[sets] chunk decode {score}: {int((~same).sum())} of {same.size} queries differ at a near-tie",
              flush=True)
    rows = same
    assert np.array_equal(pk.cpu().numpy()[rows], ref[4][rows])
    qn, odt = np_of(qq)
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    out_ref = orc.decode_attend(qn, kn, vn, odt, invf.cpu().numpy(), 1.0, sm, M - Q, got["idx"], got["newpos_k"],
                                got["newpos_q"])
    e = check_output(out, out_ref, odt, "chunk decode")
    print(f"[result] chunk decode {score} {agg} Q={Q}: kept mean {got['set_size'].mean():.0f}, out err {e:.2e}",
          flush=True)


def test_chunk_dropins_and_stats():
    import shared_selection_triton_chunked as chm
    from synthetic import planted_inputs, base_inv_freq
    H, N, D = 2, 600, 64
    q, k, v = planted_inputs(74, H, H, N, D, 0.02, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    chm.reset_chunk_stats()
    say("chunked drop-in module")
    out, usize, kept = chm.shared_chunk_attention(q, k, v, tau, invf, invf, pos_scale_a=0.5, k_max=512, measure=True)
    assert out.shape == (1, H, N, D) and usize.shape == kept.shape == (H, (N + 31) // 32)
    assert int(kept.max()) <= 512
    st = chm.get_chunk_stats()["prefill"]
    assert st["cells"] == H * ((N + 31) // 32) and 0 < st["recall_count"] <= 1 and 0 < st["utilisation"] <= 1
    with pytest.raises(AssertionError):
        chm.shared_chunk_attention(q, k, v, tau, invf, invf, k_max=512, n_chunk=100)
    P = N - 1
    idx, npk, npq = chm._decode_build_sets_chunk(q[0, :, P], k[0], tau, invf, P, 0.5, 1.0, 1.0 / math.sqrt(D), 32,
                                                 32, 512, 16, 20, measure=True)
    assert idx.shape == (H, 512) and idx.dtype == torch.int64 and npq.shape == (H,)
    kept_d = (idx < N).sum(-1)
    assert torch.all(npq == kept_d - 1).item()          # the query is the last kept key
    assert chm.get_chunk_stats()["decode"]["cells"] == H


def test_chunked_model_everything_kept_is_dense():
    """install_shared_pi_forward of the chunked module with tau = inf and every chunk selectable:
    prefill and decode reproduce the dense model (base RoPE at natural positions)."""
    import shared_selection_triton_chunked as chm
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=8192,
                      attn_implementation="eager")
    torch.manual_seed(21)
    model = LlamaForCausalLM(cfg).to(DEV, torch.float32).eval()
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, 256, (1, 300), generator=g).to(DEV)
    say("chunked model: dense known answer")

    def greedy():
        with torch.no_grad():
            r = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=5, do_sample=False,
                               output_logits=True, return_dict_in_generate=True, pad_token_id=0)
        return r.sequences, torch.stack(r.logits, 0)
    with torch.no_grad():
        ref_logits = model(ids).logits
    ref_seq, ref_steps = greedy()
    chm.install_shared_pi_forward(model, context_window=8192, n_global=8, n_local=8, k_max=1024, chunk_size=16,
                                  measure=True)
    for layer in model.model.layers:
        layer.self_attn.tau_head_vec = torch.full((4,), math.inf, device=DEV)
    with torch.no_grad():
        logits = model(ids).logits
    err = float((logits - ref_logits).abs().max())
    seq, steps = greedy()
    derr = float((steps - ref_steps).abs().max())
    print(f"[result] chunked model: prefill logits err {err:.2e}, decode {derr:.2e}", flush=True)
    assert err < 2e-3 and derr < 2e-3 and torch.equal(seq, ref_seq)
