"""CPU tests that pin the PQ Union and PQ Stream oracles (oracle/sta_oracle_pq.c).

Pins, per oracle function:
  build_sets_pq    -- the reference's _build_sets_pq on 6 synthetic (votes, bits, wvotes) inputs
                      (tests/golden/build_sets_pq_golden.npz): equal, except among keys whose rank
                      value ties at the overflow cut, where torch.topk's choice is unspecified.
  select_bits      -- votes / bits / wvotes of the reference's _select_bits_kernel under the
                      Triton interpreter (pq_composed_golden.npz, fp32).
  gather_attn_mask -- the reference's composed shared_pq_attention output given its own sets, and
                      the reference's independent torch golden pq_attention_torch end to end.
  pqstream         -- the reference's fused _pqstream_kernel under the interpreter (out, span,
                      kept, blocks, skipped) and its torch golden pqstream_attention_torch; the
                      tau=inf / advance="full" case also against dense causal RoPE attention
                      computed here in float64.
"""
import math
import os

import numpy as np

from parity_helpers import PQ_SET_NAMES, compare_pq_sets, pq_rank_values

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_build_sets_pq_matches_reference(oracle):
    g = _load("build_sets_pq_golden.npz")
    n = int(g["ncases"])
    assert n >= 6
    tie_tiles = 0
    for i in range(n):
        p = f"c{i}_"
        ng, nl, T, kmax, qb, mode = (int(x) for x in g[p + "params"])
        votes, bits, wv = g[p + "votes"], g[p + "bits"], g[p + "wvotes"]
        res = oracle.build_sets_pq(votes, bits, wv, ng, nl, T, kmax, qb, mode)
        got = dict(zip(PQ_SET_NAMES, res))
        ref = {k: g[p + k] for k in PQ_SET_NAMES}
        tie_tiles += compare_pq_sets(got, ref, pq_rank_values(votes, wv, mode), votes.shape[-1])
    # the freq and tie cases must exercise the tie rule at least once
    assert tie_tiles > 0


def test_build_sets_pq_budget_zero_keeps_forced_prefix(oracle):
    """n_forced > k_max: budget clamps to 0, the kept set is the forced set and only its first
    k_max keys reach a slot (perquery.py:398-433)."""
    g = _load("build_sets_pq_golden.npz")
    p = "c5_"
    ng, nl, T, kmax, qb, mode = (int(x) for x in g[p + "params"])
    res = oracle.build_sets_pq(g[p + "votes"], g[p + "bits"], g[p + "wvotes"], ng, nl, T, kmax, qb, mode)
    idx, mask, kept = res[0], res[3], res[5]
    assert (kept > kmax).any()
    over = kept > kmax
    assert np.all(mask[over] == -1)          # every slot holds a forced key
    assert np.all(idx[over][:, :ng] == np.arange(ng))


def test_select_bits_matches_reference(oracle):
    g = _load("pq_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, kmax, mode, qb = g[p + "params"]
        q, k = g[p + "q"], g[p + "k"]
        sm = 1.0 / math.sqrt(q.shape[-1])
        a = oracle.select_bits(q, k, oracle.F32, g[p + "tau"], g[p + "inv_freq_a"], float(psa),
                               float(rsa), sm, 32, int(qb), int(mode))
        assert np.array_equal(a["votes"], g[p + "votes"]), i
        assert np.array_equal(a["bits"], g[p + "bits"]), i
        if int(mode) > 0:
            np.testing.assert_allclose(a["wvotes"], g[p + "wvotes"], rtol=2e-6, atol=1e-6)
        # votes are the popcount of the bits
        pc = np.zeros_like(a["votes"])
        for r in range(32):
            pc += (a["bits"].view(np.uint32) >> np.uint32(r)).astype(np.int64).astype(np.int32) & 1
        assert np.array_equal(pc, a["votes"])


def test_pq_sets_and_output_match_reference(oracle):
    g = _load("pq_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, kmax, mode, qb = g[p + "params"]
        ng, nl, kmax, mode, qb = int(ng), int(nl), int(kmax), int(mode), int(qb)
        q, k, v = g[p + "q"], g[p + "k"], g[p + "v"]
        N = q.shape[1]
        sm = 1.0 / math.sqrt(q.shape[-1])
        votes, bits, wv = g[p + "votes"], g[p + "bits"], g[p + "wvotes"]
        res = oracle.build_sets_pq(votes, bits, wv, ng, nl, 32, kmax, qb, mode)
        compare_pq_sets(dict(zip(PQ_SET_NAMES, res)), {k_: g[p + k_] for k_ in PQ_SET_NAMES},
                        pq_rank_values(votes, wv, mode), N)
        # Kernel C given the reference's own sets
        out = oracle.gather_attn_mask(q, k, v, oracle.F32, g[p + "idx"], g[p + "newpos_k"],
                                      g[p + "newpos_q"], g[p + "mask"], g[p + "inv_freq_c"], 1.0, sm,
                                      32, kmax, 64, qb)
        np.testing.assert_allclose(out, g[p + "out"], atol=2e-5, rtol=1e-5)
        # end to end against the reference's independent torch golden.  Not for freq ranking
        # under overflow (the choice among tied vote counts is torch.topk's, and differs between
        # the reference's own two paths) and not for margin ranking (pq_attention_torch ranks by
        # expmass whatever select_score says, perquery.py:594-598, unlike the kernel path)
        if p + "out_torch" in g.files and (mode == 2 or not g[p + "overflow"].any()):
            full = oracle.shared_pq_attention(q, k, v, oracle.F32, g[p + "tau"], g[p + "inv_freq_a"],
                                              g[p + "inv_freq_c"], float(psa), float(rsa), sm, ng, nl,
                                              32, kmax, 64, qb, ["freq", "margin", "expmass"][mode])
            np.testing.assert_allclose(full[0], g[p + "out_torch"], atol=2e-5, rtol=1e-5)


def test_pqstream_matches_reference(oracle):
    g = _load("pqstream_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, bn, full, skip = g[p + "params"]
        q, k, v = g[p + "q"], g[p + "k"], g[p + "v"]
        out, span, kept, blocks, skipped, _ = oracle.pqstream(
            q, k, v, oracle.F32, g[p + "tau"], g[p + "inv_freq_a"], g[p + "inv_freq_c"], float(psa),
            float(rsa), None, int(ng), int(nl), 32, int(bn), "full" if full else "max", bool(skip))
        assert np.array_equal(span, g[p + "span"]), i
        assert np.array_equal(kept, g[p + "kept"]), i
        assert np.array_equal(blocks, g[p + "blocks"]), i
        assert np.array_equal(skipped, g[p + "skipped"]), i
        np.testing.assert_allclose(out, g[p + "out"], atol=2e-5, rtol=1e-5)
        np.testing.assert_allclose(out, g[p + "out_torch"], atol=2e-5, rtol=1e-5)
    # the skip path and the no-skip path were both exercised
    assert float(g["c3_skipped"].sum()) > 0 and float(g["c4_skipped"].sum()) == 0


def test_pqstream_full_advance_is_dense_rope_attention(oracle):
    """tau=inf with advance="full": every causal key is kept, d advances by the slots each block
    occupies, so npq - npk = qpos - j and the kernel is dense causal attention with base RoPE
    (pqstream_kernel.py:291-302).  Checked in float64 with complex rotations."""
    rng = np.random.default_rng(5)
    H, N, D = 1, 150, 64
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    v = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = (1.0 / (10000.0 ** (np.arange(0, D, 2) / D))).astype(np.float32)
    out, span, kept, blocks, skipped, _ = oracle.pqstream(
        q, k, v, oracle.F32, np.full(H, np.inf, np.float32), invf * 0.5, invf, 0.7, 1.3, None, 4, 8,
        32, 32, "full", True)
    half = D // 2
    pos = np.arange(N)
    rot = np.exp(1j * pos[:, None] * invf.astype(np.float64)[None, :])
    qc = (q[0, :, :half] + 1j * q[0, :, half:]) * rot
    kc = (k[0, :, :half] + 1j * k[0, :, half:]) * rot
    s = (qc[:, None, :] * np.conj(kc[None, :, :])).real.sum(-1) / math.sqrt(D)
    s = np.where(pos[:, None] >= pos[None, :], s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    ref = w @ v[0].astype(np.float64)
    np.testing.assert_allclose(out[0], ref, atol=2e-4, rtol=1e-4)
    assert np.array_equal(kept[0], pos + 1)
    nt = (N + 31) // 32
    assert np.array_equal(span[0], np.minimum(np.arange(nt) * 32 + 32, N).astype(np.float32))
