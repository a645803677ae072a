"""CPU tests that pin the oracle's weighted ranking of the shared path (select_score "margin" /
"expmass", shared_selection_triton_exact_2.py:126-138, 299-302) before the device is compared
against it.

Pins:
  build_sets with wvotes  -- bit-exact against the reference's own _build_sets on 19 vote /
                             weighted-vote tensors (tests/golden/build_sets_weighted_golden.npz:
                             fallback, measure, truncation, ragged tiles, q_pos_base, pct 0 / 22.5 /
                             100, an empty tile, tied weighted votes and the frequency tiebreak).
  the zero-weight invariant -- all weighted votes 0 ranks by fl(1e-6 votes), a strictly increasing
                             function of the votes, so the sets equal the frequency ranking's.
  select_vote wmode 1 / 2 -- votes equal and weighted votes within a few fp32 ulps of the
                             reference's Kernel A under the Triton interpreter (fp32 inputs).
  the composition         -- sets from the reference's votes / weighted votes bit-exact, and the
                             output given the reference's sets within 2e-5
                             (tests/golden/composed_weighted_golden.npz).
"""
import os

import numpy as np

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SET_NAMES = ["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen", "orig_overflow",
             "kpct_meas", "overflow20"]


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _same(got, ref):
    if ref.dtype == np.float32:
        return np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    return np.array_equal(got.astype(ref.dtype), ref)


def test_weighted_build_sets_matches_reference_goldens(oracle):
    g = _load("build_sets_weighted_golden.npz")
    n = int(g["ncases"])
    assert n >= 19
    for i in range(n):
        p = f"c{i}_"
        ps, ng, nl, pct, T, kmax, qb, meas, _ = g[p + "params"]
        res = oracle.build_sets(g[p + "votes"], float(ps), int(ng), int(nl), float(pct), int(T), int(kmax),
                                int(qb), bool(meas), wvotes=g[p + "wvotes"])
        for name, got in zip(SET_NAMES, res):
            assert _same(got, g[p + name]), (i, name)


def test_zero_weights_rank_like_frequency(oracle):
    g = _load("build_sets_weighted_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        ps, ng, nl, pct, T, kmax, qb, meas, _ = g[p + "params"]
        args = (float(ps), int(ng), int(nl), float(pct), int(T), int(kmax), int(qb), bool(meas))
        votes = g[p + "votes"]
        w = oracle.build_sets(votes, *args, wvotes=np.zeros(votes.shape, np.float32))
        f = oracle.build_sets(votes, *args)
        for name, a, b in zip(SET_NAMES, w, f):
            assert _same(a, b), (i, name)


def test_weighted_votes_match_reference_kernel_a_fp32(oracle):
    g = _load("composed_weighted_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm, wmode = g[p + "params"]
        a = oracle.select_vote(g[p + "q"], g[p + "k"], oracle.F32, g[p + "tau"], g[p + "inv_freq"], float(ps),
                               1.0, float(sm), int(tile), int(qb), wmode=int(wmode))
        assert np.array_equal(a["votes"], g[p + "votes"]), i
        ref = g[p + "wvotes"]
        assert np.array_equal(a["wvotes"] == 0, ref == 0), i
        err = np.abs(a["wvotes"].astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
        assert float(err.max()) < 1e-5, (i, float(err.max()))


def test_weighted_composition_matches_reference_fp32(oracle):
    g = _load("composed_weighted_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm, wmode = g[p + "params"]
        res = oracle.build_sets(g[p + "votes"], float(ps), int(ng), int(nl), float(pct), int(tile), int(kmax),
                                int(qb), False, wvotes=g[p + "wvotes"])
        for name, got in zip(SET_NAMES, res):
            assert _same(got, g[p + name]), (i, name)
        out = oracle.gather_attn(g[p + "q"], g[p + "k"], g[p + "v"], oracle.F32, g[p + "idx"], g[p + "newpos_k"],
                                 g[p + "newpos_q"], g[p + "inv_freq"], 1.0, float(sm), int(tile), int(kmax),
                                 64, int(qb))
        assert np.max(np.abs(out - g[p + "out"])) < 2e-5, i
        # end to end through the oracle's own weighted votes
        o, ss, ks, ch, oo, km, o20, ex = oracle.shared_pi_attention(
            g[p + "q"], g[p + "k"], g[p + "v"], oracle.F32, g[p + "tau"], g[p + "inv_freq"], float(ps), 1.0,
            pct=float(pct), sm_scale=float(sm), n_global=int(ng), n_local=int(nl), tile=int(tile),
            k_max=int(kmax), q_pos_base=int(qb), select_score={1: "margin", 2: "expmass"}[int(wmode)])
        assert np.array_equal(ex["idx"], g[p + "idx"]), i
        assert np.max(np.abs(o - g[p + "out"])) < 2e-5, i
