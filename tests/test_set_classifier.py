"""CPU tests of the set-level parity classifier the GPU tests use (tests/parity_helpers.py).

The GPU side is played by the oracle itself with votes changed on the CPU: changes at band keys
must be accepted and counted (the key itself, keys moved by the shifted cut, keys moved by the
truncation boundary), and a change planted at a key outside the band must be rejected.
"""
import math

import numpy as np
import pytest

from parity_helpers import classify_set_diffs, classify_pq_set_diffs, pq_rank_values


def _case(oracle, band_eps):
    rng = np.random.default_rng(11)
    H, N, D, T = 2, 768, 64, 64
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)
    a = oracle.select_vote(q, k, oracle.F32, np.full(H, 2.5, np.float32), invf, 1.0, 1.0,
                           1.0 / math.sqrt(D), T, band_eps=band_eps, want_band=True)
    return a, T


def _sets(oracle, votes, T, k_max):
    r = oracle.build_sets(votes, 1.0, 8, 8, 30.0, T, k_max, want_cut=True)
    return {"idx": r[0]}, r[9]


@pytest.mark.parametrize("k_max", [64, 200, 4096])
def test_band_flips_are_classified(oracle, k_max):
    a, T = _case(oracle, band_eps=0.05)
    band = a["band"]
    assert band.sum() > 50
    votes_o = a["votes"]
    votes_g = votes_o.copy()
    rng = np.random.default_rng(3)
    hit = np.argwhere(band > 0)
    pick = hit[rng.choice(len(hit), size=min(40, len(hit)), replace=False)]
    for h, t, j in pick:                                 # each band key loses or gains one vote
        votes_g[h, t, j] = max(0, votes_g[h, t, j] + (1 if rng.random() < 0.5 else -1))
    sg, cg = _sets(oracle, votes_g, T, k_max)
    so, co = _sets(oracle, votes_o, T, k_max)
    c = classify_set_diffs(votes_g, votes_o, band, sg, so, cg, co, T, k_max, 8, 8)
    assert c["keys"] == c["band"] + c["cut"] + c["trunc"]
    assert c["tiles_differ"] > 0


def test_planted_flip_outside_band_fails(oracle):
    a, T = _case(oracle, band_eps=1e-3)
    band = a["band"]
    votes_o = a["votes"]
    so, co = _sets(oracle, votes_o, T, 4096)
    # a kept, non-forced key outside the band loses all its votes: a real selection error
    h, t = 0, 8
    j_all = np.arange(votes_o.shape[-1])
    forced = (j_all < 8) | ((j_all >= t * T - 7) & (j_all <= t * T + T - 1))
    cand = np.nonzero((band[h, t] == 0) & (votes_o[h, t] >= co[h, t]) & (votes_o[h, t] > 0) & ~forced)[0]
    j = int(cand[0])
    votes_g = votes_o.copy()
    votes_g[h, t, j] = 0
    sg, cg = _sets(oracle, votes_g, T, 4096)
    with pytest.raises(AssertionError):
        classify_set_diffs(votes_g, votes_o, band, sg, so, cg, co, T, 4096, 8, 8)


def test_pq_classifier(oracle):
    rng = np.random.default_rng(5)
    H, N, D = 1, 512, 64
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)
    a = oracle.select_bits(q, k, oracle.F32, np.full(H, 2.0, np.float32), invf, 1.0, 1.0,
                           1.0 / math.sqrt(D), 32, 0, 2, band_eps=0.05, want_band=True)
    names = ["idx", "newpos_k", "newpos_q", "mask", "usize", "kept_size", "overflow"]
    ro = dict(zip(names, oracle.build_sets_pq(a["votes"], a["bits"], a["wvotes"], 4, 4, 32, 96, 0, 2)))
    # the GPU side: weighted votes perturbed at the fp32-summation level everywhere
    wv = a["wvotes"] * np.float32(1 + 1e-6)
    rg = dict(zip(names, oracle.build_sets_pq(a["votes"], a["bits"], wv, 4, 4, 32, 96, 0, 2)))
    c = classify_pq_set_diffs(a["band"], rg, ro, pq_rank_values(a["votes"], wv, 2),
                              pq_rank_values(a["votes"], a["wvotes"], 2), N)
    assert c["keys"] == c["band"] + c["cut"]
    # a planted error: an unkept key outside the band gets a large weighted vote on the GPU side
    t = int(np.nonzero(ro["overflow"][0])[0][-1])
    row = ro["idx"][0, t]
    kept = set(row[row < N].tolist())
    cand = [j for j in range(8, t * 32 - 40) if j not in kept and a["band"][0, t, j] == 0]
    wv_bad = a["wvotes"].copy()
    wv_bad[0, t, cand[0]] = a["wvotes"][0, t].max() * 2
    rb = dict(zip(names, oracle.build_sets_pq(a["votes"], a["bits"], wv_bad, 4, 4, 32, 96, 0, 2)))
    with pytest.raises(AssertionError):
        classify_pq_set_diffs(a["band"], rb, ro, pq_rank_values(a["votes"], wv_bad, 2),
                              pq_rank_values(a["votes"], a["wvotes"], 2), N)
