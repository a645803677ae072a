"""CPU tests that pin the chunk-granular selection oracle (oracle/sta_oracle_chunk.c).

The reference module (shared_selection_triton_chunked.py) imports chunk_recall_core, which is not
in the reference tree, so it cannot run here and no fixture of its outputs exists; parity is
pinned by what the reference's own text fixes and by properties of the rule:

  * budget arithmetic: the worked numbers of its docstrings (chunked.py:25-36, 132-141: 7 forced
    chunks / 112 slots and n_chunk = 249 at C = 16, 3 chunks / 384 slots at C = 128);
  * the prefill rule (_build_sets_chunk, :149-243, forced chunks as chunk_attention_torch states
    them, :368-376) as properties of every (head, tile) on random votes: the forced visible chunks
    are kept, min(n_chunk, candidates) others are, every kept candidate chunk is valued at least as
    high as every dropped one (equal values: the lower chunk index wins), the kept keys are exactly
    those chunks' keys up to the tile's last query, dense ranks, sentinels, the pooled mask, the
    query ranks, usize and the passers counter -- for freq / expmass, sum / mean, a nonzero
    q_pos_base and a ragged last tile;
  * the decode rule (_decode_build_sets_chunk, :411-489) equals the prefill rule with one-query
    tiles built from the same scores (two restatements through different inputs);
  * known answer: with every chunk selectable (n_chunk >= nC) the kept set of every tile is every
    causal key, the ranks are the positions, and the composed attention is dense causal RoPE
    attention (float64 numpy).
"""
import math

import numpy as np
import pytest

from oracle import sta_oracle as orc


def test_budget_arithmetic_matches_the_reference_docstrings():
    assert orc.n_forced_chunks(16, 32, 32, 32) == 7                     # 7 chunks = 112 slots
    assert orc.derive_n_chunk(4096, 16, 32, 32, 32) == 249
    assert orc.n_forced_chunks(128, 32, 32, 32) == 3                    # 3 chunks = 384 slots


def _chunk_values(vr, wr, C, N, weighted, mean):
    nC = (N + C - 1) // C
    val = np.zeros(nC, np.float64)
    for c in range(nC):
        seg = slice(c * C, min(N, (c + 1) * C))
        cand = vr[seg] > 0
        x = (wr[seg] if weighted else vr[seg]).astype(np.float64)
        m = x[cand].sum()
        val[c] = m / max(1, int(cand.sum())) if mean else m
    return val


def _check_tile(vr, wr, idx, npk, npq, mask, us, ks, pk, t, T, C, N, k_max, n_chunk, q_pos_base, ng, nl,
                weighted, mean):
    nC = (N + C - 1) // C
    r0 = q_pos_base + t * T
    last_q = r0 + T - 1
    lim = min(last_q, N - 1)
    vis = np.arange(nC) * C <= last_q
    glob = np.arange(nC) < (ng + C - 1) // C
    loc = (np.arange(nC) >= max(0, r0 - nl + 1) // C) & (np.arange(nC) <= last_q // C)
    forced = (glob | loc) & vis
    cand = vis & ~forced
    kept_keys = idx[idx < N]
    assert np.all(np.diff(kept_keys) > 0) and len(kept_keys) == ks
    assert np.all(idx[ks:] == N) and np.all(npk[ks:] == 0) and np.array_equal(npk[:ks], np.arange(ks))
    assert np.array_equal(mask, np.where(np.arange(k_max) < ks, -1, 0))
    K = np.zeros(nC, bool)
    K[np.unique(kept_keys // C)] = True
    assert np.all(K[forced]) and not np.any(K & ~vis)
    sel = K & cand
    assert sel.sum() == min(n_chunk, cand.sum())
    val = _chunk_values(vr, wr, C, N, weighted, mean)
    if sel.any() and (cand & ~K).any():
        lo_sel = val[sel].min()
        hi_drop = val[cand & ~K].max()
        assert lo_sel >= hi_drop
        if lo_sel == hi_drop:      # equal values: the selected ones have the lower chunk indices
            assert np.flatnonzero(sel & (val == lo_sel)).max() < np.flatnonzero(cand & ~K & (val == lo_sel)).min()
    expect = np.array([j for j in range(lim + 1) if K[j // C]], np.int64)
    assert np.array_equal(kept_keys, expect)
    for i in range(T):
        qp = min(r0 + i, N - 1)
        assert npq[i] == np.sum(expect <= qp) - 1
    assert us == int(np.sum(vr[:min(N, last_q + 1)] > 0))
    assert pk == int(np.sum(vr[expect] > 0))


@pytest.mark.parametrize("score,agg,q_pos_base", [("freq", "sum", 0), ("expmass", "sum", 0),
                                                   ("expmass", "mean", 0), ("margin", "sum", 40),
                                                   ("freq", "mean", 7)])
def test_prefill_rule_properties(score, agg, q_pos_base):
    rng = np.random.default_rng(hash((score, agg, q_pos_base)) % 2**32)
    H, N, T, C, ng, nl, n_chunk = 2, 333, 32, 16, 20, 24, 5
    nt = (N + T - 1) // T
    k_max = (orc.n_forced_chunks(C, ng, nl, T) + n_chunk) * C
    votes = np.zeros((H, nt, N), np.int32)
    wv = np.zeros((H, nt, N), np.float32)
    for t in range(nt):
        hi = min(N, q_pos_base + (t + 1) * T)
        v = rng.integers(0, 4, size=(H, hi)) * (rng.random((H, hi)) < 0.3)
        if score == "freq":                           # integer chunk sums: many ties
            v = v * (rng.random((H, hi)) < 0.5)
        votes[:, t, :hi] = v
        wv[:, t, :hi] = np.where(v > 0, rng.random((H, hi)).astype(np.float32) * v, 0)
    idx, npk, npq, mask, us, ks, pk = orc.build_sets_chunk(votes, wv, ng, nl, T, k_max, C, n_chunk, q_pos_base,
                                                           score, agg)
    assert int(ks.max()) <= k_max
    for h in range(H):
        for t in range(nt):
            _check_tile(votes[h, t], wv[h, t], idx[h, t], npk[h, t], npq[h, t], mask[h, t], us[h, t], ks[h, t],
                        pk[h, t], t, T, C, N, k_max, n_chunk, q_pos_base, ng, nl, score != "freq", agg == "mean")


@pytest.mark.parametrize("score,agg", [("expmass", "sum"), ("freq", "sum"), ("expmass", "mean")])
def test_decode_rule_equals_one_query_tiles(score, agg):
    rng = np.random.default_rng(11)
    H, Q, M, C, ng, nl, n_chunk, k_max = 2, 40, 500, 16, 16, 20, 6, 512
    scores = (rng.standard_normal((H, Q, M)) * 2).astype(np.float32)
    if score == "freq":
        scores = np.round(scores * 2) / 2                              # ties in the keep counts
    tau = np.array([2.0, 3.5], np.float32)
    q_pos0 = M - Q
    idx, npk, npq, ks, pk = orc.decode_build_sets_chunk(scores, tau, q_pos0, ng, nl, k_max, C, n_chunk, score, agg)
    # the prefill rule with tiles of one query at q_pos0 + i, votes / weighted votes of that query
    votes = np.zeros((H, Q, M), np.int32)
    wv = np.zeros((H, Q, M), np.float32)
    for h in range(H):
        for i in range(Q):
            m = q_pos0 + i + 1
            row = scores[h, i, :m]
            mx = row.max()
            keep = row >= np.float32(mx - tau[h])
            votes[h, i, :m] = keep
            wv[h, i, :m] = np.where(keep, np.exp(row - mx), 0).astype(np.float32)
    ref = orc.build_sets_chunk(votes, wv, ng, nl, 1, k_max, C, n_chunk, q_pos0, score, agg)
    for h in range(H):
        for i in range(Q):
            m = q_pos0 + i + 1
            k = ks[h, i]
            assert k == ref[5][h, i]
            assert np.array_equal(idx[h, i, :k], ref[0][h, i, :k]) and np.all(idx[h, i, k:] == m)
            assert np.array_equal(npk[h, i], ref[1][h, i])
            assert npq[h, i] == ref[2][h, i, 0]
            assert pk[h, i] == ref[6][h, i]
            assert q_pos0 + i in set(idx[h, i, :k].tolist())


def _rope64(x, pos, invf):
    ang = np.asarray(pos, np.float64)[..., None] * invf.astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h].astype(np.float64), x[..., h:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def test_every_chunk_selectable_is_dense_causal_attention():
    rng = np.random.default_rng(3)
    H, N, D, C = 2, 200, 64, 16
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    v = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / D))).astype(np.float32)
    nC = (N + C - 1) // C
    k_max = (orc.n_forced_chunks(C, 16, 16, 32) + nC) * C
    out, us, ks, ex = orc.shared_chunk_attention(q, k, v, orc.F32, np.full(H, 1.0, np.float32), invf, invf, 0.5,
                                                 1.0, n_global=16, n_local=16, k_max=k_max, chunk_size=C,
                                                 n_chunk=nC)
    nt = (N + 31) // 32
    for t in range(nt):
        lim = min(N, (t + 1) * 32)
        assert np.all(ks[:, t] == lim)
        assert np.array_equal(ex["newpos_q"][:, t], np.broadcast_to(np.minimum(np.arange(t * 32, t * 32 + 32), N - 1),
                                                                  (H, 32)))
    for h in range(H):
        qr = _rope64(q[h], np.arange(N), invf)
        kr = _rope64(k[h], np.arange(N), invf)
        s = qr @ kr.T / math.sqrt(D)
        s = np.where(np.tril(np.ones((N, N), bool)), s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        ref = (p / p.sum(-1, keepdims=True)) @ v[h].astype(np.float64)
        np.testing.assert_allclose(out[h], ref, atol=2e-5, rtol=2e-5)
