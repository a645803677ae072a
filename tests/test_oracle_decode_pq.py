"""CPU oracle of the per-query (PQ) selection rule, pinned to the reference's own functions.

The rule is _decode_build_sets_pq (shared_selection_triton_perquery.py:651-720): per query,
keep = s >= fl(max - tau) plus the forced global / local / self keys; above k_max the forced keys
plus the top-(k_max - n_forced) others by score (an exact budget); positions are dense ranks
over the final set.  It is the decode rule of the per-query file and, run at every position, its
prefill_mode="perquery" prefill (config 3: "capped at 2048 keys per query by score rank").

  * decode_build_sets_pq == the reference on 11 crafted score rows (cap, deep cap, ties at the
    cut, budget 0, all keys forced, a single key, k_max > M, no forced window, tau 0 / tight /
    wide) -- tests/golden/decode_pq_sets_golden.npz; among equal scores at the cut the reference's
    torch.topk choice is unspecified, so there only the tie members may differ;
  * the sets the reference built from its Triton scores and from its torch scores, and both
    attends (_decode_attend_torch_pq / _decode_attend_kernelC_pq) on them;
  * the per-query prefill (every position P over the cache prefix K[:, :P + 1]) in the batched
    form -- tests/golden/prefill_pq_perquery_golden.npz;
  * closed forms: every key kept -> dense ranks equal positions; under the cap the set is the
    forced keys plus the best-scored others, restated with numpy's stable argsort.
"""
import math
import os

import numpy as np

from oracle import sta_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _same_up_to_ties(idx, ref_idx, s, M, forced):
    """Sets equal, or differing only among keys of one score value v that no common non-forced
    kept key undercuts (the topk tie at the cut); returns the number of rows with a tie
    difference.  forced: the set of forced keys."""
    nd = 0
    for r in range(idx.shape[0]):
        a = set(idx[r][idx[r] < M].tolist())
        b = set(ref_idx[r][ref_idx[r] < M].tolist())
        if a == b:
            continue
        nd += 1
        assert len(a) == len(b), r
        diff = a ^ b
        vals = {float(s[r, j]) for j in diff}
        assert len(vals) == 1, (r, sorted(diff)[:8])
        v = vals.pop()
        assert all(float(s[r, j]) >= v for j in (a & b) - forced), r
    return nd


def test_decode_build_sets_pq_matches_reference_goldens():
    g = _load("decode_pq_sets_golden.npz")
    ties = 0
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ng, nl, km = (int(x) for x in g[p + "params"])
        s = g[p + "scores"]
        H, M = s.shape
        idx, npk, npq, size, us, ov = orc.decode_build_sets_pq(s[:, None, :], g[p + "tau"], qp, ng, nl, km)
        idx, npk, npq = idx[:, 0], npk[:, 0], npq[:, 0]
        ref_idx = g[p + "idx"]
        forced = set(range(min(ng, M))) | set(range(max(0, qp - nl + 1), qp + 1))
        nd = _same_up_to_ties(idx, ref_idx, s, M, forced)
        ties += nd
        if nd == 0:
            assert np.array_equal(idx.astype(np.int64), ref_idx), i
            assert np.array_equal(npk, g[p + "newpos_k"]), i
        assert np.array_equal(npq, g[p + "newpos_q"]), i
        # dense ranks: slot r holds rank r; the query itself is the last kept key
        valid = idx < M
        assert np.array_equal(npk[valid], np.nonzero(valid)[1].astype(np.float32)), i
        assert np.array_equal(size, valid.sum(-1)[:, None]), i
        # measurement counters: |keep| and the overflow flag, recomputed from the scores
        thr = (s.max(-1) - g[p + "tau"]).astype(np.float32)
        assert np.array_equal(us[:, 0], (s >= thr[:, None]).sum(-1)), i
    assert ties <= 2       # only the quantised-score case has ties at the cut


def test_decode_pq_scores_sets_and_attends_match_reference():
    g = _load("decode_pq_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, km, sm = g[p + "params"]
        qp, ng, nl, km = int(qp), int(ng), int(nl), int(km)
        q, k, v = g[p + "q"], g[p + "k"], g[p + "v"]
        ia, ic = g[p + "inv_freq_a"], g[p + "inv_freq_c"]
        H, M = k.shape[0], k.shape[1]
        s = orc.decode_scores(q[:, None, :], k, orc.F32, ia, float(ps), float(rs), float(sm), qp)
        ref = g[p + "scores_triton"]
        assert np.max(np.abs(s[:, 0] - ref)) <= 2e-6 * max(1.0, float(np.abs(ref).max())), i
        taus = np.full(H, tau, np.float32)
        # sets from the reference's own Triton scores: equal
        idx, npk, npq, *_ = orc.decode_build_sets_pq(ref[:, None, :], taus, qp, ng, nl, km)
        assert np.array_equal(idx[:, 0].astype(np.int64), g[p + "idx"]), i
        assert np.array_equal(npk[:, 0], g[p + "newpos_k"]) and np.array_equal(npq[:, 0], g[p + "newpos_q"]), i
        # sets from the oracle's scores against the reference's torch-score sets
        idx2, *_ = orc.decode_build_sets_pq(s, taus, qp, ng, nl, km)
        assert np.array_equal(idx2[:, 0].astype(np.int64), g[p + "idx_torch_scores"]), i
        # both attends: base RoPE (inv_freq_c, scale 1) at the dense ranks
        for causal, name in ((False, "out_torch"), (True, "out_kernelc")):
            out = orc.decode_attend(q[:, None, :], k, v, orc.F32, ic, 1.0, float(sm), qp, idx, npk, npq,
                                    causal=causal)[:, 0]
            np.testing.assert_allclose(out, g[p + name], atol=2e-5, rtol=2e-5, err_msg=f"{i} {name}")


def test_perquery_prefill_matches_reference_loop():
    """prefill_mode="perquery": every position P selects over K[:, :P + 1] (perquery.py:905-924);
    the batched oracle (Q = N queries over one cache of N keys) reproduces the loop."""
    g = _load("prefill_pq_perquery_golden.npz")
    ps, rs, tau, ng, nl, km, sm = g["params"]
    ng, nl, km = int(ng), int(nl), int(km)
    q, k, v = g["q"], g["k"], g["v"]
    H, N, D = q.shape
    s = orc.decode_scores(q, k, orc.F32, g["inv_freq_a"], float(ps), float(rs), float(sm), 0)
    idx, npk, npq, size, us, ov = orc.decode_build_sets_pq(s, np.full(H, tau, np.float32), 0, ng, nl, km)
    # the reference's torch scores and these fp32 dots differ by ulps: sets may differ only at
    # keys within 1e-5 of a row's threshold or cut; count such rows and check the rest exactly
    ref_idx = g["idx"]
    same = np.all(idx.astype(np.int64) == ref_idx, axis=-1)
    assert same.mean() > 0.99, same.mean()
    for h, i in np.argwhere(~same):
        a = set(idx[h, i][idx[h, i] <= i].tolist())
        b = set(ref_idx[h, i][ref_idx[h, i] <= i].tolist())
        row = s[h, i, :i + 1]
        thr = np.float32(row.max() - tau)
        kept = sorted(a & b, key=lambda j: row[j])
        cut = row[kept[0]] if kept else thr
        for j in a ^ b:
            assert min(abs(row[j] - thr), abs(row[j] - cut)) < 1e-5, (h, i, j)
    assert np.array_equal(npk[same], g["newpos_k"][same]) and np.array_equal(npq[same], g["newpos_q"][same])
    out = orc.decode_attend(q, k, v, orc.F32, g["inv_freq_c"], 1.0, float(sm), 0, idx, npk, npq)
    np.testing.assert_allclose(out[same], g["out"][same], atol=2e-5, rtol=2e-5)
    assert ov.any() and (~ov).any()


def test_closed_forms():
    rng = np.random.default_rng(4)
    H, Q, M, km, ng, nl = 2, 5, 400, 60, 8, 8
    s = rng.standard_normal((H, Q, M)).astype(np.float32)
    q0 = M - Q
    # every key kept: tau = inf and k_max >= M -> slot r holds key r, dense ranks = positions
    idx, npk, npq, size, us, ov = orc.decode_build_sets_pq(s, np.full(H, np.inf, np.float32), q0, ng, nl, M)
    for i in range(Q):
        m = M - (Q - 1 - i)
        assert np.array_equal(idx[:, i, :m], np.broadcast_to(np.arange(m), (H, m)))
        assert np.array_equal(npk[:, i, :m], np.broadcast_to(np.arange(m, dtype=np.float32), (H, m)))
        assert np.all(npq[:, i] == q0 + i) and not ov[:, i].any()
    # the cap: forced keys + the best-scored others, by a stable argsort
    idx, npk, npq, size, us, ov = orc.decode_build_sets_pq(s, np.full(H, 3.0, np.float32), q0, ng, nl, km)
    for h in range(H):
        for i in range(Q):
            m, p = M - (Q - 1 - i), q0 + i
            row = s[h, i, :m]
            forced = np.zeros(m, bool)
            forced[:ng] = True
            forced[max(0, p - nl + 1):p + 1] = True
            keep = row >= np.float32(row.max() - np.float32(3.0))
            kp = keep | forced
            if kp.sum() > km:
                cand = np.nonzero(kp & ~forced)[0]
                order = cand[np.argsort(-row[cand], kind="stable")]
                fin = forced.copy()
                fin[order[:km - forced.sum()]] = True
            else:
                fin = kp
            want = np.nonzero(fin)[0][:km]
            got = idx[h, i][idx[h, i] < m]
            assert np.array_equal(got, want), (h, i)
            assert npq[h, i] == fin.sum() - 1
