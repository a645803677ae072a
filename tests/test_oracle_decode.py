"""CPU oracle of the decode path, pinned to the reference's own decode functions.

  * decode_build_sets == _decode_build_sets (exact_2.py:527-604) bit for bit on 13 crafted score
    tensors (cap, tie-inclusive cuts, budget <= 0, pct_decode < 100, q_pos inside the cache,
    single key, all keys forced) -- tests/golden/decode_sets_golden.npz;
  * decode_scores against the Triton _decode_select_kernel (exact_2.py:235-271) run under the
    interpreter, and the sets the reference built from those scores;
  * decode_attend against _decode_attend_torch (:608-623) and, with causal=True, against
    _decode_attend_kernelC (:626-655);
  * the batched form (Q queries over one cache) against spi_forward's per-token loop
    (:743-762) -- tests/golden/decode_sequence_golden.npz;
  * closed forms: every key kept -> dense ranks (newpos = position) and the plain softmax
    attention under native RoPE.
"""
import math
import os

import numpy as np

from oracle import sta_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_decode_build_sets_matches_reference_goldens():
    g = _load("decode_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, ng, nl, km, pctd = g[p + "params"]
        s = g[p + "scores"]
        idx, npk, npq, size = orc.decode_build_sets(s[:, None, :], g[p + "tau"], int(qp), float(ps), int(ng),
                                                     int(nl), int(km), float(pctd))
        assert np.array_equal(idx[:, 0].astype(np.int64), g[p + "idx"]), i
        assert _bits_equal(npk[:, 0], g[p + "newpos_k"]), i
        assert _bits_equal(npq[:, 0], g[p + "newpos_q"]), i
        M = s.shape[1]
        # set_size counts the whole set; the reference keeps its first k_max positions
        assert np.array_equal(np.minimum(size[:, 0], int(km)), (g[p + "idx"] < M).sum(-1)), i


def test_decode_scores_sets_and_attend_match_reference():
    g = _load("decode_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, km, pctd, sm = g[p + "params"]
        qp, ng, nl, km = int(qp), int(ng), int(nl), int(km)
        q, k, v, invf = g[p + "q"], g[p + "k"], g[p + "v"], g[p + "inv_freq"]
        H, M = k.shape[0], k.shape[1]
        s = orc.decode_scores(q[:, None, :], k, orc.F32, invf, float(ps), float(rs), float(sm), qp)[:, 0]
        ref = g[p + "scores_triton"]
        assert np.max(np.abs(s - ref)) <= 2e-6 * max(1.0, float(np.abs(ref).max())), i
        taus = np.full(H, tau, np.float32)
        # sets from the reference's own scores: bit for bit
        idx, npk, npq, _ = orc.decode_build_sets(ref[:, None, :], taus, qp, float(ps), ng, nl, km, float(pctd))
        assert np.array_equal(idx[:, 0].astype(np.int64), g[p + "idx"]), i
        assert _bits_equal(npk[:, 0], g[p + "newpos_k"]) and _bits_equal(npq[:, 0], g[p + "newpos_q"]), i
        # sets from the oracle's scores equal those of the reference's torch scores (no key of
        # these inputs lies within the scores' rounding of a cut)
        idx2, _, _, _ = orc.decode_build_sets(s[:, None, :], taus, qp, float(ps), ng, nl, km, float(pctd))
        assert np.array_equal(idx2[:, 0].astype(np.int64), g[p + "idx_torch_scores"]), i
        for causal, name in ((False, "out_torch"), (True, "out_kernelc")):
            out = orc.decode_attend(q[:, None, :], k, v, orc.F32, invf, float(rs), float(sm), qp,
                                    g[p + "idx"][:, None, :], g[p + "newpos_k"][:, None, :],
                                    g[p + "newpos_q"][:, None], causal=causal)[:, 0]
            assert np.max(np.abs(out - g[p + name])) < 2e-5, (i, name)
        # q_pos inside the cache: the two attends differ (keys past q_pos), as in the reference
        if qp < M - 1:
            assert np.max(np.abs(g[p + "out_torch"] - g[p + "out_kernelc"])) > 1e-3


def test_decode_batched_matches_per_token_loop():
    g = _load("decode_sequence_golden.npz")
    P0, Q, ps, rs, tau, ng, nl, km, pctd, sm = g["params"]
    P0, Q, ng, nl, km = int(P0), int(Q), int(ng), int(nl), int(km)
    q, k, v, invf = g["q"], g["k"], g["v"], g["inv_freq"]
    H, M = k.shape[0], k.shape[1]
    assert M == P0 + Q
    s = orc.decode_scores(q, k, orc.F32, invf, float(ps), float(rs), float(sm), P0)
    for i in range(Q):   # query i sees exactly the prefix [0, P0 + i]
        assert np.all(np.isnan(s[:, i, P0 + i + 1:])) and not np.any(np.isnan(s[:, i, :P0 + i + 1]))
    idx, npk, npq, _ = orc.decode_build_sets(s, np.full(H, tau, np.float32), P0, float(ps), ng, nl, km,
                                             float(pctd))
    assert np.array_equal(idx.astype(np.int64), g["idx"])   # sentinel P + 1 per query
    assert _bits_equal(npk, g["newpos_k"]) and _bits_equal(npq, g["newpos_q"])
    out = orc.decode_attend(q, k, v, orc.F32, invf, float(rs), float(sm), P0, idx, npk, npq)
    assert np.max(np.abs(out - g["out"])) < 2e-5


def _dense_reference(q, k, v, invf, qpos, sm):
    """Softmax attention of one query over keys 0..M-1 at native RoPE positions, float64."""
    def rot(x, pos):
        ang = np.outer(np.asarray(pos, np.float64), invf.astype(np.float64))
        h = x.shape[-1] // 2
        x1, x2 = x[..., :h].astype(np.float64), x[..., h:].astype(np.float64)
        return np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)], -1)
    qr = rot(q[None, :], [qpos])[0]
    kr = rot(k, np.arange(k.shape[0]))
    s = kr @ qr * sm
    w = np.exp(s - s.max())
    return (w[:, None] * v.astype(np.float64)).sum(0) / w.sum()


def test_decode_everything_kept_is_dense_attention():
    rng = np.random.default_rng(5)
    H, M, D = 2, 300, 64
    q = rng.standard_normal((H, 1, D)).astype(np.float32)
    k = rng.standard_normal((H, M, D)).astype(np.float32)
    v = rng.standard_normal((H, M, D)).astype(np.float32)
    invf = (1.0 / (10000.0 ** (np.arange(0, D, 2) / D))).astype(np.float32)
    sm = 1.0 / math.sqrt(D)
    s = orc.decode_scores(q, k, orc.F32, invf, 0.5, 1.0, sm, M - 1)
    # tau = inf keeps every key; with k_max >= M nothing is capped; ranks are the positions
    idx, npk, npq, size = orc.decode_build_sets(s, np.full(H, np.inf, np.float32), M - 1, 0.5, 4, 4, M + 7)
    assert np.all(size == M)
    assert np.array_equal(idx[:, 0, :M], np.broadcast_to(np.arange(M), (H, M)))
    assert np.all(idx[:, 0, M:] == M)
    assert np.array_equal(npk[:, 0, :M], np.broadcast_to(np.arange(M, dtype=np.float32), (H, M)))
    assert np.all(npq == M - 1)
    out = orc.decode_attend(q, k, v, orc.F32, invf, 1.0, sm, M - 1, idx, npk, npq)
    for h in range(H):
        ref = _dense_reference(q[h, 0], k[h], v[h], invf, M - 1, sm)
        assert np.max(np.abs(out[h, 0] - ref)) < 1e-5


def test_decode_cap_keeps_forced_and_top_scores():
    """Under the cap the set is the forced keys plus the best-scored others (distinct scores)."""
    rng = np.random.default_rng(9)
    H, M, km, ng, nl = 3, 400, 50, 5, 7
    s = rng.permutation(M * H).reshape(H, 1, M).astype(np.float32) / 7.0
    idx, _, _, size = orc.decode_build_sets(s, np.full(H, 1e9, np.float32), M - 1, 1.0, ng, nl, km)
    for h in range(H):
        forced = set(range(ng)) | set(range(M - nl, M))
        others = [j for j in np.argsort(-s[h, 0]) if j not in forced][:km - len(forced)]
        assert set(idx[h, 0].tolist()) == forced | set(int(j) for j in others)
        assert size[h, 0] == km
