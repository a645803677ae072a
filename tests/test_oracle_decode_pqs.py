"""CPU oracle of PQ Stream's per-query decode rule, pinned to the reference's own functions.

The rule is _decode_build_sets_pqs (pqstream_kernel.py:695-797): per query, every threshold passer
plus the forced global / local / self keys (no cap), at streamed positions -- blocks of block_n
keys aligned at 0, walked from the query backwards, a key sitting at the kept count of the more
recent blocks plus its natural offset inside its block.  The attend is base RoPE at those
positions with the query at 0.

  * decode_build_sets_pqs == the reference bit for bit (idx, newpos_k including -0 for the query,
    newpos_q) on 9 crafted score rows (block_n 32 / 64, sparse blocks, ties, all keys forced, a
    single key, a partial last block, no forced window, a long row) --
    tests/golden/decode_pqs_sets_golden.npz;
  * the composed decode (the reference's torch scores, both attends);
  * the per-query prefill loop (prefill_mode="perquery") in the batched form;
  * closed form: tau = inf keeps every key, and then the streamed distance of key j is q_pos - j.
"""
import os

import numpy as np

from oracle import sta_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_decode_build_sets_pqs_matches_reference_goldens():
    g = _load("decode_pqs_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ng, nl, bn = (int(x) for x in g[p + "params"])
        s = g[p + "scores"]
        ref_idx = g[p + "idx"]
        idx, npk, npq, size, span, skp = orc.decode_build_sets_pqs(s[:, None, :], g[p + "tau"], qp, ng, nl, bn,
                                                                   k_max=ref_idx.shape[-1])
        assert np.array_equal(idx[:, 0].astype(np.int64), ref_idx), i
        assert np.array_equal(npk[:, 0].view(np.uint32), g[p + "newpos_k"].view(np.uint32)), i
        assert np.array_equal(npq[:, 0], g[p + "newpos_q"]), i
        M = s.shape[1]
        assert np.array_equal(size[:, 0], (ref_idx < M).sum(-1)), i


def test_decode_pqs_composed_matches_reference():
    g = _load("decode_pqs_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, bn, sm = g[p + "params"]
        qp, ng, nl, bn = int(qp), int(ng), int(nl), int(bn)
        q, k, v, invf = g[p + "q"], g[p + "k"], g[p + "v"], g[p + "inv_freq"]
        H, M = k.shape[0], k.shape[1]
        s = orc.decode_scores(q[:, None, :], k, orc.F32, invf, float(ps), float(rs), float(sm), qp)
        idx, npk, npq, *_ = orc.decode_build_sets_pqs(s, np.full(H, tau, np.float32), qp, ng, nl, bn,
                                                      k_max=g[p + "idx"].shape[-1])
        assert np.array_equal(idx[:, 0].astype(np.int64), g[p + "idx"]), i
        assert np.array_equal(npk[:, 0], g[p + "newpos_k"]), i
        for causal, name in ((False, "out_torch"), (True, "out_triton")):
            out = orc.decode_attend(q[:, None, :], k, v, orc.F32, invf, 1.0, float(sm), qp, idx, npk, npq,
                                    causal=causal)[:, 0]
            np.testing.assert_allclose(out, g[p + name], atol=2e-5, rtol=2e-5, err_msg=f"{i} {name}")


def test_pqs_perquery_prefill_matches_reference_loop():
    g = _load("prefill_pqs_perquery_golden.npz")
    ps, rs, tau, ng, nl, bn, sm = g["params"]
    ng, nl, bn = int(ng), int(nl), int(bn)
    q, k, v = g["q"], g["k"], g["v"]
    H, N, D = q.shape
    s = orc.decode_scores(q, k, orc.F32, g["inv_freq"], float(ps), float(rs), float(sm), 0)
    idx, npk, npq, size, span, skp = orc.decode_build_sets_pqs(s, np.full(H, tau, np.float32), 0, ng, nl, bn)
    same = size == g["set_size"]
    assert same.mean() > 0.99
    out = orc.decode_attend(q, k, v, orc.F32, g["inv_freq"], 1.0, float(sm), 0, idx, npk, npq)
    np.testing.assert_allclose(out[same], g["out"][same], atol=2e-5, rtol=2e-5)


def test_every_key_kept_streams_natural_distances():
    rng = np.random.default_rng(2)
    H, Q, M, bn = 2, 3, 300, 32
    s = rng.standard_normal((H, Q, M)).astype(np.float32)
    q0 = M - Q
    idx, npk, npq, size, span, skp = orc.decode_build_sets_pqs(s, np.full(H, np.inf, np.float32), q0, 4, 4, bn)
    for i in range(Q):
        m = M - (Q - 1 - i)
        assert np.array_equal(idx[:, i, :m], np.broadcast_to(np.arange(m), (H, m)))
        assert np.array_equal(-npk[:, i, :m], np.broadcast_to((q0 + i - np.arange(m)).astype(np.float32), (H, m)))
        assert np.all(span[:, i] == q0 + i) and np.all(skp[:, i] == 0)
