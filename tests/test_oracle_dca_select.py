"""CPU pins of the config-4 oracle: DCA positions with exact-max selection over the inter-chunk keys.

No reference file combines DCA (dca_kernel.py, dense) with threshold selection; the oracle
composes pinned parts -- DCA's rotations (oracle_dca's tables, pinned to the reference's DCA
prefill in test_oracle_dca.py), Kernel A's keep rule and _build_sets (oracle_build_sets, pinned to
the reference's own vectors in test_oracle.py) -- and these tests pin the composition:
  * tau = inf, pct = 100, k_max >= N keeps every inter key: the output is the dense DCA prefill;
  * N <= 2 L (no inter keys): the output is the dense DCA prefill for any selection parameters;
  * the votes against a float64 brute force of the inter scores (within the 1e-3 band);
  * each tile's sets equal _build_sets applied to that tile's inter votes as its own key axis;
  * the attention given the sets against a float64 brute force over the union of the selected
    inter keys and the local (own + previous chunk) keys.
"""
import math

import numpy as np

from oracle import sta_oracle as orc


def _inputs(seed, H, Hkv, N, D, dt=np.float32):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, N, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, N, D)).astype(np.float32)
    u = rng.standard_normal(D).astype(np.float32)
    u /= np.linalg.norm(u)
    planted = rng.choice(N, size=max(1, N // 50), replace=False)
    k[:, planted] += 3.0 * u
    q += u
    return q, k, v


def _invf(D):
    return (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)


# chunk 320 with local window 64: L = 256, pretraining length 512
S, W, C = 320, 64, 512


def test_infinite_tau_is_dense_dca():
    H, N, D = 2, 1100, 64
    q, k, v = _inputs(1, H, H, N, D)
    invf = _invf(D)
    out, sets, _ = orc.dca_select_attention(q, k, v, orc.F32, invf, S, C, W, np.full(H, np.inf, np.float32),
                                            pct=100.0, k_max=N, n_global=4)
    dense = orc.dca_attention(q, k, v, orc.F32, invf, S, C, W)
    np.testing.assert_allclose(out, dense, atol=1e-5, rtol=1e-5)
    # every inter key of every tile selected
    L = S - W
    for t in range(sets[0].shape[1]):
        c = (t * 64) // L
        ext = (c - 1) * L if c >= 2 else 0
        assert np.all(sets[2][:, t] == ext)


def test_no_inter_keys_is_dense_dca():
    H, N, D = 2, 2 * (S - W), 64
    q, k, v = _inputs(2, H, H, N, D)
    invf = _invf(D)
    out, sets, a = orc.dca_select_attention(q, k, v, orc.F32, invf, S, C, W, np.full(H, 0.5, np.float32),
                                            pct=30.0, k_max=8, n_global=4)
    np.testing.assert_allclose(out, orc.dca_attention(q, k, v, orc.F32, invf, S, C, W), atol=1e-5, rtol=1e-5)
    assert not a["votes"].any() and not sets[2].any()


def _rotated_f64(q, k, invf, N, L, ms):
    """float64 DCA rotations (no dtype rounding): keys at j mod L, queries at the inter position."""
    D = q.shape[-1]
    def rot(x, t):
        ang = np.outer(t, invf.astype(np.float64))
        c, s = np.cos(ang) * ms, np.sin(ang) * ms
        x1, x2 = x[..., :D // 2].astype(np.float64), x[..., D // 2:].astype(np.float64)
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    kr = rot(k, np.arange(N) % L)
    pin = min(2 * L - 1, S)
    qr = rot(q, np.full(N, pin))
    return qr, kr


def test_votes_against_float64_brute_force():
    H, N, D = 1, 1300, 64
    q, k, v = _inputs(3, H, H, N, D)
    invf = _invf(D)
    tau = np.full(H, 2.0, np.float32)
    a = orc.dca_inter_votes(q, k, orc.F32, invf, S, C, W, tau, want_band=True)
    L = S - W
    ms = orc.dca_mscale(N, C)
    qr, kr = _rotated_f64(q[0], k[0], invf, N, L, ms)
    sm = 1.0 / math.sqrt(D)
    nt = (N + 63) // 64
    vb = np.zeros((nt, N), np.int64)
    for t in range(nt):
        c = (t * 64) // L
        ext = (c - 1) * L if c >= 2 else 0
        if not ext:
            continue
        s = (qr[t * 64:t * 64 + 64] @ kr[:ext].T) * sm
        m = s.max(-1, keepdims=True)
        vb[t, :ext] = (s >= m - 2.0).sum(0)
        np.testing.assert_allclose(a["row_max"][0, t * 64:t * 64 + 64], m[:, 0], atol=1e-4)
    d = np.abs(vb - a["votes"][0])
    assert np.all(d <= a["band"][0])
    assert (a["votes"] > 0).sum() > 1000


def test_tile_subset_equals_the_full_evaluation():
    """dca_inter_votes(tiles=...) evaluates only the listed tiles: their votes, band counts and row
    maxima equal the full evaluation's, every other tile keeps zero votes and a NaN row max."""
    H, Hkv, N, D = 2, 1, 1500, 64
    q, k, _ = _inputs(5, H, Hkv, N, D)
    invf = _invf(D)
    tau = np.full(H, 2.5, np.float32)
    full = orc.dca_inter_votes(q, k, orc.F32, invf, S, C, W, tau, want_band=True)
    tiles = [9, 15, 23]
    part = orc.dca_inter_votes(q, k, orc.F32, invf, S, C, W, tau, want_band=True, tiles=tiles)
    nt = (N + 63) // 64
    keep = np.zeros(nt, bool)
    keep[tiles] = True
    rows = np.repeat(keep, 64)[:N]
    assert np.array_equal(part["votes"][:, keep], full["votes"][:, keep])
    assert np.array_equal(part["band"][:, keep], full["band"][:, keep])
    assert not part["votes"][:, ~keep].any() and not part["band"][:, ~keep].any()
    assert np.array_equal(part["row_max"][:, rows], full["row_max"][:, rows])
    assert np.isnan(part["row_max"][:, ~rows]).all()
    assert (full["votes"][:, keep] > 0).sum() > 100


def test_sets_are_build_sets_on_each_tiles_inter_axis():
    H, N, D = 2, 1500, 64
    q, k, v = _inputs(4, H, H, N, D)
    invf = _invf(D)
    a = orc.dca_inter_votes(q, k, orc.F32, invf, S, C, W, np.full(H, 3.0, np.float32))
    km, ng = 96, 8
    sets = orc.dca_build_sets(a["votes"], S, W, ng, 30.0, km)
    L = S - W
    nt = a["votes"].shape[1]
    for h in range(H):
        for t in range(nt):
            c = (t * 64) // L
            ext = (c - 1) * L if c >= 2 else 0
            if not ext:
                assert sets[2][h, t] == 0
                continue
            ref = orc.build_sets(a["votes"][h:h + 1, t:t + 1, :ext], 1.0, ng, 0, 30.0, 64, km, q_pos_base=t * 64)
            assert np.array_equal(sets[0][h, t], ref[0][0, 0]), (h, t)
            for j, name in ((1, 3), (2, 4), (3, 5)):
                assert sets[j][h, t] == ref[name][0, 0], (h, t, name)
    assert (sets[2] > km).any(), "no tile overflows: the cap path is not exercised"


def test_attention_given_sets_against_brute_force():
    H, N, D = 1, 1000, 64
    q, k, v = _inputs(5, H, H, N, D)
    invf = _invf(D)
    out, sets, _ = orc.dca_select_attention(q, k, v, orc.F32, invf, S, C, W, np.full(H, 2.5, np.float32),
                                            pct=30.0, k_max=64, n_global=4)
    L = S - W
    ms = orc.dca_mscale(N, C)
    D2 = D // 2
    def rot(x, t):
        ang = np.outer(np.atleast_1d(t), invf.astype(np.float64))
        c, s = np.cos(ang) * ms, np.sin(ang) * ms
        x1, x2 = x[..., :D2].astype(np.float64), x[..., D2:].astype(np.float64)
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    kr = rot(k[0], np.arange(N) % L)
    sm = 1.0 / math.sqrt(D)
    for i in (5, 300, 700, 999):
        c, t = i // L, i // 64
        lo = (c - 1) * L if c >= 2 else 0
        nsel = min(int(sets[2][0, t]), 64)
        sel = sets[0][0, t, :nsel]
        pid = i % L
        keys, scores = [], []
        for j in sel:
            keys.append(j)
            scores.append(float((rot(q[0, i], min(2 * L - 1, S)) @ kr[j])[0]) * sm)
        for j in range(lo, i + 1):
            pos = pid if j // L == c else min(pid + L, S)
            keys.append(j)
            scores.append(float((rot(q[0, i], pos) @ kr[j])[0]) * sm)
        sc = np.array(scores)
        p = np.exp(sc - sc.max())
        ref = (p[:, None] * v[0, keys].astype(np.float64)).sum(0) / p.sum()
        np.testing.assert_allclose(out[0, i], ref, atol=1e-5, rtol=1e-5)
