"""CPU tests that pin the oracle (oracle/sta_oracle.c) before anything is compared against it.

Pins, per oracle function:
  build_sets   -- bit-exact against the reference's own _build_sets on 14 vote tensors
                  (tests/golden/build_sets_golden.npz), plus an independent histogram
                  formulation of the top-k% cut and the fp32 budget quirk.
  select_vote  -- votes/row_counts against the reference's Kernel A under the Triton interpreter
                  (fp32 and bf16 inputs), and row max against a float64 brute force.
  gather_attn  -- the composed reference pipeline's output (fp32) and the identity-reposition
                  known answer: tau=inf, pct=100, k_max>=N reduces to dense causal RoPE attention,
                  computed here independently in float64 with complex rotations.
  rope_rotate  -- norm scaling by rope_scale, identity at position 0 and the relative-position
                  property of the rotation.
"""
import math
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SET_NAMES = ["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen", "orig_overflow",
             "kpct_meas", "overflow20"]


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def base_inv_freq(D, theta):
    return (1.0 / (theta ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)


# ------------------------------------------------------------------------------------------------
# build_sets
# ------------------------------------------------------------------------------------------------
def test_build_sets_matches_reference_goldens(oracle):
    g = _load("build_sets_golden.npz")
    n = int(g["ncases"])
    assert n >= 14
    for i in range(n):
        p = f"c{i}_"
        ps, ng, nl, pct, T, kmax, qb, meas = g[p + "params"]
        res = oracle.build_sets(g[p + "votes"], float(ps), int(ng), int(nl), float(pct), int(T),
                                int(kmax), int(qb), bool(meas))
        for name, got in zip(SET_NAMES, res):
            ref = g[p + name]
            if ref.dtype == np.float32:
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (i, name)
            else:
                assert np.array_equal(got.astype(ref.dtype), ref), (i, name)


def test_budget_is_float32_ceil(oracle):
    """U=50, p=30: ceil(float32(0.3)*50) = 16, the rational ceil(15.0) would be 15."""
    v = np.zeros((1, 1, 256), np.int32)
    v[0, 0, 100:150] = np.arange(1, 51)
    res = oracle.build_sets(v, 1.0, 0, 1, 30.0, 64, 2048)
    assert int(res[3][0, 0]) == 16


def _hist_reference(votes, forced, steps, K_ord, kmax):
    """Independent formulation: the (b+1)-th largest vote from a histogram of integer votes."""
    N = votes.size
    U = int((votes > 0).sum())
    top = int(votes.max())
    ge = np.array([(votes >= v).sum() for v in range(top + 2)])       # C(v) = #(votes >= v)
    resolved, chosen, cut = False, 0, None
    for p in steps:
        budget = max(1, math.ceil(float(np.float32(np.float32(p / 100.0) * np.float32(U)))))
        b = min(max(budget - 1, 0), K_ord - 1)
        vcut = max(v for v in range(top + 1) if ge[v] >= b + 1)
        size = int(ge[vcut]) + int((forced & (votes < vcut)).sum())
        if not resolved:
            cut = vcut
            if size <= kmax:
                resolved, chosen = True, p
    return chosen, int(ge[cut]), int(ge[cut] + (forced & (votes < cut)).sum())


def test_build_sets_histogram_equivalence(oracle):
    rng = np.random.default_rng(7)
    H, nt, N, T = 3, 6, 400, 64
    for trial in range(4):
        votes = rng.binomial(T, 0.1 + 0.2 * trial, size=(H, nt, N)).astype(np.int32)
        kmax = [2048, 200, 150, 120][trial]
        res = oracle.build_sets(votes, 1.0, 16, 16, 30.0, T, kmax)
        K_ord = math.ceil(0.3 * N)
        kj = np.arange(N)
        for h in range(H):
            for t in range(nt):
                forced = (kj < 16) | ((kj >= t * T - 15) & (kj <= t * T + T - 1))
                ch, ss, ks = _hist_reference(votes[h, t], forced, [30, 25, 20], K_ord, kmax)
                assert int(res[5][h, t]) == ch
                assert int(res[3][h, t]) == ss
                assert int(res[4][h, t]) == ks


def test_identity_positions_when_everything_is_kept(oracle):
    """All keys kept (votes>0 everywhere causal, pct=100): newpos = max(j*s, prev+1) = j for s<=1."""
    H, N, T = 1, 300, 32
    nt = (N + T - 1) // T
    votes = np.zeros((H, nt, N), np.int32)
    for t in range(nt):
        votes[0, t, :min(N, (t + 1) * T)] = 1
    for ps in (1.0, 0.5, 1.0 / 3.0):
        idx, npk, npq, *_ = oracle.build_sets(votes, ps, 0, 1, 100.0, T, 512)
        for t in range(nt):
            hi = min(N, (t + 1) * T)
            assert np.array_equal(idx[0, t, :hi], np.arange(hi))
            assert np.all(idx[0, t, hi:] == N)
            assert np.array_equal(npk[0, t, :hi], np.arange(hi, dtype=np.float32))
            qp = np.minimum(np.arange(t * T, t * T + T), N - 1)
            assert np.array_equal(npq[0, t], qp.astype(np.float32))


# ------------------------------------------------------------------------------------------------
# select_vote
# ------------------------------------------------------------------------------------------------
def _band_ok(got, ref, band):
    """votes may differ only by queries whose score sits within the tolerance band."""
    return np.all(np.abs(got.astype(np.int64) - ref.astype(np.int64)) <= band)


def test_select_vote_matches_reference_fp32(oracle):
    g = _load("composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm = g[p + "params"]
        a = oracle.select_vote(g[p + "q"], g[p + "k"], oracle.F32, g[p + "tau"], g[p + "inv_freq"],
                               float(ps), 1.0, float(sm), int(tile), int(qb), band_eps=1e-5,
                               want_band=True)
        assert _band_ok(a["votes"], g[p + "votes"], a["band"]), i
        assert np.array_equal(a["votes"], g[p + "votes"]), i
        assert np.array_equal(a["row_counts"], g[p + "row_counts"]), i


def test_select_vote_matches_reference_bf16(oracle):
    g = _load("kernel_a_bf16_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, ps, sm = g[p + "params"]
        a = oracle.select_vote(g[p + "q"], g[p + "k"], oracle.BF16, g[p + "tau"], g[p + "inv_freq"],
                               float(ps), 1.0, float(sm), int(tile), 0, band_eps=1e-5, want_band=True)
        assert _band_ok(a["votes"], g[p + "votes"], a["band"]), i
        diff = int(np.abs(a["votes"] - g[p + "votes"]).sum())
        assert diff <= 2, diff
        assert int(np.abs(a["row_counts"] - g[p + "row_counts"]).sum()) <= 2


def _rope64(x, pos, inv_freq, rope_scale=1.0):
    """float64 rotation through complex numbers: (x1 + i x2) * e^{i pos f} * rope_scale."""
    half = x.shape[-1] // 2
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:].astype(np.float64)
    z = z * np.exp(1j * np.asarray(pos, np.float64)[..., None] * inv_freq.astype(np.float64)) * rope_scale
    return np.concatenate([z.real, z.imag], axis=-1)


def test_row_max_brute_force(oracle):
    rng = np.random.default_rng(3)
    H, N, D, T = 2, 150, 64, 32
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = base_inv_freq(D, 10000.0)
    sm = 1.0 / math.sqrt(D)
    a = oracle.select_vote(q, k, oracle.F32, np.full(H, 4.0, np.float32), invf, 0.5, 1.0, sm, T)
    pos = np.arange(N) * np.float64(np.float32(0.5))
    for h in range(H):
        s = _rope64(q[h], pos, invf) @ _rope64(k[h], pos, invf).T * sm
        s[np.triu_indices(N, 1)] = -np.inf
        m = s.max(1)
        assert np.max(np.abs(a["row_max"][h] - m)) < 1e-4
        keep = s >= (m[:, None] - 4.0)
        nt = (N + T - 1) // T
        for t in range(nt):
            ref = keep[t * T:(t + 1) * T].sum(0)
            close = (np.abs(s[t * T:(t + 1) * T] - (m[t * T:(t + 1) * T, None] - 4.0)) < 1e-4).sum(0)
            assert np.all(np.abs(a["votes"][h, t] - ref) <= close)


# ------------------------------------------------------------------------------------------------
# gather / composition
# ------------------------------------------------------------------------------------------------
def test_composed_matches_reference_fp32(oracle):
    g = _load("composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm = g[p + "params"]
        out, ss, ks, ch, oo, km, o20, ex = oracle.shared_pi_attention(
            g[p + "q"], g[p + "k"], g[p + "v"], oracle.F32, g[p + "tau"], g[p + "inv_freq"], float(ps),
            1.0, pct=float(pct), sm_scale=float(sm), n_global=int(ng), n_local=int(nl),
            tile=int(tile), k_max=int(kmax), q_pos_base=int(qb))
        assert np.array_equal(ex["idx"], g[p + "idx"]), i
        assert np.array_equal(ex["newpos_k"], g[p + "newpos_k"]), i
        assert np.array_equal(ex["newpos_q"], g[p + "newpos_q"]), i
        for name, got in zip(["shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas",
                              "overflow20"], [ss, ks, ch, oo, km, o20]):
            assert np.array_equal(got.astype(g[p + name].dtype), g[p + name]), (i, name)
        ref = g[p + "out"]
        assert np.max(np.abs(out - ref)) < 2e-5, (i, float(np.max(np.abs(out - ref))))


def test_hybrid_matches_reference_fp32(oracle):
    g = _load("composed_golden.npz")
    tile, kmax, pct, ng, nl, ps_a, rs_a, ps_c, rs_c = g["hyb_params"]
    out, ss, ks, ch, oo, km, o20, ex = oracle.shared_pi_attention(
        g["hyb_q"], g["hyb_k"], g["hyb_v"], oracle.F32, g["hyb_tau"], g["hyb_inv_freq_a"], float(ps_a),
        float(rs_a), g["hyb_inv_freq_c"], float(ps_c), float(rs_c), pct=float(pct),
        n_global=int(ng), n_local=int(nl), tile=int(tile), k_max=int(kmax))
    assert np.array_equal(ks, g["hyb_kept_size"])
    assert np.array_equal(ss, g["hyb_shared_size"])
    assert np.array_equal(o20, g["hyb_overflow20"])
    assert np.max(np.abs(out - g["hyb_out"])) < 2e-5


def test_identity_kat_is_dense_rope_attention(oracle):
    """tau=inf, pct=100, k_max >= N: every causal key kept at its own position, so the pipeline
    is dense causal attention with native RoPE (positions j), here in float64."""
    rng = np.random.default_rng(11)
    H, N, D, T = 2, 200, 64, 32
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    v = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = base_inv_freq(D, 10000.0)
    sm = 1.0 / math.sqrt(D)
    out, *_ = oracle.shared_pi_attention(q, k, v, oracle.F32, np.full(H, np.inf, np.float32), invf,
                                         1.0, 1.0, pct=100.0, sm_scale=sm, tile=T, k_max=256)
    pos = np.arange(N)
    for h in range(H):
        qz = q[h, :, :D // 2] + 1j * q[h, :, D // 2:]
        kz = k[h, :, :D // 2] + 1j * k[h, :, D // 2:]
        rel = np.exp(1j * (pos[:, None, None] - pos[None, :, None]) * invf.astype(np.float64))
        s = np.real(np.einsum("qf,kf,qkf->qk", qz, np.conj(kz), rel)) * sm
        s[np.triu_indices(N, 1)] = -np.inf
        a = np.exp(s - s.max(1, keepdims=True))
        ref = (a / a.sum(1, keepdims=True)) @ v[h].astype(np.float64)
        assert np.max(np.abs(out[h] - ref)) < 1e-5


def test_rope_invariants(oracle):
    rng = np.random.default_rng(5)
    D = 128
    x = rng.standard_normal((64, D)).astype(np.float32)
    invf = base_inv_freq(D, 500000.0)
    r0 = oracle.rope_rotate(x, oracle.F32, np.zeros(64, np.float32), invf, 1.25)
    assert np.max(np.abs(r0 - 1.25 * x)) < 1e-6
    pos = rng.integers(0, 30000, 64).astype(np.float32)
    r = oracle.rope_rotate(x, oracle.F32, pos, invf, 1.25)
    assert np.allclose(np.linalg.norm(r, axis=1), 1.25 * np.linalg.norm(x, axis=1), rtol=1e-5)
    # relative position: <R(a) x, R(b) y> depends on b - a only (checked at integer shifts)
    y = rng.standard_normal((64, D)).astype(np.float32)
    a = rng.integers(0, 1000, 64).astype(np.float32)
    d = 37.0
    s1 = (oracle.rope_rotate(x, oracle.F32, a, invf, 1.0) *
          oracle.rope_rotate(y, oracle.F32, a + d, invf, 1.0)).sum(1)
    s2 = (x * oracle.rope_rotate(y, oracle.F32, np.full(64, d, np.float32), invf, 1.0)).sum(1)
    assert np.max(np.abs(s1 - s2)) < 1e-3
    # half-split pairing: dims i and i + D/2 form one complex number rotated by the fp32 angle
    ang32 = (pos[:, None] * invf[None, :]).astype(np.float32).astype(np.float64)
    z = (x[:, :D // 2] + 1j * x[:, D // 2:]).astype(np.complex128) * np.exp(1j * ang32) * 1.25
    assert np.max(np.abs(r - np.concatenate([z.real, z.imag], axis=1))) < 2e-5


def test_bf16_round_trip(oracle):
    x = np.array([1.0, 1.00390625, 1.005859375, -3.14159, 65504.0, 1e-30], np.float32)
    b = oracle.round_to_dtype(x, oracle.BF16)
    back = oracle.to_f32(b, oracle.BF16)
    assert back[0] == 1.0 and back[1] == 1.0            # tie rounds to even
    assert back[2] == np.float32(1.0078125)
    assert abs(back[3] + 3.140625) < 1e-6
