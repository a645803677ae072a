"""GPU parity of the per-query rule (config 3 as written): every query keeps its own threshold
passers plus the forced keys, capped at k_max by score rank, with dense-rank positions
(_decode_build_sets_pq, shared_selection_triton_perquery.py:651-720), run at every prompt position
(prefill_mode="perquery", :905-924) and at decode.

Layers, as for the other paths:
  1. scores: the GPU's per-key scores against the oracle's (a few fp32 ulps);
  2. sets given the GPU's scores: the oracle's rule reproduces idx, newpos and the counters bit
     for bit (equal scores at the cap's cut are taken in ascending key order on both sides);
  3. sets against the oracle's own sets (from its own scores): every differing key lies within
     1e-3 of its query's threshold m - tau or of its query's cap cut; counted and reported;
  4. output given the GPU's sets: the oracle's attend within 1e-4 (fp32) or 2e-2 abs + 1e-2 rel.
Against the reference's fixtures: its _decode_build_sets_pq on crafted score rows, its composed
decode (Triton scores, torch / Kernel C attends) and its per-query prefill loop.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, check_output, np_of

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda:0"


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def classify_pq_rows(idx_g, idx_o, s_o, tau, q_pos0, M, n_global, n_local, k_max):
    """Per-query sets: keys in one side's set only, each within BAND of its query's threshold or
    of the oracle's cap cut (the smallest kept non-forced score of a capped query).  Returns
    (rows that differ, keys, threshold-band keys, cut-band keys)."""
    H, Q, _ = idx_g.shape
    rows = keys = nthr = ncut = 0
    for h in range(H):
        for i in range(Q):
            m, p = M - (Q - 1 - i), q_pos0 + i
            a = set(idx_g[h, i][idx_g[h, i] < m].tolist())
            b = set(idx_o[h, i][idx_o[h, i] < m].tolist())
            if a == b:
                continue
            rows += 1
            row = s_o[h, i, :m]
            thr = np.float32(row.max() - np.float32(tau[h]))
            forced = set(range(min(n_global, m))) | set(range(max(0, p - n_local + 1), p + 1))
            nf = [j for j in b if j not in forced]
            cut = min(float(row[j]) for j in nf) if (nf and len(b) >= k_max) else None
            for j in a ^ b:
                keys += 1
                if abs(float(row[j]) - float(thr)) <= BAND:
                    nthr += 1
                elif cut is not None and abs(float(row[j]) - cut) <= BAND:
                    ncut += 1
                else:
                    raise AssertionError(f"head {h} query {i} key {j}: score {row[j]} is neither within "
                                         f"{BAND} of the threshold {thr} nor of the cap cut {cut}")
    return rows, keys, nthr, ncut


def _check_perquery(q, k, v, tau, invf_a, ps, rs, invf_c, q_pos0, ng, nl, k_max, what, sample_rows=None):
    """Scores, sets and attend of Q queries (H, Q, D) at q_pos0.. over the cache k, v (Hkv, M, D)."""
    import _sta_native as native
    H, Q, D = q.shape
    M = k.shape[1]
    sm = 1.0 / math.sqrt(D)
    say(f"{what}: H={H} Hkv={k.shape[0]} Q={Q} M={M} D={D} k_max={k_max} {q.dtype}")
    r = native.decode_attention(q, k, v, tau, invf_a, q_pos0, ps, rs, sm, ng, nl, k_max, 100.0, False,
                                want_scores=True, inv_freq_c=invf_c, pos_scale_c=1.0, rope_scale_c=1.0, rule="pq")
    torch.cuda.synchronize()
    qn, dt = np_of(q)
    kn, _ = np_of(k)
    vn, _ = np_of(v)
    tau_n = tau.cpu().numpy()
    s_g = r["scores"].cpu().numpy()
    s_o = orc.decode_scores(qn, kn, dt, invf_a.cpu().numpy(), ps, rs, sm, q_pos0)
    valid = ~np.isnan(s_o)
    err = float(np.max(np.abs(s_g[valid] - s_o[valid])))
    assert err < 1e-4, f"{what}: scores differ from the oracle's by {err:.3e}"
    # sets given the GPU's scores: bit for bit
    ref = orc.decode_build_sets_pq(np.where(valid, s_g, np.float32(0)), tau_n, q_pos0, ng, nl, k_max)
    got = {n: r[n].cpu().numpy() for n in ("idx", "newpos_k", "newpos_q", "set_size", "usize", "overflow")}
    for name, rv in zip(("idx", "newpos_k", "newpos_q", "set_size", "usize", "overflow"), ref):
        assert np.array_equal(got[name], rv), f"{what}: {name} differs from the oracle given the GPU's scores"
    # sets against the oracle's own
    own = orc.decode_build_sets_pq(np.where(valid, s_o, np.float32(0)), tau_n, q_pos0, ng, nl, k_max)
    rows, keys, nthr, ncut = classify_pq_rows(got["idx"], own[0], s_o, tau_n, q_pos0, M, ng, nl, k_max)
    print(f"[sets] {what}: {rows} of {H * Q} queries' sets differ from the oracle's; {keys} keys: {nthr} "
          f"within 1e-3 of the threshold, {ncut} within 1e-3 of the cap cut", flush=True)
    # the attend given the GPU's sets
    if sample_rows is not None:
        qs = np.asarray(sample_rows)
        out_ref = orc.decode_attend(qn[:, qs], kn, vn, dt, invf_c.cpu().numpy(), 1.0, sm, 0,
                                    got["idx"][:, qs], got["newpos_k"][:, qs], got["newpos_q"][:, qs])
        out_g = r["out"].float().cpu().numpy()[:, qs]
    else:
        out_ref = orc.decode_attend(qn, kn, vn, dt, invf_c.cpu().numpy(), 1.0, sm, q_pos0, got["idx"],
                                    got["newpos_k"], got["newpos_q"])
        out_g = r["out"].float().cpu().numpy()
    e = check_output(out_g, out_ref, dt, what)
    print(f"[result] {what}: score err {err:.2e}, capped queries {int(got['overflow'].sum())} of "
          f"{got['overflow'].size}, set size mean {got['set_size'].mean():.1f}, max out err {e:.2e}", flush=True)
    return r, got


def test_pq_decode_sets_match_reference_goldens():
    """Selection alone from the reference's crafted score rows."""
    import _sta_native as native
    g = _gold("decode_pq_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ng, nl, km = (int(x) for x in g[p + "params"])
        s = g[p + "scores"]
        H, M = s.shape
        say(f"pq decode sets golden {i}")
        plan = native.DecodePlan(torch.zeros(H, 1, 64, device=DEV), torch.zeros(H, M, 64, device=DEV), None,
                                 torch.from_numpy(g[p + "tau"]), torch.ones(32), qp, k_max=km, n_global=ng,
                                 n_local=nl, rule="pq")
        r = plan.build_sets(torch.from_numpy(s).to(DEV).reshape(H, 1, M))
        ref = orc.decode_build_sets_pq(s[:, None, :], g[p + "tau"], qp, ng, nl, km)
        for name, rv in zip(("idx", "newpos_k", "newpos_q", "set_size", "usize", "overflow"), ref):
            assert np.array_equal(r[name].cpu().numpy(), rv), (i, name)
        # against the reference itself (its topk order among tied scores at the cut is unspecified)
        idx = r["idx"].cpu().numpy()[:, 0].astype(np.int64)
        same = np.all(idx == g[p + "idx"], axis=-1)
        if not same.all():
            assert i == 3, f"case {i}: sets differ from the reference outside the tie case"
        assert np.array_equal(r["newpos_q"].cpu().numpy()[:, 0], g[p + "newpos_q"]), i


def _crafted_rows(kind, H, Q, M, rng):
    """Score rows (H, Q, M) fp32 that reach each path of the per-query selection's cut search."""
    s = rng.standard_normal((H, Q, M)).astype(np.float32)
    if kind == "tied_cut":          # most passers share one value: the cut bin holds them all
        s[..., ::3] = np.float32(1.0)
    elif kind == "clustered":       # > 512 distinct values within a few hundred ulps at the cut
        c = np.float32(1.5) + np.arange(M, dtype=np.float32) * np.float32(2.0 ** -22)
        s[..., ::2] = c[::2]
    elif kind == "quantised":       # few distinct values: many exact ties everywhere
        s = np.round(s * 4.0).astype(np.float32) / np.float32(4.0)
    elif kind == "near_zero":       # the cut among values ~1e-3 under a threshold near -8: a value
        s = s * np.float32(1e-3)    # bin's edges are far more ulps apart than the search window
        s[..., ::97] = np.float32(8.0)
    return s


@pytest.mark.parametrize("kind,tau,Q,M", [("plain", 4.0, 1, 3000), ("plain", 4.0, 300, 3000),
                                          ("tied_cut", 4.0, 1, 3000), ("tied_cut", 4.0, 300, 3000),
                                          ("clustered", 4.0, 1, 3000), ("clustered", 4.0, 300, 3000),
                                          ("quantised", 4.0, 300, 3000), ("plain", float("inf"), 300, 3000),
                                          ("quantised", 0.0, 300, 3000), ("plain", -1.0, 1, 3000),
                                          ("plain", 4.0, 300, 16383), ("tied_cut", 4.0, 1, 16384),
                                          ("plain", 4.0, 300, 20000), ("tied_cut", 4.0, 300, 20000),
                                          ("clustered", 4.0, 1, 20000), ("plain", float("inf"), 300, 20000),
                                          ("plain", 4.0, 2100, 3000), ("tied_cut", 4.0, 2100, 8192),
                                          ("clustered", 4.0, 2100, 16384), ("quantised", 0.0, 2100, 6000),
                                          ("plain", 4.0, 2100, 3001), ("near_zero", 16.0, 300, 3000),
                                          ("near_zero", 16.0, 2100, 8192)])
def test_pq_select_crafted_rows(kind, tau, Q, M):
    """The per-query rule's selection from crafted score rows bit for bit against the oracle:
    exact ties at the cut, clusters of distinct values finer than the value bins (the key-space
    refinement), quantised scores, a cut among values near 0 under a threshold near -8 (the value
    bin's edges not found near their nominal values: the per-key bin test), tau = inf (every key
    passes), tau = 0 and tau < 0.  Batches of
    300 queries take the 512-thread kernels, single queries the 1024-thread ones; rows of up to
    16384 keys the register-resident kernel, longer ones the LDS-staged kernel; batches of 4200
    rows as the per-query prefill's launches have them."""
    import _sta_native as native
    H, km = 2, 700
    rng = np.random.default_rng(abs(hash((kind, Q))) % 2**32)
    s = _crafted_rows(kind, H, Q, M, rng)
    qp = M - Q
    say(f"pq crafted select: {kind} tau={tau} H={H} Q={Q} M={M} k_max={km}")
    plan = native.DecodePlan(torch.zeros(H, Q, 64, device=DEV), torch.zeros(H, M, 64, device=DEV), None,
                             torch.full((H,), tau), torch.ones(32), qp, k_max=km, n_global=16, n_local=16,
                             rule="pq")
    r = plan.build_sets(torch.from_numpy(s).to(DEV))
    ref = orc.decode_build_sets_pq(s, np.full(H, tau, np.float32), qp, 16, 16, km)
    for name, rv in zip(("idx", "newpos_k", "newpos_q", "set_size", "usize", "overflow"), ref):
        assert np.array_equal(r[name].cpu().numpy(), rv), name
    print(f"[result] pq crafted select {kind} tau={tau} Q={Q} M={M}: capped {int(ref[5].sum())} of {H * Q}, "
          f"set size mean {ref[3].mean():.1f}", flush=True)


def test_pq_decode_composed_reference_goldens():
    import shared_selection_triton_perquery as pqm
    g = _gold("decode_pq_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, km, sm = g[p + "params"]
        qp, ng, nl, km = int(qp), int(ng), int(nl), int(km)
        q, K, V = (torch.from_numpy(g[p + n]).to(DEV) for n in ("q", "k", "v"))
        ia, ic = torch.from_numpy(g[p + "inv_freq_a"]).to(DEV), torch.from_numpy(g[p + "inv_freq_c"]).to(DEV)
        H = q.shape[0]
        taus = torch.full((H,), float(tau))
        _check_perquery(q[:, None, :], K, V, taus.to(DEV), ia, float(ps), float(rs), ic, qp, ng, nl, km,
                        f"pq decode composed golden {i}")
        # the drop-in's one-query helpers against the reference's outputs
        say(f"pq decode drop-ins, golden {i}")
        s = pqm._decode_scores_kernel(q, K, ia, qp, float(ps), float(rs), float(sm))
        ref_s = g[p + "scores_triton"]
        assert np.max(np.abs(s.cpu().numpy() - ref_s)) <= 2e-6 * max(1.0, float(np.abs(ref_s).max()))
        idx, npk, npq = pqm._decode_build_sets_pq(q, K, taus, ia, qp, float(ps), float(rs), float(sm), ng, nl, km)
        if np.array_equal(idx.cpu().numpy(), g[p + "idx"]):
            out_t = pqm._decode_attend_torch_pq(q, K, V, idx, npk, npq, ic, float(sm))
            out_c = pqm._decode_attend_kernelC_pq(q, K, V, idx, npk, npq, ic, float(sm), km, q_pos=qp)
            np.testing.assert_allclose(out_t.cpu().numpy(), g[p + "out_torch"], atol=1e-4, rtol=1e-4)
            np.testing.assert_allclose(out_c.cpu().numpy(), g[p + "out_kernelc"], atol=1e-4, rtol=1e-4)


def test_perquery_prefill_matches_reference_loop():
    """prefill_mode="perquery" at every position of a 300-token prompt (fp32) against the
    reference's per-token loop."""
    import shared_selection_triton_perquery as pqm
    g = _gold("prefill_pq_perquery_golden.npz")
    ps, rs, tau, ng, nl, km, sm = g["params"]
    ng, nl, km = int(ng), int(nl), int(km)
    q, k, v = (torch.from_numpy(g[n]).to(DEV) for n in ("q", "k", "v"))
    H, N, D = q.shape
    ia, ic = torch.from_numpy(g["inv_freq_a"]).to(DEV), torch.from_numpy(g["inv_freq_c"]).to(DEV)
    taus = torch.full((H,), float(tau), device=DEV)
    r, got = _check_perquery(q, k, v, taus, ia, float(ps), float(rs), ic, 0, ng, nl, km, "pq prefill golden")
    same = np.all(got["idx"].astype(np.int64) == g["idx"], axis=-1)
    assert same.mean() > 0.99
    np.testing.assert_allclose(r["out"].cpu().numpy()[same], g["out"][same], atol=1e-4, rtol=1e-4)
    # the drop-in's one-call per-query prefill gives the same output
    say("perquery prefill drop-in")
    pqm.reset_overflow_stats()
    out, usize, size, ovf = pqm.perquery_prefill_attention(q[None], k[None], v[None], taus, ia, ic, float(ps),
                                                          float(rs), float(sm), ng, nl, km)
    assert torch.equal(out[0], r["out"])
    assert torch.equal(size, r["set_size"][:, :]) and torch.equal(ovf, r["overflow"])
    st = pqm.get_overflow_stats()["decode"]
    assert st["total_cells"] == H * N and st["overflow_cells"] == int(ovf.sum().item())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_perquery_bf16_gqa_cap(dt):
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, N, D = 4, 2, 1500, 128
    q, k, v = planted_inputs(61, H, Hkv, N, D, 0.01, dt, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    _check_perquery(q[0], k[0], v[0], torch.full((H,), 4.0, device=DEV), invf, 0.25, 1.0, invf, 0, 32, 32, 256,
                    f"pq per-query prefill {dt} GQA k_max 256")


def test_perquery_config3_shape_deep_rows():
    """Config 3's shape (N=16384, d128, bf16, tau 4, PI 1/4, k_max 2048) on two heads: the last
    384 positions (where the cap binds) and the first 128, through the batched per-query path."""
    from synthetic import CONFIGS
    c = CONFIGS["c3q"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    invf = invf.to(DEV)
    tau = torch.full((2,), c.tau, device=DEV)
    kk, vv = k[0, :2], v[0, :2]
    Q = 384
    _check_perquery(q[0, :2, c.N - Q:], kk, vv, tau, invf, ps, rs, invf, c.N - Q, c.n_global, c.n_local, c.k_max,
                    "config 3 shape, last 384 positions, 2 heads", sample_rows=list(range(0, Q, 16)))
    _check_perquery(q[0, :2, :128], kk[:, :128], vv[:, :128], tau, invf, ps, rs, invf, 0, c.n_global, c.n_local,
                    c.k_max, "config 3 shape, first 128 positions, 2 heads")


@pytest.mark.parametrize("D,dt", [(128, torch.bfloat16), (64, torch.float32), (128, torch.float16)])
def test_grouped_attend_any_positions(D, dt):
    """The batched per-query attend (16 queries per workgroup, the dense-rank (cos, sin) table in
    LDS): a batch of 40 queries (a partial last group) against the oracle given the GPU's sets;
    the same queries in batches of 10 (the split attend) within the output tolerance; and the
    attend alone over sets with positions that are not the slot indices (newpos_k + 2.5,
    newpos_q + 2.5) against the oracle: sets from the caller take the split attend, which reads
    every slot's position."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, Q = 2, 900, 40
    q, k, v = planted_inputs(91, H, H, N, D, 0.02, dt, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    q0 = N - Q
    qq, kk, vv = q[0, :, q0:], k[0], v[0]
    sm = 1.0 / math.sqrt(D)
    say(f"grouped per-query attend: H={H} Q={Q} M={N} D={D} {dt}")
    plan = native.DecodePlan(qq, kk, vv, tau, invf, q0, 0.5, 1.0, sm, 16, 16, 256, 100.0, False,
                             inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0, rule="pq")
    r = plan.run()
    torch.cuda.synchronize()
    got = {n: r[n].clone() for n in ("out", "idx", "newpos_k", "newpos_q", "set_size")}
    assert int(r["overflow"].sum()) > 0, "the cap binds for some queries"
    qn, dtc = np_of(qq)
    kn, _ = np_of(kk)
    vn, _ = np_of(vv)
    invf_n = invf.cpu().numpy()
    out_ref = orc.decode_attend(qn, kn, vn, dtc, invf_n, 1.0, sm, q0, got["idx"].cpu().numpy(),
                                got["newpos_k"].cpu().numpy(), got["newpos_q"].cpu().numpy())
    e1 = check_output(got["out"].float().cpu().numpy(), out_ref, dtc, "grouped attend")
    # the same queries through the split attend (batches below 16 queries)
    worst = 0.0
    for i0 in range(0, Q, 10):
        r1 = native.decode_attention(qq[:, i0:i0 + 10], kk[:, :q0 + i0 + 10], vv[:, :q0 + i0 + 10], tau, invf,
                                     q0 + i0, 0.5, 1.0, sm, 16, 16, 256, 100.0, False, inv_freq_c=invf,
                                     pos_scale_c=1.0, rope_scale_c=1.0, rule="pq")
        torch.cuda.synchronize()
        assert torch.equal(r1["idx"], got["idx"][:, i0:i0 + 10]), "sets do not depend on the batch"
        worst = max(worst, (r1["out"].float() - got["out"][:, i0:i0 + 10].float()).abs().max().item())
    tol = 1e-5 if dt == torch.float32 else 2e-2
    assert worst <= tol, f"grouped vs split attend differ by {worst:.3e}"
    # positions that are not the slot indices
    npk = torch.where(got["idx"] < N, got["newpos_k"] + 2.5, got["newpos_k"])
    npq = got["newpos_q"] + 2.5
    out2 = plan.attend(got["idx"], npk, npq, got["set_size"]).clone()
    torch.cuda.synchronize()
    out_ref2 = orc.decode_attend(qn, kn, vn, dtc, invf_n, 1.0, sm, q0, got["idx"].cpu().numpy(), npk.cpu().numpy(),
                                 npq.cpu().numpy())
    e2 = check_output(out2.float().cpu().numpy(), out_ref2, dtc, "grouped attend, shifted positions")
    assert (out2.float() - got["out"].float()).abs().max().item() > 0, "the shifted positions changed the output"
    print(f"[result] grouped attend {D} {dt}: max out err {e1:.2e}, vs split {worst:.2e}, shifted positions "
          f"{e2:.2e}", flush=True)


def test_perquery_config3_sampled_positions_whole_sequence():
    """Config 3 as written (N=16384, d128, bf16, tau 4, PI 1/4, k_max 2048) at every 257th position
    of two heads, from the first query to the last: scores against the oracle's, sets given the
    GPU's scores bit for bit, sets against the oracle's own (every differing key classified) and
    the attend given the GPU's sets."""
    import _sta_native as native
    from synthetic import CONFIGS
    c = CONFIGS["c3q"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    invf_d = invf.to(DEV)
    invf_n = invf.numpy()
    sm = 1.0 / math.sqrt(c.D)
    positions = list(range(0, c.N, 257)) + [c.N - 1]
    names = ("idx", "newpos_k", "newpos_q", "set_size", "usize", "overflow")
    for h in (0, 1):
        say(f"config 3 sampled positions: head {h}, {len(positions)} queries")
        tau = torch.full((1,), c.tau, device=DEV)
        tau_n = tau.cpu().numpy()
        tot = {"rows": 0, "keys": 0, "thr": 0, "cut": 0, "capped": 0}
        worst_s = worst_o = 0.0
        for p in positions:
            qq, kk, vv = q[0, h:h + 1, p:p + 1], k[0, h:h + 1, :p + 1], v[0, h:h + 1, :p + 1]
            r = native.decode_attention(qq, kk, vv, tau, invf_d, p, ps, rs, sm, c.n_global, c.n_local, c.k_max, 100.0,
                                        False, want_scores=True, inv_freq_c=invf_d, pos_scale_c=1.0,
                                        rope_scale_c=1.0, rule="pq")
            torch.cuda.synchronize()
            qn, dt = np_of(qq)
            kn, _ = np_of(kk)
            vn, _ = np_of(vv)
            s_g = r["scores"].cpu().numpy()
            s_o = orc.decode_scores(qn, kn, dt, invf_n, ps, rs, sm, p)
            worst_s = max(worst_s, float(np.max(np.abs(s_g - s_o))))
            assert worst_s < 1e-4, f"position {p}: scores differ from the oracle's by {worst_s:.3e}"
            got = {n: r[n].cpu().numpy() for n in names}
            ref = orc.decode_build_sets_pq(s_g, tau_n, p, c.n_global, c.n_local, c.k_max)
            for name, rv in zip(names, ref):
                assert np.array_equal(got[name], rv), f"position {p}: {name} differs given the GPU's scores"
            own = orc.decode_build_sets_pq(s_o, tau_n, p, c.n_global, c.n_local, c.k_max)
            rows, keys, nthr, ncut = classify_pq_rows(got["idx"], own[0], s_o, tau_n, p, p + 1, c.n_global,
                                                      c.n_local, c.k_max)
            for n_, x in zip(("rows", "keys", "thr", "cut"), (rows, keys, nthr, ncut)):
                tot[n_] += x
            tot["capped"] += int(got["overflow"].sum())
            out_ref = orc.decode_attend(qn, kn, vn, dt, invf_n, 1.0, sm, p, got["idx"], got["newpos_k"],
                                        got["newpos_q"])
            worst_o = max(worst_o, check_output(r["out"].float().cpu().numpy(), out_ref, dt, f"position {p}"))
        print(f"[sets] config 3 as written, head {h}, every 257th position ({len(positions)} queries, "
              f"{tot['capped']} capped): {tot['rows']} queries' sets differ from the oracle's; {tot['keys']} keys: "
              f"{tot['thr']} within 1e-3 of the threshold, {tot['cut']} within 1e-3 of the cap cut, 0 other",
              flush=True)
        print(f"[result] config 3 head {h}: max score err {worst_s:.2e}, max out err {worst_o:.2e}", flush=True)


def test_perquery_full_prefill_plan_config3_structure():
    """The whole config-3 prefill (32 heads x 16384 positions) through the head-grouped plan:
    structural invariants on every query and the output of sampled rows of one head against the
    oracle given the GPU's own selection (recomputed for those rows)."""
    import _sta_native as native
    from synthetic import CONFIGS
    c = CONFIGS["c3q"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    invf = invf.to(DEV)
    say("config 3 per-query prefill plan, full size")
    plan = native.PerQueryPrefillPlan(q, k, v, torch.full((c.H,), c.tau, device=DEV), invf, invf, ps, rs,
                                      n_global=c.n_global, n_local=c.n_local, k_max=c.k_max)
    r = plan.run()
    torch.cuda.synchronize()
    size, us, ov = r["set_size"], r["usize"], r["overflow"]
    pos = torch.arange(c.N, device=DEV)
    assert torch.all(size <= c.k_max) and torch.all(size >= 1) and torch.all(size <= pos[None] + 1)
    # capped queries keep exactly k_max keys; the others their passers plus at most 64 forced keys
    assert torch.all(size[ov] == c.k_max)
    assert torch.all(size[~ov] >= us[~ov]) and torch.all(size[~ov] <= us[~ov] + c.n_global + c.n_local)
    assert torch.isfinite(r["out"].float()).all()
    print(f"[result] config 3 per-query prefill: capped queries {int(ov.sum())} of {ov.numel()}, set size mean "
          f"{size.float().mean().item():.1f}, passers mean {us.float().mean().item():.1f}", flush=True)
    # sampled rows of head 5: the plan's output equals a direct per-query call on those rows
    h, rows = 5, [100, 4000, 9000, 16383]
    for rr in rows:
        d = native.decode_attention(q[0, h:h + 1, rr:rr + 1], k[0, h:h + 1, :rr + 1], v[0, h:h + 1, :rr + 1],
                                    torch.full((1,), c.tau), invf, rr, ps, rs, None, c.n_global, c.n_local, c.k_max,
                                    inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0, rule="pq")
        e = (d["out"][0, 0].float() - r["out"][h, rr].float()).abs().max().item()
        assert e <= 2e-2, (rr, e)



def test_perquery_prefill_split_attend_without_key_positions():
    """The plan passes no newpos_k (the per-query rule's positions are the slot indices).  Chunks
    of 10 queries take the split attend, which then reads the slot index as the position: bit for
    bit the direct decode calls on the same chunks, which pass newpos_k."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D = 2, 300, 64
    q, k, v = planted_inputs(85, H, H, N, D, 0.02, torch.float32, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    say("per-query prefill: split attend (chunks of 10) without newpos_k against direct decode calls")
    plan = native.PerQueryPrefillPlan(q, k, v, tau, invf, invf, 0.5, 1.0, None, 8, 8, 64, query_chunk=10).run()
    torch.cuda.synchronize()
    capped = 0
    for i0 in range(0, N, 10):
        i1 = min(N, i0 + 10)
        d = native.decode_attention(q[0, :, i0:i1], k[0, :, :i1], v[0, :, :i1], tau, invf, i0, 0.5, 1.0, None, 8, 8,
                                    64, inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0, rule="pq")
        assert torch.equal(d["out"], plan["out"][:, i0:i1]), i0
        assert torch.equal(d["overflow"].bool(), plan["overflow"][:, i0:i1]), i0
        capped += int(d["overflow"].sum())
    assert capped > 0


def test_perquery_prefill_chunking_is_transparent():
    """The per-query prefill over chunks of positions (each a decode batch over its cache prefix)
    gives the one-batch run's outputs bit for bit: a query's scores, set and attend depend on
    neither the chunking nor the head grouping."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, N, D = 4, 2, 2500, 128
    q, k, v = planted_inputs(83, H, Hkv, N, D, 0.01, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 4.0, device=DEV)
    say("per-query prefill: chunks of 1000 and 2 heads per group against one batch")
    whole = native.PerQueryPrefillPlan(q, k, v, tau, invf, invf, 0.25, 1.0, None, 16, 16, 256,
                                       query_chunk=None).run()
    whole = {n: t.clone() for n, t in whole.items()}
    parts = native.PerQueryPrefillPlan(q, k, v, tau, invf, invf, 0.25, 1.0, None, 16, 16, 256, heads_per_group=2,
                                       query_chunk=1000).run()
    torch.cuda.synchronize()
    assert int(whole["overflow"].sum()) > 0          # the cap binds somewhere
    for name in ("out", "set_size", "usize", "overflow"):
        assert torch.equal(whole[name], parts[name]), name
