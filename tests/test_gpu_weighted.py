"""GPU parity of the shared path's weighted ranking (select_score "margin" / "expmass",
shared_selection_triton_exact_2.py:126-138, 277-426 with wvotes) through the C ABI.

  * _build_sets with weighted votes: bit-exact against the reference's own outputs on the 19
    golden tensors (tests/golden/build_sets_weighted_golden.npz);
  * the whole prefill on the reference's fp32 golden inputs and on planted bf16 / fp16 inputs,
    checked in layers: votes differ from the oracle's only inside the 1e-3 band; where the votes
    agree the weighted votes agree to 1e-5 relative; the oracle's weighted _build_sets applied to
    the GPU's own votes and weighted votes reproduces every set and statistic bit for bit; the
    oracle's Kernel C applied to the GPU's sets reproduces the output within tolerance.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, SET_NAMES, check_output, check_votes, gpu_sets_numpy, np_of, out_f32

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


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _same(got, ref):
    if ref.dtype == np.float32:
        return np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    return np.array_equal(got.astype(ref.dtype), ref)


def test_weighted_build_sets_matches_reference_goldens():
    import _sta_native as native
    g = _load("build_sets_weighted_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        ps, ng, nl, pct, T, kmax, qb, meas, _ = g[p + "params"]
        say(f"weighted build_sets golden case {i}: votes {g[p + 'votes'].shape} k_max {int(kmax)} pct {pct}")
        res = native.build_sets(torch.from_numpy(g[p + "votes"]).to(DEV), float(ps), int(ng), int(nl), float(pct),
                                int(T), int(kmax), int(qb), bool(meas),
                                wvotes=torch.from_numpy(g[p + "wvotes"]).to(DEV))
        torch.cuda.synchronize()
        for name, got in zip(SET_NAMES, res):
            assert _same(got.cpu().numpy(), g[p + name]), (i, name)


def _check_weighted(q, k, v, tau, invf, ps, rs, tile, k_max, select_score, pct=30.0, n_global=32, n_local=32,
                    q_pos_base=0, measure=False, what=""):
    import _sta_native as native
    H, N, D = q.shape[1], q.shape[2], q.shape[3]
    sm = 1.0 / math.sqrt(D)
    wmode = orc.WMODES[select_score]
    say(f"{what}: H={H} Hkv={k.shape[1]} N={N} D={D} tile={tile} k_max={k_max} {q.dtype} {select_score}")
    r = native.shared_attention(q, k, v, tau, invf, ps, rs, invf, ps, rs, pct=pct, sm_scale=sm, n_global=n_global,
                                n_local=n_local, tile=tile, k_max=k_max, q_pos_base=q_pos_base, measure=measure,
                                want_votes=True, want_row_max=True, select_score=select_score)
    torch.cuda.synchronize()
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    a = orc.select_vote(qn, kn, dt, tau.cpu().numpy(), invf.cpu().numpy(), ps, rs, sm, tile, q_pos_base,
                        band_eps=BAND, want_band=True, wmode=wmode)
    votes_g = r["votes"].cpu().numpy()
    wv_g = r["wvotes"].cpu().numpy()
    ndiff, nband = check_votes(votes_g, a["votes"], a["band"])
    same = votes_g == a["votes"]
    ref = a["wvotes"].astype(np.float64)
    err = np.abs(wv_g - ref)[same]
    # each keeping row adds a weight computed from a score that carries the three-product error
    # (typically ~1e-6, bounded by 3 * 2^-16 sum|q_i k_i| * sm_scale)
    tol = (1e-5 * np.abs(ref) + 2e-5 * a["votes"])[same] + 1e-7
    assert np.all(err <= tol), f"{what}: weighted votes differ by {float((err / tol).max()):.2f} x tolerance"
    sets_g = gpu_sets_numpy(r)
    refs = orc.build_sets(votes_g, ps, n_global, n_local, pct, tile, k_max, q_pos_base, measure, wvotes=wv_g)
    for name, rr in zip(SET_NAMES, refs):
        assert _same(sets_g[name], rr), (what, name)
    out_ref = orc.gather_attn(qn, kn, vn, dt, sets_g["idx"], sets_g["newpos_k"], sets_g["newpos_q"],
                              invf.cpu().numpy(), rs, sm, tile, k_max, 64, q_pos_base)
    e = check_output(out_f32(r["out"]), out_ref, dt, what)
    print(f"[result] {what}: vote entries differing {ndiff} (band pairs {nband}), max out err {e:.2e}, "
          f"kept mean {sets_g['kept_size'].mean():.1f}, overflow20 {int(sets_g['overflow20'].sum())}", flush=True)
    return r, sets_g


def test_weighted_composed_reference_goldens_fp32():
    g = _load("composed_weighted_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm, wmode = g[p + "params"]
        q = torch.from_numpy(g[p + "q"])[None].to(DEV)
        k = torch.from_numpy(g[p + "k"])[None].to(DEV)
        v = torch.from_numpy(g[p + "v"])[None].to(DEV)
        mode = {1: "margin", 2: "expmass"}[int(wmode)]
        r, sets_g = _check_weighted(q, k, v, torch.from_numpy(g[p + "tau"]), torch.from_numpy(g[p + "inv_freq"]),
                                    float(ps), 1.0, int(tile), int(kmax), mode, pct=float(pct), n_global=int(ng),
                                    n_local=int(nl), q_pos_base=int(qb), what=f"weighted golden case {i}")
        if np.array_equal(r["votes"].cpu().numpy(), g[p + "votes"]) and np.array_equal(sets_g["idx"], g[p + "idx"]):
            # no band key flipped and no cut moved: the reference's own output, end to end
            assert np.max(np.abs(out_f32(r["out"]) - g[p + "out"])) < 1e-4, i


@pytest.mark.parametrize("case", [
    # (H, Hkv, N, D, dtype, tile, k_max, select_score, pct, q_pos_base, measure)
    (2, 2, 1500, 128, torch.bfloat16, 64, 256, "expmass", 30.0, 0, False),
    (2, 1, 1200, 128, torch.bfloat16, 64, 2048, "margin", 30.0, 0, True),
    (2, 2, 777, 64, torch.float16, 32, 96, "margin", 22.5, 13, True),
    (3, 3, 640, 64, torch.float32, 32, 120, "expmass", 25.0, 0, False),
])
def test_weighted_three_layer(case):
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, N, D, dt, tile, kmax, mode, pct, qb, meas = case
    q, k, v = planted_inputs(9, H, Hkv, N, D, 0.02, dt, DEV)
    invf = base_inv_freq(D, 10000.0)
    _check_weighted(q, k, v, torch.full((H,), 5.0), invf.to(DEV), 0.5, 1.0, tile, kmax, mode, pct=pct,
                    q_pos_base=qb, measure=meas, what=f"weighted {mode} {dt} N={N} tile={tile}")


@pytest.mark.parametrize("mode", ["expmass", "margin"])
def test_weighted_empty_union_stages_every_key(mode):
    """tau < 0 on one head: no key passes, every rank value is zero and the cut falls on the keys
    past the causal end too (the select kernel then stages all N keys, not just the causal ones);
    the other head selects normally."""
    from synthetic import base_inv_freq, planted_inputs
    H, N, D = 2, 900, 64
    q, k, v = planted_inputs(13, H, H, N, D, 0.02, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0)
    _check_weighted(q, k, v, torch.tensor([-1.0, 5.0]), invf.to(DEV), 0.5, 1.0, 64, 200, mode,
                    what=f"weighted {mode}, empty union on head 0")


def test_weighted_dropin_entry_points():
    """select_score through the reference's entry points (exact_2 / YaRN / hybrid) and _build_sets."""
    import shared_selection_triton_exact_2 as ex2
    import shared_selection_triton_hybrid_exact as hyb
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D = 2, 900, 128
    q, k, v = planted_inputs(11, H, H, N, D, 0.02, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 5.0)
    say("weighted drop-in entry points")
    for mode in ("margin", "expmass"):
        res = ex2.shared_pi_attention(q, k, v, tau, invf, pos_scale=0.5, pct=30.0, tile=64, k_max=200,
                                      select_score=mode)
        r = native.shared_attention(q, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, pct=30.0, tile=64, k_max=200,
                                    select_score=mode)
        assert torch.equal(res[0][0], r["out"])
        assert torch.equal(res[2], r["kept_size"].long())
        h = hyb.shared_pi_attention(q, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, pct=30.0, tile=64, k_max=200,
                                    select_score=mode)
        assert torch.equal(h[0], res[0])
        votes, _, _, wv = native.select_vote(q, k, tau, invf, 0.5, 1.0, 1.0 / math.sqrt(D), 64, select_score=mode)
        sets = ex2._build_sets(votes, 0.5, 32, 32, 30.0, 64, 200, wvotes=wv, select_score=mode)
        assert torch.equal(sets[0], r["idx"])
        # freq ranking ignores the weighted votes, as the reference does (exact_2.py:299-300)
        f = ex2._build_sets(votes, 0.5, 32, 32, 30.0, 64, 200, wvotes=wv, select_score="freq")
        f0 = ex2._build_sets(votes, 0.5, 32, 32, 30.0, 64, 200)
        assert torch.equal(f[0], f0[0])
    with pytest.raises(KeyError):
        ex2.shared_pi_attention(q, k, v, tau, invf, select_score="bogus")


def test_weighted_config1_shape_one_head():
    """config 1's shape and geometry on one head with expmass ranking (the harness default)."""
    from synthetic import CONFIGS, planted_inputs
    c = CONFIGS["c1"]
    q, k, v = planted_inputs(0, 1, 1, c.N, c.D, c.frac, c.dtype, DEV)
    invf, ps, rs = c.geometry()
    _check_weighted(q, k, v, torch.full((1,), c.tau), invf.to(DEV), ps, rs, c.tile, c.k_max, "expmass",
                    what="config 1 shape, one head, expmass")


def test_weighted_long_rows_dense_votes():
    """Rows too long for the rank keys in LDS (N = 40000 at k_max 2048): the select kernel reads
    the keys from the vote rows at every pass; bit-exact against the oracle's _build_sets on the
    same dense votes, with tied weighted votes at the cuts and the measure loop."""
    import _sta_native as native
    N, nt, T, kmax = 40000, 6, 64, 2048
    g = np.random.default_rng(21)
    votes = g.integers(0, T + 1, size=(1, nt, N)).astype(np.int32)
    votes[:, :, g.random(N) < 0.5] = 0
    wv = (votes * g.random((1, nt, N)) * 3.0).astype(np.float32)
    wv[:, :, 5000:9000] = wv[:, :, 9000:13000]
    for pct, meas in ((30.0, False), (22.5, True)):
        say(f"weighted long rows, dense votes, N={N}, pct {pct}")
        qb = N - nt * T
        res = native.build_sets(torch.from_numpy(votes).to(DEV), 0.5, 32, 32, pct, T, kmax, qb, meas,
                                wvotes=torch.from_numpy(wv).to(DEV))
        torch.cuda.synchronize()
        refs = orc.build_sets(votes, 0.5, 32, 32, pct, T, kmax, qb, meas, wvotes=wv)
        for name, got, rr in zip(SET_NAMES, res, refs):
            assert _same(got.cpu().numpy(), rr), name


def test_weighted_long_rows_fused():
    """The fused prefill with expmass ranking past the LDS limit (N = 37000, one head): sets
    bit-exact against the oracle's _build_sets on the GPU's own votes and weighted votes."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D, T, kmax = 1, 37000, 64, 64, 2048
    q, k, v = planted_inputs(17, H, H, N, D, 0.02, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 5.0)
    say(f"weighted long rows, fused, N={N}")
    r = native.shared_attention(q, k, v, tau, invf, 1 / 3, 1.0, invf, 1 / 3, 1.0, pct=30.0, tile=T, k_max=kmax,
                                want_votes=True, select_score="expmass")
    torch.cuda.synchronize()
    votes_g, wv_g = r["votes"].cpu().numpy(), r["wvotes"].cpu().numpy()
    sets_g = gpu_sets_numpy(r)
    refs = orc.build_sets(votes_g, 1 / 3, 32, 32, 30.0, T, kmax, 0, False, wvotes=wv_g)
    for name, rr in zip(SET_NAMES, refs):
        assert _same(sets_g[name], rr), name
    assert torch.isfinite(r["out"].float()).all()
    print(f"[result] weighted long rows fused: kept mean {sets_g['kept_size'].mean():.1f}, "
          f"overflow20 {int(sets_g['overflow20'].sum())}", flush=True)
