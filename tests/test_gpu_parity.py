"""GPU parity: the HIP path through the C ABI against the CPU oracle and the reference goldens.

Selection is compared under the band rule (see parity_helpers); outputs within 1e-4 (fp32) or
2e-2 abs + 1e-2 rel (bf16 / fp16).  Each test prints the case it runs before touching the GPU.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import (BAND, check_output, check_sets_given_votes, check_votes,
                            classify_set_diffs, gpu_sets_numpy, np_of, out_f32, report_set_diffs,
                            SET_NAMES)

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


def _t(a):
    """numpy -> device tensor; uint16 arrays hold bf16 bit patterns."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def full_check(q, k, v, tau, invf_a, ps_a, rs_a, invf_c=None, ps_c=None, rs_c=None, pct=30.0,
               n_global=32, n_local=32, tile=64, k_max=2048, q_pos_base=0, measure=False, what=""):
    """Run the device path once and apply the three-layer check; returns a small report."""
    import _sta_native as native
    if invf_c is None:
        invf_c, ps_c, rs_c = invf_a, ps_a, rs_a
    H, N, D = q.shape[1], q.shape[2], q.shape[3]
    sm = 1.0 / math.sqrt(D)
    say(f"{what}: H={H} Hkv={k.shape[1]} N={N} D={D} tile={tile} k_max={k_max} dtype={q.dtype}")
    r = native.shared_attention(q, k, v, tau, invf_a, ps_a, rs_a, invf_c, ps_c, rs_c, pct=pct,
                                sm_scale=sm, n_global=n_global, n_local=n_local, tile=tile, k_max=k_max,
                                q_pos_base=q_pos_base, measure=measure, want_votes=True,
                                want_row_max=True)
    torch.cuda.synchronize()
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    a = orc.select_vote(qn, kn, dt, tau.cpu().numpy(), invf_a.cpu().numpy(), ps_a, rs_a, sm, tile,
                        q_pos_base, band_eps=BAND, want_band=True)
    votes_g = r["votes"].cpu().numpy()
    ndiff, nband = check_votes(votes_g, a["votes"], a["band"])
    rm = r["row_max"].cpu().numpy()
    assert np.max(np.abs(rm - a["row_max"])) < 1e-4, "row max"
    sets_g = gpu_sets_numpy(r)
    check_sets_given_votes(votes_g, sets_g, ps_c, n_global, n_local, pct, tile, k_max, q_pos_base,
                           measure)
    sd = set_level_diffs(votes_g, a, ps_c, n_global, n_local, pct, tile, k_max, q_pos_base, measure, what)
    if ndiff == 0:  # no band key flipped: the GPU sets are the oracle's end to end
        assert sd["keys"] == 0
    out_ref = orc.gather_attn(qn, kn, vn, dt, sets_g["idx"], sets_g["newpos_k"], sets_g["newpos_q"],
                              invf_c.cpu().numpy(), rs_c, sm, tile, k_max, 64, q_pos_base)
    err = check_output(out_f32(r["out"]), out_ref, dt, what)
    print(f"[result] {what}: vote entries differing {ndiff} (band pairs {nband}), max out err {err:.2e}, "
          f"kept mean {sets_g['kept_size'].mean():.1f}, overflow20 {int(sets_g['overflow20'].sum())}",
          flush=True)
    return r, sets_g


def set_level_diffs(votes_g, a, ps_c, n_global, n_local, pct, tile, k_max, q_pos_base=0,
                    measure=False, what="", heads=None):
    """The GPU's selected sets (from its own votes) against the oracle's sets built from the
    oracle's own votes: every differing key classified (band / shifted cut / truncation) and the
    counts printed.  `heads` selects the oracle's heads matching votes_g."""
    votes_o, band = a["votes"], a["band"]
    if heads is not None:
        votes_o, band = votes_o[heads], band[heads]
    ref_g = orc.build_sets(votes_g, ps_c, n_global, n_local, pct, tile, k_max, q_pos_base, measure,
                           want_cut=True)
    ref_o = orc.build_sets(votes_o, ps_c, n_global, n_local, pct, tile, k_max, q_pos_base, measure,
                           want_cut=True)
    c = classify_set_diffs(votes_g, votes_o, band, {"idx": ref_g[0]}, {"idx": ref_o[0]}, ref_g[9],
                           ref_o[9], tile, k_max, n_global, n_local, q_pos_base)
    report_set_diffs(what, c)
    return c


# ------------------------------------------------------------------------------------------
# stage-level parity against the reference's own vectors
# ------------------------------------------------------------------------------------------
def test_build_sets_matches_reference_goldens():
    import _sta_native as native
    g = _gold("build_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        ps, ng, nl, pct, T, kmax, qb, meas = g[p + "params"]
        say(f"build_sets golden case {i}")
        res = native.build_sets(_t(g[p + "votes"]), float(ps), int(ng), int(nl), float(pct), int(T),
                                int(kmax), int(qb), bool(meas))
        for name, got in zip(SET_NAMES, res):
            got = got.cpu().numpy()
            ref = g[p + name]
            if ref.dtype == np.float32:
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (i, name)
            else:
                assert np.array_equal(got.astype(ref.dtype), ref), (i, name)


def test_kernel_a_matches_reference_goldens_fp32():
    import _sta_native as native
    g = _gold("composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm = g[p + "params"]
        say(f"kernel A fp32 golden case {i}")
        votes, rc, rm = native.select_vote(_t(g[p + "q"]), _t(g[p + "k"]), _t(g[p + "tau"]),
                                           _t(g[p + "inv_freq"]), float(ps), 1.0, float(sm), int(tile),
                                           int(qb))
        a = orc.select_vote(g[p + "q"], g[p + "k"], orc.F32, g[p + "tau"], g[p + "inv_freq"], float(ps),
                            1.0, float(sm), int(tile), int(qb), band_eps=BAND, want_band=True)
        ndiff, nband = check_votes(votes.cpu().numpy(), g[p + "votes"], a["band"])
        check_votes(rc.cpu().numpy(), g[p + "row_counts"], a["band_rows"])
        print(f"[result] kernel A fp32 golden {i}: vote entries differing {ndiff} of {nband} band pairs",
              flush=True)


def test_kernel_a_matches_reference_goldens_bf16():
    import _sta_native as native
    g = _gold("kernel_a_bf16_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, ps, sm = g[p + "params"]
        say(f"kernel A bf16 golden case {i}")
        q = _t(g[p + "q"])
        k = _t(g[p + "k"])
        votes, rc, rm = native.select_vote(q, k, _t(g[p + "tau"]), _t(g[p + "inv_freq"]), float(ps), 1.0,
                                           float(sm), int(tile), 0)
        a = orc.select_vote(g[p + "q"], g[p + "k"], orc.BF16, g[p + "tau"], g[p + "inv_freq"], float(ps),
                            1.0, float(sm), int(tile), 0, band_eps=BAND, want_band=True)
        check_votes(votes.cpu().numpy(), g[p + "votes"], a["band"])


def test_composed_matches_reference_goldens_fp32():
    """The whole path against the reference's composed run.  Tiles whose votes equal the
    reference's must reproduce its sets and output; every other tile may differ only through
    band keys (votes within the band, sets exact given the votes, output exact given the sets)."""
    import _sta_native as native
    import shared_selection_triton_exact_2 as st
    g = _gold("composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        tile, kmax, pct, ng, nl, ps, qb, sm = g[p + "params"]
        tile, kmax, ng, nl, qb = int(tile), int(kmax), int(ng), int(nl), int(qb)
        say(f"composed fp32 golden case {i}")
        q, k, v = (_t(g[p + n])[None] for n in "qkv")
        tau, invf = _t(g[p + "tau"]), _t(g[p + "inv_freq"])
        r = native.shared_attention(q, k, v, tau, invf, float(ps), 1.0, invf, float(ps), 1.0,
                                    pct=float(pct), sm_scale=float(sm), n_global=ng, n_local=nl,
                                    tile=tile, k_max=kmax, q_pos_base=qb, want_votes=True)
        a = orc.select_vote(g[p + "q"], g[p + "k"], orc.F32, g[p + "tau"], g[p + "inv_freq"], float(ps),
                            1.0, float(sm), tile, qb, band_eps=BAND, want_band=True)
        votes = r["votes"].cpu().numpy()
        ndiff, _ = check_votes(votes, g[p + "votes"], a["band"])
        sets = gpu_sets_numpy(r)
        check_sets_given_votes(votes, sets, float(ps), ng, nl, float(pct), tile, kmax, qb)
        same_tile = np.all(votes == g[p + "votes"], axis=-1)                       # (H, nt)
        for name in SET_NAMES:
            ref = g[p + name]
            assert np.array_equal(sets[name][same_tile].astype(ref.dtype), ref[same_tile]), (i, name)
        out = r["out"].cpu().numpy()
        H, N, _ = out.shape
        rows_same = np.repeat(same_tile, tile, axis=1)[:, :N]                    # (H, N)
        check_output(out[rows_same], g[p + "out"][rows_same], orc.F32, f"golden {i} (same tiles)")
        out_ref = orc.gather_attn(g[p + "q"], g[p + "k"], g[p + "v"], orc.F32, sets["idx"],
                                  sets["newpos_k"], sets["newpos_q"], g[p + "inv_freq"], 1.0, float(sm),
                                  tile, kmax, 64, qb)
        check_output(out, out_ref, orc.F32, f"golden {i} (given sets)")
        print(f"[result] composed golden {i}: tiles with a band flip {int((~same_tile).sum())}, "
              f"vote entries differing {ndiff}", flush=True)
        # the drop-in entry point: same tensors, the reference's return types
        res = st.shared_pi_attention(q, k, v, tau, invf, pos_scale=float(ps), pct=float(pct),
                                     sm_scale=float(sm), n_global=ng, n_local=nl, tile=tile, k_max=kmax,
                                     q_pos_base=qb)
        assert torch.equal(res[0][0], r["out"])
        for name, got in zip(["shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas",
                              "overflow20"], res[1:]):
            assert got.dtype == torch.from_numpy(g[p + name]).dtype, (i, name)
            assert np.array_equal(got.cpu().numpy(), sets[name].astype(g[p + name].dtype)), (i, name)


def test_hybrid_matches_reference_golden_fp32():
    import shared_selection_triton_hybrid_exact as hy
    g = _gold("composed_golden.npz")
    tile, kmax, pct, ng, nl, ps_a, rs_a, ps_c, rs_c = g["hyb_params"]
    say("hybrid golden")
    q, k, v = (_t(g["hyb_" + n])[None] for n in "qkv")
    res = hy.shared_pi_attention(q, k, v, _t(g["hyb_tau"]), _t(g["hyb_inv_freq_a"]), float(ps_a),
                                 float(rs_a), _t(g["hyb_inv_freq_c"]), float(ps_c), float(rs_c),
                                 pct=float(pct), n_global=int(ng), n_local=int(nl), tile=int(tile),
                                 k_max=int(kmax))
    import _sta_native as native
    r = native.shared_attention(q, k, v, _t(g["hyb_tau"]), _t(g["hyb_inv_freq_a"]), float(ps_a), float(rs_a),
                                _t(g["hyb_inv_freq_c"]), float(ps_c), float(rs_c), pct=float(pct),
                                n_global=int(ng), n_local=int(nl), tile=int(tile), k_max=int(kmax),
                                want_votes=True)
    assert torch.equal(res[0][0], r["out"])
    sm = 1.0 / math.sqrt(g["hyb_q"].shape[-1])
    # the oracle's hybrid votes equal the reference's (pinned on the CPU)
    a = orc.select_vote(g["hyb_q"], g["hyb_k"], orc.F32, g["hyb_tau"], g["hyb_inv_freq_a"], float(ps_a),
                        float(rs_a), sm, int(tile), band_eps=BAND, want_band=True)
    votes = r["votes"].cpu().numpy()
    check_votes(votes, a["votes"], a["band"])
    same = np.all(votes == a["votes"], axis=-1)
    for j, name in enumerate(["shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas",
                              "overflow20"]):
        assert np.array_equal(res[1 + j].cpu().numpy()[same], g["hyb_" + name][same]), name
    rows = np.repeat(same, int(tile), axis=1)[:, :g["hyb_q"].shape[1]]
    check_output(res[0][0].cpu().numpy()[rows], g["hyb_out"][rows], orc.F32, "hybrid")


def test_gather_given_oracle_sets_bf16():
    """Kernel C alone on bf16 inputs, from the oracle's own idx/newpos."""
    import _sta_native as native
    from synthetic import planted_inputs, base_inv_freq
    H, N, D, T, kmax = 2, 640, 128, 64, 256
    q, k, v = planted_inputs(5, H, H, N, D, 0.02, torch.bfloat16)
    qn, dt = np_of(q[0]); kn, _ = np_of(k[0]); vn, _ = np_of(v[0])
    invf = base_inv_freq(D, 10000.0)
    sm = 1.0 / math.sqrt(D)
    a = orc.select_vote(qn, kn, dt, np.full(H, 5.0, np.float32), invf.numpy(), 0.5, 1.0, sm, T)
    idx, npk, npq, *_ = orc.build_sets(a["votes"], 0.5, 32, 32, 30.0, T, kmax)
    say("gather alone, bf16")
    out = native.gather_attention(q.to(DEV), k.to(DEV), v.to(DEV), invf.to(DEV), torch.from_numpy(idx),
                                  torch.from_numpy(npk), torch.from_numpy(npq), sm, 1.0, T, kmax)
    ref = orc.gather_attn(qn, kn, vn, dt, idx, npk, npq, invf.numpy(), 1.0, sm, T, kmax)
    check_output(out.float().cpu().numpy(), ref, dt, "gather bf16")


# ------------------------------------------------------------------------------------------
# end to end on seeded synthetic inputs
# ------------------------------------------------------------------------------------------
def test_config0_end_to_end_fp32():
    from synthetic import CONFIGS
    c = CONFIGS["c0"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    full_check(q, k, v, torch.full((c.H,), c.tau), invf.to(DEV), ps, rs, tile=c.tile, k_max=c.k_max,
               what="config 0")


def test_pi_bf16_d128_truncation():
    """config-1 geometry (PI 1/3, tile 64, bf16, d128) at N=4096 with k_max=512, so the 30->25->20
    fallback and the unresolved-tile truncation both occur."""
    from synthetic import planted_inputs, base_inv_freq, pi_pos_scale
    H, N, D = 4, 4096, 128
    q, k, v = planted_inputs(1, H, H, N, D, 0.01, torch.bfloat16, DEV)
    _, sets = full_check(q, k, v, torch.full((H,), 5.0), base_inv_freq(D, 10000.0).to(DEV),
                         pi_pos_scale(4096, 12288), 1.0, tile=64, k_max=512, what="PI bf16 truncation")
    assert sets["overflow20"].any()
    assert ((sets["chosen"] == 25) | (sets["chosen"] == 20)).any()


def test_yarn_gqa_bf16():
    from synthetic import planted_inputs, yarn_inv_freq
    H, Hkv, N, D = 8, 2, 2048, 128
    q, k, v = planted_inputs(2, H, Hkv, N, D, 0.005, torch.bfloat16, DEV)
    invf, msc = yarn_inv_freq(D, 500000.0, 4.0, 8192)
    full_check(q, k, v, torch.full((H,), 5.0), invf.to(DEV), 1.0, msc, tile=64, k_max=300,
               what="YaRN GQA bf16")


def test_hybrid_fp16_ragged_tile32():
    from synthetic import planted_inputs, yarn_inv_freq, base_inv_freq
    H, N, D = 4, 1000, 64
    q, k, v = planted_inputs(3, H, H, N, D, 0.02, torch.float16, DEV)
    invf_a, msc = yarn_inv_freq(D, 10000.0, 3.0, 512)
    full_check(q, k, v, torch.full((H,), 4.0), invf_a.to(DEV), 1.0, msc,
               base_inv_freq(D, 10000.0).to(DEV), 0.25, 1.0, tile=32, k_max=128, n_global=8,
               n_local=16, measure=True, what="hybrid fp16 ragged tile 32")


@pytest.mark.parametrize("N", [1, 5, 33, 64, 65])
def test_tiny_sequences(N):
    from synthetic import planted_inputs, base_inv_freq
    q, k, v = planted_inputs(4, 2, 2, N, 64, 0.1, torch.bfloat16, DEV)
    full_check(q, k, v, torch.full((2,), 3.0), base_inv_freq(64, 10000.0).to(DEV), 1.0, 1.0, tile=64,
               k_max=16, n_global=4, n_local=4, what=f"tiny N={N}")


def test_q_pos_base_and_pct_variants():
    from synthetic import planted_inputs, base_inv_freq
    q, k, v = planted_inputs(6, 2, 2, 300, 64, 0.05, torch.float32, DEV)
    for pct, qb in [(25.0, 0), (22.5, 17), (0.0, 0), (100.0, 5)]:
        full_check(q, k, v, torch.full((2,), 3.0), base_inv_freq(64, 10000.0).to(DEV), 0.5, 1.0,
                   pct=pct, tile=32, k_max=64, n_global=4, n_local=8, q_pos_base=qb, measure=True,
                   what=f"pct {pct} q_pos_base {qb}")


def test_strided_inputs_match_contiguous():
    """(B, N, H, D).transpose(1, 2) inputs, as the model's projections produce them."""
    import shared_selection_triton_exact_2 as st
    from synthetic import base_inv_freq
    g = torch.Generator("cpu").manual_seed(9)
    x = torch.randn(1, 512, 4, 128, generator=g).to(torch.bfloat16).to(DEV)
    q = x.transpose(1, 2)
    k = (x * 0.5).transpose(1, 2)
    v = (x * 2.0).transpose(1, 2)
    invf = base_inv_freq(128, 10000.0).to(DEV)
    tau = torch.full((4,), 5.0)
    say("strided inputs")
    a = st.shared_pi_attention(q, k, v, tau, invf, pos_scale=0.5, tile=64, k_max=128)
    b = st.shared_pi_attention(q.contiguous(), k.contiguous(), v.contiguous(), tau, invf, pos_scale=0.5,
                               tile=64, k_max=128)
    for x1, x2 in zip(a, b):
        assert torch.equal(x1, x2)


def test_identity_kat_dense_rope_attention():
    """tau=inf, pct=100, k_max >= N: dense causal attention with native RoPE, in float64."""
    from synthetic import planted_inputs, base_inv_freq
    import shared_selection_triton_exact_2 as st
    H, N, D = 2, 512, 128
    for dtype, tol in [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)]:
        q, k, v = planted_inputs(8, H, H, N, D, 0.02, dtype, DEV)
        invf = base_inv_freq(D, 10000.0)
        say(f"identity KAT {dtype}")
        out = st.shared_pi_attention(q, k, v, torch.full((H,), float("inf")), invf.to(DEV), pct=100.0,
                                     tile=64, k_max=N)[0][0].double().cpu()
        qd, kd, vd = (x[0].double().cpu() for x in (q, k, v))
        pos = torch.arange(N, dtype=torch.float64)
        ang = pos[:, None] * invf.double()[None, :]
        def rot(x):
            z = torch.complex(x[..., :D // 2], x[..., D // 2:]) * torch.polar(torch.ones_like(ang), ang)
            return torch.cat([z.real, z.imag], -1)
        s = rot(qd) @ rot(kd).transpose(-1, -2) / math.sqrt(D)
        s = s.masked_fill(torch.triu(torch.ones(N, N, dtype=torch.bool), 1), float("-inf"))
        ref = torch.softmax(s, -1) @ vd
        err = (out - ref).abs().max().item()
        assert err < tol, (dtype, err)


def test_config1_full_size_head_spot_check():
    """config 1 at full size (32 heads x 12288 x d128, bf16): structural invariants on every tile,
    the three-layer oracle check on six heads and the set-level comparison with the oracle's own
    sets (every differing key classified and counted)."""
    import _sta_native as native
    from synthetic import CONFIGS
    c = CONFIGS["c1"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    invf = invf.to(DEV)
    tau = torch.full((c.H,), c.tau)
    say("config 1 full size")
    r = native.shared_attention(q, k, v, tau, invf, ps, rs, invf, ps, rs, pct=c.pct, tile=c.tile,
                                k_max=c.k_max, want_votes=True, want_row_max=True)
    torch.cuda.synchronize()
    idx = r["idx"]
    ks = r["kept_size"]
    nvalid = torch.clamp(ks, max=c.k_max)
    slot = torch.arange(c.k_max, device=DEV)
    valid = slot[None, None, :] < nvalid[..., None]
    assert torch.all(torch.where(valid, idx < c.N, idx == c.N))
    d = idx[..., 1:] - idx[..., :-1]
    assert torch.all(torch.where(valid[..., 1:], d > 0, torch.ones_like(d, dtype=torch.bool)))
    assert torch.isfinite(r["out"].float()).all()
    print(f"[result] config 1: kept mean {ks.float().mean().item():.1f}, "
          f"overflow20 {int(r['overflow20'].sum())}, chosen {torch.unique(r['chosen']).tolist()}", flush=True)
    # six heads, every tile of each (the deepest tiles carry the truncation path)
    heads = [0, 7, 13, 21, 26, 31]
    total = {"tiles": 0, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0, "trunc": 0}
    for h in heads:
        qh, kh, vh = q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1]
        qn, dt = np_of(qh[0]); kn, _ = np_of(kh[0]); vn, _ = np_of(vh[0])
        a = orc.select_vote(qn, kn, dt, np.full(1, c.tau, np.float32), invf.cpu().numpy(), ps, rs,
                            1.0 / math.sqrt(c.D), c.tile, band_eps=BAND, want_band=True)
        votes_g = r["votes"][h:h + 1].cpu().numpy()
        ndiff, nband = check_votes(votes_g, a["votes"], a["band"])
        sets_g = {n: r[n][h:h + 1].cpu().numpy() for n in SET_NAMES}
        check_sets_given_votes(votes_g, sets_g, ps, c.n_global, c.n_local, c.pct, c.tile, c.k_max)
        sd = set_level_diffs(votes_g, a, ps, c.n_global, c.n_local, c.pct, c.tile, c.k_max,
                             what=f"config 1 head {h}")
        for n in total:
            total[n] += sd[n]
        out_ref = orc.gather_attn(qn, kn, vn, dt, sets_g["idx"], sets_g["newpos_k"], sets_g["newpos_q"],
                                  invf.cpu().numpy(), rs, 1.0 / math.sqrt(c.D), c.tile, c.k_max, 64)
        err = check_output(r["out"][h:h + 1].float().cpu().numpy(), out_ref, dt, f"c1 head {h}")
        print(f"[result] config 1 head {h}: vote entries differing {ndiff} (band pairs {nband}), "
              f"max out err {err:.2e}", flush=True)
    report_set_diffs(f"config 1, heads {heads}", total)


def test_config2_full_length_gqa_group():
    """config 2's geometry at full length (YaRN factor 4 from 8192, theta 5e5, 32768 tokens,
    d128, bf16) on one GQA group of two query heads sharing a KV head, three-layer check."""
    from synthetic import CONFIGS, planted_inputs
    c = CONFIGS["c2"]
    q, k, v = planted_inputs(0, 2, 1, c.N, c.D, c.frac, c.dtype, DEV)
    invf, ps, rs = c.geometry()
    tau = torch.full((2,), c.tau, device=DEV)
    full_check(q, k, v, tau, invf.to(DEV), ps, rs, pct=c.pct, tile=c.tile, k_max=c.k_max,
               n_global=c.n_global, n_local=c.n_local, what="config 2 full length, 2 q heads / 1 kv head")


def test_config2_full_size_three_gqa_groups():
    """config 2 as written (32 query heads over 8 KV heads, 32768 tokens, YaRN, bf16) in one call,
    then two query heads of each of three GQA groups (KV heads 0, 3, 7) against the oracle: votes
    within the band, sets given the votes bit for bit, the set-level comparison with the
    oracle's own sets, and the outputs given the GPU's sets."""
    import _sta_native as native
    from synthetic import CONFIGS
    c = CONFIGS["c2"]
    q, k, v = c.inputs(DEV)
    invf, ps, rs = c.geometry()
    invf = invf.to(DEV)
    say("config 2 full size, 32 q heads / 8 kv heads")
    r = native.shared_attention(q, k, v, torch.full((c.H,), c.tau), invf, ps, rs, invf, ps, rs, pct=c.pct,
                                tile=c.tile, k_max=c.k_max, want_votes=True, want_row_max=True)
    torch.cuda.synchronize()
    G = c.H // c.Hkv
    total = {"tiles": 0, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0, "trunc": 0}
    for kvh, heads in ((0, [0, 1]), (3, [12, 14]), (7, [29, 31])):
        assert all(h // G == kvh for h in heads)
        qn, dt = np_of(q[0, heads])
        kn, _ = np_of(k[0, kvh:kvh + 1])
        vn, _ = np_of(v[0, kvh:kvh + 1])
        a = orc.select_vote(qn, kn, dt, np.full(len(heads), c.tau, np.float32), invf.cpu().numpy(), ps, rs,
                            1.0 / math.sqrt(c.D), c.tile, band_eps=BAND, want_band=True)
        votes_g = r["votes"][heads].cpu().numpy()
        ndiff, nband = check_votes(votes_g, a["votes"], a["band"])
        assert np.max(np.abs(r["row_max"][heads].cpu().numpy() - a["row_max"])) < 1e-4, "row max"
        sets_g = {n: r[n][heads].cpu().numpy() for n in SET_NAMES}
        check_sets_given_votes(votes_g, sets_g, ps, c.n_global, c.n_local, c.pct, c.tile, c.k_max)
        sd = set_level_diffs(votes_g, a, ps, c.n_global, c.n_local, c.pct, c.tile, c.k_max,
                             what=f"config 2 kv head {kvh}")
        for n in total:
            total[n] += sd[n]
        out_ref = orc.gather_attn(qn, kn, vn, dt, sets_g["idx"], sets_g["newpos_k"], sets_g["newpos_q"],
                                  invf.cpu().numpy(), rs, 1.0 / math.sqrt(c.D), c.tile, c.k_max, 64)
        err = check_output(r["out"][heads].float().cpu().numpy(), out_ref, dt, f"c2 kv head {kvh}")
        print(f"[result] config 2 q heads {heads} (kv head {kvh}): vote entries differing {ndiff} "
              f"(band pairs {nband}), max out err {err:.2e}", flush=True)
    report_set_diffs("config 2 full size, q heads 0 1 12 14 29 31", total)


@pytest.mark.parametrize("k_max", [2048, 10000])
def test_build_sets_slot_paths(k_max):
    """_build_sets on random votes with the kept slots staged in LDS (k_max 2048) and written
    straight from the compaction (k_max 10000: the staged slots would pass 80 KB of LDS):
    bit-exact against the oracle either way."""
    import _sta_native as native
    rng = np.random.default_rng(97)
    H, T, N = 2, 64, 12000
    nt = (N + T - 1) // T
    votes = rng.integers(0, 65, size=(H, nt, N)).astype(np.int32)
    votes[votes < 40] = 0                                  # most keys unvoted, as in real tiles
    say(f"build_sets slot paths: k_max={k_max}")
    res = native.build_sets(torch.from_numpy(votes).to(DEV), 1.0 / 3.0, 32, 32, 30.0, T, k_max, 0, True)
    ref = orc.build_sets(votes, 1.0 / 3.0, 32, 32, 30.0, T, k_max, 0, True)
    for name, got, r in zip(SET_NAMES, res, ref):
        got = got.cpu().numpy()
        r = np.asarray(r)
        if r.dtype == np.float32:
            assert np.array_equal(got.view(np.uint32), r.view(np.uint32)), name
        else:
            assert np.array_equal(got.astype(r.dtype), r), name
