"""GPU parity of the per-query variant (PQ Union) through the C ABI.

Layers, as for the shared path:
  1. bits: per (head, tile, key) the GPU's keep bits may differ from the oracle's only in rows
     whose score lies within BAND of that row's threshold (popcount of the XOR <= band count);
     weighted votes agree to fp32 rounding where the bits agree;
  2. sets given the GPU's own votes / bits / wvotes: the oracle's _build_sets_pq reproduces idx,
     newpos, mask and the statistics bit for bit (both take tied rank values in key order);
  3. output given the GPU's sets: the oracle's masked Kernel C within 1e-4 (fp32) or 2e-2 abs +
     1e-2 rel (bf16).
Against the reference's own fixtures: _build_sets_pq through the device, and the composed
shared_pq_attention where the sets agree.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import (BAND, PQ_SET_NAMES, check_output, classify_pq_set_diffs, compare_pq_sets,
                            np_of, out_f32, pq_rank_values, report_pq_set_diffs)

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


def _np(r):
    """device tensors -> numpy (half-precision tensors are upcast to fp32)"""
    def one(v):
        if not torch.is_tensor(v):
            return v
        if v.dtype in (torch.bfloat16, torch.float16):
            v = v.float()
        return v.cpu().numpy()
    return {k: one(v) for k, v in r.items()}


def check_bits(bits_g, bits_o, band):
    x = (bits_g.view(np.uint32) ^ bits_o.view(np.uint32)).astype(np.uint64)
    pc = np.zeros(x.shape, np.int64)
    for r in range(32):
        pc += ((x >> np.uint64(r)) & np.uint64(1)).astype(np.int64)
    bad = pc > band
    assert not bad.any(), f"{int(bad.sum())} keys differ in more rows than the band allows"
    return int((pc > 0).sum())


def pq_full_check(q, k, v, tau, invf_a, ps_a, rs_a, invf_c, n_global=32, n_local=32, k_max=2048,
                  q_pos_base=0, select_score="expmass", what=""):
    import _sta_native as native
    H, N, D = q.shape[1], q.shape[2], q.shape[3]
    sm = 1.0 / math.sqrt(D)
    mode = native.SCORES[select_score]
    say(f"{what}: H={H} Hkv={k.shape[1]} N={N} D={D} k_max={k_max} {select_score} dtype={q.dtype}")
    r = native.pq_attention(q, k, v, tau, invf_a, invf_c, ps_a, rs_a, sm, n_global, n_local, 32, k_max,
                            q_pos_base, select_score, want_votes=True, want_row_max=True)
    torch.cuda.synchronize()
    g = _np(r)
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    a = orc.select_bits(qn, kn, dt, tau.cpu().numpy(), invf_a.cpu().numpy(), ps_a, rs_a, sm, 32,
                        q_pos_base, mode, band_eps=BAND, want_band=True)
    ndiff = check_bits(g["bits"], a["bits"], a["band"])
    pc = np.zeros_like(g["votes"])
    for rr in range(32):
        pc += (g["bits"].view(np.uint32) >> np.uint32(rr)).astype(np.int32) & 1
    assert np.array_equal(pc, g["votes"]), "votes are not the popcount of the bits"
    assert np.max(np.abs(g["row_max"] - a["row_max"])) < 1e-4, "row max"
    if mode > 0:
        same = g["bits"] == a["bits"]
        np.testing.assert_allclose(g["wvotes"][same], a["wvotes"][same], rtol=2e-5, atol=2e-5)
    # sets given the GPU's own votes / bits / wvotes: bit-exact
    ref = orc.build_sets_pq(g["votes"], g["bits"], g["wvotes"], n_global, n_local, 32, k_max, q_pos_base, mode)
    for name, rv in zip(PQ_SET_NAMES, ref):
        gv = g[name]
        if rv.dtype == np.float32:
            assert np.array_equal(gv.view(np.uint32), rv.view(np.uint32)), name
        else:
            assert np.array_equal(gv.astype(np.int64), rv.astype(np.int64)), name
    # sets against the oracle's sets from the oracle's own bits: every differing key classified
    ro = orc.build_sets_pq(a["votes"], a["bits"], a["wvotes"], n_global, n_local, 32, k_max, q_pos_base, mode)
    sd = classify_pq_set_diffs(a["band"], g, dict(zip(PQ_SET_NAMES, ro)),
                               pq_rank_values(g["votes"], g["wvotes"], mode),
                               pq_rank_values(a["votes"], a["wvotes"], mode), N)
    report_pq_set_diffs(what, sd)
    if ndiff == 0 and mode == 0:
        assert sd["keys"] == 0
    out_ref = orc.gather_attn_mask(qn, kn, vn, dt, g["idx"], g["newpos_k"], g["newpos_q"], g["mask"],
                                   invf_c.cpu().numpy(), 1.0, sm, 32, k_max, 64, q_pos_base)
    err = check_output(out_f32(r["out"]), out_ref, dt, what)
    print(f"[result] {what}: keys with flipped bits {ndiff} (band pairs {int(a['band'].sum())}), max out "
          f"err {err:.2e}, kept mean {g['kept_size'].mean():.1f}, overflow {int(g['overflow'].sum())}/"
          f"{g['overflow'].size}", flush=True)
    return r, a


def test_pq_build_sets_goldens():
    import _sta_native as native
    g = _gold("build_sets_pq_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        ng, nl, T, kmax, qb, mode = (int(x) for x in g[p + "params"])
        say(f"build_sets_pq golden {i}")
        votes, bits, wv = g[p + "votes"], g[p + "bits"], g[p + "wvotes"]
        res = native.pq_build_sets(torch.from_numpy(votes).to(DEV), torch.from_numpy(bits).to(DEV),
                                   torch.from_numpy(wv).to(DEV), ng, nl, T, kmax, qb,
                                   ["freq", "margin", "expmass"][mode])
        got = {n: t.cpu().numpy() for n, t in zip(PQ_SET_NAMES, res)}
        compare_pq_sets(got, {n: g[p + n] for n in PQ_SET_NAMES}, pq_rank_values(votes, wv, mode),
                        votes.shape[-1])
        # and the oracle's tie rule exactly
        ref = orc.build_sets_pq(votes, bits, wv, ng, nl, T, kmax, qb, mode)
        for name, rv in zip(PQ_SET_NAMES, ref):
            assert np.array_equal(np.asarray(got[name]).astype(np.float64), rv.astype(np.float64)), (i, name)


def _radix_case(seed, N, nt, kind):
    """Dense (1, nt, N) votes / bits / wvotes that steer _build_sets_pq's budget cut through one
    path of the device's radix select."""
    g = np.random.default_rng(seed)
    votes = g.integers(1, 33, size=(1, nt, N)).astype(np.int32)
    votes[:, :, g.random(N) < 0.2] = 0                       # some keys outside the union
    bits = g.integers(-2**31, 2**31 - 1, size=(1, nt, N), dtype=np.int64).astype(np.int32)
    if kind == "wide_bin":
        # ~4000 candidates share key bits 31..20 (values in [1, 1.125)) and hold the cut: more
        # than the LDS list holds, so the remaining bits resolve over all keys
        wv = (1.0 + 0.125 * g.random((1, nt, N))).astype(np.float32)
        wv[:, :, :100] = 4.0 + g.random((1, nt, 100)).astype(np.float32)
        wv[:, :, 200:260] = wv[:, :, 300:360]                 # exact ties
    elif kind == "list_bin":
        # the cut's bin holds a few hundred keys: the list path, with ties at the cut
        wv = (0.01 + 10.0 * g.random((1, nt, N)) ** 3).astype(np.float32)
        wv[:, :, 1000:1400] = wv[:, :, 1400:1800]
    elif kind == "nonpositive":
        # the cut falls among negative rank values (caller-given weighted votes), with ties
        wv = -(0.001 + np.abs(g.normal(size=(1, nt, N)))).astype(np.float32)
        wv[:, :, :100] = -wv[:, :, :100]
        wv[:, :, 1000:1200] = wv[:, :, 1200:1400]
    elif kind == "big_votes":
        # caller votes of 2047 and more hold the statistic: the full float-key radix
        votes = np.where(votes > 0, g.integers(2000, 2100, size=(1, nt, N)), 0).astype(np.int32)
        wv = np.zeros((1, nt, N), np.float32)
    else:   # "small_votes": the vote count is the level-1 digit
        wv = np.zeros((1, nt, N), np.float32)
    return votes, bits, wv


@pytest.mark.parametrize("kind,mode,N", [("wide_bin", 2, 6000), ("list_bin", 1, 6000), ("nonpositive", 1, 6000),
                                         ("big_votes", 0, 6000), ("small_votes", 0, 6000), ("wide_bin", 2, 40000),
                                         ("list_bin", 2, 40000), ("small_votes", 0, 40000)])
def test_pq_build_sets_radix_paths(kind, mode, N):
    """Every path of the device's budget cut (vote-count digit, weighted list, weighted bin too wide
    for the list, caller votes of 2047 and more, non-positive rank values) against the oracle, bit
    for bit, with exact ties at the cut; at N = 40000 the rank keys outgrow the LDS and every pass
    reads them from the vote rows."""
    import _sta_native as native
    nt, T, kmax, ng, nl = 3, 32, 256, 8, 8
    votes, bits, wv = _radix_case(7, N, nt, kind)
    say(f"pq radix path {kind}, rank mode {mode}, N={N}")
    res = native.pq_build_sets(torch.from_numpy(votes).to(DEV), torch.from_numpy(bits).to(DEV),
                               torch.from_numpy(wv).to(DEV), ng, nl, T, kmax, N - nt * T,
                               ["freq", "margin", "expmass"][mode])
    got = {n: t.cpu().numpy() for n, t in zip(PQ_SET_NAMES, res)}
    ref = orc.build_sets_pq(votes, bits, wv, ng, nl, T, kmax, N - nt * T, mode)
    assert bool(np.asarray(got["overflow"]).all())
    for name, rv in zip(PQ_SET_NAMES, ref):
        assert np.array_equal(np.asarray(got[name]).astype(np.float64), rv.astype(np.float64)), name


def test_pq_composed_goldens():
    import _sta_native as native
    g = _gold("pq_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, kmax, mode, qb = g[p + "params"]
        ng, nl, kmax, mode, qb = int(ng), int(nl), int(kmax), int(mode), int(qb)
        sc = ["freq", "margin", "expmass"][mode]
        q, k, v = (torch.from_numpy(g[p + n]).to(DEV)[None] for n in ("q", "k", "v"))
        tau = torch.from_numpy(g[p + "tau"]).to(DEV)
        ia, ic = torch.from_numpy(g[p + "inv_freq_a"]).to(DEV), torch.from_numpy(g[p + "inv_freq_c"]).to(DEV)
        r, a = pq_full_check(q, k, v, tau, ia, float(psa), float(rsa), ic, ng, nl, kmax, qb, sc,
                             what=f"pq composed golden {i} ({sc})")
        got = {n: r[n].cpu().numpy() for n in PQ_SET_NAMES}
        if np.array_equal(got["mask"].astype(np.int64), g[p + "mask"].astype(np.int64)) and \
                np.array_equal(got["idx"], g[p + "idx"]):
            np.testing.assert_allclose(r["out"].cpu().numpy(), g[p + "out"], atol=1e-4, rtol=1e-4)
        else:
            # only keys tied at the overflow cut (freq ranking) may differ from the reference
            assert mode == 0, f"case {i}: sets differ from the reference outside the freq tie rule"
            compare_pq_sets(got, {n: g[p + n] for n in PQ_SET_NAMES},
                            pq_rank_values(g[p + "votes"], g[p + "wvotes"], mode), q.shape[2])


@pytest.mark.parametrize("mode", ["expmass", "freq", "margin"])
def test_pq_bf16_overflow(mode):
    from synthetic import planted_inputs, base_inv_freq
    H, N, D = 4, 1536, 128
    q, k, v = planted_inputs(31, H, H, N, D, 0.01, torch.bfloat16, DEV)
    tau = torch.full((H,), 4.0, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    pq_full_check(q, k, v, tau, invf, 0.25, 1.0, invf, 32, 32, 384, 0, mode, what=f"pq bf16 overflow {mode}")


def test_pq_gqa_fp16_qbase():
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, N, D = 4, 2, 999, 64
    q, k, v = planted_inputs(32, H, Hkv, N, D, 0.02, torch.float16, DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    pq_full_check(q, k, v, tau, invf * 0.5, 1.0, 1.1386294, invf, 8, 16, 200, 40, "expmass",
                  what="pq gqa fp16 q_pos_base 40")


def test_pq_dropin_and_errors():
    import shared_selection_triton_perquery as pq
    from synthetic import planted_inputs, base_inv_freq
    H, N, D = 2, 300, 64
    q, k, v = planted_inputs(33, H, H, N, D, 0.02, torch.bfloat16, DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    say("pq drop-in module")
    pq.reset_overflow_stats()
    out, usize, kept, ovf = pq.shared_pq_attention(q, k, v, tau, invf, invf, pos_scale_a=0.5, k_max=128)
    assert out.shape == (1, H, N, D) and out.dtype == torch.bfloat16
    assert usize.dtype == torch.int32 and kept.dtype == torch.int32 and ovf.dtype == torch.bool
    st = pq.get_overflow_stats()["prefill"]
    assert st["total_cells"] == H * ((N + 31) // 32)
    with pytest.raises(AssertionError):
        pq.shared_pq_attention(q, k, v, tau, invf, invf, tile=64)
    with pytest.raises(AssertionError):
        pq.shared_pq_attention(q, k, v, tau, invf, invf, n_global=64, n_local=64, k_max=128)


def test_pq_config3_full_size_one_head():
    """Config 3 at full size (N=16384, d128, bf16, tau 4, PI 1/4, k_max 2048) for two heads."""
    from synthetic import CONFIGS
    cfg = CONFIGS["c3"]
    q, k, v = cfg.inputs(DEV)
    q, k, v = q[:, :2].contiguous(), k[:, :2].contiguous(), v[:, :2].contiguous()
    invf, ps, rs = cfg.geometry()
    invf = invf.to(DEV)
    tau = torch.full((2,), cfg.tau, device=DEV)
    pq_full_check(q, k, v, tau, invf, ps, rs, invf, cfg.n_global, cfg.n_local, cfg.k_max, 0,
                  cfg.select_score, what="config 3 full size, 2 heads")
