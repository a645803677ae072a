"""GPU: the screened pass 1 of the score kernel against the three-product sweep and the oracle.

The score kernel's pass 1 (exact row max, shared_selection_triton_exact_2.py:87-103) normally
sweeps with one bf16 product per score and evaluates exactly only the keys that can hold a row's
maximum; STA_EXACT_PASS1=1 forces the three-product sweep.  Both must give the oracle's row max
(within 1e-4) and votes that differ from the oracle's only inside the 1e-3 band.  Inputs with
tied scores make the screen inconclusive, which sends the workgroup to the three-product sweep:
those cases check that fallback.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, check_votes, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _kernel_a(q, k, tau, invf, ps, rs, tile, q_pos_base, exact):
    import _sta_native as native
    old = os.environ.pop("STA_EXACT_PASS1", None)
    try:
        if exact:
            os.environ["STA_EXACT_PASS1"] = "1"
        votes, _, rm = native.select_vote(q, k, tau, invf, ps, rs, 1.0 / math.sqrt(q.shape[-1]), tile,
                                          q_pos_base)
        torch.cuda.synchronize()
    finally:
        os.environ.pop("STA_EXACT_PASS1", None)
        if old is not None:
            os.environ["STA_EXACT_PASS1"] = old
    return votes.cpu().numpy(), rm.cpu().numpy()


def _check_both(q, k, tau, invf, ps, rs, tile, q_pos_base, what):
    say(what)
    D = q.shape[-1]
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    a = orc.select_vote(qn, kn, dt, tau.cpu().numpy(), invf.cpu().numpy(), ps, rs, 1.0 / math.sqrt(D), tile,
                        q_pos_base, band_eps=BAND, want_band=True)
    res = {}
    for exact in (False, True):
        votes, rm = _kernel_a(q, k, tau, invf.to(DEV), ps, rs, tile, q_pos_base, exact)
        err = float(np.max(np.abs(rm - a["row_max"])))
        assert err < 1e-4, f"{what} (exact={exact}): row max differs from the oracle by {err:.3e}"
        ndiff, nband = check_votes(votes, a["votes"], a["band"])
        res[exact] = (votes, rm, ndiff)
        print(f"[result] {what} exact_pass1={exact}: row max err {err:.2e}, vote entries differing "
              f"{ndiff} (band pairs {nband})", flush=True)
    # the two sweeps find the same maxima up to the rounding of the dropped lo.lo term
    d = float(np.max(np.abs(res[False][1] - res[True][1])))
    assert d < 1e-4, f"{what}: screened and three-product row maxima differ by {d:.3e}"
    return res


@pytest.mark.parametrize("case", [
    # (H, Hkv, N, D, dtype, tile, q_pos_base, pos_scale)
    (2, 1, 3000, 128, torch.bfloat16, 64, 0, 0.25),
    (2, 2, 1000, 64, torch.float32, 32, 0, 1.0),
    (4, 2, 4133, 128, torch.bfloat16, 64, 37, 1.0 / 3.0),
    (2, 2, 2049, 128, torch.float16, 32, 0, 0.5),
])
def test_screened_pass1_matches_exact_sweep(case):
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, N, D, dt, tile, qpb, ps = case
    q, k, _ = planted_inputs(3, H, Hkv, N, D, 0.01, dt, DEV)
    invf = base_inv_freq(D, 10000.0)
    tau = torch.full((H,), 5.0)
    _check_both(q, k, tau, invf, ps, 1.0, tile, qpb,
                f"screened vs exact pass 1: H={H} Hkv={Hkv} N={N} D={D} {dt} tile={tile} q_pos_base={qpb}")


def test_screened_pass1_ties_fall_back():
    """Every key of a head identical (all of a row's scores tie) and some query rows zero: the
    screen cannot single out a maximum, so those workgroups take the three-product sweep."""
    from synthetic import base_inv_freq
    H, N, D = 2, 1500, 128
    g = torch.Generator("cpu").manual_seed(5)
    q = torch.randn(1, H, N, D, generator=g)
    q[:, :, 300:700] = 0.0
    k = torch.randn(1, H, N, D, generator=g)
    k[:, 0] = k[:, 0, :1]                      # head 0: one key repeated
    q, k = q.to(torch.bfloat16).to(DEV), k.to(torch.bfloat16).to(DEV)
    invf = base_inv_freq(D, 10000.0)
    tau = torch.full((H,), 5.0)
    # position-free geometry (pos_scale 0): repeated keys give exactly tied scores
    _check_both(q, k, tau, invf, 0.0, 1.0, 64, 0, "tied scores: repeated keys, zero query rows")


def test_screened_pass1_full_length_config1_head():
    """config 1's shape and geometry on one head (12288 keys): the screened sweep against the
    oracle and the three-product sweep."""
    from synthetic import CONFIGS, planted_inputs
    c = CONFIGS["c1"]
    q, k, _ = planted_inputs(0, 1, 1, c.N, c.D, c.frac, c.dtype, DEV)
    invf, ps, rs = c.geometry()
    _check_both(q, k, torch.full((1,), c.tau), invf, ps, rs, c.tile, 0, "config 1 shape, one head")


def test_tau_zero_keeps_each_rows_best_key():
    """tau = 0: every valid row keeps its own maximum (qk == m passes the reference's keep test,
    exact_2.py:121), with the screened pass 1 as with the three-product one.  The screen's row max
    comes from fp32 dots of the (hi + lo) operands and pass 2 scores with three bf16 products, so
    the threshold is capped just below the maximum; keys within that cap of m are band keys."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D, tile = 2, 2000, 128, 64
    q, k, _ = planted_inputs(12, H, H, N, D, 0.01, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.zeros(H)
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    a = orc.select_vote(qn, kn, dt, tau.numpy(), invf.cpu().numpy(), 0.5, 1.0, 1.0 / math.sqrt(D), tile,
                        band_eps=BAND, want_band=True)
    for exact in (False, True):
        say(f"tau 0, exact_pass1={exact}")
        old = os.environ.pop("STA_EXACT_PASS1", None)
        try:
            if exact:
                os.environ["STA_EXACT_PASS1"] = "1"
            votes, rc, rm = native.select_vote(q, k, tau, invf, 0.5, 1.0, 1.0 / math.sqrt(D), tile)
            torch.cuda.synchronize()
        finally:
            os.environ.pop("STA_EXACT_PASS1", None)
            if old is not None:
                os.environ["STA_EXACT_PASS1"] = old
        rc = rc.cpu().numpy()
        assert (rc >= 1).all(), f"exact_pass1={exact}: {int((rc < 1).sum())} rows keep no key"
        ndiff, nband = check_votes(votes.cpu().numpy(), a["votes"], a["band"])
        print(f"[result] tau 0 exact_pass1={exact}: min row count {int(rc.min())}, vote entries "
              f"differing {ndiff} (band pairs {nband})", flush=True)


def test_negative_tau_keeps_no_key():
    """tau < 0 puts the threshold above every row's maximum: the reference keeps no key
    (exact_2.py:121), with the screened pass 1 as with the three-product one."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D, tile = 2, 1500, 128, 64
    q, k, _ = planted_inputs(14, H, H, N, D, 0.01, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.tensor([-0.5, -3.0])
    for exact in (False, True):
        say(f"tau < 0, exact_pass1={exact}")
        old = os.environ.pop("STA_EXACT_PASS1", None)
        try:
            if exact:
                os.environ["STA_EXACT_PASS1"] = "1"
            votes, rc, _ = native.select_vote(q, k, tau, invf, 0.5, 1.0, 1.0 / math.sqrt(D), tile)
            torch.cuda.synchronize()
        finally:
            os.environ.pop("STA_EXACT_PASS1", None)
            if old is not None:
                os.environ["STA_EXACT_PASS1"] = old
        assert int(votes.abs().sum()) == 0 and int(rc.abs().sum()) == 0, f"exact_pass1={exact}"


def _gathered(fn):
    """fn() with STA_SCREEN_GATHER=1: the screen takes its candidate keys from the K fragments."""
    old = os.environ.pop("STA_SCREEN_GATHER", None)
    os.environ["STA_SCREEN_GATHER"] = "1"
    try:
        r = fn()
        torch.cuda.synchronize()
    finally:
        os.environ.pop("STA_SCREEN_GATHER", None)
        if old is not None:
            os.environ["STA_SCREEN_GATHER"] = old
    return r


@pytest.mark.parametrize("case", [
    # (H, Hkv, N, D, dtype, q_pos_base, pos_scale)
    (2, 1, 3000, 128, torch.bfloat16, 0, 1.0 / 3.0),
    (2, 2, 2049, 128, torch.float16, 37, 0.5),
    (2, 2, 1000, 64, torch.float32, 0, 1.0),
])
def test_screen_candidates_rebuilt_from_table_match_fragment_gathers(case):
    """The screen scores its candidate keys from the raw K rows and the K rope's (cos, sin) table;
    STA_SCREEN_GATHER=1 makes the same kernel gather those keys from the K fragments instead.  The
    rebuild repeats the rope pre-kernel's fp32 rotation and split, so both feed the matrix cores
    the same bits and the row maxima agree bit for bit, on the shared path and the per-query one."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, N, D, dt, qpb, ps = case
    say(f"table vs fragment candidates: H={H} Hkv={Hkv} N={N} D={D} {dt} q_pos_base={qpb}")
    q, k, _ = planted_inputs(21, H, Hkv, N, D, 0.01, dt, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 4.0)
    sm = 1.0 / math.sqrt(D)
    shared = lambda: native.select_vote(q, k, tau, invf, ps, 1.0, sm, 32, qpb)[2]
    pq = lambda: native.pq_select_bits(q, k, tau, invf, ps, 1.0, sm, 32, qpb)["row_max"]
    for name, fn in (("shared", shared), ("per-query", pq)):
        rm_table = fn()
        torch.cuda.synchronize()
        rm_gather = _gathered(fn)
        nd = int((rm_table != rm_gather).sum())
        print(f"[result] {name}: row maxima differing {nd} of {rm_table.numel()}", flush=True)
        assert nd == 0, f"{name}: {nd} row maxima differ between the table rebuild and the gathers"
