"""GPU parity of config 4: DCA positions with exact-max selection over the inter-chunk keys
(sta_dca_attention with select = 1) against the config-4 oracle.

Layers, as for the shared path:
  1. votes over each 64-query tile's inter keys within the 1e-3 band of the oracle's, row max
     within 1e-4;
  2. sets given the GPU's votes: the oracle's per-tile _build_sets reproduces idx and every
     statistic bit for bit;
  3. sets against the oracle's own sets: every differing key classified (band key, shifted cut,
     truncation boundary) and counted;
  4. output given the GPU's sets within 1e-4 (fp32) or 2e-2 abs + 1e-2 rel (bf16 / fp16).
KAT: tau = inf, pct = 100, k_max >= N keeps every inter key, which is the dense DCA prefill.
"""
import math

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, check_output, check_votes, classify_set_diffs, np_of, report_set_diffs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NAMES = ["idx", "shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas", "overflow20"]


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _invf(D, theta=10000.0):
    return 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))


def check_dca_select(q, k, v, s, c, w, tau, pct, k_max, n_global, what, rows=None):
    import _sta_native as native
    H, N, D = q.shape[1], q.shape[2], q.shape[3]
    L = s - w
    invf = _invf(D)
    say(f"{what}: H={H} Hkv={k.shape[1]} N={N} D={D} chunk {s} window {w} (L {L}) k_max={k_max} {q.dtype}")
    r = native.dca_select_attention(q, k, v, invf.to(DEV), s, c, w, torch.full((H,), tau), pct, k_max, n_global,
                                    want_votes=True, want_row_max=True)
    torch.cuda.synchronize()
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    a = orc.dca_inter_votes(qn, kn, dt, invf.numpy(), s, c, w, np.full(H, tau, np.float32), want_band=True)
    votes_g = r["votes"].cpu().numpy()
    ndiff, nband = check_votes(votes_g, a["votes"], a["band"])
    rm = r["row_max"].cpu().numpy()
    fin = np.isfinite(a["row_max"])
    assert np.array_equal(fin, np.isfinite(rm)), "rows with inter keys differ"
    assert np.max(np.abs(rm[fin] - a["row_max"][fin]), initial=0.0) < 1e-4, "row max"
    got = {n: r[n].cpu().numpy() for n in NAMES}
    ref_g = orc.dca_build_sets(votes_g, s, w, n_global, pct, k_max, want_cut=True)
    for name, rv in zip(NAMES, ref_g):
        assert np.array_equal(got[name].astype(np.int64), rv.astype(np.int64)), f"{what}: {name} given the votes"
    # set level: per tile, the inter key axis [0, ext) with the tile's start as its position base
    ref_o = orc.dca_build_sets(a["votes"], s, w, n_global, pct, k_max, want_cut=True)
    nt = votes_g.shape[1]
    tot = {"tiles": 0, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0, "trunc": 0}
    for h in range(H):
        for t in range(nt):
            cq = (t * 64) // L
            ext = (cq - 1) * L if cq >= 2 else 0
            tot["tiles"] += 1
            if not ext:
                continue
            sl = (slice(h, h + 1), slice(t, t + 1))
            cnt = classify_set_diffs(votes_g[sl][..., :ext], a["votes"][sl][..., :ext], a["band"][sl][..., :ext],
                                     {"idx": ref_g[0][sl]}, {"idx": ref_o[0][sl]}, ref_g[7][sl], ref_o[7][sl],
                                     64, k_max, n_global, 0, q_pos_base=t * 64)
            for n in ("tiles_differ", "keys", "band", "cut", "trunc"):
                tot[n] += cnt[n]
    report_set_diffs(what, tot)
    out_ref = orc.dca_select_attn(qn, kn, vn, dt, invf.numpy(), s, c, w, got["idx"], got["kept_size"], rows=rows)
    out_g = r["out"].float().cpu().numpy()
    if rows is not None:
        out_g, out_ref = out_g[:, rows], out_ref[:, rows]
    e = check_output(out_g, out_ref, dt, what)
    print(f"[result] {what}: vote entries differing {ndiff} (band pairs {nband}), kept mean "
          f"{got['kept_size'].mean():.1f}, overflow20 {int(got['overflow20'].sum())}, max out err {e:.2e}",
          flush=True)
    return r


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_dca_select_three_layer(dt):
    from synthetic import planted_inputs
    H, Hkv, N, D = 4, 2, 2600, 64
    q, k, v = planted_inputs(41, H, Hkv, N, D, 0.02, dt, DEV)
    # chunk 576, window 64: L = 512; tiles of chunk >= 2 select among up to 2 L inter keys
    check_dca_select(q, k, v, 576, 1024, 64, 3.0, 30.0, 192, 8, f"dca select {dt}")


def test_dca_select_d128_truncation():
    from synthetic import planted_inputs
    H, N, D = 2, 4200, 128
    q, k, v = planted_inputs(42, H, H, N, D, 0.01, torch.bfloat16, DEV)
    r = check_dca_select(q, k, v, 704, 2048, 64, 5.0, 30.0, 128, 32, "dca select d128, k_max 128")
    assert r["overflow20"].any()


def test_dca_select_infinite_tau_is_dense():
    import _sta_native as native
    from synthetic import planted_inputs
    H, N, D = 2, 1800, 128
    q, k, v = planted_inputs(43, H, H, N, D, 0.02, torch.bfloat16, DEV)
    s, c, w = 320, 512, 64
    invf = _invf(D).to(DEV)
    say("dca select, tau inf, pct 100, k_max N")
    r = native.dca_select_attention(q, k, v, invf, s, c, w, torch.full((H,), float("inf")), 100.0, N, 4)
    dense = native.dca_attention(q, k, v, invf, s, c, w)
    torch.cuda.synchronize()
    e = (r["out"].float() - dense.float()).abs().max().item()
    assert e <= 2e-2, e
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    ref = orc.dca_attention(qn, kn, vn, dt, invf.cpu().numpy(), s, c, w)
    check_output(r["out"].float().cpu().numpy(), ref, dt, "dca select tau inf vs dense oracle")
    print(f"[result] tau inf: max |select - dense| on the GPU {e:.2e}", flush=True)


def test_config4_geometry_16k_one_head():
    """Config 4's chunking (chunk 4096, window 512, pretraining 4096: L = 3584) and selection
    (tau 5, top 30%, k_max 2048, 32 global keys) at 16384 tokens on one head, full three-layer."""
    from synthetic import CONFIGS, planted_inputs
    cfg = CONFIGS["c4"]
    q, k, v = planted_inputs(0, 1, 1, 16384, cfg.D, cfg.frac, cfg.dtype, DEV)
    s, c, w = cfg.dca
    rows = list(range(0, 16384, 97)) + [16383]
    check_dca_select(q, k, v, s, c, w, cfg.tau, cfg.pct, cfg.k_max, cfg.n_global, "config 4 geometry, 16k, 1 head",
                     rows=rows)


def test_config4_full_size_structure_and_sampled_rows():
    """Config 4 at full size (32 heads x 65536 x d128 bf16): structural invariants of every tile's
    selection; head 0's sets rebuilt by the oracle from the GPU's votes (all 1024 tiles, bit for
    bit); votes and sets of eight deep tiles of head 0 (past position 50k, up to 60928 inter keys)
    against the oracle's own votes and sets, every differing key classified; and 48 sampled rows
    of two heads against the oracle given the GPU's sets."""
    import _sta_native as native
    from synthetic import CONFIGS
    cfg = CONFIGS["c4"]
    q, k, v = cfg.inputs(DEV)
    s, c, w = cfg.dca
    L = s - w
    invf = _invf(cfg.D).to(DEV)
    say("config 4 full size")
    r = native.dca_select_attention(q, k, v, invf, s, c, w, torch.full((cfg.H,), cfg.tau), cfg.pct, cfg.k_max,
                                    cfg.n_global, want_votes=True, want_row_max=True)
    torch.cuda.synchronize()
    nt = (cfg.N + 63) // 64
    t = torch.arange(nt, device=DEV)
    ext = torch.where(t * 64 // L >= 2, (t * 64 // L - 1) * L, torch.zeros_like(t))
    ks, idx = r["kept_size"], r["idx"]
    assert torch.all(ks <= ext[None]) and torch.all((ks > 0) == (ext[None] > 0))
    nvalid = ks.clamp(max=cfg.k_max)
    slot = torch.arange(cfg.k_max, device=DEV)
    valid = slot[None, None] < nvalid[..., None]
    assert torch.all(torch.where(valid, idx < ext[None, :, None], torch.ones_like(valid)))
    d = idx[..., 1:] - idx[..., :-1]
    assert torch.all(torch.where(valid[..., 1:], d > 0, torch.ones_like(d, dtype=torch.bool)))
    assert torch.isfinite(r["out"].float()).all()
    print(f"[result] config 4: kept mean {ks[:, 112:].float().mean().item():.1f} over tiles with inter keys, "
          f"overflow20 {int(r['overflow20'].sum())} of {ks.numel()}", flush=True)

    # head 0: sets given the GPU's votes on every tile, then eight deep tiles against the oracle
    h = 0
    deep = [790, 830, 870, 910, 950, 990, 1010, nt - 1]
    say(f"config 4 head {h}: oracle votes of tiles {deep}")
    votes_g = r["votes"][h:h + 1].cpu().numpy().astype(np.int32)
    got = {n: r[n][h:h + 1].cpu().numpy() for n in NAMES}
    ref_g = orc.dca_build_sets(votes_g, s, w, cfg.n_global, cfg.pct, cfg.k_max, want_cut=True)
    for name, rv in zip(NAMES, ref_g):
        assert np.array_equal(got[name].astype(np.int64), rv.astype(np.int64)), f"head {h}: {name} given the votes"
    qn, dt = np_of(q[0, h:h + 1])
    kn, _ = np_of(k[0, h:h + 1])
    vn, _ = np_of(v[0, h:h + 1])
    a = orc.dca_inter_votes(qn, kn, dt, invf.cpu().numpy(), s, c, w, np.full(1, cfg.tau, np.float32),
                            want_band=True, tiles=deep)
    rows_deep = np.concatenate([np.arange(tt * 64, tt * 64 + 64) for tt in deep])
    rm_g = r["row_max"][h, rows_deep].cpu().numpy()
    assert np.max(np.abs(rm_g - a["row_max"][0, rows_deep])) < 1e-4, "row max of the deep tiles"
    ref_o = orc.dca_build_sets(a["votes"], s, w, cfg.n_global, cfg.pct, cfg.k_max, want_cut=True)
    tot = {"tiles": 0, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0, "trunc": 0}
    ndiff = nband = 0
    for tt in deep:
        e_t = int(ext[tt])
        sl = (slice(0, 1), slice(tt, tt + 1))
        dv, db = check_votes(votes_g[sl][..., :e_t], a["votes"][sl][..., :e_t], a["band"][sl][..., :e_t])
        ndiff += dv
        nband += db
        cnt = classify_set_diffs(votes_g[sl][..., :e_t], a["votes"][sl][..., :e_t], a["band"][sl][..., :e_t],
                                 {"idx": ref_g[0][sl]}, {"idx": ref_o[0][sl]}, ref_g[7][sl], ref_o[7][sl],
                                 64, cfg.k_max, cfg.n_global, 0, q_pos_base=tt * 64)
        tot["tiles"] += 1
        for n in ("tiles_differ", "keys", "band", "cut", "trunc"):
            tot[n] += cnt[n]
    print(f"[result] config 4 head {h}, deep tiles: vote entries differing {ndiff} (band pairs {nband}), "
          f"inter keys {int(ext[deep[0]])}..{int(ext[deep[-1]])}", flush=True)
    report_set_diffs(f"config 4 full size, head {h}, {len(deep)} deep tiles", tot)
    out_ref = orc.dca_select_attn(qn, kn, vn, dt, invf.cpu().numpy(), s, c, w, got["idx"], got["kept_size"],
                                  rows=rows_deep[::8])
    e = check_output(r["out"][h:h + 1, rows_deep[::8]].float().cpu().numpy(), out_ref[:, rows_deep[::8]], dt,
                     f"config 4 head {h} deep rows")
    print(f"[result] config 4 head {h}: {len(rows_deep[::8])} deep rows, max out err {e:.2e}", flush=True)

    rows = list(range(5, cfg.N, cfg.N // 24))[:24] + [cfg.N - 1]
    for h in (0, 17):
        qn, dt = np_of(q[0, h:h + 1])
        kn, _ = np_of(k[0, h:h + 1])
        vn, _ = np_of(v[0, h:h + 1])
        out_ref = orc.dca_select_attn(qn, kn, vn, dt, invf.cpu().numpy(), s, c, w, r["idx"][h:h + 1].cpu().numpy(),
                                      r["kept_size"][h:h + 1].cpu().numpy(), rows=rows)
        e = check_output(r["out"][h:h + 1, rows].float().cpu().numpy(), out_ref[:, rows], dt, f"config 4 head {h}")
        print(f"[result] config 4 head {h}: {len(rows)} sampled rows, max out err {e:.2e}", flush=True)
