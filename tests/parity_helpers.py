"""Comparison helpers for the GPU parity tests (HIP path vs the CPU oracle).

The contract for selection: key-index sets match the reference exactly, except for keys whose
score lies within BAND (1e-3) of a query's threshold m - tau; such keys are counted and
reported.  Checked in three layers:
  1. votes: |votes_gpu - votes_oracle| <= (# of the tile's queries whose score for that key lies
     in the band), for every (head, tile, key);
  2. sets given votes: the oracle's _build_sets restatement applied to the GPU's own votes
     reproduces the GPU's idx / newpos / statistics bit for bit;
  3. output given sets: the oracle's Kernel C applied to the GPU's idx / newpos matches the GPU
     output within the output tolerance (fp32: 1e-4 abs; bf16/fp16: 2e-2 abs + 1e-2 rel).
Where the votes agree exactly (no band key flipped) the GPU sets equal the oracle's end to end.
"""
import numpy as np
import torch

from oracle import sta_oracle as orc

BAND = 1e-3
SET_NAMES = ["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen", "orig_overflow",
             "kpct_meas", "overflow20"]


def np_of(t):
    """device tensor -> numpy (bf16/fp16 as uint16 bit patterns) and dtype code."""
    return orc.from_torch(t)


def check_votes(votes_gpu, votes_or, band):
    d = np.abs(votes_gpu.astype(np.int64) - votes_or.astype(np.int64))
    bad = d > band
    assert not bad.any(), f"{int(bad.sum())} vote entries differ beyond the band"
    return int((d > 0).sum()), int(band.sum())


def check_sets_given_votes(votes_gpu, sets_gpu, pos_scale, n_global, n_local, pct, T, k_max,
                           q_pos_base=0, measure=False):
    ref = orc.build_sets(votes_gpu, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base, measure)
    for name, r in zip(SET_NAMES, ref):
        g = sets_gpu[name]
        if r.dtype == np.float32:
            same = np.array_equal(g.view(np.uint32), r.view(np.uint32))
        else:
            same = np.array_equal(g.astype(np.int64), r.astype(np.int64))
        if not same:
            diff = np.argwhere(g != r)
            raise AssertionError(f"{name} differs at {diff[:5].tolist()} (of {len(diff)})")
    return ref


def check_output(out_gpu, out_ref, dtype_code, what=""):
    """out_gpu: numpy float32 of the GPU output (upcast); out_ref: the oracle's fp32 accumulator."""
    finite = np.isfinite(out_ref)
    assert np.array_equal(finite, np.isfinite(out_gpu)), f"{what}: non-finite pattern differs"
    err = np.abs(out_gpu[finite] - out_ref[finite])
    if dtype_code == orc.F32:
        tol = 1e-4 + 1e-4 * np.abs(out_ref[finite])
    else:
        tol = 2e-2 + 1e-2 * np.abs(out_ref[finite])
    worst = float((err / tol).max()) if err.size else 0.0
    assert worst <= 1.0, f"{what}: max |err| {float(err.max()):.3e} exceeds tolerance (ratio {worst:.2f})"
    return float(err.max()) if err.size else 0.0


def gpu_sets_numpy(r):
    return {n: r[n].cpu().numpy() for n in SET_NAMES}


def out_f32(t):
    return t.float().cpu().numpy()


# ------------------------------------------------------------------------------------------------
# PQ Union: sets may differ only among keys tied at the overflow cut
# ------------------------------------------------------------------------------------------------
PQ_SET_NAMES = ["idx", "newpos_k", "newpos_q", "mask", "usize", "kept_size", "overflow"]


def pq_rank_values(votes, wvotes, rank_mode):
    """fl(wvotes + fl(1e-6 * votes)) (perquery.py:397), or votes for freq ranking."""
    if rank_mode == 0 or wvotes is None:
        return votes.astype(np.float32)
    return (wvotes.astype(np.float32) + np.float32(1e-6) * votes.astype(np.float32)).astype(np.float32)


def kept_mask_of(idx, N):
    H, nt, _ = idx.shape
    m = np.zeros((H, nt, N + 1), bool)
    np.put_along_axis(m, idx.astype(np.int64), True, axis=-1)
    return m[..., :N]


def compare_pq_sets(got, ref, rank_vals, N, rel=0.0):
    """got/ref: dicts of the 7 outputs.  Tiles whose kept sets agree must agree in every output;
    in the others every differing key must carry a rank value within `rel` (relative) of the
    reference's cut (its smallest kept non-forced rank value) -- equal values for exact inputs,
    where torch.topk's choice among ties is unspecified -- and the sizes must agree.
    Returns the number of tiles whose sets differ."""
    kg, kr = kept_mask_of(got["idx"], N), kept_mask_of(ref["idx"], N)
    differ = (kg != kr).any(-1)
    for n in ("usize", "kept_size", "overflow"):
        assert np.array_equal(np.asarray(got[n]).astype(np.int64), np.asarray(ref[n]).astype(np.int64)), n
    same = ~differ
    for n in ("idx", "newpos_k", "newpos_q", "mask"):
        a, b = np.asarray(got[n]), np.asarray(ref[n])
        if a.dtype == np.float32:
            eq = a.view(np.uint32) == b.view(np.uint32)
        else:
            eq = a.astype(np.int64) == b.astype(np.int64)
        assert eq[same].all(), f"{n} differs in a tile whose kept set agrees"
    for h, t in np.argwhere(differ):
        keys = np.nonzero(kg[h, t] != kr[h, t])[0]
        forced = ref["mask"][h, t] == -1
        sel = ref["idx"][h, t][(ref["idx"][h, t] < N) & ~forced]
        cut = rank_vals[h, t, sel].min()
        rv = rank_vals[h, t, keys]
        tol = rel * abs(float(cut))
        assert np.all(np.abs(rv - cut) <= tol), (h, t, keys[:8].tolist(), rv[:8].tolist(), float(cut))
    return int(differ.sum())
