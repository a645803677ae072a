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
