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


def forced_mask(nt, N, T, n_global, n_local, q_pos_base=0):
    """(nt, N) bool: global keys and each tile's local window (exact_2.py:290-293, 303)."""
    j = np.arange(N)[None, :]
    tstart = q_pos_base + np.arange(nt)[:, None] * T
    return (j < n_global) | ((j >= tstart - n_local + 1) & (j <= tstart + T - 1))


def classify_set_diffs(votes_g, votes_o, band, sets_g, sets_o, cut_g, cut_o, T, k_max, n_global,
                       n_local, q_pos_base=0, rank_g=None, rank_o=None):
    """Count the keys whose membership in the selected sets differs between the GPU (sets built
    from its own votes) and the oracle (sets built from the oracle's votes), and classify each:

      band  - the key itself has a score within BAND of the threshold m - tau of one of the
              tile's queries (its vote may legitimately differ);
      cut   - the key's rank value is the same on both sides and lies between the two sides'
              cuts v_cut (tie-inclusive, exact_2.py:330-331): a band flip elsewhere in the tile
              moved the cut (or the chosen fallback step) past it;
      trunc - the tile is truncated to its k_max smallest kept keys (exact_2.py:394-405) on
              either side and the key lies past the first key where the untruncated sets differ,
              so the truncation boundary moved with it.
    Anything else fails.  rank_* default to the votes (frequency ranking); cut_* are the oracle's
    per-tile cuts for each side's votes.  Returns a dict of counts."""
    H, nt, N = votes_g.shape
    rank_g = votes_g.astype(np.float32) if rank_g is None else rank_g
    rank_o = votes_o.astype(np.float32) if rank_o is None else rank_o
    kg, ko = kept_mask_of(sets_g["idx"], N), kept_mask_of(sets_o["idx"], N)
    forced = forced_mask(nt, N, T, n_global, n_local, q_pos_base)
    counts = {"tiles": H * nt, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0, "trunc": 0}
    for h, t in np.argwhere((kg != ko).any(-1)):
        counts["tiles_differ"] += 1
        assert (votes_g[h, t] != votes_o[h, t]).any(), f"tile ({h},{t}): sets differ with equal votes"
        fg = (rank_g[h, t] >= cut_g[h, t]) | forced[t]
        fo = (rank_o[h, t] >= cut_o[h, t]) | forced[t]
        full_diff = np.nonzero(fg != fo)[0]
        lo_c, hi_c = sorted((float(cut_g[h, t]), float(cut_o[h, t])))
        for j in full_diff:
            if band[h, t, j] > 0:
                continue
            same = rank_g[h, t, j] == rank_o[h, t, j]
            assert same and lo_c <= rank_g[h, t, j] <= hi_c, (
                f"tile ({h},{t}) key {j}: not a band key and not between the cuts "
                f"(rank {rank_g[h, t, j]} / {rank_o[h, t, j]}, cuts {lo_c} {hi_c})")
        keys = np.nonzero(kg[h, t] != ko[h, t])[0]
        first = full_diff.min() if full_diff.size else N
        truncated = fg.sum() > k_max or fo.sum() > k_max
        for j in keys:
            counts["keys"] += 1
            if j in full_diff:
                counts["band" if band[h, t, j] > 0 else "cut"] += 1
            else:
                assert truncated and j > first, (
                    f"tile ({h},{t}) key {j}: differs only after truncation but the tile is not "
                    f"truncated past an earlier difference (first {first})")
                counts["trunc"] += 1
    return counts


def report_set_diffs(what, c):
    msg = (f"[sets] {what}: {c['tiles_differ']} of {c['tiles']} tiles differ from the oracle's sets; "
           f"{c['keys']} keys: {c['band']} band keys, {c['cut']} moved by a shifted cut, "
           f"{c['trunc']} moved by the truncation boundary")
    print(msg, flush=True)
    return msg


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


def classify_pq_set_diffs(band, sets_g, sets_o, rank_g, rank_o, N, rel=1e-4):
    """PQ Union: count the keys whose membership in the tile's union set differs between the GPU
    (sets from its own bits / weighted votes) and the oracle (sets from its own), classified:

      band - one of the tile's rows has the key's score within BAND of its threshold, so the
             key's keep bit (and its weighted vote) may differ;
      cut  - the tile overflows k_max on either side (perquery.py:393-410), the key's rank value
             is the same on both sides and lies between the two sides' cuts (the smallest kept
             non-forced rank value); "same" and "between" are widened by `rel` for the fp32
             summation order of the weighted votes.
    Anything else fails.  Returns a dict of counts."""
    kg, ko = kept_mask_of(sets_g["idx"], N), kept_mask_of(sets_o["idx"], N)
    H, nt = kg.shape[:2]
    counts = {"tiles": H * nt, "tiles_differ": 0, "keys": 0, "band": 0, "cut": 0}

    def cut_of(s, rank, h, t):
        idx, mask = s["idx"][h, t], s["mask"][h, t]
        sel = idx[(idx < N) & (mask != -1)]
        return float(rank[h, t, sel].min()) if sel.size else float("inf")

    for h, t in np.argwhere((kg != ko).any(-1)):
        counts["tiles_differ"] += 1
        over = bool(sets_g["overflow"][h, t]) or bool(sets_o["overflow"][h, t])
        lo_c, hi_c = sorted((cut_of(sets_g, rank_g, h, t), cut_of(sets_o, rank_o, h, t)))
        for j in np.nonzero(kg[h, t] != ko[h, t])[0]:
            counts["keys"] += 1
            if band[h, t, j] > 0:
                counts["band"] += 1
                continue
            r = (float(rank_g[h, t, j]), float(rank_o[h, t, j]))
            same = abs(r[0] - r[1]) <= rel * max(abs(r[0]), abs(r[1]))
            ok = over and same and any(lo_c - rel * abs(lo_c) <= x <= hi_c + rel * abs(hi_c) for x in r)
            assert ok, (f"tile ({h},{t}) key {j}: not a band key and not at the overflow cut "
                        f"(rank {r}, cuts {lo_c} {hi_c}, overflow {over})")
            counts["cut"] += 1
    return counts


def report_pq_set_diffs(what, c):
    msg = (f"[sets] {what}: {c['tiles_differ']} of {c['tiles']} tiles differ from the oracle's sets; "
           f"{c['keys']} keys: {c['band']} band keys, {c['cut']} at the overflow cut")
    print(msg, flush=True)
    return msg
