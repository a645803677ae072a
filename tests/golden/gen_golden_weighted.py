#!/usr/bin/env python3
"""Write the golden vectors of the shared path's weighted ranking (select_score margin / expmass).

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden_weighted.py

Executed from the reference, because no closed form pins them:

* ``_build_sets`` (shared_selection_triton_exact_2.py:277-426) with ``wvotes`` and
  ``select_score`` "margin" / "expmass": the rank value fl(wvotes + fl(1e-6 votes)) (:299-302),
  the frequency-based union size and budgets (:296, :329), the tie-inclusive cut on fp32 rank
  values, the fallback, measure loop and truncation -- on synthetic vote / weighted-vote tensors,
  plain torch on the CPU.
* the composed prefill path with WMODE 1 / 2 (Kernel A's weighted votes, exact_2.py:126-138,
  then the weighted ``_build_sets`` and Kernel C) under ``TRITON_INTERPRET=1`` on small fp32
  shapes, recorded with the intermediate votes and weighted votes.

Every fixture stores its inputs and the reference's outputs as plain arrays in one .npz.
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from gen_golden import _import_reference, base_inv_freq, planted_inputs  # noqa: E402

OUT = HERE
SET_NAMES = ["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen", "orig_overflow",
             "kpct_meas", "overflow20"]


def gen_build_sets_weighted(ex2):
    rng = np.random.default_rng(77)

    def causal(H, nt, N, T, qb, density, mode, tau, seed, quant=None):
        r = np.random.default_rng(seed)
        votes = np.zeros((H, nt, N), np.int32)
        wv = np.zeros((H, nt, N), np.float32)
        for t in range(nt):
            hi = min(N, qb + (t + 1) * T)
            v = r.binomial(T, density, size=(H, hi)).astype(np.int32)
            votes[:, t, :hi] = v
            # a weighted vote is a sum over the keeping rows of a per-row weight
            if mode == "margin":
                w = v * r.uniform(0.0, tau, size=(H, hi))
            else:
                w = v * r.uniform(math.exp(-tau), 1.0, size=(H, hi))
            if quant is not None:   # coarse values: many exact ties among the weighted votes
                w = np.round(w / quant) * quant
            wv[:, t, :hi] = w.astype(np.float32)
        return votes, wv

    cases = []
    for mode in ("margin", "expmass"):
        v, w = causal(2, 6, 384, 64, 0, 0.3, mode, 5.0, 1)
        cases.append(dict(name=f"{mode}_plain", votes=v, wvotes=w, mode=mode, pos_scale=1.0, n_global=32,
                          n_local=32, pct=30.0, T=64, k_max=2048, q_pos_base=0, measure=False))
        v, w = causal(3, 8, 512, 64, 0, 0.6, mode, 5.0, 2)
        cases.append(dict(name=f"{mode}_cap", votes=v, wvotes=w, mode=mode, pos_scale=1.0 / 3.0, n_global=32,
                          n_local=32, pct=30.0, T=64, k_max=160, q_pos_base=0, measure=True))
        v, w = causal(2, 7, 200, 32, 0, 0.5, mode, 4.0, 3, quant=0.5)
        cases.append(dict(name=f"{mode}_ragged_ties", votes=v, wvotes=w, mode=mode, pos_scale=0.25,
                          n_global=40, n_local=16, pct=30.0, T=32, k_max=96, q_pos_base=0, measure=False))
        for i, pct in enumerate([25.0, 22.5, 100.0, 0.0]):
            v, w = causal(2, 5, 320, 64, 0, 0.5, mode, 5.0, 10 + i)
            cases.append(dict(name=f"{mode}_pct_{pct:g}", votes=v, wvotes=w, mode=mode, pos_scale=0.5,
                              n_global=8, n_local=8, pct=pct, T=64, k_max=120, q_pos_base=0,
                              measure=(i % 2 == 0)))
        v, w = causal(2, 4, 300, 64, 44, 0.4, mode, 5.0, 20)
        cases.append(dict(name=f"{mode}_qbase", votes=v, wvotes=w, mode=mode, pos_scale=0.75, n_global=16,
                          n_local=24, pct=30.0, T=64, k_max=100, q_pos_base=44, measure=True))
        v, w = causal(1, 3, 192, 64, 0, 0.3, mode, 5.0, 30)
        v[0, 1, :] = 0
        w[0, 1, :] = 0.0
        cases.append(dict(name=f"{mode}_empty_tile", votes=v, wvotes=w, mode=mode, pos_scale=1.0, n_global=4,
                          n_local=4, pct=30.0, T=64, k_max=400, q_pos_base=0, measure=False))
    # equal weighted votes with different frequencies: the 1e-6 frequency tiebreak decides
    v = np.zeros((1, 1, 256), np.int32)
    w = np.zeros((1, 1, 256), np.float32)
    v[0, 0, :200] = rng.integers(1, 64, size=200)
    w[0, 0, :200] = 2.0
    cases.append(dict(name="tiebreak", votes=v, wvotes=w, mode="margin", pos_scale=1.0, n_global=0,
                      n_local=1, pct=30.0, T=64, k_max=2048, q_pos_base=0, measure=False))

    arrays = {}
    for i, c in enumerate(cases):
        res = ex2._build_sets(torch.from_numpy(c["votes"]), c["pos_scale"], c["n_global"], c["n_local"],
                              c["pct"], c["T"], c["k_max"], q_pos_base=c["q_pos_base"], measure=c["measure"],
                              wvotes=torch.from_numpy(c["wvotes"]), select_score=c["mode"])
        p = f"c{i}_"
        arrays[p + "votes"], arrays[p + "wvotes"] = c["votes"], c["wvotes"]
        arrays[p + "params"] = np.array([c["pos_scale"], c["n_global"], c["n_local"], c["pct"], c["T"],
                                         c["k_max"], c["q_pos_base"], float(c["measure"]),
                                         {"margin": 1, "expmass": 2}[c["mode"]]], np.float64)
        for n, t in zip(SET_NAMES, res):
            arrays[p + n] = t.numpy()
        print(f"weighted build_sets case {i} {c['name']}: chosen {np.unique(res[5].numpy())}, "
              f"overflow20 {int(res[8].sum())}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "build_sets_weighted_golden.npz"), **arrays)


def run_kernel_a_weighted(mod, q, k, tau, inv_freq, sm_scale, pos_scale, rope_scale, tile, block_n,
                          q_pos_base, wmode):
    """The Kernel A launch of shared_pi_attention with WMODE > 0 (exact_2.py:448-465)."""
    Z, H, N, D = q.shape
    nt = (N + tile - 1) // tile
    qh, kh = q[0].contiguous(), k[0].contiguous()
    votes = torch.zeros((H, nt, N), dtype=torch.int32)
    row_counts = torch.zeros((H, N), dtype=torch.int32)
    wvotes = torch.zeros((H, nt, N), dtype=torch.float32)
    mod._select_vote_kernel[(nt, H)](
        qh, kh, tau.float().contiguous(), inv_freq.float().contiguous(), votes, row_counts, wvotes,
        sm_scale, float(pos_scale), float(rope_scale), int(q_pos_base),
        qh.stride(0), qh.stride(1), qh.stride(2), kh.stride(0), kh.stride(1), kh.stride(2),
        votes.stride(0), votes.stride(1), votes.stride(2), row_counts.stride(0), row_counts.stride(1),
        wvotes.stride(0), wvotes.stride(1), wvotes.stride(2),
        H, N, BLOCK_M=tile, BLOCK_N=block_n, HEAD_DIM=D, HALF_DIM=D // 2, WMODE=wmode,
        num_warps=4, num_stages=1)
    return votes, row_counts, wvotes


def gen_composed_weighted(ex2):
    cases = [
        dict(name="margin_t64", mode="margin", H=2, N=256, D=64, tile=64, k_max=2048, tau=5.0, pct=30.0,
             ng=32, nl=32, ps=1.0, qb=0, frac=0.02, seed=50),
        dict(name="expmass_cap_ragged", mode="expmass", H=2, N=200, D=64, tile=32, k_max=48, tau=3.0,
             pct=30.0, ng=4, nl=8, ps=0.5, qb=0, frac=0.05, seed=51),
        dict(name="margin_third_cap", mode="margin", H=2, N=320, D=64, tile=64, k_max=96, tau=2.5,
             pct=30.0, ng=8, nl=16, ps=1.0 / 3.0, qb=0, frac=0.02, seed=52),
        dict(name="expmass_qbase", mode="expmass", H=2, N=160, D=64, tile=32, k_max=64, tau=3.0,
             pct=30.0, ng=4, nl=8, ps=0.5, qb=16, frac=0.05, seed=53),
    ]
    arrays = {}
    for i, c in enumerate(cases):
        q, k, v = planted_inputs(c["seed"], c["H"], c["H"], c["N"], c["D"], c["frac"])
        tau = torch.full((c["H"],), c["tau"], dtype=torch.float32)
        invf = base_inv_freq(c["D"], 10000.0)
        sm = 1.0 / math.sqrt(c["D"])
        wmode = {"margin": 1, "expmass": 2}[c["mode"]]
        votes, rc, wv = run_kernel_a_weighted(ex2, q, k, tau, invf, sm, c["ps"], 1.0, c["tile"], 64, c["qb"],
                                              wmode)
        sets = ex2._build_sets(votes, c["ps"], c["ng"], c["nl"], c["pct"], c["tile"], c["k_max"],
                               q_pos_base=c["qb"], wvotes=wv, select_score=c["mode"])
        full = ex2.shared_pi_attention(q, k, v, tau, invf, pos_scale=c["ps"], pct=c["pct"], n_global=c["ng"],
                                       n_local=c["nl"], tile=c["tile"], k_max=c["k_max"], q_pos_base=c["qb"],
                                       select_score=c["mode"])
        p = f"c{i}_"
        arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = q[0].numpy(), k[0].numpy(), v[0].numpy()
        arrays[p + "tau"], arrays[p + "inv_freq"] = tau.numpy(), invf.numpy()
        arrays[p + "params"] = np.array([c["tile"], c["k_max"], c["pct"], c["ng"], c["nl"], c["ps"], c["qb"], sm,
                                         wmode], np.float64)
        arrays[p + "votes"], arrays[p + "row_counts"], arrays[p + "wvotes"] = votes.numpy(), rc.numpy(), wv.numpy()
        for n, t in zip(SET_NAMES, sets):
            arrays[p + n] = t.numpy()
        arrays[p + "out"] = full[0][0].numpy()
        for n, t in zip(["shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas", "overflow20"],
                        full[1:]):
            assert torch.equal(t, sets[SET_NAMES.index(n)]), n
        print(f"weighted composed case {i} {c['name']}: kept {sets[4].float().mean():.1f} "
              f"overflow20 {int(sets[8].sum())}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "composed_weighted_golden.npz"), **arrays)


if __name__ == "__main__":
    torch.set_num_threads(8)
    ex2, _ = _import_reference()
    gen_build_sets_weighted(ex2)
    gen_composed_weighted(ex2)
