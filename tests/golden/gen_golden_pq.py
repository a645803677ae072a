#!/usr/bin/env python3
"""Write the golden vectors of the two per-query variants (PQ Union and PQ Stream).

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden_pq.py

What is executed from the reference, and why:

* ``_build_sets_pq`` (shared_selection_triton_perquery.py:363-453), plain torch on the CPU, on
  synthetic votes / bits / weighted votes: the union, forced columns, the k_max overflow
  truncation by expmass (or freq) rank, dense ranks and the per-slot bitmask are edge semantics
  no closed form pins.
* ``shared_pq_attention`` (perquery.py:459-525) composed under ``TRITON_INTERPRET=1`` on small
  fp32 shapes, with the inputs and outputs of its ``_build_sets_pq`` call recorded on the way
  (votes, bits, wvotes from ``_select_bits_kernel``).  Also the reference's own torch golden
  ``pq_attention_torch`` (perquery.py:544-615) on the same inputs.
* ``pqstream_attention`` (pqstream_kernel.py:498-564, the fused ``_pqstream_kernel`` 174-368)
  under the interpreter on small fp32 shapes, and its torch golden ``pqstream_attention_torch``
  (pqstream_kernel.py:582-652).

Every fixture stores its inputs and the reference's outputs as plain arrays in one .npz.
"""
import math
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, OUT)
from gen_golden import planted_inputs, base_inv_freq  # noqa: E402


def _import_reference():
    os.environ.setdefault("TRITON_INTERPRET", "1")
    sys.path.insert(0, REF)
    import shared_selection_triton_perquery as pq      # noqa: E402
    import pqstream_kernel as pqs                       # noqa: E402
    return pq, pqs


# ---------------------------------------------------------------------------------------------
# _build_sets_pq on synthetic votes / bits / wvotes
# ---------------------------------------------------------------------------------------------
def synthetic_bits(H, nt, N, T, q_pos_base, density, seed, ties=False):
    r = np.random.default_rng(seed)
    bits = np.zeros((H, nt, N), np.int64)
    wv = np.zeros((H, nt, N), np.float32)
    for t in range(nt):
        hi = min(N, q_pos_base + (t + 1) * T)
        keep = r.random((H, T, hi)) < density                       # (H, rows, keys)
        for i in range(T):
            bits[:, t, :hi] |= keep[:, i, :].astype(np.int64) << i
        w = r.random((H, T, hi)).astype(np.float32)
        if ties:
            w = np.round(w * 4) / 4                                 # few distinct values
        wv[:, t, :hi] = np.where(keep, w, 0).sum(1)
    bits32 = ((bits + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)  # int32 wrap (row 31 = sign)
    votes = np.zeros((H, nt, N), np.int32)
    for i in range(T):
        votes += ((bits >> i) & 1).astype(np.int32)
    return votes, bits32, wv


def gen_build_sets_pq(pq):
    cases = [
        dict(name="no_overflow", H=2, nt=6, N=192, T=32, qb=0, dens=0.05, ng=4, nl=8, k_max=4096,
             mode="expmass", seed=1, ties=False),
        dict(name="overflow_expmass", H=2, nt=8, N=256, T=32, qb=0, dens=0.2, ng=4, nl=8, k_max=64,
             mode="expmass", seed=2, ties=False),
        dict(name="overflow_freq", H=2, nt=8, N=256, T=32, qb=0, dens=0.2, ng=4, nl=8, k_max=64,
             mode="freq", seed=3, ties=False),
        dict(name="ragged_qbase", H=2, nt=5, N=150, T=32, qb=12, dens=0.15, ng=8, nl=16, k_max=72,
             mode="expmass", seed=4, ties=False),
        dict(name="expmass_ties", H=1, nt=6, N=192, T=32, qb=0, dens=0.3, ng=2, nl=4, k_max=48,
             mode="expmass", seed=5, ties=True),
        dict(name="forced_exceeds", H=1, nt=4, N=128, T=32, qb=0, dens=0.3, ng=40, nl=32, k_max=60,
             mode="expmass", seed=6, ties=False),
    ]
    arrays = {}
    for i, c in enumerate(cases):
        votes, bits, wv = synthetic_bits(c["H"], c["nt"], c["N"], c["T"], c["qb"], c["dens"], c["seed"],
                                         c["ties"])
        res = pq._build_sets_pq(torch.from_numpy(votes), torch.from_numpy(bits), torch.from_numpy(wv),
                                c["ng"], c["nl"], c["T"], c["k_max"], q_pos_base=c["qb"],
                                select_score=c["mode"])
        p = f"c{i}_"
        arrays[p + "votes"], arrays[p + "bits"], arrays[p + "wvotes"] = votes, bits, wv
        arrays[p + "params"] = np.array([c["ng"], c["nl"], c["T"], c["k_max"], c["qb"],
                                         {"freq": 0, "margin": 1, "expmass": 2}[c["mode"]]], np.int64)
        for n, t in zip(["idx", "newpos_k", "newpos_q", "mask", "usize", "kept_size", "overflow"], res):
            arrays[p + n] = t.numpy()
        print(f"build_sets_pq case {i} {c['name']}: overflow {int(res[6].sum())}/{res[6].numel()}, "
              f"kept mean {res[5].float().mean():.1f}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "build_sets_pq_golden.npz"), **arrays)


# ---------------------------------------------------------------------------------------------
# composed PQ Union under the interpreter
# ---------------------------------------------------------------------------------------------
def gen_pq_composed(pq):
    cases = [
        dict(name="basic", H=2, N=200, D=64, tau=3.0, psa=0.5, rsa=1.0, ng=4, nl=8, k_max=4096,
             mode="expmass", qb=0, frac=0.03, seed=11, yarn=False),
        dict(name="overflow_expmass", H=2, N=256, D=64, tau=4.0, psa=0.25, rsa=1.0, ng=4, nl=8,
             k_max=72, mode="expmass", qb=0, frac=0.02, seed=12, yarn=False),
        dict(name="overflow_freq", H=2, N=256, D=64, tau=4.0, psa=0.25, rsa=1.0, ng=4, nl=8,
             k_max=72, mode="freq", qb=0, frac=0.02, seed=13, yarn=False),
        dict(name="overflow_margin", H=1, N=224, D=64, tau=3.5, psa=0.5, rsa=1.0, ng=4, nl=8,
             k_max=64, mode="margin", qb=0, frac=0.02, seed=14, yarn=False),
        dict(name="qbase", H=2, N=160, D=64, tau=3.0, psa=0.5, rsa=1.0, ng=4, nl=8, k_max=80,
             mode="expmass", qb=16, frac=0.03, seed=15, yarn=False),
        dict(name="two_geom_d128", H=1, N=128, D=128, tau=3.0, psa=1.0, rsa=1.1386294, ng=4, nl=8,
             k_max=4096, mode="expmass", qb=0, frac=0.03, seed=16, yarn=True),
    ]
    arrays = {}
    captured = {}
    orig = pq._build_sets_pq

    def spy(votes, bits, wvotes, *args, **kw):
        res = orig(votes, bits, wvotes, *args, **kw)
        captured.update(votes=votes.clone(), bits=bits.clone(), wvotes=wvotes.clone(), res=res)
        return res

    pq._build_sets_pq = spy
    try:
        for i, c in enumerate(cases):
            q, k, v = planted_inputs(c["seed"], c["H"], c["H"], c["N"], c["D"], c["frac"])
            tau = torch.full((c["H"],), c["tau"], dtype=torch.float32)
            invf_c = base_inv_freq(c["D"], 10000.0)
            invf_a = invf_c * torch.linspace(1.0, 0.25, c["D"] // 2) if c["yarn"] else invf_c
            captured.clear()
            out, usize, kept, ovf = pq.shared_pq_attention(
                q, k, v, tau, invf_a, invf_c, pos_scale_a=c["psa"], rope_scale_a=c["rsa"],
                n_global=c["ng"], n_local=c["nl"], tile=32, k_max=c["k_max"], q_pos_base=c["qb"],
                select_score=c["mode"])
            p = f"c{i}_"
            arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = q[0].numpy(), k[0].numpy(), v[0].numpy()
            arrays[p + "tau"] = tau.numpy()
            arrays[p + "inv_freq_a"], arrays[p + "inv_freq_c"] = invf_a.numpy(), invf_c.numpy()
            arrays[p + "params"] = np.array([c["psa"], c["rsa"], c["ng"], c["nl"], c["k_max"],
                                             {"freq": 0, "margin": 1, "expmass": 2}[c["mode"]],
                                             c["qb"]], np.float64)
            arrays[p + "votes"] = captured["votes"].numpy()
            arrays[p + "bits"] = captured["bits"].numpy()
            wv = captured["wvotes"]
            arrays[p + "wvotes"] = (wv.numpy() if wv.shape[-1] == c["N"]
                                    else np.zeros(captured["votes"].shape, np.float32))
            for n, t in zip(["idx", "newpos_k", "newpos_q", "mask", "usize", "kept_size", "overflow"],
                            captured["res"]):
                arrays[p + n] = t.numpy()
            arrays[p + "out"] = out[0].numpy()
            if c["qb"] == 0:
                gold = pq.pq_attention_torch(q, k, v, tau, invf_a, invf_c, pos_scale_a=c["psa"],
                                             rope_scale_a=c["rsa"], n_global=c["ng"], n_local=c["nl"],
                                             tile=32, k_max=c["k_max"], select_score=c["mode"])
                arrays[p + "out_torch"] = gold[0].numpy()
            print(f"pq composed case {i} {c['name']}: overflow {int(ovf.sum())}/{ovf.numel()}, "
                  f"kept mean {kept.float().mean():.1f}", flush=True)
    finally:
        pq._build_sets_pq = orig
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "pq_composed_golden.npz"), **arrays)


# ---------------------------------------------------------------------------------------------
# PQ Stream under the interpreter
# ---------------------------------------------------------------------------------------------
def gen_pqstream(pqs):
    cases = [
        dict(name="max", H=2, N=200, D=64, tau=3.0, psa=0.5, rsa=1.0, ng=4, nl=8, bn=32, adv="max",
             skip=True, frac=0.03, seed=21, yarn=False),
        dict(name="full_inf", H=1, N=200, D=64, tau=float("inf"), psa=1.0, rsa=1.0, ng=4, nl=8, bn=32,
             adv="full", skip=True, frac=0.03, seed=22, yarn=False),
        dict(name="bn64", H=2, N=256, D=64, tau=2.0, psa=0.25, rsa=1.0, ng=4, nl=8, bn=64, adv="max",
             skip=True, frac=0.02, seed=23, yarn=False),
        dict(name="skip_blocks", H=2, N=320, D=64, tau=0.05, psa=0.5, rsa=1.0, ng=0, nl=1, bn=32,
             adv="max", skip=True, frac=0.02, seed=24, yarn=False),
        dict(name="noskip", H=2, N=320, D=64, tau=0.05, psa=0.5, rsa=1.0, ng=0, nl=1, bn=32,
             adv="max", skip=False, frac=0.02, seed=24, yarn=False),
        dict(name="two_geom_d128", H=1, N=160, D=128, tau=3.0, psa=1.0, rsa=1.1386294, ng=4, nl=8,
             bn=32, adv="max", skip=True, frac=0.03, seed=25, yarn=True),
    ]
    arrays = {}
    for i, c in enumerate(cases):
        q, k, v = planted_inputs(c["seed"], c["H"], c["H"], c["N"], c["D"], c["frac"])
        tau = torch.full((c["H"],), c["tau"], dtype=torch.float32)
        invf_c = base_inv_freq(c["D"], 10000.0)
        invf_a = invf_c * torch.linspace(1.0, 0.25, c["D"] // 2) if c["yarn"] else invf_c
        out, span, kept, blocks, skipped = pqs.pqstream_attention(
            q, k, v, tau, invf_a, invf_c, pos_scale_a=c["psa"], rope_scale_a=c["rsa"],
            n_global=c["ng"], n_local=c["nl"], tile=32, block_n=c["bn"], pos_advance=c["adv"],
            use_skip=c["skip"])
        gold = pqs.pqstream_attention_torch(q, k, v, tau, invf_a, invf_c, pos_scale_a=c["psa"],
                                            rope_scale_a=c["rsa"], n_global=c["ng"], n_local=c["nl"],
                                            tile=32, block_n=c["bn"], pos_advance=c["adv"])
        p = f"c{i}_"
        arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = q[0].numpy(), k[0].numpy(), v[0].numpy()
        arrays[p + "tau"] = tau.numpy()
        arrays[p + "inv_freq_a"], arrays[p + "inv_freq_c"] = invf_a.numpy(), invf_c.numpy()
        arrays[p + "params"] = np.array([c["psa"], c["rsa"], c["ng"], c["nl"], c["bn"],
                                         1 if c["adv"] == "full" else 0, int(c["skip"])], np.float64)
        arrays[p + "out"] = out[0].numpy()
        arrays[p + "out_torch"] = gold[0].numpy()
        arrays[p + "span"], arrays[p + "kept"] = span.numpy(), kept.numpy()
        arrays[p + "blocks"], arrays[p + "skipped"] = blocks.numpy(), skipped.numpy()
        print(f"pqstream case {i} {c['name']}: span max {float(span.max()):.0f}, skipped "
              f"{int(skipped.sum())}/{int(blocks.sum())}, |kernel-torch| "
              f"{float((out - gold).abs().max()):.2e}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "pqstream_golden.npz"), **arrays)


if __name__ == "__main__":
    torch.set_num_threads(8)
    pq, pqs = _import_reference()
    which = sys.argv[1:] or ["sets", "composed", "stream"]
    if "sets" in which:
        gen_build_sets_pq(pq)
    if "composed" in which:
        gen_pq_composed(pq)
    if "stream" in which:
        gen_pqstream(pqs)
