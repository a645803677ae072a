#!/usr/bin/env python3
"""Write the golden vectors of the decode path (one query per call selecting its own key set).

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden_decode.py

Executed from the reference, because no closed form pins their edge semantics:

* ``_decode_build_sets`` (shared_selection_triton_exact_2.py:527-604), plain torch on the CPU,
  on given score vectors: threshold at fl(max - tau), the top-pct_decode% cut over the passers
  (fp32 budget, tie-inclusive), the forced global / local / self keys, the k_max cap by score
  over the non-forced keys (tie-inclusive cut, budget <= 0), the ascending truncation to k_max
  and the fp32 reposition recurrence; also with ``scores=None`` (its own torch scores).
* ``_decode_scores_kernel`` (:505-525, the Triton ``_decode_select_kernel`` :235-271) under the
  interpreter on fp32 inputs.
* ``_decode_attend_torch`` (:608-623) and ``_decode_attend_kernelC`` (:626-655, Kernel C with one
  real query row; interpreter, fp32) on the sets the reference itself built.
* a decode sequence: the per-token loop of spi_forward (:743-762) for a few consecutive query
  positions over one cache, every call on the cache prefix K[:, :P + 1].

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


def gen_sets_from_scores(ex2):
    """_decode_build_sets on crafted score rows (H, M)."""
    cases = []

    def randn(seed, H, M, quant=None, scale=1.0):
        r = np.random.default_rng(seed)
        s = (r.standard_normal((H, M)) * scale).astype(np.float32)
        if quant is not None:   # coarse values: many exact ties at every cut
            s = (np.round(s / quant) * quant).astype(np.float32)
        return s

    # (name, scores, tau, q_pos, pos_scale, n_global, n_local, k_max, pct_decode)
    cases.append(("plain", randn(1, 3, 500), [2.0, 1.5, 3.0], 499, 1.0, 32, 32, 1024, 100.0))
    cases.append(("cap", randn(2, 3, 700), [6.0, 6.0, 6.0], 699, 1.0 / 3.0, 8, 8, 64, 100.0))
    cases.append(("pct30", randn(3, 2, 900), [2.5, 2.5], 899, 0.5, 16, 16, 2048, 30.0))
    cases.append(("pct_cap_ties", randn(4, 3, 800, quant=0.25), [3.0, 2.0, 4.0], 799, 1.0 / 3.0, 8, 8,
                  48, 30.0))
    cases.append(("cap_ties", randn(5, 2, 600, quant=0.5), [5.0, 5.0], 599, 1.0, 4, 4, 40, 100.0))
    cases.append(("budget_nonpositive", randn(6, 2, 300), [9.0, 9.0], 299, 0.25, 8, 8, 10, 100.0))
    cases.append(("qpos_inside", randn(7, 2, 300), [2.0, 2.0], 200, 0.75, 16, 16, 128, 100.0))
    cases.append(("all_forced", randn(8, 2, 5), [1.0, 1.0], 4, 1.0, 32, 32, 64, 100.0))
    cases.append(("single_key", randn(9, 2, 1), [1.0, 1.0], 0, 1.0, 32, 32, 16, 30.0))
    cases.append(("pct_fraction", randn(10, 2, 777), [3.0, 3.0], 776, 1.0 / 3.0, 32, 32, 2048, 22.5))
    cases.append(("kmax_over_m", randn(11, 2, 100), [20.0, 20.0], 99, 0.5, 2, 2, 512, 100.0))
    cases.append(("no_local", randn(12, 2, 400), [2.0, 2.0], 399, 1.0, 0, 0, 32, 100.0))
    cases.append(("pct_small", randn(13, 2, 1000, scale=3.0), [10.0, 10.0], 999, 0.2, 32, 32, 100, 5.0))

    arrays = {}
    for i, (name, s, tau, qp, ps, ng, nl, km, pctd) in enumerate(cases):
        H, M = s.shape
        q = torch.zeros(H, 8)
        K = torch.zeros(H, M, 8)
        idx, npk, npq = ex2._decode_build_sets(q, K, torch.tensor(tau, dtype=torch.float32),
                                               base_inv_freq(8, 10000.0), qp, ps, 1.0, 1.0, ng, nl, km,
                                               pctd, scores=torch.from_numpy(s))
        p = f"c{i}_"
        arrays[p + "scores"] = s
        arrays[p + "tau"] = np.array(tau, np.float32)
        arrays[p + "params"] = np.array([qp, ps, ng, nl, km, pctd], np.float64)
        arrays[p + "idx"] = idx.numpy()
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        nvalid = (idx < M).sum(-1).numpy()
        print(f"decode sets case {i} {name}: M {M} valid slots {nvalid}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_sets_golden.npz"), **arrays)


def gen_composed(ex2):
    """Scores (Triton kernel under the interpreter and the torch path), sets and attend."""
    cases = [
        # (name, seed, H, M, D, q_pos, pos_scale, rope_scale, tau, n_global, n_local, k_max, pct_decode)
        ("d64_pi", 21, 2, 700, 64, 699, 0.5, 1.0, 5.0, 32, 32, 256, 100.0),
        ("d128_cap", 22, 2, 900, 128, 899, 1.0 / 3.0, 1.0, 5.0, 16, 16, 96, 100.0),
        ("d64_pct_yarn", 23, 3, 513, 64, 512, 1.0, 1.1386294, 4.0, 8, 8, 2048, 30.0),
        ("d128_inside", 24, 2, 400, 128, 250, 0.25, 1.0, 5.0, 32, 32, 200, 100.0),
    ]
    arrays = {}
    for i, (name, seed, H, M, D, qp, ps, rs, tau, ng, nl, km, pctd) in enumerate(cases):
        qa, ka, va = planted_inputs(seed, H, H, M, D, 0.02)
        q = qa[0, :, qp, :].contiguous()        # (H, D): the query at position qp
        K, V = ka[0].contiguous(), va[0].contiguous()
        invf = base_inv_freq(D, 10000.0)
        taus = torch.full((H,), tau)
        sm = 1.0 / math.sqrt(D)
        s_tri = ex2._decode_scores_kernel(q, K, invf, qp, ps, rs, sm, block_n=64)
        idx_t, npk_t, npq_t = ex2._decode_build_sets(q, K, taus, invf, qp, ps, rs, sm, ng, nl, km, pctd)
        idx, npk, npq = ex2._decode_build_sets(q, K, taus, invf, qp, ps, rs, sm, ng, nl, km, pctd,
                                               scores=s_tri)
        out_t = ex2._decode_attend_torch(q, K, V, idx, npk, npq, invf, rs, sm)
        out_c = ex2._decode_attend_kernelC(q, K, V, idx, npk, npq, invf, rs, sm, km, q_pos=qp, block_k=32)
        p = f"c{i}_"
        arrays[p + "q"] = q.numpy()
        arrays[p + "k"] = K.numpy()
        arrays[p + "v"] = V.numpy()
        arrays[p + "inv_freq"] = invf.numpy()
        arrays[p + "params"] = np.array([qp, ps, rs, tau, ng, nl, km, pctd, sm], np.float64)
        arrays[p + "scores_triton"] = s_tri.numpy()
        arrays[p + "idx_torch_scores"] = idx_t.numpy()
        arrays[p + "newpos_k_torch_scores"] = npk_t.numpy()
        arrays[p + "newpos_q_torch_scores"] = npq_t.numpy()
        arrays[p + "idx"] = idx.numpy()
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        arrays[p + "out_torch"] = out_t.numpy()
        arrays[p + "out_kernelc"] = out_c.numpy()
        print(f"decode composed case {i} {name}: valid {(idx < M).sum(-1).numpy()}, "
              f"torch-vs-triton-score sets equal {bool(torch.equal(idx, idx_t))}, "
              f"attend torch vs kernelC {float((out_t - out_c).abs().max()):.2e}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_composed_golden.npz"), **arrays)


def gen_sequence(ex2):
    """The per-token loop of spi_forward (exact_2.py:743-762): query P over the cache prefix."""
    H, N, D = 2, 600, 64
    qa, ka, va = planted_inputs(31, H, H, N, D, 0.02)
    invf = base_inv_freq(D, 10000.0)
    taus = torch.full((H,), 5.0)
    sm = 1.0 / math.sqrt(D)
    ps, rs, ng, nl, km, pctd = 0.5, 1.0, 32, 32, 128, 100.0
    P0, Q = 590, 10
    Kf, Vf, qf = ka[0], va[0], qa[0]
    outs, idxs, npks, npqs = [], [], [], []
    for i in range(Q):
        P = P0 + i
        Ki, Vi, qi = Kf[:, :P + 1, :], Vf[:, :P + 1, :], qf[:, P, :]
        idx, npk, npq = ex2._decode_build_sets(qi, Ki, taus, invf, P, ps, rs, sm, ng, nl, km, pctd)
        outs.append(ex2._decode_attend_torch(qi, Ki, Vi, idx, npk, npq, invf, rs, sm))
        idxs.append(idx)
        npks.append(npk)
        npqs.append(npq)
    arrays = {
        "q": qf[:, P0:P0 + Q, :].numpy(), "k": Kf[:, :P0 + Q, :].numpy(), "v": Vf[:, :P0 + Q, :].numpy(),
        "inv_freq": invf.numpy(), "params": np.array([P0, Q, ps, rs, 5.0, ng, nl, km, pctd, sm], np.float64),
        "idx": torch.stack(idxs, 1).numpy(), "newpos_k": torch.stack(npks, 1).numpy(),
        "newpos_q": torch.stack(npqs, 1).numpy(), "out": torch.stack(outs, 1).numpy(),
    }
    print(f"decode sequence: positions {P0}..{P0 + Q - 1}", flush=True)
    np.savez_compressed(os.path.join(OUT, "decode_sequence_golden.npz"), **arrays)


def main():
    torch.set_num_threads(8)
    ex2, _ = _import_reference()
    gen_sets_from_scores(ex2)
    gen_composed(ex2)
    gen_sequence(ex2)


if __name__ == "__main__":
    main()
