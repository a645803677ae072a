#!/usr/bin/env python3
"""Write the golden vectors of the per-query (PQ) decode rule, which is also the prefill rule of
config 3 ("each query keeps its own keys ... capped at 2048 keys per query by score rank").

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden_decode_pq.py

Executed from the reference (shared_selection_triton_perquery.py), because no closed form pins
their edge semantics:

* ``_decode_build_sets_pq`` (:651-720), plain torch on the CPU, on given score rows: threshold
  at fl(max - tau), the forced global / local / self keys, the k_max cap as forced + the
  top-(k_max - n_forced) non-forced keys by score (an exact budget through torch.topk), and the
  dense-rank positions over the final set; also with ``scores=None`` (its own torch scores).
* ``_decode_attend_torch_pq`` (:723-740) and ``_decode_attend_kernelC_pq`` (:743-778, the PQ
  Kernel C with one real query row; interpreter, fp32) on the sets the reference built.
* the per-query prefill of ``install_shared_pi_forward(prefill_mode="perquery")`` (:905-924):
  every position P of a short sequence selects over the cache prefix K[:, :P + 1] and attends
  it, with the torch selection and the torch attend.

Every fixture stores its inputs and the reference's outputs as plain arrays in one .npz.
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from gen_golden import REF, base_inv_freq, planted_inputs  # noqa: E402

OUT = HERE


def _import_pq():
    os.environ.setdefault("TRITON_INTERPRET", "1")
    sys.path.insert(0, REF)
    import shared_selection_triton_perquery as pq          # noqa: E402
    return pq


def gen_sets_from_scores(pq):
    """_decode_build_sets_pq on crafted score rows (H, M); q_pos = M - 1 as the reference asks."""
    def randn(seed, H, M, quant=None, scale=1.0):
        r = np.random.default_rng(seed)
        s = (r.standard_normal((H, M)) * scale).astype(np.float32)
        if quant is not None:   # coarse values: exact ties at the cap's cut
            s = (np.round(s / quant) * quant).astype(np.float32)
        return s

    # (name, scores, tau, n_global, n_local, k_max)
    cases = [
        ("plain", randn(1, 3, 500), [2.0, 1.5, 3.0], 32, 32, 1024),
        ("cap", randn(2, 3, 700), [6.0, 6.0, 6.0], 8, 8, 64),
        ("cap_deep", randn(3, 2, 3000), [4.0, 4.0], 32, 32, 256),
        ("cap_ties", randn(5, 2, 600, quant=0.5), [5.0, 5.0], 4, 4, 40),
        ("budget_zero", randn(6, 2, 300), [9.0, 9.0], 5, 5, 10),
        ("all_forced", randn(8, 2, 5), [1.0, 1.0], 32, 32, 64),
        ("single_key", randn(9, 2, 1), [1.0, 1.0], 4, 4, 16),
        ("kmax_over_m", randn(11, 2, 100), [20.0, 20.0], 2, 2, 512),
        ("no_forced_window", randn(12, 2, 400), [2.0, 2.0], 0, 0, 32),
        ("wide_tau", randn(13, 2, 1000, scale=3.0), [10.0, 10.0], 32, 32, 100),
        ("tight_tau", randn(14, 3, 800), [0.25, 0.5, 0.0], 16, 16, 128),
    ]
    arrays = {}
    for i, (name, s, tau, ng, nl, km) in enumerate(cases):
        H, M = s.shape
        qp = M - 1
        q = torch.zeros(H, 8)
        K = torch.zeros(H, M, 8)
        idx, npk, npq = pq._decode_build_sets_pq(q, K, torch.tensor(tau, dtype=torch.float32),
                                                 base_inv_freq(8, 10000.0), qp, 1.0, 1.0, 1.0, ng, nl, km,
                                                 scores=torch.from_numpy(s))
        p = f"c{i}_"
        arrays[p + "scores"] = s
        arrays[p + "tau"] = np.array(tau, np.float32)
        arrays[p + "params"] = np.array([qp, ng, nl, km], np.int64)
        arrays[p + "idx"] = idx.numpy().astype(np.int64)
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        print(f"pq decode sets case {i} {name}: M {M} valid slots {(idx < M).sum(-1).numpy()}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_pq_sets_golden.npz"), **arrays)


def gen_composed(pq):
    """Sets from the reference's torch scores and from its Triton scores, then both attends."""
    cases = [
        # (name, seed, H, M, D, pos_scale_a, rope_scale_a, tau, n_global, n_local, k_max)
        ("d64_pi", 41, 2, 700, 64, 0.5, 1.0, 4.0, 32, 32, 256),
        ("d128_cap", 42, 2, 900, 128, 0.25, 1.0, 4.0, 16, 16, 96),
        ("d64_yarn_scale", 43, 3, 513, 64, 1.0, 1.1386294, 3.0, 8, 8, 2048),
    ]
    arrays = {}
    for i, (name, seed, H, M, D, ps, rs, tau, ng, nl, km) in enumerate(cases):
        qa, ka, va = planted_inputs(seed, H, H, M, D, 0.02)
        qp = M - 1
        q = qa[0, :, qp, :].contiguous()
        K, V = ka[0].contiguous(), va[0].contiguous()
        invf_a = base_inv_freq(D, 10000.0) * (0.5 if rs != 1.0 else 1.0)
        invf_c = base_inv_freq(D, 10000.0)
        taus = torch.full((H,), tau)
        sm = 1.0 / math.sqrt(D)
        s_tri = pq._decode_scores_kernel(q, K, invf_a, qp, ps, rs, sm, block_n=64)
        idx_t, npk_t, npq_t = pq._decode_build_sets_pq(q, K, taus, invf_a, qp, ps, rs, sm, ng, nl, km)
        idx, npk, npq = pq._decode_build_sets_pq(q, K, taus, invf_a, qp, ps, rs, sm, ng, nl, km, scores=s_tri)
        out_t = pq._decode_attend_torch_pq(q, K, V, idx, npk, npq, invf_c, sm)
        out_c = pq._decode_attend_kernelC_pq(q, K, V, idx, npk, npq, invf_c, sm, km, q_pos=qp, block_k=32)
        p = f"c{i}_"
        arrays[p + "q"] = q.numpy()
        arrays[p + "k"] = K.numpy()
        arrays[p + "v"] = V.numpy()
        arrays[p + "inv_freq_a"] = invf_a.numpy()
        arrays[p + "inv_freq_c"] = invf_c.numpy()
        arrays[p + "params"] = np.array([qp, ps, rs, tau, ng, nl, km, sm], np.float64)
        arrays[p + "scores_triton"] = s_tri.numpy()
        arrays[p + "idx_torch_scores"] = idx_t.numpy().astype(np.int64)
        arrays[p + "newpos_k_torch_scores"] = npk_t.numpy()
        arrays[p + "newpos_q_torch_scores"] = npq_t.numpy()
        arrays[p + "idx"] = idx.numpy().astype(np.int64)
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        arrays[p + "out_torch"] = out_t.numpy()
        arrays[p + "out_kernelc"] = out_c.numpy()
        print(f"pq decode composed case {i} {name}: valid {(idx < M).sum(-1).numpy()}, "
              f"torch-vs-triton-score sets equal {bool(torch.equal(idx, idx_t))}, "
              f"attend torch vs kernelC {float((out_t - out_c).abs().max()):.2e}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_pq_composed_golden.npz"), **arrays)


def gen_prefill(pq):
    """The per-query prefill loop (perquery.py:905-924, select and attend backends "torch")."""
    H, N, D = 2, 300, 64
    qa, ka, va = planted_inputs(51, H, H, N, D, 0.02)
    invf_a = base_inv_freq(D, 10000.0)
    invf_c = base_inv_freq(D, 10000.0)
    taus = torch.full((H,), 4.0)
    sm = 1.0 / math.sqrt(D)
    ps, rs, ng, nl, km = 0.25, 1.0, 8, 8, 48
    Kf, Vf, qf = ka[0], va[0], qa[0]
    outs, idxs, npks, npqs = [], [], [], []
    for P in range(N):
        Ki, Vi, qi = Kf[:, :P + 1, :], Vf[:, :P + 1, :], qf[:, P, :]
        idx, npk, npq = pq._decode_build_sets_pq(qi, Ki, taus, invf_a, P, ps, rs, sm, ng, nl, km)
        outs.append(pq._decode_attend_torch_pq(qi, Ki, Vi, idx, npk, npq, invf_c, sm))
        idxs.append(idx.numpy().astype(np.int64))
        npks.append(npk.numpy())
        npqs.append(npq.numpy())
    arrays = {
        "q": qf.numpy(), "k": Kf.numpy(), "v": Vf.numpy(), "inv_freq_a": invf_a.numpy(),
        "inv_freq_c": invf_c.numpy(), "params": np.array([ps, rs, 4.0, ng, nl, km, sm], np.float64),
        "idx": np.stack(idxs, 1), "newpos_k": np.stack(npks, 1), "newpos_q": np.stack(npqs, 1),
        "out": torch.stack(outs, 1).numpy(),
    }
    print(f"pq per-query prefill: {N} positions, capped rows {(np.stack(idxs, 1) < N).sum(-1).max()}",
          flush=True)
    np.savez_compressed(os.path.join(OUT, "prefill_pq_perquery_golden.npz"), **arrays)


def main():
    torch.set_num_threads(8)
    pq = _import_pq()
    gen_sets_from_scores(pq)
    gen_composed(pq)
    gen_prefill(pq)


if __name__ == "__main__":
    main()
