#!/usr/bin/env python3
"""Write the golden vectors of PQ Stream's decode rule (one query per call, streamed positions).

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden_decode_pqs.py

Executed from the reference (pqstream_kernel.py), because no closed form pins their edge semantics:

* ``_decode_build_sets_pqs`` (:695-797), plain torch on the CPU, on given score rows: threshold
  at fl(max - tau), the forced global / local / self keys, no cap, and the streamed positions
  (aligned blocks descending from the query, base = kept count of the more recent blocks, natural
  offset inside the block); also with ``scores=None`` (its own torch scores);
* ``_decode_attend_torch`` (:800-817) and ``_decode_attend_triton`` (:820-850, interpreter, fp32)
  on the sets the reference built;
* the per-query prefill of ``install_pqstream_forward(prefill_mode="perquery")`` (:975-993):
  every position P of a short sequence over the cache prefix K[:, :P + 1], torch backends.
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


def _import_pqs():
    os.environ.setdefault("TRITON_INTERPRET", "1")
    sys.path.insert(0, REF)
    import pqstream_kernel as pqs                          # noqa: E402
    return pqs


def gen_sets_from_scores(pqs):
    def randn(seed, H, M, quant=None, scale=1.0):
        r = np.random.default_rng(seed)
        s = (r.standard_normal((H, M)) * scale).astype(np.float32)
        if quant is not None:
            s = (np.round(s / quant) * quant).astype(np.float32)
        return s

    # (name, scores, tau, n_global, n_local, block_n)
    cases = [
        ("plain32", randn(1, 3, 500), [2.0, 1.5, 3.0], 32, 32, 32),
        ("plain64", randn(2, 2, 700), [1.0, 2.5], 8, 8, 64),
        ("sparse_blocks", randn(3, 2, 1500, scale=3.0), [0.5, 1.0], 4, 4, 32),
        ("ties", randn(5, 2, 600, quant=0.5), [1.0, 2.0], 4, 4, 32),
        ("all_forced", randn(8, 2, 5), [1.0, 1.0], 32, 32, 32),
        ("single_key", randn(9, 2, 1), [1.0, 1.0], 4, 4, 32),
        ("partial_block", randn(11, 2, 97), [0.0, 20.0], 2, 2, 32),
        ("no_forced_window", randn(12, 2, 400), [2.0, 2.0], 0, 0, 64),
        ("long", randn(13, 2, 3000), [3.0, 1.5], 32, 32, 32),
    ]
    arrays = {}
    for i, (name, s, tau, ng, nl, bn) in enumerate(cases):
        H, M = s.shape
        qp = M - 1
        q = torch.zeros(H, 8)
        K = torch.zeros(H, M, 8)
        idx, npk, npq = pqs._decode_build_sets_pqs(q, K, torch.tensor(tau, dtype=torch.float32),
                                                   base_inv_freq(8, 10000.0), qp, 1.0, 1.0, 1.0, ng, nl, bn,
                                                   scores=torch.from_numpy(s))
        p = f"c{i}_"
        arrays[p + "scores"] = s
        arrays[p + "tau"] = np.array(tau, np.float32)
        arrays[p + "params"] = np.array([qp, ng, nl, bn], np.int64)
        arrays[p + "idx"] = idx.numpy().astype(np.int64)
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        print(f"pqs decode sets case {i} {name}: M {M} kept {(idx < M).sum(-1).numpy()}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_pqs_sets_golden.npz"), **arrays)


def gen_composed(pqs):
    cases = [
        # (name, seed, H, M, D, pos_scale_a, rope_scale_a, tau, n_global, n_local, block_n)
        ("d64_pi", 61, 2, 700, 64, 0.5, 1.0, 3.0, 32, 32, 32),
        ("d128_bn64", 62, 2, 900, 128, 0.25, 1.0, 2.0, 16, 16, 64),
    ]
    arrays = {}
    for i, (name, seed, H, M, D, ps, rs, tau, ng, nl, bn) in enumerate(cases):
        qa, ka, va = planted_inputs(seed, H, H, M, D, 0.02)
        qp = M - 1
        q = qa[0, :, qp, :].contiguous()
        K, V = ka[0].contiguous(), va[0].contiguous()
        invf = base_inv_freq(D, 10000.0)
        taus = torch.full((H,), tau)
        sm = 1.0 / math.sqrt(D)
        idx, npk, npq = pqs._decode_build_sets_pqs(q, K, taus, invf, qp, ps, rs, sm, ng, nl, bn)
        out_t = pqs._decode_attend_torch(q, K, V, idx, npk, npq, invf, sm)
        out_c = pqs._decode_attend_triton(q, K, V, idx, npk, npq, invf, sm, q_pos=qp, block_k=32)
        p = f"c{i}_"
        arrays[p + "q"] = q.numpy()
        arrays[p + "k"] = K.numpy()
        arrays[p + "v"] = V.numpy()
        arrays[p + "inv_freq"] = invf.numpy()
        arrays[p + "params"] = np.array([qp, ps, rs, tau, ng, nl, bn, sm], np.float64)
        arrays[p + "idx"] = idx.numpy().astype(np.int64)
        arrays[p + "newpos_k"] = npk.numpy()
        arrays[p + "newpos_q"] = npq.numpy()
        arrays[p + "out_torch"] = out_t.numpy()
        arrays[p + "out_triton"] = out_c.numpy()
        print(f"pqs decode composed case {i} {name}: kept {(idx < M).sum(-1).numpy()}, "
              f"attend torch vs triton {float((out_t - out_c).abs().max()):.2e}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "decode_pqs_composed_golden.npz"), **arrays)


def gen_prefill(pqs):
    H, N, D = 2, 260, 64
    qa, ka, va = planted_inputs(71, H, H, N, D, 0.02)
    invf = base_inv_freq(D, 10000.0)
    taus = torch.full((H,), 2.5)
    sm = 1.0 / math.sqrt(D)
    ps, rs, ng, nl, bn = 0.25, 1.0, 8, 8, 32
    Kf, Vf, qf = ka[0], va[0], qa[0]
    outs, sizes = [], []
    for P in range(N):
        Ki, Vi, qi = Kf[:, :P + 1, :], Vf[:, :P + 1, :], qf[:, P, :]
        idx, npk, npq = pqs._decode_build_sets_pqs(qi, Ki, taus, invf, P, ps, rs, sm, ng, nl, bn)
        outs.append(pqs._decode_attend_torch(qi, Ki, Vi, idx, npk, npq, invf, sm))
        sizes.append((idx < P + 1).sum(-1).numpy())
    arrays = {"q": qf.numpy(), "k": Kf.numpy(), "v": Vf.numpy(), "inv_freq": invf.numpy(),
              "params": np.array([ps, rs, 2.5, ng, nl, bn, sm], np.float64),
              "set_size": np.stack(sizes, 1), "out": torch.stack(outs, 1).numpy()}
    print(f"pqs per-query prefill: {N} positions", flush=True)
    np.savez_compressed(os.path.join(OUT, "prefill_pqs_perquery_golden.npz"), **arrays)


def main():
    torch.set_num_threads(8)
    pqs = _import_pqs()
    gen_sets_from_scores(pqs)
    gen_composed(pqs)
    gen_prefill(pqs)


if __name__ == "__main__":
    main()
