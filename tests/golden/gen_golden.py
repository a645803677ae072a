#!/usr/bin/env python3
"""Write the golden input/output vectors the oracle is pinned against.

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    TRITON_INTERPRET=1 python tests/golden/gen_golden.py

Only the functions that no closed form or invariant pins are executed from the reference:

* ``_build_sets`` (shared_selection_triton_exact_2.py:277-426) -- plain torch on the CPU.  Its
  fp32 budget rounding (ceil(float32(p/100) * U)), tie-inclusive cut, 30->25->20 fallback,
  pct=0 special case, measure loop, unresolved-tile truncation and fp32 reposition recurrence are
  exactly the edge semantics the oracle must reproduce bit for bit.
* the composed prefill path ``_select_vote_kernel`` -> ``_build_sets`` -> ``_gather_attn_kernel``
  (exact_2.py:50-140, 146-225, 432-486) under ``TRITON_INTERPRET=1`` on small fp32 shapes (the
  interpreter's fp32 dots are exact; its bf16 dot and fp32->bf16 store are not, so Kernel C is
  only recorded for fp32 inputs), including ragged last tiles, the k_max truncation path,
  q_pos_base > 0 and a hybrid two-geometry case (hybrid_exact.py:450-510).
* Kernel A alone on bf16 inputs (its dots see fp32 operands after the rotation, which the
  interpreter computes exactly).

Every fixture stores its inputs and the reference's outputs as plain arrays in one .npz.
"""
import math
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))


def _import_reference():
    os.environ.setdefault("TRITON_INTERPRET", "1")
    sys.path.insert(0, REF)
    import shared_selection_triton_exact_2 as ex2          # noqa: E402
    import shared_selection_triton_hybrid_exact as hyb     # noqa: E402
    return ex2, hyb


def planted_inputs(seed, H, Hkv, N, D, frac, dtype=torch.float32):
    """Gaussian Q, K, V with planted keys (+3 u_h) and every query shifted by +1 u_h."""
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(1, H, N, D, generator=g)
    k = torch.randn(1, Hkv, N, D, generator=g)
    v = torch.randn(1, Hkv, N, D, generator=g)
    u = torch.nn.functional.normalize(torch.randn(Hkv, D, generator=g), dim=-1)
    planted = torch.randperm(N, generator=g)[:max(1, round(frac * N))]
    for h in range(Hkv):
        k[0, h, planted] += 3.0 * u[h]
    grp = H // Hkv
    for h in range(H):
        q[0, h] += 1.0 * u[h // grp]
    return q.to(dtype), k.to(dtype), v.to(dtype)


def base_inv_freq(D, theta):
    return 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))


# ---------------------------------------------------------------------------------------------
# _build_sets on synthetic vote tensors
# ---------------------------------------------------------------------------------------------
def gen_build_sets(ex2):
    cases = []
    rng = np.random.default_rng(1234)

    def causal_votes(H, nt, N, T, q_pos_base, density, seed):
        r = np.random.default_rng(seed)
        v = np.zeros((H, nt, N), np.int32)
        for t in range(nt):
            hi = min(N, q_pos_base + (t + 1) * T)
            v[:, t, :hi] = r.binomial(T, density, size=(H, hi))
        return v

    # 1. typical freq votes, cap never binds
    cases.append(dict(name="plain", votes=causal_votes(2, 6, 384, 64, 0, 0.3, 1), pos_scale=1.0,
                      n_global=32, n_local=32, pct=30.0, T=64, k_max=2048, q_pos_base=0, measure=False))
    # 2. cap binds: fallback 30 -> 25 -> 20 and unresolved truncation, PI reposition
    cases.append(dict(name="cap_fallback", votes=causal_votes(3, 8, 512, 64, 0, 0.6, 2),
                      pos_scale=1.0 / 3.0, n_global=32, n_local=32, pct=30.0, T=64, k_max=160,
                      q_pos_base=0, measure=False))
    # 3. same with measure=True (1% steps below the floor)
    c = dict(cases[-1]); c.update(name="cap_measure", measure=True, k_max=140)
    cases.append(c)
    # 4. ragged last tile, tile 32, n_global > tile, pos_scale 0.25
    cases.append(dict(name="ragged_t32", votes=causal_votes(2, 7, 200, 32, 0, 0.5, 3), pos_scale=0.25,
                      n_global=40, n_local=16, pct=30.0, T=32, k_max=96, q_pos_base=0, measure=False))
    # 5. pct variants: 25 (steps [25,20]), 22.5 (round-half-even -> 22), 20, 10, 100, 0
    for i, pct in enumerate([25.0, 22.5, 20.0, 10.0, 100.0, 0.0]):
        cases.append(dict(name=f"pct_{pct:g}", votes=causal_votes(2, 5, 320, 64, 0, 0.5, 10 + i),
                          pos_scale=0.5, n_global=8, n_local=8, pct=pct, T=64, k_max=120,
                          q_pos_base=0, measure=(i % 2 == 0)))
    # 6. q_pos_base > 0 (decode-style tile origin), small k_max
    cases.append(dict(name="qbase", votes=causal_votes(2, 4, 300, 64, 44, 0.4, 20), pos_scale=0.75,
                      n_global=16, n_local=24, pct=30.0, T=64, k_max=100, q_pos_base=44,
                      measure=True))
    # 7. budget rounding: U = 50 distinct positive votes -> fp32 budget 16, rational 15
    v = np.zeros((1, 1, 256), np.int32)
    v[0, 0, 100:150] = np.arange(1, 51)
    cases.append(dict(name="budget_u50", votes=v, pos_scale=1.0, n_global=0, n_local=1, pct=30.0,
                      T=64, k_max=2048, q_pos_base=0, measure=False))
    # 8. heavy ties: votes in {0, T} only
    vt = (rng.random((2, 4, 256)) < 0.5).astype(np.int32) * 64
    cases.append(dict(name="ties", votes=vt, pos_scale=1.0, n_global=4, n_local=4, pct=30.0, T=64,
                      k_max=64, q_pos_base=0, measure=True))
    # 9. a tile where no query kept anything (U = 0 -> v_cut = 0 keeps every key)
    vz = causal_votes(1, 3, 192, 64, 0, 0.3, 30)
    vz[0, 1, :] = 0
    cases.append(dict(name="empty_tile", votes=vz, pos_scale=1.0, n_global=4, n_local=4, pct=30.0,
                      T=64, k_max=400, q_pos_base=0, measure=False))

    arrays = {}
    for i, c in enumerate(cases):
        votes = torch.from_numpy(c["votes"])
        res = ex2._build_sets(votes, c["pos_scale"], c["n_global"], c["n_local"], c["pct"], c["T"],
                              c["k_max"], q_pos_base=c["q_pos_base"], measure=c["measure"])
        names = ["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen",
                 "orig_overflow", "kpct_meas", "overflow20"]
        p = f"c{i}_"
        arrays[p + "votes"] = c["votes"]
        arrays[p + "params"] = np.array([c["pos_scale"], c["n_global"], c["n_local"], c["pct"], c["T"],
                                         c["k_max"], c["q_pos_base"], float(c["measure"])], np.float64)
        for n, t in zip(names, res):
            arrays[p + n] = t.numpy()
        print(f"build_sets case {i} {c['name']}: chosen {np.unique(res[5].numpy())}, "
              f"overflow20 {int(res[8].sum())}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "build_sets_golden.npz"), **arrays)


# ---------------------------------------------------------------------------------------------
# composed prefill path under the interpreter
# ---------------------------------------------------------------------------------------------
def run_kernel_a(mod, q, k, tau, inv_freq, sm_scale, pos_scale, rope_scale, tile, block_n, q_pos_base):
    """The Kernel A launch exactly as shared_pi_attention issues it (exact_2.py:440-465)."""
    Z, H, N, D = q.shape
    nt = (N + tile - 1) // tile
    qh, kh = q[0].contiguous(), k[0].contiguous()
    votes = torch.zeros((H, nt, N), dtype=torch.int32)
    row_counts = torch.zeros((H, N), dtype=torch.int32)
    wvotes = torch.zeros((H, 1, 1), dtype=torch.float32)
    mod._select_vote_kernel[(nt, H)](
        qh, kh, tau.float().contiguous(), inv_freq.float().contiguous(), votes, row_counts, wvotes,
        sm_scale, float(pos_scale), float(rope_scale), int(q_pos_base),
        qh.stride(0), qh.stride(1), qh.stride(2), kh.stride(0), kh.stride(1), kh.stride(2),
        votes.stride(0), votes.stride(1), votes.stride(2), row_counts.stride(0), row_counts.stride(1),
        wvotes.stride(0), wvotes.stride(1), wvotes.stride(2),
        H, N, BLOCK_M=tile, BLOCK_N=block_n, HEAD_DIM=D, HALF_DIM=D // 2, WMODE=0,
        num_warps=4, num_stages=1)
    return votes, row_counts


def run_kernel_c(mod, q, k, v, inv_freq, idx, npk, npq, sm_scale, rope_scale, tile, block_k, k_max,
                 q_pos_base):
    """The Kernel C launch exactly as shared_pi_attention issues it (exact_2.py:471-485)."""
    Z, H, N, D = q.shape
    nt = (N + tile - 1) // tile
    qh, kh, vh = q[0].contiguous(), k[0].contiguous(), v[0].contiguous()
    out = torch.empty((H, N, D), dtype=q.dtype)
    mod._gather_attn_kernel[(nt, H)](
        qh, kh, vh, inv_freq.float().contiguous(), idx, npk, npq, out,
        sm_scale, float(rope_scale), int(q_pos_base),
        qh.stride(0), qh.stride(1), qh.stride(2), kh.stride(0), kh.stride(1), kh.stride(2),
        vh.stride(0), vh.stride(1), vh.stride(2), idx.stride(0), idx.stride(1), idx.stride(2),
        npk.stride(0), npk.stride(1), npk.stride(2), npq.stride(0), npq.stride(1), npq.stride(2),
        out.stride(0), out.stride(1), out.stride(2),
        H, N, BLOCK_M=tile, BLOCK_K=block_k, K_MAX=k_max, HEAD_DIM=D, HALF_DIM=D // 2,
        num_warps=4, num_stages=1)
    return out


def gen_composed(ex2, hyb):
    cases = [
        # name, H, N, D, tile, k_max, tau, pct, n_global, n_local, pos_scale, theta, q_pos_base, frac
        dict(name="c0_like", H=2, N=256, D=64, tile=64, k_max=2048, tau=5.0, pct=30.0, ng=32, nl=32,
             ps=1.0, theta=10000.0, qb=0, frac=0.02, seed=0),
        dict(name="pi_cap_ragged", H=2, N=200, D=64, tile=32, k_max=48, tau=3.0, pct=30.0, ng=4, nl=8,
             ps=0.5, theta=10000.0, qb=0, frac=0.05, seed=1),
        dict(name="pi_third_t64", H=2, N=320, D=64, tile=64, k_max=96, tau=2.5, pct=30.0, ng=8, nl=16,
             ps=1.0 / 3.0, theta=10000.0, qb=0, frac=0.02, seed=2),
        dict(name="identity_kat", H=1, N=130, D=64, tile=32, k_max=256, tau=float("inf"), pct=100.0,
             ng=32, nl=32, ps=1.0, theta=10000.0, qb=0, frac=0.02, seed=3),
        dict(name="qbase", H=2, N=160, D=64, tile=32, k_max=64, tau=3.0, pct=30.0, ng=4, nl=8,
             ps=0.5, theta=10000.0, qb=16, frac=0.05, seed=4),
    ]
    arrays = {}
    for i, c in enumerate(cases):
        q, k, v = planted_inputs(c["seed"], c["H"], c["H"], c["N"], c["D"], c["frac"])
        tau = torch.full((c["H"],), c["tau"], dtype=torch.float32)
        invf = base_inv_freq(c["D"], c["theta"])
        sm = 1.0 / math.sqrt(c["D"])
        votes, rc = run_kernel_a(ex2, q, k, tau, invf, sm, c["ps"], 1.0, c["tile"], 64, c["qb"])
        sets = ex2._build_sets(votes, c["ps"], c["ng"], c["nl"], c["pct"], c["tile"], c["k_max"],
                               q_pos_base=c["qb"])
        idx, npk, npq = sets[0], sets[1], sets[2]
        out = run_kernel_c(ex2, q, k, v, invf, idx, npk, npq, sm, 1.0, c["tile"], 64, c["k_max"], c["qb"])
        # the public entry point, for the end-to-end record (same launches as above)
        full = ex2.shared_pi_attention(q, k, v, tau, invf, pos_scale=c["ps"], pct=c["pct"],
                                       n_global=c["ng"], n_local=c["nl"], tile=c["tile"],
                                       k_max=c["k_max"], q_pos_base=c["qb"])
        assert torch.equal(full[0][0], out)
        p = f"c{i}_"
        arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = q[0].numpy(), k[0].numpy(), v[0].numpy()
        arrays[p + "tau"], arrays[p + "inv_freq"] = tau.numpy(), invf.numpy()
        arrays[p + "params"] = np.array([c["tile"], c["k_max"], c["pct"], c["ng"], c["nl"], c["ps"],
                                         c["qb"], sm], np.float64)
        arrays[p + "votes"], arrays[p + "row_counts"] = votes.numpy(), rc.numpy()
        for n, t in zip(["idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen",
                         "orig_overflow", "kpct_meas", "overflow20"], sets):
            arrays[p + n] = t.numpy()
        arrays[p + "out"] = out.numpy()
        print(f"composed case {i} {c['name']}: kept {sets[4].float().mean():.1f} "
              f"overflow20 {int(sets[8].sum())}", flush=True)
    arrays["ncases"] = np.array(len(cases))

    # hybrid: Kernel A under a YaRN-like geometry, _build_sets + Kernel C under PI
    H, N, D, tile, k_max = 2, 224, 64, 32, 80
    q, k, v = planted_inputs(7, H, H, N, D, 0.03)
    tau = torch.full((H,), 3.5, dtype=torch.float32)
    invf_a = base_inv_freq(D, 10000.0) * torch.linspace(1.0, 0.25, D // 2)
    invf_c = base_inv_freq(D, 10000.0)
    res = hyb.shared_pi_attention(q, k, v, tau, invf_a, 1.0, 1.1386294, invf_c, 0.4, 1.0, pct=30.0,
                                  n_global=8, n_local=8, tile=tile, k_max=k_max)
    arrays["hyb_q"], arrays["hyb_k"], arrays["hyb_v"] = q[0].numpy(), k[0].numpy(), v[0].numpy()
    arrays["hyb_tau"], arrays["hyb_inv_freq_a"], arrays["hyb_inv_freq_c"] = (
        tau.numpy(), invf_a.numpy(), invf_c.numpy())
    arrays["hyb_params"] = np.array([tile, k_max, 30.0, 8, 8, 1.0, 1.1386294, 0.4, 1.0], np.float64)
    for n, t in zip(["out", "shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas",
                     "overflow20"], res):
        arrays["hyb_" + n] = t[0].numpy() if n == "out" else t.numpy()
    print("hybrid case done", flush=True)
    np.savez_compressed(os.path.join(OUT, "composed_golden.npz"), **arrays)


def gen_kernel_a_bf16(ex2):
    arrays = {}
    for i, (H, N, D, tile, ps) in enumerate([(2, 256, 64, 64, 1.0), (2, 192, 128, 32, 1.0 / 3.0)]):
        q, k, _ = planted_inputs(40 + i, H, H, N, D, 0.02, dtype=torch.bfloat16)
        tau = torch.full((H,), 5.0, dtype=torch.float32)
        invf = base_inv_freq(D, 10000.0)
        sm = 1.0 / math.sqrt(D)
        votes, rc = run_kernel_a(ex2, q, k, tau, invf, sm, ps, 1.0, tile, 64, 0)
        p = f"c{i}_"
        arrays[p + "q"] = q[0].view(torch.int16).numpy().view(np.uint16)
        arrays[p + "k"] = k[0].view(torch.int16).numpy().view(np.uint16)
        arrays[p + "tau"], arrays[p + "inv_freq"] = tau.numpy(), invf.numpy()
        arrays[p + "params"] = np.array([tile, ps, sm], np.float64)
        arrays[p + "votes"], arrays[p + "row_counts"] = votes.numpy(), rc.numpy()
        print(f"kernel A bf16 case {i}: votes sum {int(votes.sum())}", flush=True)
    arrays["ncases"] = np.array(2)
    np.savez_compressed(os.path.join(OUT, "kernel_a_bf16_golden.npz"), **arrays)


if __name__ == "__main__":
    torch.set_num_threads(8)
    ex2, hyb = _import_reference()
    gen_build_sets(ex2)
    gen_composed(ex2, hyb)
    gen_kernel_a_bf16(ex2)
