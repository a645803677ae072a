"""GPU parity of the decode path (sta_decode_*) through the C ABI.

  * selection from given scores: bit for bit against the reference's _decode_build_sets
    (tests/golden/decode_sets_golden.npz) and against the oracle on crafted score tensors with
    heavy ties, the cap, pct_decode < 100 and caches longer than the LDS key store;
  * scores, sets and attend against the reference's decode functions on fp32 inputs
    (tests/golden/decode_composed_golden.npz) and the batched form against its per-token loop
    (tests/golden/decode_sequence_golden.npz);
  * planted bf16 / fp16 / fp32 inputs with GQA, checked in layers: scores within rounding of the
    oracle's; the oracle's selection applied to the GPU's own scores reproduces every set bit for
    bit; the oracle's attend applied to the GPU's sets reproduces the output within tolerance.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import check_output, np_of, out_f32

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda:0"


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _plan_for_scores(scores, tau, q_pos0, pos_scale, ng, nl, km, pctd, D=64):
    """A decode plan whose selection runs on given scores (H, Q, M)."""
    import _sta_native as native
    H, Q, M = scores.shape
    q = torch.zeros((H, Q, D), device=DEV)
    k = torch.zeros((H, M, D), device=DEV)
    invf = torch.ones(D // 2, device=DEV)
    return native.DecodePlan(q, k, None, torch.as_tensor(tau, dtype=torch.float32), invf, q_pos0, pos_scale, 1.0,
                             1.0, ng, nl, km, pctd)


def test_decode_sets_match_reference_goldens():
    import shared_selection_triton_exact_2 as ex2
    g = _load("decode_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, ng, nl, km, pctd = g[p + "params"]
        s = g[p + "scores"]
        H, M = s.shape
        say(f"decode sets golden case {i}: H={H} M={M} k_max={int(km)} pct_decode={pctd}")
        q = torch.zeros((H, 64), device=DEV)
        K = torch.zeros((H, M, 64), device=DEV)
        idx, npk, npq = ex2._decode_build_sets(q, K, torch.from_numpy(g[p + "tau"]), torch.ones(32), int(qp),
                                               float(ps), 1.0, 1.0, int(ng), int(nl), int(km), float(pctd),
                                               scores=torch.from_numpy(s))
        torch.cuda.synchronize()
        assert idx.dtype == torch.int64
        assert np.array_equal(idx.cpu().numpy(), g[p + "idx"]), i
        assert _bits_equal(npk.cpu().numpy(), g[p + "newpos_k"]), i
        assert _bits_equal(npq.cpu().numpy(), g[p + "newpos_q"]), i


@pytest.mark.parametrize("case", [
    # (seed, H, Q, M, k_max, n_global, n_local, pct_decode, quant, pos_scale)
    (1, 3, 4, 3000, 256, 32, 32, 100.0, None, 1.0 / 3.0),
    (2, 2, 3, 5000, 64, 8, 8, 30.0, 0.25, 0.5),          # ties at both cuts
    (3, 2, 2, 1200, 10, 8, 8, 100.0, None, 1.0),          # budget_c <= 0: forced keys only
    (4, 2, 5, 800, 4096, 0, 0, 7.5, 0.5, 0.25),           # k_max above M, heavy ties in the pct cut
    (5, 2, 2, 40000, 2048, 32, 32, 100.0, None, 1.0 / 3.0),   # the global key store (past LDS)
    (6, 1, 3, 45000, 300, 16, 16, 25.0, 0.125, 1.0),      # global store with the pct and cap cuts
    (7, 4, 1, 1, 8, 32, 32, 100.0, None, 1.0),            # a single key
    # batches of H * Q >= 512 queries take the 512-thread selection instance
    (8, 4, 160, 2500, 256, 32, 32, 100.0, None, 1.0 / 3.0),
    (9, 2, 300, 3000, 64, 8, 8, 30.0, 0.25, 0.5),         # ties at both cuts
    (10, 1, 512, 36000, 300, 16, 16, 25.0, 0.125, 1.0),   # its global key store
    # no top-pct cut: the register selection (every key equal to the cap cut kept)
    (11, 2, 3, 5000, 64, 8, 8, 100.0, 0.25, 0.5),         # ties at the cap cut
    (12, 2, 300, 3001, 64, 8, 8, 100.0, 0.25, 0.5),       # a batch, ties, rows of odd length
    (13, 1, 2, 16384, 512, 16, 16, 100.0, None, 0.25),    # the longest batch row in registers
    (14, 1, 2, 16385, 512, 16, 16, 100.0, None, 0.25),    # past it: a few queries, 6 groups
    (15, 2, 2, 32768, 2048, 32, 32, 100.0, 0.25, 1.0 / 3.0),   # 8 groups of 1024 threads, ties
    (16, 1, 2, 32769, 2048, 32, 32, 100.0, None, 1.0 / 3.0),   # one key past it (LDS store)
])
def test_decode_select_matches_oracle_on_crafted_scores(case):
    seed, H, Q, M, km, ng, nl, pctd, quant, ps = case
    rng = np.random.default_rng(seed)
    s = (rng.standard_normal((H, Q, M)) * 2.0).astype(np.float32)
    if quant is not None:
        s = (np.round(s / quant) * quant).astype(np.float32)
    tau = rng.uniform(2.0, 8.0, H).astype(np.float32)
    q_pos0 = M - Q
    say(f"decode select crafted: H={H} Q={Q} M={M} k_max={km} pct={pctd} quant={quant}")
    size = _check_crafted(s, tau, q_pos0, ps, ng, nl, km, pctd)
    print(f"[result] crafted select: set sizes {size.ravel()[:6].tolist()}", flush=True)


def test_decode_scores_sets_attend_match_reference():
    import shared_selection_triton_exact_2 as ex2
    g = _load("decode_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, km, pctd, sm = g[p + "params"]
        qp, ng, nl, km = int(qp), int(ng), int(nl), int(km)
        q = torch.from_numpy(g[p + "q"]).to(DEV)
        K = torch.from_numpy(g[p + "k"]).to(DEV)
        V = torch.from_numpy(g[p + "v"]).to(DEV)
        invf = torch.from_numpy(g[p + "inv_freq"])
        H, M = K.shape[0], K.shape[1]
        say(f"decode composed golden case {i}: H={H} M={M} q_pos={qp}")
        s = ex2._decode_scores_kernel(q, K, invf, qp, float(ps), float(rs), float(sm)).cpu().numpy()
        ref = g[p + "scores_triton"]
        assert np.max(np.abs(s - ref)) <= 2e-6 * max(1.0, float(np.abs(ref).max())), i
        taus = torch.full((H,), float(tau))
        idx, npk, npq = ex2._decode_build_sets(q, K, taus, invf, qp, float(ps), float(rs), float(sm), ng, nl, km,
                                               float(pctd))
        # layer 2: the oracle's selection on the GPU's own scores
        oi, on, oq, _ = orc.decode_build_sets(s[:, None, :], taus.numpy(), qp, float(ps), ng, nl, km, float(pctd))
        assert np.array_equal(idx.cpu().numpy(), oi[:, 0].astype(np.int64)), i
        assert _bits_equal(npk.cpu().numpy(), on[:, 0]) and _bits_equal(npq.cpu().numpy(), oq[:, 0]), i
        # no key of these inputs sits within the scores' rounding of a cut: the reference's own sets
        assert np.array_equal(idx.cpu().numpy(), g[p + "idx"]), i
        idx_r = torch.from_numpy(g[p + "idx"])
        npk_r = torch.from_numpy(g[p + "newpos_k"])
        npq_r = torch.from_numpy(g[p + "newpos_q"])
        out_t = ex2._decode_attend_torch(q, K, V, idx_r, npk_r, npq_r, invf, float(rs), float(sm))
        out_c = ex2._decode_attend_kernelC(q, K, V, idx_r, npk_r, npq_r, invf, float(rs), float(sm), km, qp)
        assert out_t.shape == (H, K.shape[2]) and out_t.dtype == q.dtype
        check_output(out_f32(out_t), g[p + "out_torch"], orc.F32, f"attend torch case {i}")
        check_output(out_f32(out_c), g[p + "out_kernelc"], orc.F32, f"attend kernelC case {i}")


def test_decode_batched_matches_per_token_loop():
    import _sta_native as native
    g = _load("decode_sequence_golden.npz")
    P0, Q, ps, rs, tau, ng, nl, km, pctd, sm = g["params"]
    P0, Q, ng, nl, km = int(P0), int(Q), int(ng), int(nl), int(km)
    q = torch.from_numpy(g["q"]).to(DEV)
    k = torch.from_numpy(g["k"]).to(DEV)
    v = torch.from_numpy(g["v"]).to(DEV)
    say(f"decode batched sequence: Q={Q} positions {P0}..{P0 + Q - 1}")
    r = native.decode_attention(q, k, v, torch.full((q.shape[0],), float(tau)), torch.from_numpy(g["inv_freq"]),
                                P0, float(ps), float(rs), float(sm), ng, nl, km, float(pctd))
    torch.cuda.synchronize()
    assert np.array_equal(r["idx"].cpu().numpy().astype(np.int64), g["idx"])   # sentinel P + 1 per query
    assert _bits_equal(r["newpos_k"].cpu().numpy(), g["newpos_k"])
    assert _bits_equal(r["newpos_q"].cpu().numpy(), g["newpos_q"])
    check_output(out_f32(r["out"]), g["out"], orc.F32, "batched decode")


def _check_crafted(s, tau, q_pos0, ps, ng, nl, km, pctd):
    """The selection from given scores against the oracle's, bit for bit; returns the set sizes."""
    plan = _plan_for_scores(s, tau, q_pos0, ps, ng, nl, km, pctd)
    r = plan.build_sets(torch.from_numpy(s).to(DEV))
    torch.cuda.synchronize()
    idx, npk, npq, size = orc.decode_build_sets(s, tau, q_pos0, ps, ng, nl, km, pctd)
    assert np.array_equal(r["idx"].cpu().numpy(), idx)
    assert _bits_equal(r["newpos_k"].cpu().numpy(), npk)
    assert _bits_equal(r["newpos_q"].cpu().numpy(), npq)
    assert np.array_equal(r["set_size"].cpu().numpy(), size)
    return size


@pytest.mark.parametrize("tau", [0.0, float("inf"), -1.0, 1e-3])
def test_decode_select_shared_rule_thresholds(tau):
    """The shared rule without a top-pct cut at thresholds the value bins do not cover (tau = 0, inf:
    key-space bins), at none (tau < 0: only the forced keys pass) and with a narrow band, on rows
    with exact ties, against the oracle bit for bit."""
    rng = np.random.default_rng(21)
    H, Q, M, km = 2, 3, 4000, 128
    s = (rng.standard_normal((H, Q, M)) * 2.0).astype(np.float32)
    s[..., ::7] = np.round(s[..., ::7])
    say(f"decode select shared rule: tau={tau}")
    size = _check_crafted(s, np.full(H, tau, np.float32), M - Q, 0.5, 8, 8, km, 100.0)
    print(f"[result] shared rule tau={tau}: set sizes {size.ravel().tolist()}", flush=True)


@pytest.mark.parametrize("case", [
    # (H, Hkv, Q, M, D, dtype, k_max, pct_decode, causal, pos_scale, rope_scale)
    (4, 2, 1, 3000, 128, torch.bfloat16, 512, 100.0, False, 1.0 / 3.0, 1.0),
    (8, 2, 4, 2500, 64, torch.float16, 200, 30.0, True, 0.5, 1.1386294),
    (2, 2, 3, 1800, 64, torch.float32, 1024, 100.0, False, 1.0, 1.0),
    (4, 4, 2, 39000, 128, torch.bfloat16, 2048, 100.0, False, 1.0 / 3.0, 1.0),   # global key store
    (2, 1, 16, 700, 128, torch.bfloat16, 96, 50.0, True, 0.25, 1.0),
    # batches of 64+ queries take their scores from the matrix cores (fragments + score rows)
    (4, 2, 200, 1500, 128, torch.bfloat16, 256, 100.0, False, 0.5, 1.0),
    (2, 2, 96, 900, 64, torch.float16, 128, 30.0, True, 1.0, 1.1386294),
    # sets of about 20000 keys: more than 256 attend splits per query
    (2, 2, 1, 30000, 64, torch.bfloat16, 24000, 100.0, False, 1.0 / 3.0, 1.0),
])
def test_decode_three_layer(case):
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, Hkv, Q, M, D, dt, km, pctd, causal, ps, rs = case
    say(f"decode three-layer: H={H} Hkv={Hkv} Q={Q} M={M} D={D} {dt} k_max={km} pct={pctd} causal={causal}")
    qa, k, v = planted_inputs(17, H, Hkv, M, D, 0.01, dt, DEV)
    q = qa[0, :, M - Q:, :].contiguous()                 # the last Q positions query the cache
    invf = base_inv_freq(D, 10000.0)
    tau = torch.full((H,), 5.0)
    sm = 1.0 / math.sqrt(D)
    q_pos0 = M - Q
    r = native.decode_attention(q, k, v, tau, invf, q_pos0, ps, rs, sm, 32, 32, km, pctd, causal, want_scores=True)
    torch.cuda.synchronize()
    qn, dc = np_of(q)
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    s_ref = orc.decode_scores(qn, kn, dc, invf.numpy(), ps, rs, sm, q_pos0)
    s_gpu = r["scores"].cpu().numpy()
    valid = ~np.isnan(s_ref)
    # fp32 rotation + dot: a few ulps of |q| |k| (the rotation keeps the norms, times rope_scale^2)
    qmax = np.sqrt((orc.to_f32(qn, dc).astype(np.float64) ** 2).sum(-1)).max()
    kmax = np.sqrt((orc.to_f32(kn, dc).astype(np.float64) ** 2).sum(-1)).max()
    tol = 4e-6 * qmax * kmax * rs * rs * sm + 1e-6
    assert np.max(np.abs(s_gpu[valid] - s_ref[valid])) <= tol
    idx, npk, npq, size = orc.decode_build_sets(s_gpu, tau.numpy(), q_pos0, ps, 32, 32, km, pctd)
    assert np.array_equal(r["idx"].cpu().numpy(), idx)
    assert _bits_equal(r["newpos_k"].cpu().numpy(), npk) and _bits_equal(r["newpos_q"].cpu().numpy(), npq)
    assert np.array_equal(r["set_size"].cpu().numpy(), size)
    out_ref = orc.decode_attend(qn, kn, vn, dc, invf.numpy(), rs, sm, q_pos0, idx, npk, npq, causal=causal)
    e = check_output(out_f32(r["out"]), out_ref, dc, "decode three-layer")
    print(f"[result] decode three-layer: set sizes {size.ravel()[:8].tolist()}, max out err {e:.2e}", flush=True)


def test_decode_rejects_bad_arguments():
    import _sta_native as native
    q = torch.zeros((2, 3, 64), device=DEV)
    k = torch.zeros((2, 10, 64), device=DEV)
    with pytest.raises(RuntimeError, match="q_pos0"):
        native.decode_attention(q, k, k, torch.ones(2), torch.ones(32), 8, k_max=4)   # 8 + 3 > 10
    with pytest.raises(RuntimeError, match="head_dim"):
        native.decode_attention(torch.zeros((2, 1, 96), device=DEV), torch.zeros((2, 10, 96), device=DEV),
                                torch.zeros((2, 10, 96), device=DEV), torch.ones(2), torch.ones(48), 9, k_max=4)
    with pytest.raises(RuntimeError, match="CPU"):
        native.decode_attention(q.cpu(), k, k, torch.ones(2), torch.ones(32), 7, k_max=4)


def test_decode_hybrid_two_geometries():
    """Selection under YaRN (a-triple), reposition with PI pos_scale_c, attend under base RoPE:
    the hybrid file's decode (hybrid_exact.py:551-629, 776-800), through its drop-in helpers."""
    import _sta_native as native
    import shared_selection_triton_hybrid_exact as hyb
    from synthetic import base_inv_freq, planted_inputs, yarn_inv_freq
    H, M, D = 4, 2600, 128
    qa, k, v = planted_inputs(23, H, H, M, D, 0.01, torch.bfloat16, DEV)
    q = qa[0, :, M - 1, :].contiguous()                 # (H, D): the newest position
    invf_a, msc = yarn_inv_freq(D, 500000.0, 4.0, 8192, 32.0, 1.0)
    invf_c = base_inv_freq(D, 10000.0)
    ps_c, sm = 1.0 / 3.0, 1.0 / math.sqrt(D)
    tau = torch.full((H,), 5.0)
    say("decode hybrid: YaRN selection, PI reposition, base-RoPE attend")
    idx, npk, npq = hyb._decode_build_sets(q, k[0], tau, invf_a, M - 1, 1.0, msc, sm, 32, 32, 300, 100.0, ps_c)
    out = hyb._decode_attend_torch(q, k[0], v[0], idx, npk, npq, invf_c, 1.0, sm)
    r = native.decode_attention(q, k, v, tau, invf_a, M - 1, 1.0, msc, sm, 32, 32, 300, 100.0, want_scores=True,
                                inv_freq_c=invf_c, pos_scale_c=ps_c, rope_scale_c=1.0)
    torch.cuda.synchronize()
    assert torch.equal(idx.to(torch.int32), r["idx"][:, 0]) and torch.equal(out, r["out"][:, 0])
    qn, dc = np_of(q[:, None, :])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    s_gpu = r["scores"].cpu().numpy()
    s_ref = orc.decode_scores(qn, kn, dc, invf_a.numpy(), 1.0, msc, sm, M - 1)
    assert np.max(np.abs(s_gpu - s_ref)) < 1e-4
    oi, on, oq, _ = orc.decode_build_sets(s_gpu, tau.numpy(), M - 1, ps_c, 32, 32, 300)
    assert np.array_equal(r["idx"].cpu().numpy(), oi)
    assert _bits_equal(r["newpos_k"].cpu().numpy(), on) and _bits_equal(r["newpos_q"].cpu().numpy(), oq)
    ref = orc.decode_attend(qn, kn, vn, dc, invf_c.numpy(), 1.0, sm, M - 1, oi, on, oq)
    check_output(out_f32(r["out"]), ref, dc, "decode hybrid")


@pytest.mark.parametrize("case", [
    # (rule, H, Hkv, Q, M, D, dtype, k_max, pct_decode, causal): the selection kernel each reaches
    ("pq", 2, 1, 200, 1500, 128, torch.bfloat16, 256, 100.0, False),     # the row in registers
    ("pq", 2, 2, 70, 20000, 64, torch.bfloat16, 2048, 100.0, False),     # the row in LDS
    ("shared", 2, 2, 96, 900, 64, torch.float16, 128, 30.0, True),       # the general selection
    ("pq", 2, 1, 65, 39000, 64, torch.bfloat16, 1024, 100.0, False),     # the global key store
    ("pq", 4, 2, 100, 3000, 128, torch.float32, 512, 100.0, False),      # fp32 fragments
    ("shared", 2, 1, 80, 2000, 64, torch.bfloat16, 256, 100.0, False),   # the shared rule in registers
    ("stream", 2, 2, 70, 1500, 64, torch.bfloat16, 4096, 100.0, False),  # PQ Stream positions
])
def test_decode_tiled_scores_match_row_major(case):
    """A batch's scores that only the selection of the same call reads leave the score rows kernel
    in 64 x 32 tiles; a call that also returns them writes (H, Q, M) rows.  Both calls give the
    same sets and outputs bit for bit (Q not a multiple of 64, M not a multiple of 32), and every
    selection kernel reads both layouts."""
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    rule, H, Hkv, Q, M, D, dt, km, pctd, causal = case
    say(f"tiled vs row-major scores: {rule} H={H} Hkv={Hkv} Q={Q} M={M} D={D} {dt} k_max={km}")
    qa, k, v = planted_inputs(29, H, Hkv, M, D, 0.01, dt, DEV)
    q = qa[0, :, M - Q:, :].contiguous()
    invf = base_inv_freq(D, 10000.0)
    tau = torch.full((H,), 4.0)
    kw = {"pq": dict(inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0, rule="pq"),
          "stream": dict(inv_freq_c=invf, pos_scale_c=1.0, rope_scale_c=1.0, rule="stream", block_n=32),
          "shared": {}}[rule]
    runs = [native.decode_attention(q, k, v, tau, invf, M - Q, 0.5, 1.0, None, 16, 16, km, pctd, causal,
                                    want_scores=ws, **kw) for ws in (False, True)]
    torch.cuda.synchronize()
    tiled, rows = runs
    names = ["out", "idx", "newpos_q", "set_size"] + (["usize", "overflow"] if rule == "pq" else ["newpos_k"])
    for name in names:
        assert torch.equal(tiled[name], rows[name]), name
    assert int((tiled["set_size"] > 0).sum()) == H * Q
