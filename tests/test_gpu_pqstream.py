"""GPU parity of PQ Stream through the C ABI.

Layers:
  1. keep bits: the threshold bits the sweep applied (computed inside the fused sweep, read out
     through sta_pqstream_args.bits) equal the score kernel's pass 2 (sta_pq_select_bits) bit for
     bit, and differ from the oracle's only in rows whose score lies within BAND of the row's
     threshold;
  2. given the GPU's bits, the oracle's restatement of the fused kernel reproduces span, kept,
     blocks and skipped exactly, and the output within 1e-4 (fp32) or 2e-2 abs + 1e-2 rel
     (bf16 / fp16).
The reference's own fixtures (its fused kernel under the Triton interpreter, fp32) are compared
end to end.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, check_output, np_of, out_f32

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


def check_bits(bits_g, bits_o, band):
    x = (bits_g.view(np.uint32) ^ bits_o.view(np.uint32)).astype(np.uint64)
    pc = np.zeros(x.shape, np.int64)
    for r in range(32):
        pc += ((x >> np.uint64(r)) & np.uint64(1)).astype(np.int64)
    bad = pc > band
    assert not bad.any(), f"{int(bad.sum())} keys differ in more rows than the band allows"
    return int((pc > 0).sum())


def stream_check(q, k, v, tau, ia, psa, rsa, ic, ng=32, nl=32, bn=32, adv="max", skip=True, what="",
                 band_check=True):
    import _sta_native as native
    H, N, D = q.shape[1], q.shape[2], q.shape[3]
    sm = 1.0 / math.sqrt(D)
    say(f"{what}: H={H} Hkv={k.shape[1]} N={N} D={D} block_n={bn} advance={adv} skip={skip} {q.dtype}")
    r = native.pqstream_attention(q, k, v, tau, ia, ic, psa, rsa, sm, ng, nl, 32, bn, adv, 0, skip, want_bits=True,
                                  fused="fused")
    ru = native.pqstream_attention(q, k, v, tau, ia, ic, psa, rsa, sm, ng, nl, 32, bn, adv, 0, skip, want_bits=True,
                                   fused="unfused")
    b = native.pq_select_bits(q, k, tau, ia, psa, rsa, sm, 32, 0, "freq")
    torch.cuda.synchronize()
    # the fused sweep's own keep bits equal the score kernel's pass 2, and the two sweeps agree
    # bit for bit
    bits_g = r["bits"].cpu().numpy()
    assert np.array_equal(bits_g, b["bits"].cpu().numpy()), f"{what}: the fused sweep's keep bits differ from pass 2's"
    assert np.array_equal(ru["bits"].cpu().numpy(), bits_g), f"{what}: the unfused sweep read other bits"
    for name in ("out", "span", "kept", "blocks", "skipped"):
        assert torch.equal(r[name], ru[name]), f"{what}: fused and unfused sweeps differ in {name}"
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    ndiff = -1
    if band_check:
        a = orc.select_bits(qn, kn, dt, tau.cpu().numpy(), ia.cpu().numpy(), psa, rsa, sm, 32, 0, 0,
                            band_eps=BAND, want_band=True)
        ndiff = check_bits(bits_g, a["bits"], a["band"])
    o = orc.pqstream(qn, kn, vn, dt, tau.cpu().numpy(), ia.cpu().numpy(), ic.cpu().numpy(), psa, rsa, sm,
                     ng, nl, 32, bn, adv, skip, bits_in=bits_g, want_band=False)
    for name, ref in zip(("span", "kept", "blocks", "skipped"), o[1:5]):
        got = r[name].cpu().numpy()
        assert np.array_equal(got, ref), f"{what}: {name} differs at {np.argwhere(got != ref)[:4].tolist()}"
    err = check_output(out_f32(r["out"]), o[0], dt, what)
    print(f"[result] {what}: keys with flipped bits {ndiff}, max out err {err:.2e}, span max "
          f"{float(o[1].max()):.0f}, skipped {int(o[4].sum())}/{int(o[3].sum())}", flush=True)
    return r


def test_pqstream_goldens():
    g = np.load(os.path.join(GOLD, "pqstream_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, bn, full, skip = g[p + "params"]
        q, k, v = (torch.from_numpy(g[p + n]).to(DEV)[None] for n in ("q", "k", "v"))
        tau = torch.from_numpy(g[p + "tau"]).to(DEV)
        ia, ic = torch.from_numpy(g[p + "inv_freq_a"]).to(DEV), torch.from_numpy(g[p + "inv_freq_c"]).to(DEV)
        r = stream_check(q, k, v, tau, ia, float(psa), float(rsa), ic, int(ng), int(nl), int(bn),
                         "full" if full else "max", bool(skip), what=f"pqstream golden {i}")
        for name in ("span", "kept", "blocks", "skipped"):
            assert np.array_equal(r[name].cpu().numpy(), g[p + name]), (i, name)
        np.testing.assert_allclose(r["out"].cpu().numpy(), g[p + "out"], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("bn,adv,skip", [(32, "max", True), (64, "max", True), (32, "full", True),
                                         (32, "max", False)])
def test_pqstream_bf16(bn, adv, skip):
    from synthetic import planted_inputs, base_inv_freq
    H, N, D = 2, 1000, 128
    q, k, v = planted_inputs(41, H, H, N, D, 0.02, torch.bfloat16, DEV)
    tau = torch.full((H,), 1.0 if not skip else 3.0, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    stream_check(q, k, v, tau, invf, 0.25, 1.0, invf, 4 if not skip else 32, 8 if not skip else 32, bn, adv,
                 skip, what=f"pqstream bf16 bn={bn} {adv} skip={skip}")


def test_pqstream_fp16_gqa_two_geometries():
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, N, D = 4, 2, 777, 64
    q, k, v = planted_inputs(42, H, Hkv, N, D, 0.02, torch.float16, DEV)
    tau = torch.full((H,), 2.5, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    stream_check(q, k, v, tau, invf * 0.5, 1.0, 1.1386294, invf, 8, 16, 64, "max", True,
                 what="pqstream fp16 gqa two geometries")


def test_pqstream_dropin_and_errors():
    import pqstream_kernel as pqs
    from synthetic import planted_inputs, base_inv_freq
    H, N, D = 2, 300, 64
    q, k, v = planted_inputs(43, H, H, N, D, 0.02, torch.bfloat16, DEV)
    tau = torch.full((H,), 3.0, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    say("pqstream drop-in module")
    pqs.reset_span_stats()
    out, span, kept, blocks, skipped = pqs.pqstream_attention(q, k, v, tau, invf, invf, pos_scale_a=0.5)
    assert out.shape == (1, H, N, D) and out.dtype == torch.bfloat16
    assert span.dtype == torch.float32 and kept.dtype == torch.int32 and kept.shape == (H, N)
    st = pqs.get_overflow_stats()["prefill"]
    assert st["total_cells"] == H * ((N + 31) // 32) and st["overflow_cells"] == 0
    for bad in (dict(tile=64), dict(q_pos_base=4), dict(block_n=16)):
        with pytest.raises(AssertionError):
            pqs.pqstream_attention(q, k, v, tau, invf, invf, **bad)


def test_pqstream_config3_shape_one_head():
    """Config 3's shape (N=16384, d128, bf16, tau 4, PI 1/4 selection, base RoPE attend), one head."""
    from synthetic import CONFIGS
    cfg = CONFIGS["c3"]
    q, k, v = cfg.inputs(DEV)
    q, k, v = q[:, :1].contiguous(), k[:, :1].contiguous(), v[:, :1].contiguous()
    invf, ps, rs = cfg.geometry()
    invf = invf.to(DEV)
    tau = torch.full((1,), cfg.tau, device=DEV)
    stream_check(q, k, v, tau, invf, ps, rs, invf, cfg.n_global, cfg.n_local, 32, "max", True,
                 what="pqstream config 3 shape, 1 head", band_check=True)


# ---------------------------------------------------------------------------------------------
# decode: the stream rule per query (_decode_build_sets_pqs, pqstream_kernel.py:695-797)
# ---------------------------------------------------------------------------------------------
def _gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _kbuf(M):
    return max(1024, -(-M // 1024) * 1024)


def classify_stream_rows(idx_g, idx_o, s_o, tau, Q, M):
    """Queries whose sets differ from the oracle's own: every key in one set only must score within
    BAND of its query's threshold m - tau (the stream rule has no cap).  Returns (rows, keys)."""
    H = idx_g.shape[0]
    rows = keys = 0
    for h in range(H):
        for i in range(Q):
            m = M - (Q - 1 - i)
            a = set(idx_g[h, i][idx_g[h, i] < m].tolist())
            b = set(idx_o[h, i][idx_o[h, i] < m].tolist())
            if a == b:
                continue
            rows += 1
            row = s_o[h, i, :m]
            thr = np.float32(row.max() - np.float32(tau[h]))
            for j in a ^ b:
                keys += 1
                assert abs(float(row[j]) - float(thr)) <= BAND, \
                    f"head {h} query {i} key {j}: score {row[j]} not within {BAND} of the threshold {thr}"
    return rows, keys


def _check_stream_decode(q, k, v, tau, invf_a, ps, rs, invf_c, q_pos0, ng, nl, bn, what, causal=False):
    """Scores, stream sets and attend of Q queries (H, Q, D) at q_pos0.. over the cache (Hkv, M, D)."""
    import _sta_native as native
    H, Q, D = q.shape
    M = k.shape[1]
    sm = 1.0 / math.sqrt(D)
    k_max = _kbuf(M)
    say(f"{what}: H={H} Hkv={k.shape[0]} Q={Q} M={M} D={D} block_n={bn} k_max={k_max} {q.dtype}")
    r = native.decode_attention(q, k, v, tau, invf_a, q_pos0, ps, rs, sm, ng, nl, k_max, 100.0, causal,
                                want_scores=True, inv_freq_c=invf_c, pos_scale_c=1.0, rope_scale_c=1.0,
                                rule="stream", block_n=bn)
    torch.cuda.synchronize()
    qn, dt = np_of(q)
    kn, _ = np_of(k)
    vn, _ = np_of(v)
    tau_n = tau.cpu().numpy()
    s_g = r["scores"].cpu().numpy()
    s_o = orc.decode_scores(qn, kn, dt, invf_a.cpu().numpy(), ps, rs, sm, q_pos0)
    valid = ~np.isnan(s_o)
    err = float(np.max(np.abs(s_g[valid] - s_o[valid])))
    assert err < 1e-4, f"{what}: scores differ from the oracle's by {err:.3e}"
    # 2. sets given the GPU's scores: bit for bit, -0 of the query's own slot included
    ref = orc.decode_build_sets_pqs(np.where(valid, s_g, np.float32(0)), tau_n, q_pos0, ng, nl, bn, k_max=k_max)
    got = {n: r[n].cpu().numpy() for n in ("idx", "newpos_k", "newpos_q", "set_size")}
    assert np.array_equal(got["idx"], ref[0]), f"{what}: idx differs from the oracle given the GPU's scores"
    assert np.array_equal(got["newpos_k"].view(np.uint32), ref[1].view(np.uint32)), f"{what}: newpos_k differs"
    assert np.array_equal(got["newpos_q"].view(np.uint32), ref[2].view(np.uint32)), f"{what}: newpos_q differs"
    assert np.array_equal(got["set_size"], ref[3]), f"{what}: set_size differs"
    # 3. sets against the oracle's own
    own = orc.decode_build_sets_pqs(np.where(valid, s_o, np.float32(0)), tau_n, q_pos0, ng, nl, bn, k_max=k_max)
    rows, keys = classify_stream_rows(got["idx"], own[0], s_o, tau_n, Q, M)
    print(f"[sets] {what}: {rows} of {H * Q} queries' sets differ from the oracle's; {keys} keys, all within "
          f"{BAND} of the threshold", flush=True)
    # 4. the attend given the GPU's sets
    out_ref = orc.decode_attend(qn, kn, vn, dt, invf_c.cpu().numpy(), 1.0, sm, q_pos0, got["idx"],
                                got["newpos_k"], got["newpos_q"], causal=causal)
    e = check_output(r["out"].float().cpu().numpy(), out_ref, dt, what)
    print(f"[result] {what}: score err {err:.2e}, set size mean {got['set_size'].mean():.1f}, span max "
          f"{float(ref[4].max()):.0f}, max out err {e:.2e}", flush=True)
    return r, got, ref


def test_pqs_decode_sets_match_reference_goldens():
    """Selection alone from the reference's crafted score rows: bit for bit, sentinel and -0 included."""
    import _sta_native as native
    g = _gold("decode_pqs_sets_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ng, nl, bn = (int(x) for x in g[p + "params"])
        s = g[p + "scores"]
        H, M = s.shape
        km = g[p + "idx"].shape[-1]
        say(f"stream decode sets golden {i}: M={M} block_n={bn}")
        plan = native.DecodePlan(torch.zeros(H, 1, 64, device=DEV), torch.zeros(H, M, 64, device=DEV), None,
                                 torch.from_numpy(g[p + "tau"]), torch.ones(32), qp, k_max=km, n_global=ng,
                                 n_local=nl, rule="stream", block_n=bn)
        r = plan.build_sets(torch.from_numpy(s).to(DEV).reshape(H, 1, M))
        idx = r["idx"].cpu().numpy()[:, 0]
        assert np.array_equal(idx.astype(np.int64), g[p + "idx"]), i
        assert np.array_equal(r["newpos_k"].cpu().numpy()[:, 0].view(np.uint32),
                              g[p + "newpos_k"].view(np.uint32)), i
        assert np.array_equal(r["newpos_q"].cpu().numpy()[:, 0], g[p + "newpos_q"]), i
        assert np.array_equal(r["set_size"].cpu().numpy()[:, 0], (g[p + "idx"] < M).sum(-1)), i


def test_pqs_decode_composed_reference_goldens():
    import pqstream_kernel as pqs
    g = _gold("decode_pqs_composed_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        qp, ps, rs, tau, ng, nl, bn, sm = g[p + "params"]
        qp, ng, nl, bn = int(qp), int(ng), int(nl), int(bn)
        q, K, V = (torch.from_numpy(g[p + n]).to(DEV) for n in ("q", "k", "v"))
        invf = torch.from_numpy(g[p + "inv_freq"]).to(DEV)
        H = q.shape[0]
        taus = torch.full((H,), float(tau), device=DEV)
        r, got, _ = _check_stream_decode(q[:, None, :], K, V, taus, invf, float(ps), float(rs), invf, qp, ng, nl,
                                         bn, f"stream decode composed golden {i}")
        # the drop-in's one-query helpers against the reference's outputs
        say(f"stream decode drop-ins, golden {i}")
        pqs.reset_overflow_stats()
        idx, npk, npq = pqs._decode_build_sets_pqs(q, K, taus, invf, qp, float(ps), float(rs), float(sm), ng, nl,
                                                   bn)
        st = pqs.get_overflow_stats()["decode"]
        assert st["total_cells"] == H and st["overflow_cells"] == 0
        assert idx.shape == g[p + "idx"].shape and npq.shape == (H,)
        if np.array_equal(idx.cpu().numpy(), g[p + "idx"]):
            assert np.array_equal(npk.cpu().numpy(), g[p + "newpos_k"])
            out_t = pqs._decode_attend_torch(q, K, V, idx, npk, npq, invf, float(sm))
            out_c = pqs._decode_attend_triton(q, K, V, idx, npk, npq, invf, float(sm), q_pos=qp)
            np.testing.assert_allclose(out_t.cpu().numpy(), g[p + "out_torch"], atol=1e-4, rtol=1e-4)
            np.testing.assert_allclose(out_c.cpu().numpy(), g[p + "out_triton"], atol=1e-4, rtol=1e-4)
        else:
            print(f"[sets] golden {i}: the GPU's set differs from the reference's (threshold band)", flush=True)


def test_pqs_perquery_prefill_matches_reference_loop():
    """prefill_mode="perquery" at every position of a 260-token prompt (fp32) against the
    reference's per-token loop."""
    g = _gold("prefill_pqs_perquery_golden.npz")
    ps, rs, tau, ng, nl, bn, sm = g["params"]
    ng, nl, bn = int(ng), int(nl), int(bn)
    q, k, v = (torch.from_numpy(g[n]).to(DEV) for n in ("q", "k", "v"))
    H, N, D = q.shape
    invf = torch.from_numpy(g["inv_freq"]).to(DEV)
    taus = torch.full((H,), float(tau), device=DEV)
    r, got, _ = _check_stream_decode(q, k, v, taus, invf, float(ps), float(rs), invf, 0, ng, nl, bn,
                                     "stream per-query prefill golden")
    same = got["set_size"] == g["set_size"]
    assert same.mean() > 0.99
    np.testing.assert_allclose(r["out"].cpu().numpy()[same], g["out"][same], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dt,Q,bn", [(torch.bfloat16, 1, 32), (torch.bfloat16, 96, 32), (torch.float16, 80, 64)])
def test_pqs_decode_gqa(dt, Q, bn):
    """Grouped-query decode at a few thousand keys, one query and batches served by the rows score
    kernel (Q >= 64), selection under a PI geometry, attend under base RoPE."""
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, M, D = 8, 2, 3000, 128
    q, k, v = planted_inputs(51 + Q, H, Hkv, M, D, 0.02, dt, DEV)
    qq = q[0, :, M - Q:, :].contiguous()
    invf = base_inv_freq(D, 10000.0).to(DEV)
    taus = torch.linspace(1.5, 4.0, H, device=DEV)
    _check_stream_decode(qq, k[0], v[0], taus, invf, 0.25, 1.0, invf, M - Q, 16, 16, bn,
                         f"stream decode {dt} Q={Q} block_n={bn}")


def test_pqs_decode_every_key_kept_is_natural():
    """tau = inf keeps every key, and then key j streams to -(q_pos - j): the attend is dense causal
    attention under base RoPE at natural relative positions."""
    from synthetic import planted_inputs, base_inv_freq
    H, M, D, Q = 2, 1500, 64, 70
    q, k, v = planted_inputs(57, H, H, M, D, 0.02, torch.float32, DEV)
    qq = q[0, :, M - Q:, :].contiguous()
    invf = base_inv_freq(D, 10000.0).to(DEV)
    r, got, _ = _check_stream_decode(qq, k[0], v[0], torch.full((H,), math.inf, device=DEV), invf, 0.5, 1.0, invf,
                                     M - Q, 4, 4, 32, "stream decode tau=inf")
    for i in (0, Q - 1):
        m, p = M - Q + i + 1, M - Q + i
        assert np.array_equal(got["idx"][:, i, :m], np.broadcast_to(np.arange(m), (H, m)))
        assert np.array_equal(got["newpos_k"][:, i, :m], np.broadcast_to(-(p - np.arange(m)).astype(np.float32),
                                                                         (H, m)))


@pytest.mark.parametrize("M,bn,Q", [(20000, 8, 2), (16000, 4, 1), (33000, 9, 2)])
def test_pqs_decode_many_position_blocks(M, bn, Q):
    """More position blocks than the selection's histogram has words (2500 and 4000): the block-end
    counts have an LDS region of their own; at M = 33000 the keys, histogram and 3667 block counts
    outgrow the LDS and the selection takes the global key store."""
    from synthetic import planted_inputs, base_inv_freq
    H, D = 2, 64
    q, k, v = planted_inputs(61 + bn, H, H, M, D, 0.02, torch.bfloat16, DEV)
    qq = q[0, :, M - Q:, :].contiguous()
    invf = base_inv_freq(D, 10000.0).to(DEV)
    _check_stream_decode(qq, k[0], v[0], torch.full((H,), 3.0, device=DEV), invf, 0.5, 1.0, invf, M - Q, 16, 16,
                         bn, f"stream decode M={M} block_n={bn} ({(M + bn - 1) // bn} blocks)")


def test_pqs_decode_rejects_bad_block_n():
    import _sta_native as native
    q = torch.zeros(2, 1, 64, device=DEV)
    k = torch.zeros(2, 200, 64, device=DEV)
    for bn in (0, -3):
        with pytest.raises(RuntimeError):
            native.DecodePlan(q, k, None, torch.ones(2), torch.ones(32), 199, k_max=1024, rule="stream",
                              block_n=bn).build_sets(torch.zeros(2, 1, 200, device=DEV))
