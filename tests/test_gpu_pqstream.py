"""GPU parity of PQ Stream through the C ABI.

Layers:
  1. keep bits: the GPU's threshold bits (the same score kernel, read out through
     sta_pq_select_bits) differ from the oracle's only in rows whose score lies within BAND of the
     row's threshold;
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
    r = native.pqstream_attention(q, k, v, tau, ia, ic, psa, rsa, sm, ng, nl, 32, bn, adv, 0, skip)
    b = native.pq_select_bits(q, k, tau, ia, psa, rsa, sm, 32, 0, "freq")
    torch.cuda.synchronize()
    bits_g = b["bits"].cpu().numpy()
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
