"""GPU: pass 2 with one bf16 product plus an fp6 correction (csrc/sta_score6.hip, sta_fp6.h).

For 16-bit inputs with plain votes, the shared path scores pass 2 as hi.hi in bf16 plus the
correction Q6(q_hi).Q6(k - k_hi) + Q6(q - q_hi).Q6(k_hi) in block-scaled e2m3.  Its error is
statistical (~1e-4 on unit-scale scores), so the set contract's band rule applies: every vote
entry may differ from the oracle's exact votes only by the rows whose score lies within 1e-3 of
max - tau (the oracle's band counts).  STA_EXACT_PASS2=1 runs the three-product pass 2 for
comparison.  Heads whose estimated error exceeds a quarter of the band must take the
three-product kernel: their votes equal it bit for bit.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc
from parity_helpers import BAND, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _run(q, k, v, tau, invf, ps, tile, exact2, q_pos_base=0):
    import _sta_native as native
    old = os.environ.get("STA_EXACT_PASS2")
    os.environ["STA_EXACT_PASS2"] = "1" if exact2 else "0"
    try:
        r = native.shared_attention(q, k, v, tau, invf, ps, 1.0, invf, ps, 1.0, pct=30.0,
                                    sm_scale=1.0 / math.sqrt(q.shape[-1]), tile=tile, k_max=512,
                                    q_pos_base=q_pos_base, want_votes=True, want_row_max=True)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("STA_EXACT_PASS2")
        else:
            os.environ["STA_EXACT_PASS2"] = old
    return r


def _case(H, N, D, tile, dtype, seed, scale_heads=(), scale=1.0, q_pos_base=0):
    from synthetic import base_inv_freq, planted_inputs
    print(f"[case] fp6 pass 2: H={H} N={N} D={D} tile={tile} {dtype} q_pos_base={q_pos_base} "
          f"heads scaled x{scale}: {list(scale_heads)}", flush=True)
    q, k, v = planted_inputs(seed, H, H, N, D, 0.01, dtype, DEV)
    for h in scale_heads:
        q[0, h] = (q[0, h].float() * scale).to(dtype)
        k[0, h] = (k[0, h].float() * scale).to(dtype)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 5.0)
    r6 = _run(q, k, v, tau, invf, 0.5, tile, False, q_pos_base)
    rx = _run(q, k, v, tau, invf, 0.5, tile, True, q_pos_base)
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    a = orc.select_vote(qn, kn, dt, tau.numpy(), invf.cpu().numpy(), 0.5, 1.0, 1.0 / math.sqrt(D), tile,
                        q_pos_base, band_eps=BAND, want_band=True)
    v6 = r6["votes"].cpu().numpy().astype(np.int64)
    vx = rx["votes"].cpu().numpy().astype(np.int64)
    vo = a["votes"].astype(np.int64)
    band = a["band"]
    for name, vv in (("fp6", v6), ("three-product", vx)):
        bad = np.abs(vv - vo) > band
        assert not bad.any(), f"{name} pass 2: {int(bad.sum())} vote entries differ beyond the band"
    assert torch.equal(r6["row_max"], rx["row_max"]), "row maxima come from the same screen"
    return v6, vx, band


def test_fast6_votes_within_band_unit_scale():
    v6, vx, band = _case(4, 2048, 128, 64, torch.bfloat16, 11)
    nd = int((v6 != vx).sum())
    print(f"[result] fp6 vs three-product: {nd} vote entries differ (all within the band; "
          f"band pairs {int(band.sum())})", flush=True)
    # about 1e-4 of error moves a few hundred near-threshold pairs at this size: the fp6 kernel ran
    assert nd > 0


@pytest.mark.parametrize("H,N,D,tile,dtype,qpb", [
    (2, 2000, 128, 32, torch.bfloat16, 0),      # ragged, tile 32 (two tiles per wave)
    (4, 1500, 64, 64, torch.float16, 0),        # D 64, fp16
    (2, 1800, 128, 64, torch.bfloat16, 100),    # q_pos_base > 0
])
def test_fast6_shapes_within_band(H, N, D, tile, dtype, qpb):
    v6, vx, _ = _case(H, N, D, tile, dtype, 12, q_pos_base=qpb)
    print(f"[result] {int((v6 != vx).sum())} vote entries differ from the three-product pass 2", flush=True)


def test_fast6_guard_keeps_large_norm_heads_exact():
    # head 1's rows scaled x4: its scores grow 16x, the fp6 error estimate far past the limit
    v6, vx, _ = _case(3, 2048, 128, 64, torch.bfloat16, 13, scale_heads=(1,), scale=4.0)
    assert np.array_equal(v6[1], vx[1]), "a guarded head must take the three-product pass 2"
    nd = int((v6[[0, 2]] != vx[[0, 2]]).sum())
    print(f"[result] guarded head identical; unit-scale heads differ in {nd} entries", flush=True)


# ------------------------------------------------------------------------------------------
# the RoPE pre-kernel's fp6 operands, bit for bit
# ------------------------------------------------------------------------------------------
def _a256(x):
    return (x + 255) // 256 * 256


def _region(heads, rows_pad, D):
    """Byte offsets of the fp6 planes / scales / error norms and the region's size
    (csrc/sta_kernels.h: frag_region_bytes with the fp6 operands)."""
    base = heads * rows_pad * D * 4 + heads * rows_pad * 8 + heads * 8 + heads * rows_pad * 4 + \
        heads * (rows_pad // 256 + 1) * 4
    planes = _a256(base)
    scales = planes + _a256(heads * rows_pad * D * 3 // 2)
    dnorms = scales + heads * rows_pad * 8
    return planes, scales, dnorms, dnorms + heads * rows_pad * 8 + heads * 8


def _bf16_rne(x):
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def _check_fp6_region(ws, off, x, rows_pad, what):
    import fp6_ref as F
    H, N, D = x.shape
    NU, NB, RBS = D // 32, D // 16, rows_pad // 32
    xp = np.zeros((H, rows_pad, D), np.float32)
    xp[:, :N] = x
    hi = _bf16_rne(xp)
    r = xp - hi                                    # exact in fp32
    vec = np.concatenate([hi, r], axis=2).reshape(H, rows_pad, NB, 32)
    e = F.block_exp(np.abs(vec).max(axis=3))
    code, val = F.encode(vec, e[..., None])
    planes, scales, dnorms, _ = _region(H, rows_pad, D)
    w = ws[off + planes: off + planes + H * rows_pad * D * 3 // 2].view(np.uint64).reshape(H, RBS, NU, 3, 64)
    got = np.zeros((H, RBS, NU, 64, 32), np.int64)
    for p in range(32):
        bit = 6 * p
        j, o = bit // 64, bit % 64
        f = (w[:, :, :, j, :] >> np.uint64(o)) & np.uint64(63)
        if o > 58:
            f |= (w[:, :, :, j + 1, :] << np.uint64(64 - o)) & np.uint64(63)
        got[..., p] = f.astype(np.int64)
    # unit m, lane lr + 32 g holds block 2m + g of row 32 rb + lr
    got = got.reshape(H, RBS, NU, 2, 32, 32).transpose(0, 1, 4, 2, 3, 5).reshape(H, rows_pad, NB, 32)
    bad = got != code
    assert not bad.any(), f"{what}: {int(bad.sum())} fp6 codes differ, first at {np.argwhere(bad)[0]}"
    sc = ws[off + scales: off + scales + H * RBS * 256].reshape(H, RBS, 2, 32, 4)[..., :NU]   # lane = 32 g + lr
    sc = sc.transpose(0, 1, 3, 4, 2).reshape(H, rows_pad, NB)                                # byte m, g -> block 2m + g
    assert np.array_equal(sc.astype(np.int64), e + 127), f"{what}: scales differ"
    dn = ws[off + dnorms: off + dnorms + H * rows_pad * 8].view(np.float32).reshape(H, rows_pad, 2)
    d2 = ((val - vec.astype(np.float64)) ** 2).reshape(H, rows_pad, 2, NB // 2 * 32).sum(axis=3)
    assert np.allclose(dn, np.sqrt(d2), rtol=1e-5, atol=1e-30), f"{what}: error norms differ"


@pytest.mark.parametrize("D", [128, 64])
def test_fp6_operands_bit_exact(D):
    """pos_scale 0 and rope_scale 1 + 2^-10: the rotation is the exact fp32 scaling x * rs (a
    bf16 times an 11-bit constant), so the rows, their bf16 hi parts and residuals are known on
    the CPU; some rows are scaled by 2^20 / 2^-20 or zeroed to reach the scale range's ends."""
    import _sta_native as native
    H, N, tile, kmax = 2, 300, 64, 64
    print(f"[case] fp6 operands of the RoPE pre-kernel: H={H} N={N} D={D}", flush=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 1, H, N, D, generator=g)
    x[:, :, :, 7] *= 2.0 ** 20
    x[:, :, :, 8] *= 2.0 ** -20
    x[:, :, :, 9] = 0
    q, k, v = (t.to(torch.bfloat16).to(DEV) for t in x)
    rs = 1.0 + 2.0 ** -10
    invf = torch.ones(D // 2, device=DEV)
    plan = native.SharedPlan(q, k, v, torch.full((H,), 5.0), invf, 0.0, rs, invf, 0.0, rs, tile=tile, k_max=kmax)
    plan.run()
    torch.cuda.synchronize()
    ws = plan.workspace.cpu().numpy()
    q_rows_pad = (N + tile - 1) // tile * tile
    k_rows_pad = (max(q_rows_pad, N) + 127) // 128 * 128
    qx = (q[0].float().cpu().numpy() * np.float32(rs)).astype(np.float32)
    kx = (k[0].float().cpu().numpy() * np.float32(rs)).astype(np.float32)
    _check_fp6_region(ws, 0, qx, q_rows_pad, "q")
    _check_fp6_region(ws, _a256(_region(H, q_rows_pad, D)[3]), kx, k_rows_pad, "k")
    print("[result] fp6 codes, scales and error norms equal the reference encoding", flush=True)
