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
