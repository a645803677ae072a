"""GPU parity of the DCA prefill through the C ABI.

Against the reference's own DCA prefill (tests/golden/dca_golden.npz: fp32 within 1e-4, bf16
within 2e-2 abs + 1e-2 rel, since the reference rounds each block output and the merge to bf16)
and against the oracle (oracle_dca) on larger shapes: every row for mid sizes, sampled rows for
config 4's full length.
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


def _t(a, bf16):
    a = np.ascontiguousarray(a)
    if bf16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def test_dca_goldens():
    import dca_kernel as dk
    g = np.load(os.path.join(GOLD, "dca_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        s, c, w, is_bf16 = (int(x) for x in g[p + "params"])
        q, k, v = (_t(g[p + n], is_bf16)[None] for n in ("q", "k", "v"))
        say(f"dca golden {i}: H={q.shape[1]} Hkv={k.shape[1]} N={q.shape[2]} D={q.shape[3]} s={s} c={c} w={w}")
        out = dk.dca_prefill_attention(q, k, v, s, c, w)
        torch.cuda.synchronize()
        got = out[0].float().cpu().numpy()
        ref = g[p + "out"]
        err = check_output(got, ref, orc.BF16 if is_bf16 else orc.F32, f"dca golden {i}")
        print(f"[result] dca golden {i}: max err vs reference {err:.2e}", flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dca_against_oracle(dtype):
    import dca_kernel as dk
    from synthetic import planted_inputs, base_inv_freq
    H, Hkv, N, D = 2, 1, 1000, 128
    s, c, w = 320, 384, 64            # L = 256: four chunks and a ragged fifth
    q, k, v = planted_inputs(61, H, Hkv, N, D, 0.01, dtype, DEV)
    say(f"dca vs oracle {dtype}: H={H} Hkv={Hkv} N={N} D={D} s={s} c={c} w={w}")
    out = dk.dca_prefill_attention(q, k, v, s, c, w)
    torch.cuda.synchronize()
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    ref = orc.dca_attention(qn, kn, vn, dt, base_inv_freq(D, 10000.0).numpy(), s, c, w)
    err = check_output(out_f32(out[0]), ref, dt, f"dca {dtype}")
    print(f"[result] dca {dtype}: max err {err:.2e}", flush=True)


def test_dca_config4_sampled_rows():
    """Config 4's length (N=65536, chunk 4096, local window 512, pretraining length 4096), one
    head, 96 query rows spread over every chunk checked against the oracle."""
    import dca_kernel as dk
    from synthetic import CONFIGS, planted_inputs
    cfg = CONFIGS["c4"]
    q, k, v = planted_inputs(0, 1, 1, cfg.N, cfg.D, cfg.frac, cfg.dtype, DEV)
    invf, _, _ = cfg.geometry()
    say(f"dca config 4: N={cfg.N} D={cfg.D} s={cfg.dca[0]} c={cfg.dca[1]} w={cfg.dca[2]}")
    out = dk.dca_prefill_attention(q, k, v, cfg.dca[0], cfg.dca[1], cfg.dca[2], inv_freq=invf)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([rng.integers(0, cfg.N, 90), [0, 1, 3583, 3584, 7168, cfg.N - 1]]))
    qn, dt = np_of(q[0])
    kn, _ = np_of(k[0])
    vn, _ = np_of(v[0])
    ref = orc.dca_attention(qn, kn, vn, dt, invf.numpy(), cfg.dca[0], cfg.dca[1], cfg.dca[2],
                            rows=rows.astype(np.int32))
    got = out_f32(out[0])
    err = check_output(got[:, rows], ref[:, rows], dt, "dca config 4 rows")
    print(f"[result] dca config 4 ({len(rows)} rows): max err {err:.2e}", flush=True)


def test_dca_rejects_unaligned_chunks():
    import dca_kernel as dk
    q = torch.zeros(1, 1, 128, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError):
        dk.dca_prefill_attention(q, q, q, 100, 4096, 20)   # L = 80
    with pytest.raises(AssertionError):
        dk.dca_prefill_attention(q, q, q, 100, 4096, 100)
