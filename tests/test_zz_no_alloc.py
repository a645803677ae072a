"""GPU: the allocation-free entry point sta_shared_attention_noalloc (include/sta.h) against
sta_shared_attention on the same inputs, through the C ABI.

Both run the same kernels; only the workspace differs (the library's fixed scratch array instead
of a caller buffer), so every output must be bit-identical.  Two calls in a row, the second with
a smaller input (the array keeps the first call's contents), and a shape whose workspace exceeds
the array must be refused with STA_ERR_WORKSPACE before anything runs.
"""
import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NAMES = ["out", "idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen", "orig_overflow",
         "kpct_meas", "overflow20", "votes"]


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _sta_native
    _sta_native.lib()


def _run_both(H, Hkv, N, D, dtype, tile, k_max, seed, select_score="freq"):
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    print(f"[case] noalloc vs workspace: H={H} Hkv={Hkv} N={N} D={D} {dtype} tile={tile} "
          f"k_max={k_max} {select_score}", flush=True)
    q, k, v = planted_inputs(seed, H, Hkv, N, D, 0.01, dtype, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 5.0)
    kw = dict(pct=30.0, tile=tile, k_max=k_max, want_votes=True, select_score=select_score)
    a = native.shared_attention(q, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, **kw)
    b = native.shared_attention_noalloc(q, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, **kw)
    torch.cuda.synchronize()
    for n in NAMES:
        assert torch.equal(a[n], b[n]), f"{n} differs between the two entry points"
    print(f"[result] H={H} N={N}: all {len(NAMES)} outputs identical, kept mean "
          f"{a['kept_size'].float().mean().item():.1f}", flush=True)


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: a larger shape; second: a smaller one over the array's leftover contents
    _run_both(8, 2, 3000, 128, torch.bfloat16, 64, 512, 1)
    _run_both(4, 4, 777, 64, torch.float16, 32, 128, 2)


def test_noalloc_weighted_ranking():
    _run_both(4, 4, 1500, 128, torch.bfloat16, 64, 256, 3, select_score="expmass")


def test_noalloc_rejects_shape_above_scratch():
    import _sta_native as native
    from synthetic import base_inv_freq
    H, N, D = 32, 8192, 128       # workspace ~ 0.5 GB, above the 64 MiB array
    q = torch.zeros(1, H, N, D, dtype=torch.bfloat16, device=DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    print("[case] noalloc above the scratch size", flush=True)
    with pytest.raises(RuntimeError, match="scratch"):
        native.shared_attention_noalloc(q, q, q, torch.full((H,), 5.0), invf, 1.0, 1.0, invf, 1.0, 1.0,
                                        tile=64, k_max=256)
