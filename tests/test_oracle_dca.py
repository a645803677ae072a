"""CPU tests that pin the DCA oracle (oracle_dca in oracle/sta_oracle_pq.c).

Pins:
  * the reference's own DCA prefill (dca_kernel.py:372-489 with its tables :166-231 and the
    PyTorch attention path + log-sum-exp merge :292-366) on 4 fixtures covering intra / succ /
    inter positions, GQA, mscale above the pretraining length, fp32 and bf16 model dtypes
    (tests/golden/dca_golden.npz);
  * a known answer: with every query in the first chunk (N <= chunk_size - local_window) DCA is
    dense causal attention with native RoPE (the query and key tables coincide), computed here in
    float64 with complex rotations;
  * row sampling: computing selected rows gives the same values as the full computation.
"""
import math
import os

import numpy as np

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inv_freq(D):
    return (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)


def test_dca_matches_reference(oracle):
    g = np.load(os.path.join(GOLD, "dca_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        s, c, w, is_bf16 = (int(x) for x in g[p + "params"])
        dt = oracle.BF16 if is_bf16 else oracle.F32
        q, k, v = g[p + "q"], g[p + "k"], g[p + "v"]
        out = oracle.dca_attention(q, k, v, dt, _inv_freq(q.shape[-1]), s, c, w)
        ref = g[p + "out"]
        if dt == oracle.F32:
            np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-5)
        else:
            # the reference rounds each of its three block outputs and the merge to bf16
            np.testing.assert_allclose(out, ref, atol=2e-2, rtol=1e-2)
            assert float(np.abs(out - ref).mean()) < 2e-3


def test_dca_single_chunk_is_dense_rope_attention(oracle):
    rng = np.random.default_rng(7)
    H, N, D = 1, 100, 64
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    v = rng.standard_normal((H, N, D)).astype(np.float32)
    invf = _inv_freq(D)
    out = oracle.dca_attention(q, k, v, oracle.F32, invf, 160, 4096, 32)   # L = 128 > N, mscale 1
    half = D // 2
    pos = np.arange(N)
    rot = np.exp(1j * pos[:, None] * invf.astype(np.float64)[None, :])
    qc = (q[0, :, :half] + 1j * q[0, :, half:]) * rot
    kc = (k[0, :, :half] + 1j * k[0, :, half:]) * rot
    sc = (qc[:, None, :] * np.conj(kc[None, :, :])).real.sum(-1) / math.sqrt(D)
    sc = np.where(pos[:, None] >= pos[None, :], sc, -np.inf)
    wgt = np.exp(sc - sc.max(-1, keepdims=True))
    wgt /= wgt.sum(-1, keepdims=True)
    np.testing.assert_allclose(out[0], wgt @ v[0].astype(np.float64), atol=2e-5, rtol=1e-5)


def test_dca_row_sampling(oracle):
    g = np.load(os.path.join(GOLD, "dca_golden.npz"), allow_pickle=False)
    s, c, w, _ = (int(x) for x in g["c0_params"])
    q, k, v = g["c0_q"], g["c0_k"], g["c0_v"]
    full = oracle.dca_attention(q, k, v, oracle.F32, _inv_freq(64), s, c, w)
    rows = np.array([0, 63, 64, 127, 128, 299], np.int32)
    part = oracle.dca_attention(q, k, v, oracle.F32, _inv_freq(64), s, c, w, rows=rows)
    np.testing.assert_array_equal(part[:, rows], full[:, rows])
    assert np.isnan(part[:, 1]).all()
