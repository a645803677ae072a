"""CPU tests that pin the DCA decode oracle (oracle_dca_decode, oracle_dca_rotate_keys in
oracle/sta_oracle_pq.c) to the reference's own forward with a KV cache.

  * the reference's dca_forward (dca_kernel.py:372-525) on a module with pass-through projections
    and a transformers DynamicCache, prefill then decode steps (tests/golden/dca_decode_golden.npz,
    written by tests/golden/gen_golden_dca_decode.py): the cache's rotated keys equal the oracle's
    bit for bit in bf16 / fp16 (fp32: within the fp32 cosine's last bit), every decode output
    equals the oracle's bit for bit in bf16 / fp16 and within 1e-6 in fp32 -- including the
    case whose decode outgrows the table, where the factor changes mid-generation and the earlier
    cached keys keep the old one;
  * the prefill output against the oracle's prefill at the recorded factor;
  * closed forms: a cache inside one chunk is plain RoPE attention (float64 numpy); a decode step
    in a later chunk equals the prefill's last row (same positions, one softmax) in fp32.
"""
import math
import os

import numpy as np
import torch

from oracle import sta_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inv_freq(D):
    # ChunkLlamaRotaryEmbedding's frequencies (dca_kernel.py:176), computed by torch as it does
    return (1.0 / (10000 ** (torch.arange(0, D, 2).float() / D))).numpy()


def _values(a, dt):
    if dt == orc.F32:
        return a.astype(np.float32)
    if dt == orc.BF16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.view(np.float16).astype(np.float32)


def _cases():
    g = np.load(os.path.join(GOLD, "dca_decode_golden.npz"), allow_pickle=False)
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        s, c, w, N, T, dt = (int(x) for x in g[p + "params"])
        yield i, g, p, s, c, w, N, T, dt


def test_cached_keys_match_reference():
    for i, g, p, s, c, w, N, T, dt in _cases():
        k = g[p + "k"]
        ms = g[p + "mscale"].astype(np.float32)
        D = k.shape[-1]
        parts = [orc.dca_rotate_keys(k[:, :N], dt, _inv_freq(D), s, w, ms[0])]
        parts += [orc.dca_rotate_keys(k[:, N + t:N + t + 1], dt, _inv_freq(D), s, w, ms[1 + t], pos0=N + t)
                  for t in range(T)]
        got = np.concatenate(parts, axis=1)
        ref = _values(g[p + "krot"], dt)
        if dt == orc.F32:
            np.testing.assert_allclose(got, ref, atol=1e-6, rtol=0, err_msg=str(i))
        else:
            assert np.array_equal(got, ref), i


def test_decode_steps_match_reference():
    for i, g, p, s, c, w, N, T, dt in _cases():
        q, v, krot, out = g[p + "q"], g[p + "v"], g[p + "krot"], g[p + "out"]
        ms = g[p + "mscale"].astype(np.float32)
        D = q.shape[-1]
        for t in range(T):
            m = N + t + 1
            o = orc.dca_decode(q[:, N + t], krot[:, :m], v[:, :m], dt, _inv_freq(D), s, w, ms[1 + t])
            if dt == orc.F32:
                np.testing.assert_allclose(o, out[:, N + t], atol=1e-6, rtol=0, err_msg=f"{i} step {t}")
            else:
                assert np.array_equal(o, out[:, N + t]), (i, t)
    # the table factor changes inside case 1's decode, and only there
    g = np.load(os.path.join(GOLD, "dca_decode_golden.npz"), allow_pickle=False)
    assert g["c1_mscale"][0] == 1.0 and g["c1_mscale"][-1] > 1.0
    assert len(set(g["c0_mscale"].tolist())) == 1


def test_prefill_matches_reference_at_recorded_factor():
    for i, g, p, s, c, w, N, T, dt in _cases():
        q, k, v, out = g[p + "q"], g[p + "k"], g[p + "v"], g[p + "out"]
        D = q.shape[-1]
        pre = orc.dca_attention(q[:, :N], k[:, :N], v[:, :N], dt, _inv_freq(D), s, c, w,
                                mscale=float(g[p + "mscale"][0]))
        tol = 1e-5 if dt == orc.F32 else 2e-2
        np.testing.assert_allclose(pre, out[:, :N], atol=tol, rtol=tol, err_msg=str(i))


def _rope64(x, pos, invf):
    """Plain RoPE (rotate-half pairs) in float64."""
    ang = np.asarray(pos, np.float64)[..., None] * invf.astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h].astype(np.float64), x[..., h:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def test_single_chunk_decode_is_plain_rope_attention():
    rng = np.random.default_rng(5)
    H, Hkv, M, D = 4, 2, 150, 64
    s, w = 288, 32                                     # L = 256 > M: every key intra, factor 1
    q = rng.standard_normal((H, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, M, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, M, D)).astype(np.float32)
    invf = _inv_freq(D)
    krot = orc.dca_rotate_keys(k, orc.F32, invf, s, w, 1.0)
    out = orc.dca_decode(q, krot, v, orc.F32, invf, s, w, 1.0)
    qr = _rope64(q, M - 1, invf)
    kr = _rope64(k, np.arange(M)[None, :], invf)
    for h in range(H):
        sc = kr[h // 2] @ qr[h] / math.sqrt(D)
        p = np.exp(sc - sc.max())
        ref = (p / p.sum()) @ v[h // 2].astype(np.float64)
        np.testing.assert_allclose(out[h], ref, atol=2e-5, rtol=2e-5)


def test_decode_equals_prefill_last_row_in_every_chunk_position():
    rng = np.random.default_rng(6)
    H, Hkv, D = 2, 1, 64
    s, c, w = 96, 4096, 32                             # L = 64
    invf = _inv_freq(D)
    for M in (40, 64, 65, 127, 128, 129, 200, 333):    # inside chunk 0, 1, 2 and later
        q = rng.standard_normal((H, M, D)).astype(np.float32)
        k = rng.standard_normal((Hkv, M, D)).astype(np.float32)
        v = rng.standard_normal((Hkv, M, D)).astype(np.float32)
        pre = orc.dca_attention(q, k, v, orc.F32, invf, s, c, w, rows=[M - 1], mscale=1.0)
        krot = orc.dca_rotate_keys(k, orc.F32, invf, s, w, 1.0)
        dec = orc.dca_decode(q[:, M - 1], krot, v, orc.F32, invf, s, w, 1.0)
        np.testing.assert_allclose(dec, pre[:, M - 1], atol=2e-5, rtol=2e-5, err_msg=str(M))
