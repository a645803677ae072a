"""CPU: the reference modules' torch helpers and goldens, as the drop-ins re-export them
(sparse-thresholded-attention_amd/_torch_golden.py).

- every drop-in exposes the names a caller of the reference module imports;
- _rope_rotate against the rotation as a complex product in float64;
- pq_attention_torch and pqstream_attention_torch against the reference's own torch goldens'
  outputs, which the committed fixtures hold (out_torch, written by tests/golden/gen_golden_pq.py
  from the reference under TRITON_INTERPRET=1);
- chunk_attention_torch against the oracle's chunk path (the reference module cannot be imported:
  its chunk_recall_core dependency is absent);
- the DCA helpers against closed forms: the six tables, table RoPE against _rope_rotate, and the
  log-sum-exp merge against one softmax over the concatenated scores.
"""
import importlib
import math
import os

import numpy as np
import pytest
import torch

from oracle import sta_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

NAMES = {
    "shared_selection_triton_exact_2": ["_rope_rotate"],
    "shared_selection_triton_exact": ["_rope_rotate"],
    "shared_selection_triton_YaRN_exact": ["_rope_rotate"],
    "shared_selection_triton_hybrid_exact": ["_rope_rotate"],
    "shared_selection_triton_perquery": ["_rope_rotate", "pq_attention_torch"],
    "pqstream_kernel": ["_rope_rotate", "pqstream_attention_torch"],
    "shared_selection_triton_chunked": ["_rope_rotate", "chunk_attention_torch"],
    "dca_kernel": ["flash_attn_status", "ChunkLlamaRotaryEmbedding", "_rotate_half", "apply_rotary_pos_emb",
                   "_fa_block", "_merge_lse", "get_mscale"],
}


@pytest.mark.parametrize("module", sorted(NAMES))
def test_drop_ins_expose_the_reference_helpers(module):
    m = importlib.import_module(module)
    for name in NAMES[module]:
        assert callable(getattr(m, name)), f"{module}.{name}"


def test_rope_rotate_is_the_complex_rotation():
    from shared_selection_triton_exact_2 import _rope_rotate
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 50, 64, generator=g)
    pos = torch.arange(50).float() * 0.37
    invf = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    got = _rope_rotate(x, pos, invf, 1.25).double()
    z = torch.complex(x[..., :32].double(), x[..., 32:].double())
    ang = pos.double()[:, None] * invf.double()[None]
    w = z * torch.polar(torch.full_like(ang, 1.25), ang)
    want = torch.cat((w.real, w.imag), dim=-1)
    assert torch.allclose(got, want, atol=2e-5, rtol=0)
    # position 0 is the identity times rope_scale; a bf16 input is rotated in fp32
    assert torch.equal(_rope_rotate(x, torch.zeros(50), invf, 1.0), x)
    assert _rope_rotate(x.bfloat16(), pos, invf, 1.0).dtype == torch.float32


def _gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_pq_attention_torch_matches_the_reference_golden():
    from shared_selection_triton_perquery import pq_attention_torch
    g = _gold("pq_composed_golden.npz")
    n = 0
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        if p + "out_torch" not in g.files:
            continue
        psa, rsa, ng, nl, km, mode, qb = g[p + "params"]
        q, k, v = (torch.from_numpy(g[p + x])[None] for x in ("q", "k", "v"))
        out = pq_attention_torch(q, k, v, torch.from_numpy(g[p + "tau"]), torch.from_numpy(g[p + "inv_freq_a"]),
                                 torch.from_numpy(g[p + "inv_freq_c"]), pos_scale_a=float(psa), rope_scale_a=float(rsa),
                                 n_global=int(ng), n_local=int(nl), tile=32, k_max=int(km),
                                 select_score=["freq", "margin", "expmass"][int(mode)])
        err = float(np.max(np.abs(out[0].numpy() - g[p + "out_torch"])))
        assert err < 2e-5, f"case {i}: {err:.3e}"
        n += 1
    assert n >= 3


def test_pqstream_attention_torch_matches_the_reference_golden():
    from pqstream_kernel import pqstream_attention_torch
    g = _gold("pqstream_golden.npz")
    for i in range(int(g["ncases"])):
        p = f"c{i}_"
        psa, rsa, ng, nl, bn, full, skip = g[p + "params"]
        q, k, v = (torch.from_numpy(g[p + x])[None] for x in ("q", "k", "v"))
        out = pqstream_attention_torch(q, k, v, torch.from_numpy(g[p + "tau"]), torch.from_numpy(g[p + "inv_freq_a"]),
                                       torch.from_numpy(g[p + "inv_freq_c"]), pos_scale_a=float(psa),
                                       rope_scale_a=float(rsa), n_global=int(ng), n_local=int(nl), tile=32,
                                       block_n=int(bn), pos_advance="full" if full else "max")
        err = float(np.max(np.abs(out[0].numpy() - g[p + "out_torch"])))
        assert err < 2e-5, f"case {i}: {err:.3e}"


@pytest.mark.parametrize("mode,agg", [("expmass", "sum"), ("freq", "mean")])
def test_chunk_attention_torch_matches_the_oracle(mode, agg):
    from shared_selection_triton_chunked import chunk_attention_torch
    from synthetic import base_inv_freq, planted_inputs
    H, N, D = 2, 300, 64
    q, k, v = planted_inputs(31, H, H, N, D, 0.03, torch.float32, "cpu")
    invf = base_inv_freq(D, 10000.0)
    tau = torch.full((H,), 3.0)
    kw = dict(n_global=4, n_local=8, tile=32, k_max=96, chunk_size=8)
    out = chunk_attention_torch(q, k, v, tau, invf, invf, pos_scale_a=0.5, select_score=mode, chunk_agg=agg, **kw)
    ref = orc.shared_chunk_attention(q[0].numpy(), k[0].numpy(), v[0].numpy(), orc.F32, tau.numpy(), invf.numpy(),
                                     invf.numpy(), pos_scale_a=0.5, select_score=mode, chunk_agg=agg, **kw)
    ref_out = ref[0] if isinstance(ref, tuple) else ref
    err = float(np.max(np.abs(out[0].numpy() - ref_out)))
    assert err < 2e-5, err


def test_dca_tables_and_table_rope():
    import dca_kernel as dk
    s, w, c, dim = 320, 64, 512, 64
    rot = dk.ChunkLlamaRotaryEmbedding(dim, max_position_embeddings=c, chunk_size=s, local_window=w)
    L = s - w
    tabs = rot(torch.zeros(1, dtype=torch.float32), seq_len=c)
    assert [t.shape[0] for t in tabs] == [L, L, L, L, c, c]
    invf = dk.base_inv_freq(dim)
    assert torch.allclose(tabs[4][:, :dim // 2], torch.cos(torch.outer(torch.arange(c).float() % L, invf)), atol=1e-6)
    assert torch.allclose(tabs[2][-1, :dim // 2], torch.cos(float(min(2 * L - 1, s)) * invf), atol=1e-6)
    # a longer call rebuilds every table with the length factor and headroom
    n = 3 * c
    tabs = rot(torch.zeros(1), seq_len=n)
    f = dk.get_mscale(n / c)
    assert rot.max_seq_len == n + 512 and abs(rot._last_mscale - f) < 1e-12
    assert torch.allclose(tabs[0][:, :dim // 2], torch.cos(torch.outer(torch.arange(L).float(), invf)) * f, atol=1e-6)
    # table RoPE at key positions equals _rope_rotate at j mod L times the factor
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, 2, 40, dim, generator=g)
    pid = torch.arange(100, 140)[None]
    got = dk.apply_rotary_pos_emb(x, tabs[4], tabs[5], pid)
    from _torch_golden import _rope_rotate
    want = _rope_rotate(x[0], (pid[0] % L).float(), invf, f)[None]
    assert torch.allclose(got, want, atol=1e-5)
    assert "HIP" in dk.flash_attn_status()


def test_dca_lse_merge_is_one_softmax():
    import dca_kernel as dk
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 5, 16, generator=g)
    k = torch.randn(1, 2, 30, 16, generator=g)
    v = torch.randn(1, 2, 30, 16, generator=g)
    sm = 1.0 / math.sqrt(16)
    parts = [dk._fa_block(q, k[:, :, a:b], v[:, :, a:b], False, sm) for a, b in ((0, 7), (7, 19), (19, 30))]
    parts.append(dk._fa_block(q, k[:, :, :0], v[:, :, :0], False, sm))        # an empty block
    merged = dk._merge_lse(parts)
    whole = torch.softmax(torch.matmul(q, k.transpose(-1, -2)) * sm, dim=-1) @ v
    assert torch.allclose(merged, whole, atol=1e-5)
    out, lse = dk._fa_block(q[:, :, :5], k[:, :, :5], v[:, :, :5], True, sm)   # causal square block
    sc = (q @ k[:, :, :5].transpose(-1, -2)) * sm
    sc = sc.masked_fill(torch.ones(5, 5, dtype=torch.bool).triu(1), float("-inf"))
    assert torch.allclose(lse, torch.logsumexp(sc, -1), atol=1e-6)
    assert torch.allclose(out, torch.softmax(sc, -1) @ v[:, :, :5], atol=1e-6)
