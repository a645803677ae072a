"""GPU: the allocation-free entry point recorded into a HIP graph (torch.cuda.graph) and replayed.

sta_shared_attention_noalloc allocates nothing and issues no memset, so a caller can capture it.
The graph is replayed several times with the program's own eager work and synchronisations in
between; every replay must reproduce the eager result bit for bit, including after the inputs
were overwritten in place (the graph reads them at replay time) and after the outputs were
cleared.
"""
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


@pytest.mark.parametrize("select_score", ["freq", "expmass"])
def test_noalloc_graph_replays_match_eager(select_score):
    import _sta_native as native
    from synthetic import base_inv_freq, planted_inputs
    H, N, D, tile, k_max = 4, 1500, 128, 64, 256
    print(f"[case] graph capture of the no-alloc entry point, {select_score}", flush=True)
    q, k, v = planted_inputs(31, H, H, N, D, 0.01, torch.bfloat16, DEV)
    q2, _, _ = planted_inputs(32, H, H, N, D, 0.01, torch.bfloat16, DEV)
    invf = base_inv_freq(D, 10000.0).to(DEV)
    tau = torch.full((H,), 5.0, device=DEV)
    kw = dict(pct=30.0, tile=tile, k_max=k_max, want_votes=True, select_score=select_score)
    q_buf = q.clone()
    plan = native.NoallocPlan(q_buf, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, **kw)
    plan.run()                     # resolves the scratch address before capture
    torch.cuda.synchronize()

    def eager(qx):
        return native.shared_attention(qx, k, v, tau, invf, 0.5, 1.0, invf, 0.5, 1.0, **kw)

    ref1, ref2 = eager(q), eager(q2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run()
    torch.cuda.synchronize()
    for rep, (src, ref) in enumerate([(q, ref1), (q2, ref2), (q, ref1), (q2, ref2)]):
        q_buf.copy_(src)                                  # new inputs in place
        for n in NAMES:
            plan.out[n].zero_()                           # the replay must write every output
        _ = eager(q2)                                     # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n in NAMES:
            assert torch.equal(plan.out[n], ref[n]), f"replay {rep}: {n} differs from the eager run"
    print(f"[result] {select_score}: 4 replays identical to the eager runs", flush=True)
