"""Common body of the shared-selection prefill entry points (PI_exact, exact, YaRN_exact, hybrid).

The reference's four files share Kernel A, _build_sets and Kernel C and differ only in the
(inv_freq, pos_scale, rope_scale) triples their entry points pass
(shared_selection_triton_exact_2.py:432-486, shared_selection_triton_exact.py:376-423,
shared_selection_triton_YaRN_exact.py:442-496, shared_selection_triton_hybrid_exact.py:450-510);
here all of them call one HIP path through the C ABI.
"""
import math

import torch

import _sta_native as native

_WMODES = {"freq": 0, "margin": 1, "expmass": 2}


def _check_select_score(select_score):
    if select_score not in _WMODES:
        raise KeyError(select_score)  # the reference's dict lookup (exact_2.py:450)


def _pct_steps(pct):
    start = native.start_pct_of(pct)
    return [start] + [c for c in (25, 20) if c < start]


def report_measure(chosen, orig_overflow, overflow20, pct, k_max):
    """The measure=True messages of exact_2.py:373-381 (one host sync, as in the reference)."""
    adjusted = orig_overflow & ~overflow20
    if bool(adjusted.any()):
        vals, counts = torch.unique(chosen[adjusted].detach().cpu(), return_counts=True)
        summary = ", ".join(f"{int(v)}%:{int(c)}" for v, c in zip(vals, counts))
        print(f"Adjusted top-pct to fit k_max={k_max}: {summary} (requested {pct:g}%).", flush=True)
    if bool(overflow20.any()):
        print(f"WARNING: {int(overflow20.sum().item())} (head,tile) sets still exceed k_max={k_max} "
              f"even at top {_pct_steps(pct)[-1]}%; gather will truncate those tiles.", flush=True)


def shared_prefill(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                   rope_scale_c, pct, sm_scale, n_global, n_local, tile, k_max, q_pos_base, measure,
                   select_score):
    _check_select_score(select_score)
    Z, H, N, D = q.shape
    assert Z == 1
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    r = native.shared_attention(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c,
                                pos_scale_c, rope_scale_c, pct=pct, sm_scale=sm_scale,
                                n_global=n_global, n_local=n_local, tile=tile, k_max=k_max,
                                q_pos_base=q_pos_base, measure=measure, select_score=select_score)
    if measure:
        report_measure(r["chosen"], r["orig_overflow"], r["overflow20"], pct, k_max)
    return (r["out"].unsqueeze(0), r["shared_size"].long(), r["kept_size"].long(), r["chosen"],
            r["orig_overflow"], r["kpct_meas"], r["overflow20"])


def build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
               wvotes=None, select_score="freq"):
    """_build_sets (exact_2.py:277-426) on the device.  Same 9-tuple.  As in the reference, the
    weighted votes rank the keys only when select_score is not "freq" and wvotes is given
    (exact_2.py:299-302)."""
    _check_select_score(select_score)
    use_w = select_score != "freq" and wvotes is not None
    res = native.build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max,
                            q_pos_base=q_pos_base, measure=measure, wvotes=wvotes if use_w else None)
    if measure:
        report_measure(res[5], res[6], res[8], pct, k_max)
    return res
