"""ctypes binding of libsta_hip.so (the C ABI declared in include/sta.h).

The library is built in-tree by build.py.  There is no other code path: if the library is
missing, cannot be loaded, or the tensors are not on a HIP device, these functions raise.
PyTorch is used only for device memory and the current stream.
"""
import ctypes
import math
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsta_hip.so")
_LIB = None

STA_OK = 0
DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
EXPORTS = ["sta_abi_version", "sta_last_error", "sta_shared_workspace_size", "sta_shared_attention",
           "sta_shared_attention_noalloc",
           "sta_select_vote", "sta_build_sets", "sta_build_sets_weighted", "sta_gather_attention",
           "sta_pq_workspace_size", "sta_pq_attention", "sta_pq_select_bits", "sta_pq_build_sets",
           "sta_pq_gather_attention", "sta_chunk_attention", "sta_chunk_build_sets",
           "sta_pqstream_workspace_size", "sta_pqstream_attention",
           "sta_dca_workspace_size", "sta_dca_attention", "sta_dca_rotate_keys", "sta_dca_decode_workspace_size",
           "sta_dca_decode", "sta_decode_workspace_size", "sta_decode_scores",
           "sta_decode_build_sets", "sta_decode_build_sets_chunk", "sta_decode_attend", "sta_decode_attention"]
SCORES = {"freq": 0, "margin": 1, "expmass": 2}


class ShareArgs(ctypes.Structure):
    """Mirror of sta_shared_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_head_stride", ctypes.c_int64), ("q_tok_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("tau", ctypes.c_void_p),
        ("inv_freq_a", ctypes.c_void_p), ("pos_scale_a", ctypes.c_float), ("rope_scale_a", ctypes.c_float),
        ("inv_freq_c", ctypes.c_void_p), ("pos_scale_c", ctypes.c_float), ("rope_scale_c", ctypes.c_float),
        ("sm_scale", ctypes.c_float),
        ("start_pct", ctypes.c_int32), ("n_global", ctypes.c_int32), ("n_local", ctypes.c_int32),
        ("tile", ctypes.c_int32), ("k_max", ctypes.c_int32), ("q_pos_base", ctypes.c_int32),
        ("measure", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("idx", ctypes.c_void_p), ("newpos_k", ctypes.c_void_p),
        ("newpos_q", ctypes.c_void_p), ("shared_size", ctypes.c_void_p), ("kept_size", ctypes.c_void_p),
        ("chosen", ctypes.c_void_p), ("orig_overflow", ctypes.c_void_p), ("kpct_meas", ctypes.c_void_p),
        ("overflow20", ctypes.c_void_p),
        ("votes", ctypes.c_void_p), ("row_counts", ctypes.c_void_p), ("row_max", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", ctypes.c_void_p),
        ("select_score", ctypes.c_int32), ("wvotes", ctypes.c_void_p),
    ]


class PqArgs(ctypes.Structure):
    """Mirror of sta_pq_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_head_stride", ctypes.c_int64), ("q_tok_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("tau", ctypes.c_void_p),
        ("inv_freq_a", ctypes.c_void_p), ("pos_scale_a", ctypes.c_float), ("rope_scale_a", ctypes.c_float),
        ("inv_freq_c", ctypes.c_void_p), ("sm_scale", ctypes.c_float),
        ("n_global", ctypes.c_int32), ("n_local", ctypes.c_int32), ("tile", ctypes.c_int32),
        ("k_max", ctypes.c_int32), ("q_pos_base", ctypes.c_int32), ("select_score", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("idx", ctypes.c_void_p), ("newpos_k", ctypes.c_void_p),
        ("newpos_q", ctypes.c_void_p), ("mask", ctypes.c_void_p), ("usize", ctypes.c_void_p),
        ("kept_size", ctypes.c_void_p), ("overflow", ctypes.c_void_p),
        ("votes", ctypes.c_void_p), ("bits", ctypes.c_void_p), ("wvotes", ctypes.c_void_p),
        ("row_counts", ctypes.c_void_p), ("row_max", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", ctypes.c_void_p),
    ]


class StreamArgsC(ctypes.Structure):
    """Mirror of sta_pqstream_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_head_stride", ctypes.c_int64), ("q_tok_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("tau", ctypes.c_void_p),
        ("inv_freq_a", ctypes.c_void_p), ("pos_scale_a", ctypes.c_float), ("rope_scale_a", ctypes.c_float),
        ("inv_freq_c", ctypes.c_void_p), ("sm_scale", ctypes.c_float),
        ("n_global", ctypes.c_int32), ("n_local", ctypes.c_int32), ("tile", ctypes.c_int32),
        ("block_n", ctypes.c_int32), ("pos_advance", ctypes.c_int32), ("use_skip", ctypes.c_int32),
        ("q_pos_base", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("span", ctypes.c_void_p), ("kept", ctypes.c_void_p),
        ("blocks", ctypes.c_void_p), ("skipped", ctypes.c_void_p), ("row_max", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", ctypes.c_void_p), ("bits", ctypes.c_void_p), ("fused", ctypes.c_int32),
    ]


STREAM_FUSED = {"auto": 0, "fused": 1, "unfused": 2}


class DcaArgsC(ctypes.Structure):
    """Mirror of sta_dca_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_head_stride", ctypes.c_int64), ("q_tok_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("inv_freq", ctypes.c_void_p),
        ("chunk_size", ctypes.c_int32), ("pretrain_len", ctypes.c_int32), ("local_window", ctypes.c_int32),
        ("scale", ctypes.c_float), ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", ctypes.c_void_p),
        ("select", ctypes.c_int32), ("tau", ctypes.c_void_p), ("start_pct", ctypes.c_int32),
        ("k_max", ctypes.c_int32), ("n_global", ctypes.c_int32), ("measure", ctypes.c_int32),
        ("idx", ctypes.c_void_p), ("shared_size", ctypes.c_void_p), ("kept_size", ctypes.c_void_p),
        ("chosen", ctypes.c_void_p), ("orig_overflow", ctypes.c_void_p), ("kpct_meas", ctypes.c_void_p),
        ("overflow20", ctypes.c_void_p), ("votes", ctypes.c_void_p), ("row_max", ctypes.c_void_p),
        ("mscale", ctypes.c_float),
    ]


class ChunkParamsC(ctypes.Structure):
    """Mirror of sta_chunk_params (include/sta.h)."""
    _fields_ = [("chunk_size", ctypes.c_int32), ("n_chunk", ctypes.c_int32), ("chunk_agg", ctypes.c_int32),
                ("passers_kept", ctypes.c_void_p)]


CHUNK_AGG = {"sum": 0, "mean": 1}


class DcaRotateArgsC(ctypes.Structure):
    """Mirror of sta_dca_rotate_args (include/sta.h)."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("x_head_stride", ctypes.c_int64), ("x_tok_stride", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_head_stride", ctypes.c_int64), ("out_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("heads", ctypes.c_int32), ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("pos0", ctypes.c_int32), ("inv_freq", ctypes.c_void_p),
        ("chunk_size", ctypes.c_int32), ("local_window", ctypes.c_int32), ("mscale", ctypes.c_float),
    ]


class DcaDecodeArgsC(ctypes.Structure):
    """Mirror of sta_dca_decode_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_head_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v", ctypes.c_void_p), ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32), ("M", ctypes.c_int32),
        ("D", ctypes.c_int32), ("inv_freq", ctypes.c_void_p),
        ("chunk_size", ctypes.c_int32), ("local_window", ctypes.c_int32),
        ("mscale", ctypes.c_float), ("scale", ctypes.c_float), ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class DecodeArgsC(ctypes.Structure):
    """Mirror of sta_decode_args (include/sta.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_head_stride", ctypes.c_int64), ("q_tok_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64), ("k_tok_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("v_tok_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("Q", ctypes.c_int32), ("M", ctypes.c_int32), ("D", ctypes.c_int32),
        ("tau", ctypes.c_void_p), ("inv_freq_a", ctypes.c_void_p),
        ("pos_scale_a", ctypes.c_float), ("rope_scale_a", ctypes.c_float), ("pos_scale_c", ctypes.c_float),
        ("inv_freq_c", ctypes.c_void_p), ("rope_scale_c", ctypes.c_float), ("sm_scale", ctypes.c_float),
        ("q_pos0", ctypes.c_int32), ("n_global", ctypes.c_int32), ("n_local", ctypes.c_int32),
        ("k_max", ctypes.c_int32), ("pct_decode", ctypes.c_double), ("causal", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("idx", ctypes.c_void_p), ("newpos_k", ctypes.c_void_p),
        ("newpos_q", ctypes.c_void_p), ("set_size", ctypes.c_void_p), ("scores", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", ctypes.c_void_p),
        ("rule", ctypes.c_int32), ("usize", ctypes.c_void_p), ("overflow", ctypes.c_void_p),
        ("block_n", ctypes.c_int32),
    ]


RULES = {"shared": 0, "pq": 1, "stream": 2}    # STA_RULE_SHARED / STA_RULE_PQ / STA_RULE_STREAM


def lib():
    """Load libsta_hip.so once; raise loudly if it is absent."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              f"`python sparse-thresholded-attention_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        L.sta_abi_version.restype = ctypes.c_int
        L.sta_last_error.restype = ctypes.c_char_p
        L.sta_shared_workspace_size.restype = ctypes.c_size_t
        L.sta_shared_workspace_size.argtypes = [ctypes.POINTER(ShareArgs)]
        for name in ("sta_shared_attention", "sta_shared_attention_noalloc", "sta_select_vote",
                     "sta_gather_attention"):
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(ShareArgs), ctypes.c_void_p]
        L.sta_build_sets.restype = ctypes.c_int
        L.sta_build_sets.argtypes = [ctypes.POINTER(ShareArgs), ctypes.c_void_p, ctypes.c_int32,
                                     ctypes.c_void_p]
        L.sta_build_sets_weighted.restype = ctypes.c_int
        L.sta_build_sets_weighted.argtypes = [ctypes.POINTER(ShareArgs), ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_int32, ctypes.c_void_p]
        L.sta_pq_workspace_size.restype = ctypes.c_size_t
        L.sta_pq_workspace_size.argtypes = [ctypes.POINTER(PqArgs)]
        for name in ("sta_pq_attention", "sta_pq_select_bits", "sta_pq_gather_attention"):
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(PqArgs), ctypes.c_void_p]
        L.sta_pq_build_sets.restype = ctypes.c_int
        L.sta_pq_build_sets.argtypes = [ctypes.POINTER(PqArgs), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
        L.sta_pqstream_workspace_size.restype = ctypes.c_size_t
        L.sta_pqstream_workspace_size.argtypes = [ctypes.POINTER(StreamArgsC)]
        L.sta_pqstream_attention.restype = ctypes.c_int
        L.sta_pqstream_attention.argtypes = [ctypes.POINTER(StreamArgsC), ctypes.c_void_p]
        L.sta_dca_workspace_size.restype = ctypes.c_size_t
        L.sta_dca_workspace_size.argtypes = [ctypes.POINTER(DcaArgsC)]
        L.sta_dca_attention.restype = ctypes.c_int
        L.sta_dca_attention.argtypes = [ctypes.POINTER(DcaArgsC), ctypes.c_void_p]
        L.sta_decode_workspace_size.restype = ctypes.c_size_t
        L.sta_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgsC)]
        for name in ("sta_decode_attend", "sta_decode_attention"):
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(DecodeArgsC), ctypes.c_void_p]
        for name in ("sta_decode_scores", "sta_decode_build_sets"):
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(DecodeArgsC), ctypes.c_void_p, ctypes.c_void_p]
        L.sta_chunk_attention.restype = ctypes.c_int
        L.sta_chunk_attention.argtypes = [ctypes.POINTER(PqArgs), ctypes.POINTER(ChunkParamsC), ctypes.c_void_p]
        L.sta_chunk_build_sets.restype = ctypes.c_int
        L.sta_chunk_build_sets.argtypes = [ctypes.POINTER(PqArgs), ctypes.POINTER(ChunkParamsC), ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
        L.sta_decode_build_sets_chunk.restype = ctypes.c_int
        L.sta_decode_build_sets_chunk.argtypes = [ctypes.POINTER(DecodeArgsC), ctypes.POINTER(ChunkParamsC),
                                                  ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
        L.sta_dca_rotate_keys.restype = ctypes.c_int
        L.sta_dca_rotate_keys.argtypes = [ctypes.POINTER(DcaRotateArgsC), ctypes.c_void_p]
        L.sta_dca_decode_workspace_size.restype = ctypes.c_size_t
        L.sta_dca_decode_workspace_size.argtypes = [ctypes.POINTER(DcaDecodeArgsC)]
        L.sta_dca_decode.restype = ctypes.c_int
        L.sta_dca_decode.argtypes = [ctypes.POINTER(DcaDecodeArgsC), ctypes.c_void_p]
        if L.sta_abi_version() != 5:
            raise ImportError("libsta_hip.so ABI version mismatch")
        _LIB = L
    return _LIB


def _check(rc, what):
    if rc != STA_OK:
        msg = lib().sta_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _heads_view(x):
    """(1, H, N, D) or (H, N, D) -> (H, N, D) view with unit dim stride and 16-byte rows."""
    if x.dim() == 4:
        assert x.shape[0] == 1, "batch size must be 1"
        x = x[0]
    esz = x.element_size()
    if (x.stride(2) != 1 or (x.stride(0) * esz) % 16 or (x.stride(1) * esz) % 16
            or x.data_ptr() % 16):
        x = x.contiguous()
    return x


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def start_pct_of(pct):
    """max(0, int(round(pct))) with Python's round-half-even (exact_2.py:309)."""
    return max(0, int(round(pct)))


def _fill_common(a, q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                 rope_scale_c, sm_scale, pct, n_global, n_local, tile, k_max, q_pos_base, measure,
                 select_score="freq"):
    H, N, D = q.shape
    a.q, a.k = _ptr(q), _ptr(k)
    a.v = _ptr(v) if v is not None else None
    a.q_head_stride, a.q_tok_stride = q.stride(0), q.stride(1)
    a.k_head_stride, a.k_tok_stride = k.stride(0), k.stride(1)
    if v is not None:
        a.v_head_stride, a.v_tok_stride = v.stride(0), v.stride(1)
    a.dtype = DTYPES[q.dtype]
    a.H, a.Hkv, a.N, a.D = H, k.shape[0], N, D
    a.tau = _ptr(tau)
    a.inv_freq_a, a.pos_scale_a, a.rope_scale_a = _ptr(inv_freq_a), float(pos_scale_a), float(rope_scale_a)
    a.inv_freq_c, a.pos_scale_c, a.rope_scale_c = _ptr(inv_freq_c), float(pos_scale_c), float(rope_scale_c)
    a.sm_scale = float(sm_scale)
    a.start_pct = start_pct_of(pct)
    a.n_global, a.n_local, a.tile, a.k_max = int(n_global), int(n_local), int(tile), int(k_max)
    a.q_pos_base, a.measure = int(q_pos_base), int(bool(measure))
    a.select_score = SCORES[select_score]


def _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c):
    if not q.is_cuda:
        raise RuntimeError("sparse-thresholded attention runs on a HIP device only; got a CPU tensor")
    if q.dtype not in DTYPES:
        raise TypeError(f"unsupported dtype {q.dtype}")
    dev = q.device
    qh = _heads_view(q)
    kh = _heads_view(k.to(dev))
    vh = _heads_view(v.to(dev)) if v is not None else None
    if kh.dtype != qh.dtype or (vh is not None and vh.dtype != qh.dtype):
        raise TypeError("q, k and v must share one dtype")
    tau = tau.to(device=dev, dtype=torch.float32).contiguous()
    ifa = inv_freq_a.to(device=dev, dtype=torch.float32).contiguous()
    ifc = inv_freq_c.to(device=dev, dtype=torch.float32).contiguous() if inv_freq_c is not None else ifa
    return qh, kh, vh, tau, ifa, ifc


def _workspace(a, dev):
    n = lib().sta_shared_workspace_size(ctypes.byref(a))
    if n == 0:
        _check(-1, "sta_shared_workspace_size")
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    assert ws.data_ptr() % 256 == 0
    a.workspace, a.workspace_bytes = _ptr(ws), n
    return ws


class SharedPlan:
    """Outputs and workspace for one shape, allocated once; run() launches the whole prefill path
    on the current stream and allocates nothing.  Successive runs overwrite the outputs."""

    def __init__(self, q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                 rope_scale_c, pct=30.0, sm_scale=None, n_global=32, n_local=32, tile=32,
                 k_max=1024, q_pos_base=0, measure=False, want_votes=False, want_row_max=False,
                 want_row_counts=False, select_score="freq"):
        qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
        H, N, D = qh.shape
        self.device = qh.device
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        self.args = a = ShareArgs()
        _fill_common(a, qh, kh, vh, tau, ifa, pos_scale_a, rope_scale_a, ifc, pos_scale_c, rope_scale_c,
                     sm_scale, pct, n_global, n_local, tile, k_max, q_pos_base, measure, select_score)
        self._keep = (qh, kh, vh, tau, ifa, ifc)
        self.out = _alloc_outputs(a, H, N, D, qh.dtype, tile, k_max, self.device, want_votes,
                                  want_row_max, want_row_counts, want_wvotes=want_votes and select_score != "freq")
        self.workspace = _workspace(a, self.device)
        self._events = None

    def run(self, events=None):
        """events: None or 5 recorded torch.cuda.Event(enable_timing=True) marking the stages."""
        if events is not None:
            self._events = (ctypes.c_void_p * 5)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_shared_attention(ctypes.byref(self.args), _stream(self.device)),
               "sta_shared_attention")
        return self.out


def _alloc_outputs(a, H, N, D, dtype, tile, k_max, dev, want_votes, want_row_max, want_row_counts,
                   want_wvotes=False):
    nt = (N + tile - 1) // tile
    r = {
        "out": torch.empty((H, N, D), dtype=dtype, device=dev),
        "idx": torch.empty((H, nt, k_max), dtype=torch.int32, device=dev),
        "newpos_k": torch.empty((H, nt, k_max), dtype=torch.float32, device=dev),
        "newpos_q": torch.empty((H, nt, tile), dtype=torch.float32, device=dev),
        "shared_size": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "kept_size": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "chosen": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "orig_overflow": torch.empty((H, nt), dtype=torch.bool, device=dev),
        "kpct_meas": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "overflow20": torch.empty((H, nt), dtype=torch.bool, device=dev),
    }
    if want_votes:
        r["votes"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
    if want_row_max:
        r["row_max"] = torch.empty((H, N), dtype=torch.float32, device=dev)
    if want_row_counts:
        r["row_counts"] = torch.empty((H, N), dtype=torch.int32, device=dev)
    if want_wvotes:
        r["wvotes"] = torch.empty((H, nt, N), dtype=torch.float32, device=dev)
    for name in ("out", "idx", "newpos_k", "newpos_q", "shared_size", "kept_size", "chosen",
                 "orig_overflow", "kpct_meas", "overflow20"):
        setattr(a, name, _ptr(r[name]))
    a.votes = _ptr(r.get("votes"))
    a.row_max = _ptr(r.get("row_max"))
    a.row_counts = _ptr(r.get("row_counts"))
    a.wvotes = _ptr(r.get("wvotes"))
    return r


def shared_attention(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                     rope_scale_c, pct=30.0, sm_scale=None, n_global=32, n_local=32, tile=32,
                     k_max=1024, q_pos_base=0, measure=False, want_votes=False, want_row_max=False,
                     want_row_counts=False, select_score="freq"):
    """Run the whole prefill path on the device.  q (1,H,N,D) / k, v (1,Hkv,N,D).
    Returns a dict of device tensors (see include/sta.h for their meaning; with want_votes and a
    weighted select_score also "wvotes").  The workspace is released on return; the caching
    allocator hands it out again only to work queued later on the same stream."""
    plan = SharedPlan(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                      rope_scale_c, pct, sm_scale, n_global, n_local, tile, k_max, q_pos_base, measure,
                      want_votes, want_row_max, want_row_counts, select_score)
    return plan.run()


NOALLOC_SCRATCH_BYTES = 64 << 20   # STA_NOALLOC_SCRATCH_BYTES (include/sta.h)


def shared_attention_noalloc(q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c,
                             pos_scale_c, rope_scale_c, pct=30.0, sm_scale=None, n_global=32,
                             n_local=32, tile=32, k_max=1024, q_pos_base=0, measure=False,
                             want_votes=False, want_row_max=False, select_score="freq"):
    """The whole prefill path through sta_shared_attention_noalloc: the library's fixed scratch
    array replaces the workspace, so no device memory is allocated for it (the outputs still
    are, here).  Same results as shared_attention."""
    qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
    H, N, D = qh.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    a = ShareArgs()
    _fill_common(a, qh, kh, vh, tau, ifa, pos_scale_a, rope_scale_a, ifc, pos_scale_c, rope_scale_c,
                 sm_scale, pct, n_global, n_local, tile, k_max, q_pos_base, measure, select_score)
    out = _alloc_outputs(a, H, N, D, qh.dtype, tile, k_max, qh.device, want_votes, want_row_max, False,
                         want_wvotes=want_votes and select_score != "freq")
    a.workspace, a.workspace_bytes = None, 0
    _check(lib().sta_shared_attention_noalloc(ctypes.byref(a), _stream(qh.device)),
           "sta_shared_attention_noalloc")
    return out


class NoallocPlan:
    """Outputs for one shape allocated once; run() launches the whole prefill path through
    sta_shared_attention_noalloc on the current stream, with no workspace and no allocation, so
    it can be recorded into a HIP graph (torch.cuda.graph).  The library resolves its scratch
    array's device address on the first call on a device: run once before capturing."""

    def __init__(self, q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, pos_scale_c,
                 rope_scale_c, pct=30.0, sm_scale=None, n_global=32, n_local=32, tile=32, k_max=1024,
                 q_pos_base=0, measure=False, want_votes=False, select_score="freq"):
        qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
        H, N, D = qh.shape
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        self.device = qh.device
        a = self.args = ShareArgs()
        _fill_common(a, qh, kh, vh, tau, ifa, pos_scale_a, rope_scale_a, ifc, pos_scale_c, rope_scale_c,
                     sm_scale, pct, n_global, n_local, tile, k_max, q_pos_base, measure, select_score)
        self.out = _alloc_outputs(a, H, N, D, qh.dtype, tile, k_max, qh.device, want_votes, False, False,
                                  want_wvotes=want_votes and select_score != "freq")
        a.workspace, a.workspace_bytes = None, 0
        self._keep = (qh, kh, vh, tau, ifa, ifc)

    def run(self):
        _check(lib().sta_shared_attention_noalloc(ctypes.byref(self.args), _stream(self.device)),
               "sta_shared_attention_noalloc")
        return self.out


def select_vote(q, k, tau, inv_freq, pos_scale, rope_scale, sm_scale, tile, q_pos_base=0,
                want_row_counts=True, select_score="freq"):
    """Kernel A alone: votes (H,nt,N) int32, row_counts (H,N) int32, row_max (H,N) fp32; with a
    weighted select_score a fourth result, the weighted votes (H,nt,N) fp32."""
    qh, kh, _, tau, ifa, _ = _prep_inputs(q, k, None, tau, inv_freq, None)
    H, N, D = qh.shape
    dev = qh.device
    nt = (N + tile - 1) // tile
    a = ShareArgs()
    _fill_common(a, qh, kh, None, tau, ifa, pos_scale, rope_scale, ifa, pos_scale, rope_scale,
                 sm_scale, 30.0, 0, 0, tile, 1, q_pos_base, False, select_score)
    votes = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
    rc = torch.empty((H, N), dtype=torch.int32, device=dev) if want_row_counts else None
    rm = torch.empty((H, N), dtype=torch.float32, device=dev)
    wv = torch.empty((H, nt, N), dtype=torch.float32, device=dev) if select_score != "freq" else None
    a.votes, a.row_counts, a.row_max, a.wvotes = _ptr(votes), _ptr(rc), _ptr(rm), _ptr(wv)
    ws = _workspace(a, dev)
    _check(lib().sta_select_vote(ctypes.byref(a), _stream(dev)), "sta_select_vote")
    del ws
    if wv is not None:
        return votes, rc, rm, wv
    return votes, rc, rm


def build_sets(votes, pos_scale, n_global, n_local, pct, T, k_max, q_pos_base=0, measure=False,
               wvotes=None):
    """_build_sets on the device from int32 votes (H, nt, N) and, for weighted ranking, fp32
    wvotes (H, nt, N) (rank = fl(wvotes + fl(1e-6 votes)), exact_2.py:299-302).  Returns the
    reference's 9-tuple (exact_2.py:418-426) with shared_size / kept_size as int64 like the
    reference's sums."""
    if not votes.is_cuda:
        raise RuntimeError("build_sets runs on a HIP device only; got a CPU tensor")
    votes = votes.to(torch.int32).contiguous()
    # the library stages votes as bytes (a tile's count is at most its 32 or 64 queries) and does
    # not check them; a value outside [0, 255] would wrap, so it is rejected here (one sync, as the
    # reference's own _build_sets syncs)
    if votes.numel() and (int(votes.min()) < 0 or int(votes.max()) > 255):
        raise ValueError("votes must lie in [0, 255] (a tile's vote count is at most its tile size)")
    if wvotes is not None:
        wvotes = wvotes.to(device=votes.device, dtype=torch.float32).contiguous()
        if wvotes.shape != votes.shape:
            raise ValueError(f"wvotes {tuple(wvotes.shape)} and votes {tuple(votes.shape)} differ in shape")
    H, nt, N = votes.shape
    dev = votes.device
    a = ShareArgs()
    a.dtype, a.H, a.Hkv, a.N, a.D = 1, H, H, N, 64
    a.pos_scale_c = float(pos_scale)
    a.start_pct = start_pct_of(pct)
    a.n_global, a.n_local, a.tile, a.k_max = int(n_global), int(n_local), int(T), int(k_max)
    a.q_pos_base, a.measure = int(q_pos_base), int(bool(measure))
    idx = torch.empty((H, nt, k_max), dtype=torch.int32, device=dev)
    npk = torch.empty((H, nt, k_max), dtype=torch.float32, device=dev)
    npq = torch.empty((H, nt, T), dtype=torch.float32, device=dev)
    ss = torch.empty((H, nt), dtype=torch.int32, device=dev)
    ks = torch.empty((H, nt), dtype=torch.int32, device=dev)
    ch = torch.empty((H, nt), dtype=torch.int32, device=dev)
    oo = torch.empty((H, nt), dtype=torch.bool, device=dev)
    km = torch.empty((H, nt), dtype=torch.int32, device=dev)
    o20 = torch.empty((H, nt), dtype=torch.bool, device=dev)
    a.idx, a.newpos_k, a.newpos_q = _ptr(idx), _ptr(npk), _ptr(npq)
    a.shared_size, a.kept_size, a.chosen = _ptr(ss), _ptr(ks), _ptr(ch)
    a.orig_overflow, a.kpct_meas, a.overflow20 = _ptr(oo), _ptr(km), _ptr(o20)
    if wvotes is not None:
        a.select_score = SCORES["margin"]   # any weighted ranking: the rank value is the same
        _check(lib().sta_build_sets_weighted(ctypes.byref(a), _ptr(votes), _ptr(wvotes), nt, _stream(dev)),
               "sta_build_sets_weighted")
    else:
        _check(lib().sta_build_sets(ctypes.byref(a), _ptr(votes), nt, _stream(dev)), "sta_build_sets")
    return idx, npk, npq, ss.long(), ks.long(), ch, oo, km, o20


def gather_attention(q, k, v, inv_freq, idx, newpos_k, newpos_q, sm_scale, rope_scale, tile, k_max,
                     q_pos_base=0, kept_size=None):
    """Kernel C alone.  Returns out (H, N, D) in q.dtype."""
    qh, kh, vh, _, ifc, _ = _prep_inputs(q, k, v, torch.zeros(1), inv_freq, None)
    H, N, D = qh.shape
    dev = qh.device
    a = ShareArgs()
    _fill_common(a, qh, kh, vh, torch.zeros(1, device=dev), ifc, 1.0, rope_scale, ifc, 1.0, rope_scale,
                 sm_scale, 30.0, 0, 0, tile, k_max, q_pos_base, False)
    out = torch.empty((H, N, D), dtype=qh.dtype, device=dev)
    idx = idx.to(device=dev, dtype=torch.int32).contiguous()
    newpos_k = newpos_k.to(device=dev, dtype=torch.float32).contiguous()
    newpos_q = newpos_q.to(device=dev, dtype=torch.float32).contiguous()
    a.out, a.idx, a.newpos_k, a.newpos_q = _ptr(out), _ptr(idx), _ptr(newpos_k), _ptr(newpos_q)
    ks = kept_size.to(device=dev, dtype=torch.int32).contiguous() if kept_size is not None else None
    a.kept_size = _ptr(ks)
    _check(lib().sta_gather_attention(ctypes.byref(a), _stream(dev)), "sta_gather_attention")
    return out


# ---------------------------------------------------------------------------------------------
# PQ Union (per-query sets through the tile union + per-slot bitmask)
# ---------------------------------------------------------------------------------------------
def _fill_pq(a, q, k, v, tau, inv_freq_a, pos_scale_a, rope_scale_a, inv_freq_c, sm_scale, n_global,
             n_local, tile, k_max, q_pos_base, select_score):
    H, N, D = q.shape
    a.q, a.k = _ptr(q), _ptr(k)
    a.v = _ptr(v) if v is not None else None
    a.q_head_stride, a.q_tok_stride = q.stride(0), q.stride(1)
    a.k_head_stride, a.k_tok_stride = k.stride(0), k.stride(1)
    if v is not None:
        a.v_head_stride, a.v_tok_stride = v.stride(0), v.stride(1)
    a.dtype = DTYPES[q.dtype]
    a.H, a.Hkv, a.N, a.D = H, k.shape[0], N, D
    a.tau = _ptr(tau)
    a.inv_freq_a, a.pos_scale_a, a.rope_scale_a = _ptr(inv_freq_a), float(pos_scale_a), float(rope_scale_a)
    a.inv_freq_c = _ptr(inv_freq_c)
    a.sm_scale = float(sm_scale)
    a.n_global, a.n_local, a.tile, a.k_max = int(n_global), int(n_local), int(tile), int(k_max)
    a.q_pos_base = int(q_pos_base)
    if select_score not in SCORES:
        raise ValueError(f"select_score must be one of {sorted(SCORES)}, got {select_score!r}")
    a.select_score = SCORES[select_score]


def _pq_set_outputs(a, H, nt, tile, k_max, dev):
    r = {
        "idx": torch.empty((H, nt, k_max), dtype=torch.int32, device=dev),
        "newpos_k": torch.empty((H, nt, k_max), dtype=torch.float32, device=dev),
        "newpos_q": torch.empty((H, nt, tile), dtype=torch.float32, device=dev),
        "mask": torch.empty((H, nt, k_max), dtype=torch.int32, device=dev),
        "usize": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "kept_size": torch.empty((H, nt), dtype=torch.int32, device=dev),
        "overflow": torch.empty((H, nt), dtype=torch.bool, device=dev),
    }
    for name, t in r.items():
        setattr(a, name, _ptr(t))
    return r


def _pq_workspace(a, dev):
    n = lib().sta_pq_workspace_size(ctypes.byref(a))
    if n == 0:
        _check(-1, "sta_pq_workspace_size")
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    assert ws.data_ptr() % 256 == 0
    a.workspace, a.workspace_bytes = _ptr(ws), n
    return ws


class PqPlan:
    """Outputs and workspace of the PQ Union prefill for one shape, allocated once; run()
    launches the whole path on the current stream and allocates nothing."""

    def __init__(self, q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                 sm_scale=None, n_global=32, n_local=32, tile=32, k_max=4096, q_pos_base=0,
                 select_score="expmass", want_votes=False, want_row_max=False, want_row_counts=False):
        qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
        H, N, D = qh.shape
        self.device = dev = qh.device
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        self.args = a = PqArgs()
        _fill_pq(a, qh, kh, vh, tau, ifa, pos_scale_a, rope_scale_a, ifc, sm_scale, n_global, n_local,
                 tile, k_max, q_pos_base, select_score)
        self._keep = (qh, kh, vh, tau, ifa, ifc)
        nt = (N + tile - 1) // tile
        r = _pq_set_outputs(a, H, nt, tile, k_max, dev)
        r["out"] = torch.empty((H, N, D), dtype=qh.dtype, device=dev)
        a.out = _ptr(r["out"])
        if want_votes:
            r["votes"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
            r["bits"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
            r["wvotes"] = torch.empty((H, nt, N), dtype=torch.float32, device=dev)
        if want_row_max:
            r["row_max"] = torch.empty((H, N), dtype=torch.float32, device=dev)
        if want_row_counts:
            r["row_counts"] = torch.empty((H, N), dtype=torch.int32, device=dev)
        for name in ("votes", "bits", "wvotes", "row_max", "row_counts"):
            setattr(a, name, _ptr(r.get(name)))
        self.out = r
        self.workspace = _pq_workspace(a, dev)
        self._events = None

    def run(self, events=None):
        if events is not None:
            self._events = (ctypes.c_void_p * 5)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_pq_attention(ctypes.byref(self.args), _stream(self.device)), "sta_pq_attention")
        return self.out


def pq_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0, sm_scale=None,
                 n_global=32, n_local=32, tile=32, k_max=4096, q_pos_base=0, select_score="expmass",
                 want_votes=False, want_row_max=False, want_row_counts=False):
    """The whole PQ Union prefill on the device; returns a dict of device tensors."""
    return PqPlan(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale, n_global,
                  n_local, tile, k_max, q_pos_base, select_score, want_votes, want_row_max,
                  want_row_counts).run()


def pq_select_bits(q, k, tau, inv_freq, pos_scale, rope_scale, sm_scale, tile=32, q_pos_base=0,
                   select_score="expmass"):
    """PQ Kernel A alone: votes, bits (H,nt,N) int32, wvotes (H,nt,N) fp32, row_counts, row_max."""
    qh, kh, _, tau, ifa, _ = _prep_inputs(q, k, None, tau, inv_freq, None)
    H, N, D = qh.shape
    dev = qh.device
    nt = (N + tile - 1) // tile
    a = PqArgs()
    _fill_pq(a, qh, kh, None, tau, ifa, pos_scale, rope_scale, ifa, sm_scale, 0, 0, tile, 1, q_pos_base,
             select_score)
    r = {"votes": torch.empty((H, nt, N), dtype=torch.int32, device=dev),
         "bits": torch.empty((H, nt, N), dtype=torch.int32, device=dev),
         "wvotes": torch.empty((H, nt, N), dtype=torch.float32, device=dev),
         "row_counts": torch.empty((H, N), dtype=torch.int32, device=dev),
         "row_max": torch.empty((H, N), dtype=torch.float32, device=dev)}
    for name, t in r.items():
        setattr(a, name, _ptr(t))
    ws = _pq_workspace(a, dev)
    _check(lib().sta_pq_select_bits(ctypes.byref(a), _stream(dev)), "sta_pq_select_bits")
    del ws
    return r


def pq_build_sets(votes, bits, wvotes, n_global, n_local, T, k_max, q_pos_base=0, select_score="expmass"):
    """_build_sets_pq on the device from dense (H, nt, N) votes / bits / wvotes.  Returns the
    reference's 7-tuple (idx, newpos_k, newpos_q, mask, usize, kept_size, overflow)."""
    if not votes.is_cuda:
        raise RuntimeError("pq_build_sets runs on a HIP device only; got a CPU tensor")
    votes = votes.to(torch.int32).contiguous()
    bits = bits.to(torch.int32).contiguous()
    H, nt, N = votes.shape
    dev = votes.device
    use_w = select_score != "freq" and wvotes is not None and wvotes.shape[-1] == N
    wv = wvotes.to(torch.float32).contiguous() if use_w else None
    a = PqArgs()
    a.dtype, a.H, a.Hkv, a.N, a.D = 1, H, H, N, 64
    a.n_global, a.n_local, a.tile, a.k_max = int(n_global), int(n_local), int(T), int(k_max)
    a.q_pos_base = int(q_pos_base)
    a.select_score = SCORES[select_score] if use_w else SCORES["freq"]
    r = _pq_set_outputs(a, H, nt, T, k_max, dev)
    _check(lib().sta_pq_build_sets(ctypes.byref(a), _ptr(votes), _ptr(bits), _ptr(wv), nt, _stream(dev)),
           "sta_pq_build_sets")
    return (r["idx"], r["newpos_k"], r["newpos_q"], r["mask"], r["usize"], r["kept_size"], r["overflow"])


# ---------------------------------------------------------------------------------------------
# chunk-granular selection (chunked variant)
# ---------------------------------------------------------------------------------------------
def _chunk_params(chunk_size, n_chunk, chunk_agg, passers_kept=None):
    cp = ChunkParamsC()
    cp.chunk_size, cp.n_chunk, cp.chunk_agg = int(chunk_size), int(n_chunk), CHUNK_AGG[chunk_agg]
    cp.passers_kept = _ptr(passers_kept)
    return cp


class ChunkPlan:
    """Outputs and workspace of the chunked prefill for one shape, allocated once; run() launches
    PQ Kernel A, the chunk selection and the pooled Kernel C on the current stream and allocates
    nothing.  Outputs: out, idx, newpos_k, newpos_q, mask, usize, kept_size, passers_kept (and
    votes / bits / wvotes on request)."""

    def __init__(self, q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0, sm_scale=None,
                 n_global=32, n_local=32, tile=32, k_max=4096, chunk_size=16, n_chunk=None, q_pos_base=0,
                 select_score="expmass", chunk_agg="sum", want_votes=False):
        qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
        H, N, D = qh.shape
        self.device = dev = qh.device
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        if n_chunk is None:
            n_chunk = derive_n_chunk(k_max, chunk_size, n_global, n_local, tile)
        self.args = a = PqArgs()
        _fill_pq(a, qh, kh, vh, tau, ifa, pos_scale_a, rope_scale_a, ifc, sm_scale, n_global, n_local,
                 tile, k_max, q_pos_base, select_score)
        self._keep = (qh, kh, vh, tau, ifa, ifc)
        nt = (N + tile - 1) // tile
        r = _pq_set_outputs(a, H, nt, tile, k_max, dev)
        r["out"] = torch.empty((H, N, D), dtype=qh.dtype, device=dev)
        r["passers_kept"] = torch.empty((H, nt), dtype=torch.int32, device=dev)
        a.out = _ptr(r["out"])
        if want_votes:
            r["votes"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
            r["bits"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
            r["wvotes"] = torch.empty((H, nt, N), dtype=torch.float32, device=dev)
        for name in ("votes", "bits", "wvotes"):
            setattr(a, name, _ptr(r.get(name)))
        self.chunk = _chunk_params(chunk_size, n_chunk, chunk_agg, r["passers_kept"])
        self.out = r
        self.workspace = _pq_workspace(a, dev)
        self._events = None

    def run(self, events=None):
        """events: None or 5 recorded torch.cuda.Event(enable_timing=True), as for PqPlan."""
        if events is not None:
            self._events = (ctypes.c_void_p * 5)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_chunk_attention(ctypes.byref(self.args), ctypes.byref(self.chunk), _stream(self.device)),
               "sta_chunk_attention")
        return self.out


def n_forced_chunks(chunk_size, n_global, n_local, tile):
    """Worst-case chunks of the forced global + local keys (chunked.py:115-129)."""
    C = chunk_size
    return (n_global + C - 1) // C + (n_local + tile - 1 + C - 1) // C + 1


def derive_n_chunk(k_max, chunk_size, n_global, n_local, tile):
    """Chunks to select so that forced + selected fill k_max exactly (chunked.py:132-146)."""
    C = chunk_size
    assert k_max % C == 0, f"k_max={k_max} must be divisible by chunk_size={C}"
    nf = n_forced_chunks(C, n_global, n_local, tile)
    n = k_max // C - nf
    assert n > 0, (f"chunk_size={C} leaves no budget: forced needs {nf} chunks ({nf * C} slots) of "
                   f"k_max={k_max}. Raise k_max or lower chunk_size/n_global/n_local.")
    return n


def chunk_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0, sm_scale=None,
                    n_global=32, n_local=32, tile=32, k_max=4096, chunk_size=16, n_chunk=None, q_pos_base=0,
                    select_score="expmass", chunk_agg="sum", want_votes=False):
    """The whole chunked prefill on the device; returns a dict of device tensors."""
    return ChunkPlan(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale, n_global, n_local,
                     tile, k_max, chunk_size, n_chunk, q_pos_base, select_score, chunk_agg, want_votes).run()


def chunk_build_sets(votes, wvotes, n_global, n_local, T, k_max, chunk_size, n_chunk, q_pos_base=0,
                     select_score="expmass", chunk_agg="sum"):
    """_build_sets_chunk on the device from dense (H, nt, N) votes / wvotes.  Returns the
    reference's 6-tuple (idx, newpos_k, newpos_q, mask, usize, kept_size) and passers_kept."""
    if not votes.is_cuda:
        raise RuntimeError("chunk_build_sets runs on a HIP device only; got a CPU tensor")
    votes = votes.to(torch.int32).contiguous()
    H, nt, N = votes.shape
    dev = votes.device
    use_w = select_score != "freq" and wvotes is not None and wvotes.shape[-1] == N
    wv = wvotes.to(torch.float32).contiguous() if use_w else None
    a = PqArgs()
    a.dtype, a.H, a.Hkv, a.N, a.D = 1, H, H, N, 64
    a.n_global, a.n_local, a.tile, a.k_max = int(n_global), int(n_local), int(T), int(k_max)
    a.q_pos_base = int(q_pos_base)
    a.select_score = SCORES[select_score] if use_w else SCORES["freq"]
    r = _pq_set_outputs(a, H, nt, T, k_max, dev)
    pk = torch.empty((H, nt), dtype=torch.int32, device=dev)
    cp = _chunk_params(chunk_size, n_chunk, chunk_agg, pk)
    _check(lib().sta_chunk_build_sets(ctypes.byref(a), ctypes.byref(cp), _ptr(votes), _ptr(wv), nt, _stream(dev)),
           "sta_chunk_build_sets")
    return (r["idx"], r["newpos_k"], r["newpos_q"], r["mask"], r["usize"], r["kept_size"]), pk


def pq_gather_attention(q, k, v, inv_freq_c, idx, newpos_k, newpos_q, mask, sm_scale, tile, k_max,
                        q_pos_base=0, kept_size=None):
    """PQ Kernel C alone.  Returns out (H, N, D) in q.dtype."""
    qh, kh, vh, _, ifc, _ = _prep_inputs(q, k, v, torch.zeros(1), inv_freq_c, None)
    H, N, D = qh.shape
    dev = qh.device
    a = PqArgs()
    _fill_pq(a, qh, kh, vh, torch.zeros(1, device=dev), ifc, 1.0, 1.0, ifc, sm_scale, 0, 0, tile, k_max,
             q_pos_base, "expmass")
    out = torch.empty((H, N, D), dtype=qh.dtype, device=dev)
    keep = [t.to(device=dev, dtype=dt).contiguous() for t, dt in
            ((idx, torch.int32), (newpos_k, torch.float32), (newpos_q, torch.float32), (mask, torch.int32))]
    a.out = _ptr(out)
    a.idx, a.newpos_k, a.newpos_q, a.mask = (_ptr(t) for t in keep)
    ks = kept_size.to(device=dev, dtype=torch.int32).contiguous() if kept_size is not None else None
    a.kept_size = _ptr(ks)
    _check(lib().sta_pq_gather_attention(ctypes.byref(a), _stream(dev)), "sta_pq_gather_attention")
    return out


# ---------------------------------------------------------------------------------------------
# PQ Stream (per-query keep sets, streamed block positions, one attend sweep)
# ---------------------------------------------------------------------------------------------
ADVANCES = {"max": 0, "full": 1}


class StreamPlan:
    """Outputs and workspace of the PQ Stream prefill for one shape, allocated once; run()
    launches the whole path on the current stream and allocates nothing."""

    def __init__(self, q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                 sm_scale=None, n_global=32, n_local=32, tile=32, block_n=32, pos_advance="max",
                 q_pos_base=0, use_skip=True, want_row_max=False, want_bits=False, fused="auto"):
        """want_bits: also return bits (H, nt, N) int32, the threshold keep bits the sweep applied
        (zero past each tile's last query).  fused: "auto" (the separate keep-bit pass while its
        buffer stays within 4 GiB), "fused" (the sweep computes the keep bits) or "unfused"."""
        qh, kh, vh, tau, ifa, ifc = _prep_inputs(q, k, v, tau, inv_freq_a, inv_freq_c)
        H, N, D = qh.shape
        self.device = dev = qh.device
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        if pos_advance not in ADVANCES:
            raise KeyError(pos_advance)
        self.args = a = StreamArgsC()
        a.q, a.k, a.v = _ptr(qh), _ptr(kh), _ptr(vh)
        a.q_head_stride, a.q_tok_stride = qh.stride(0), qh.stride(1)
        a.k_head_stride, a.k_tok_stride = kh.stride(0), kh.stride(1)
        a.v_head_stride, a.v_tok_stride = vh.stride(0), vh.stride(1)
        a.dtype = DTYPES[qh.dtype]
        a.H, a.Hkv, a.N, a.D = H, kh.shape[0], N, D
        a.tau = _ptr(tau)
        a.inv_freq_a, a.pos_scale_a, a.rope_scale_a = _ptr(ifa), float(pos_scale_a), float(rope_scale_a)
        a.inv_freq_c, a.sm_scale = _ptr(ifc), float(sm_scale)
        a.n_global, a.n_local, a.tile, a.block_n = int(n_global), int(n_local), int(tile), int(block_n)
        a.pos_advance, a.use_skip, a.q_pos_base = ADVANCES[pos_advance], int(bool(use_skip)), int(q_pos_base)
        a.fused = STREAM_FUSED[fused]
        self._keep = (qh, kh, vh, tau, ifa, ifc)
        nt = (N + tile - 1) // tile
        r = {"out": torch.empty((H, N, D), dtype=qh.dtype, device=dev),
             "span": torch.empty((H, nt), dtype=torch.float32, device=dev),
             "kept": torch.empty((H, N), dtype=torch.int32, device=dev),
             "blocks": torch.empty((H, nt), dtype=torch.float32, device=dev),
             "skipped": torch.empty((H, nt), dtype=torch.float32, device=dev)}
        if want_row_max:
            r["row_max"] = torch.empty((H, N), dtype=torch.float32, device=dev)
        if want_bits:
            r["bits"] = torch.zeros((H, nt, N), dtype=torch.int32, device=dev)
        for name in ("out", "span", "kept", "blocks", "skipped", "row_max", "bits"):
            setattr(a, name, _ptr(r.get(name)))
        self.out = r
        n = lib().sta_pqstream_workspace_size(ctypes.byref(a))
        if n == 0:
            _check(-1, "sta_pqstream_workspace_size")
        self.workspace = torch.empty(n, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), n
        self._events = None

    def run(self, events=None):
        if events is not None:
            self._events = (ctypes.c_void_p * 5)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_pqstream_attention(ctypes.byref(self.args), _stream(self.device)),
               "sta_pqstream_attention")
        return self.out


def pqstream_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                       sm_scale=None, n_global=32, n_local=32, tile=32, block_n=32, pos_advance="max",
                       q_pos_base=0, use_skip=True, want_row_max=False, want_bits=False, fused="auto"):
    """The whole PQ Stream prefill on the device; returns a dict of device tensors."""
    return StreamPlan(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a, rope_scale_a, sm_scale,
                      n_global, n_local, tile, block_n, pos_advance, q_pos_base, use_skip,
                      want_row_max, want_bits, fused).run()


# ---------------------------------------------------------------------------------------------
# DCA (dense attention, dual-chunk positions)
# ---------------------------------------------------------------------------------------------
class DcaPlan:
    """Output and workspace of the DCA prefill for one shape, allocated once; run() launches the
    rotations and the attention sweep on the current stream and allocates nothing."""

    def __init__(self, q, k, v, inv_freq, chunk_size, pretrain_len, local_window, scale=None, tau=None,
                 pct=30.0, k_max=2048, n_global=32, measure=False, want_votes=False, want_row_max=False,
                 mscale=None):
        """tau given: config 4 (exact-max selection over the inter-chunk keys, 64-query tiles);
        the outputs then also hold the selection (idx, shared_size, kept_size, chosen,
        orig_overflow, kpct_meas, overflow20; votes / row_max on request).  mscale: the table
        factor (default get_mscale(N / pretrain_len))."""
        qh, kh, vh, _, ifc, _ = _prep_inputs(q, k, v, torch.zeros(1), inv_freq, None)
        H, N, D = qh.shape
        self.device = dev = qh.device
        if scale is None:
            scale = 1.0 / math.sqrt(D)
        self.args = a = DcaArgsC()
        a.q, a.k, a.v = _ptr(qh), _ptr(kh), _ptr(vh)
        a.q_head_stride, a.q_tok_stride = qh.stride(0), qh.stride(1)
        a.k_head_stride, a.k_tok_stride = kh.stride(0), kh.stride(1)
        a.v_head_stride, a.v_tok_stride = vh.stride(0), vh.stride(1)
        a.dtype = DTYPES[qh.dtype]
        a.H, a.Hkv, a.N, a.D = H, kh.shape[0], N, D
        a.inv_freq = _ptr(ifc)
        a.chunk_size, a.pretrain_len, a.local_window = int(chunk_size), int(pretrain_len), int(local_window)
        a.scale = float(scale)
        a.mscale = 0.0 if mscale is None else float(mscale)
        self._keep = (qh, kh, vh, ifc)
        self.out = {"out": torch.empty((H, N, D), dtype=qh.dtype, device=dev)}
        a.out = _ptr(self.out["out"])
        self.select = tau is not None
        if self.select:
            nt = (N + 63) // 64
            tau = tau.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
            if tau.numel() == 1 and H > 1:
                tau = tau.expand(H).contiguous()
            self._keep = self._keep + (tau,)
            a.select, a.tau, a.start_pct = 1, _ptr(tau), start_pct_of(pct)
            a.k_max, a.n_global, a.measure = int(k_max), int(n_global), int(bool(measure))
            o = self.out
            o["idx"] = torch.empty((H, nt, k_max), dtype=torch.int32, device=dev)
            for name in ("shared_size", "kept_size", "chosen", "kpct_meas"):
                o[name] = torch.empty((H, nt), dtype=torch.int32, device=dev)
            for name in ("orig_overflow", "overflow20"):
                o[name] = torch.empty((H, nt), dtype=torch.bool, device=dev)
            if want_votes:
                o["votes"] = torch.empty((H, nt, N), dtype=torch.int32, device=dev)
            if want_row_max:
                o["row_max"] = torch.empty((H, N), dtype=torch.float32, device=dev)
            for name in ("idx", "shared_size", "kept_size", "chosen", "orig_overflow", "kpct_meas", "overflow20",
                         "votes", "row_max"):
                setattr(a, name, _ptr(o.get(name)))
        n = lib().sta_dca_workspace_size(ctypes.byref(a))
        if n == 0:
            _check(-1, "sta_dca_workspace_size")
        self.workspace = torch.empty(n, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), n
        self._events = None

    def run(self, events=None):
        """events: None or recorded torch.cuda.Event(enable_timing=True): 3 (dense: rotations,
        sweep) or 5 (selection: rotations, votes, selection, attention)."""
        if events is not None:
            n = 5 if self.select else 3
            self._events = (ctypes.c_void_p * n)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_dca_attention(ctypes.byref(self.args), _stream(self.device)), "sta_dca_attention")
        return self.out


def dca_attention(q, k, v, inv_freq, chunk_size, pretrain_len, local_window, scale=None, mscale=None):
    """The DCA prefill on the device; returns out (H, N, D) in q.dtype."""
    return DcaPlan(q, k, v, inv_freq, chunk_size, pretrain_len, local_window, scale, mscale=mscale).run()["out"]


def dca_rotate_keys(k, pos0, inv_freq, chunk_size, local_window, mscale, out=None):
    """Keys k (heads, N, D) or (1, heads, N, D) at positions pos0.. rotated at (pos mod L) with the
    key table, in the model dtype -> out (heads, N, D) (allocated when not given)."""
    kh = _heads_view(k)
    if not kh.is_cuda:
        raise RuntimeError("sparse-thresholded attention runs on a HIP device only; got a CPU tensor")
    if kh.dtype not in DTYPES:
        raise TypeError(f"unsupported dtype {kh.dtype}")
    heads, N, D = kh.shape
    if out is None:
        out = torch.empty((heads, N, D), dtype=kh.dtype, device=kh.device)
    ifr = inv_freq.to(device=kh.device, dtype=torch.float32).contiguous()
    a = DcaRotateArgsC()
    a.x, a.x_head_stride, a.x_tok_stride = _ptr(kh), kh.stride(0), kh.stride(1)
    a.out, a.out_head_stride, a.out_tok_stride = _ptr(out), out.stride(0), out.stride(1)
    a.dtype, a.heads, a.N, a.D = DTYPES[kh.dtype], heads, N, D
    a.pos0, a.inv_freq = int(pos0), _ptr(ifr)
    a.chunk_size, a.local_window, a.mscale = int(chunk_size), int(local_window), float(mscale)
    _check(lib().sta_dca_rotate_keys(ctypes.byref(a), _stream(kh.device)), "sta_dca_rotate_keys")
    return out


def dca_decode(q, k, v, inv_freq, chunk_size, local_window, mscale, scale=None):
    """DCA at decode: the query q (H, D) (or (1, H, 1, D)) at position M - 1 over the cache of
    rotated keys k and values v (Hkv, M, D) (or (1, Hkv, M, D)) -> out (H, D) in q.dtype."""
    qh = q.reshape(q.shape[-3] if q.dim() == 4 else q.shape[0], q.shape[-1])
    if qh.stride(-1) != 1:
        qh = qh.contiguous()
    kh, vh = _heads_view(k), _heads_view(v)
    if not qh.is_cuda:
        raise RuntimeError("sparse-thresholded attention runs on a HIP device only; got a CPU tensor")
    if qh.dtype not in DTYPES or kh.dtype != qh.dtype or vh.dtype != qh.dtype:
        raise TypeError("q, k and v must share one supported dtype")
    H, D = qh.shape
    Hkv, M = kh.shape[0], kh.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    dev = qh.device
    ifr = inv_freq.to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty((H, D), dtype=qh.dtype, device=dev)
    a = DcaDecodeArgsC()
    a.q, a.q_head_stride = _ptr(qh), qh.stride(0)
    a.k, a.k_head_stride, a.k_tok_stride = _ptr(kh), kh.stride(0), kh.stride(1)
    a.v, a.v_head_stride, a.v_tok_stride = _ptr(vh), vh.stride(0), vh.stride(1)
    a.dtype, a.H, a.Hkv, a.M, a.D = DTYPES[qh.dtype], H, Hkv, M, D
    a.inv_freq = _ptr(ifr)
    a.chunk_size, a.local_window = int(chunk_size), int(local_window)
    a.mscale, a.scale, a.out = float(mscale), float(scale), _ptr(out)
    n = lib().sta_dca_decode_workspace_size(ctypes.byref(a))
    if n == 0:
        _check(-1, "sta_dca_decode_workspace_size")
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = _ptr(ws), n
    _check(lib().sta_dca_decode(ctypes.byref(a), _stream(dev)), "sta_dca_decode")
    return out


def dca_select_attention(q, k, v, inv_freq, chunk_size, pretrain_len, local_window, tau, pct=30.0, k_max=2048,
                         n_global=32, scale=None, measure=False, want_votes=False, want_row_max=False):
    """Config 4 on the device: DCA positions, exact-max selection over each 64-query tile's
    inter-chunk keys, dense local keys.  Returns the dict of outputs (out, idx, statistics, ...)."""
    return DcaPlan(q, k, v, inv_freq, chunk_size, pretrain_len, local_window, scale, tau, pct, k_max, n_global,
                   measure, want_votes, want_row_max).run()


# ---------------------------------------------------------------------------------------------
# decode: Q queries over one cache of M keys, query i at position q_pos0 + i seeing the keys
# [0, M - (Q - 1 - i))
# ---------------------------------------------------------------------------------------------
def _queries_view(x):
    """(H, D) one query per head, (H, Q, D) or (1, H, Q, D) -> (H, Q, D) with unit dim stride."""
    if x.dim() == 2:
        x = x.unsqueeze(1)
    return _heads_view(x)


class DecodePlan:
    """Outputs and workspace of the decode path for one shape, allocated once; run() launches the
    scores, the selection and the attend on the current stream and allocates nothing."""

    def __init__(self, q, k, v, tau, inv_freq, q_pos0, pos_scale=1.0, rope_scale=1.0, sm_scale=None,
                 n_global=32, n_local=32, k_max=1024, pct_decode=100.0, causal=False, want_scores=False,
                 inv_freq_c=None, pos_scale_c=None, rope_scale_c=None, rule="shared", block_n=32):
        """inv_freq / pos_scale / rope_scale: the selection geometry; the *_c triple (default: the
        same) repositions (pos_scale_c) and attends (inv_freq_c, rope_scale_c).  rule "shared" is
        _decode_build_sets (exact_2.py:527-604), "pq" _decode_build_sets_pq (perquery.py:651-720:
        dense ranks, exact cap budget; pass rope_scale_c=1 and the base inv_freq_c); "pq" also
        fills usize and overflow (H, Q).  "stream" is _decode_build_sets_pqs (pqstream_kernel.py:
        695-797: every passer and forced key, no cap, streamed positions over blocks of block_n
        keys walked back from the query; k_max is the slot buffer, M rounded up to 1024)."""
        if not q.is_cuda:
            raise RuntimeError("sparse-thresholded attention runs on a HIP device only; got a CPU tensor")
        if q.dtype not in DTYPES:
            raise TypeError(f"unsupported dtype {q.dtype}")
        dev = q.device
        qh = _queries_view(q)
        kh = _heads_view(k.to(dev))
        vh = _heads_view(v.to(dev)) if v is not None else None
        if kh.dtype != qh.dtype or (vh is not None and vh.dtype != qh.dtype):
            raise TypeError("q, k and v must share one dtype")
        H, Q, D = qh.shape
        M = kh.shape[1]
        self.device = dev
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        tau = tau.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if tau.numel() == 1 and H > 1:
            tau = tau.expand(H).contiguous()
        ifr = inv_freq.to(device=dev, dtype=torch.float32).contiguous()
        ifc = inv_freq_c.to(device=dev, dtype=torch.float32).contiguous() if inv_freq_c is not None else ifr
        pos_scale_c = pos_scale if pos_scale_c is None else pos_scale_c
        rope_scale_c = rope_scale if rope_scale_c is None else rope_scale_c
        self.args = a = DecodeArgsC()
        a.q, a.k = _ptr(qh), _ptr(kh)
        a.v = _ptr(vh) if vh is not None else None
        a.q_head_stride, a.q_tok_stride = qh.stride(0), qh.stride(1)
        a.k_head_stride, a.k_tok_stride = kh.stride(0), kh.stride(1)
        if vh is not None:
            a.v_head_stride, a.v_tok_stride = vh.stride(0), vh.stride(1)
        a.dtype = DTYPES[qh.dtype]
        a.H, a.Hkv, a.Q, a.M, a.D = H, kh.shape[0], Q, M, D
        a.tau, a.inv_freq_a, a.inv_freq_c = _ptr(tau), _ptr(ifr), _ptr(ifc)
        a.pos_scale_a, a.rope_scale_a, a.sm_scale = float(pos_scale), float(rope_scale), float(sm_scale)
        a.pos_scale_c, a.rope_scale_c = float(pos_scale_c), float(rope_scale_c)
        a.q_pos0, a.n_global, a.n_local, a.k_max = int(q_pos0), int(n_global), int(n_local), int(k_max)
        a.pct_decode, a.causal = float(pct_decode), int(bool(causal))
        a.rule = RULES[rule]
        a.block_n = int(block_n)
        self._keep = (qh, kh, vh, tau, ifr, ifc)
        self.out = {
            "out": torch.empty((H, Q, D), dtype=qh.dtype, device=dev),
            "idx": torch.empty((H, Q, k_max), dtype=torch.int32, device=dev),
            "newpos_k": torch.empty((H, Q, k_max), dtype=torch.float32, device=dev),
            "newpos_q": torch.empty((H, Q), dtype=torch.float32, device=dev),
            "set_size": torch.empty((H, Q), dtype=torch.int32, device=dev),
        }
        if want_scores:
            self.out["scores"] = torch.empty((H, Q, M), dtype=torch.float32, device=dev)
        if rule == "pq":
            self.out["usize"] = torch.empty((H, Q), dtype=torch.int32, device=dev)
            self.out["overflow"] = torch.empty((H, Q), dtype=torch.bool, device=dev)
        for name in ("out", "idx", "newpos_k", "newpos_q", "set_size"):
            setattr(a, name, _ptr(self.out[name]))
        a.scores = _ptr(self.out.get("scores"))
        a.usize, a.overflow = _ptr(self.out.get("usize")), _ptr(self.out.get("overflow"))
        n = lib().sta_decode_workspace_size(ctypes.byref(a))
        if n == 0:
            _check(-1, "sta_decode_workspace_size")
        self.workspace = torch.empty(n, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), n
        self._events = None

    def run(self, events=None):
        """events: None or 4 recorded torch.cuda.Event(enable_timing=True) marking the stages."""
        if events is not None:
            self._events = (ctypes.c_void_p * 4)(*[e.cuda_event for e in events])
            self.args.stage_events = ctypes.cast(self._events, ctypes.c_void_p)
        else:
            self.args.stage_events = None
        _check(lib().sta_decode_attention(ctypes.byref(self.args), _stream(self.device)), "sta_decode_attention")
        return self.out

    def scores(self, out):
        """Scores alone into out (H, Q, M) fp32."""
        _check(lib().sta_decode_scores(ctypes.byref(self.args), _ptr(out), _stream(self.device)),
               "sta_decode_scores")
        return out

    def build_sets(self, scores):
        """Selection alone from scores (H, Q, M) fp32 into idx / newpos_k / newpos_q / set_size."""
        _check(lib().sta_decode_build_sets(ctypes.byref(self.args), _ptr(scores), _stream(self.device)),
               "sta_decode_build_sets")
        return self.out

    def build_sets_chunk(self, scores, chunk_size, n_chunk, select_score="expmass", chunk_agg="sum",
                         passers_kept=None, usize=None):
        """The chunk rule (_decode_build_sets_chunk, chunked.py:411-489) from scores (H, Q, M) fp32
        into idx / newpos_k / newpos_q / set_size (the kept count); passers_kept and usize (H, Q)
        int32 receive the threshold passers among the kept keys and in all, when given."""
        cp = _chunk_params(chunk_size, n_chunk, chunk_agg, passers_kept)
        a = self.args
        saved = a.usize
        a.usize = _ptr(usize)
        try:
            _check(lib().sta_decode_build_sets_chunk(ctypes.byref(a), ctypes.byref(cp), SCORES[select_score],
                                                     _ptr(scores), _stream(self.device)),
                   "sta_decode_build_sets_chunk")
        finally:
            a.usize = saved
        return self.out

    def attend(self, idx, newpos_k, newpos_q, set_size=None):
        """Attend alone over given sets (H, Q, k_max) int32 / fp32 and (H, Q) fp32 into out."""
        a = self.args
        saved = (a.idx, a.newpos_k, a.newpos_q, a.set_size)
        a.idx, a.newpos_k, a.newpos_q = _ptr(idx), _ptr(newpos_k), _ptr(newpos_q)
        a.set_size = _ptr(set_size)
        try:
            _check(lib().sta_decode_attend(ctypes.byref(a), _stream(self.device)), "sta_decode_attend")
        finally:
            a.idx, a.newpos_k, a.newpos_q, a.set_size = saved
        return self.out["out"]


def decode_attention(q, k, v, tau, inv_freq, q_pos0, pos_scale=1.0, rope_scale=1.0, sm_scale=None,
                     n_global=32, n_local=32, k_max=1024, pct_decode=100.0, causal=False, want_scores=False,
                     inv_freq_c=None, pos_scale_c=None, rope_scale_c=None, rule="shared", block_n=32):
    """Scores, selection and attend of Q queries (H, Q, D) over the cache k, v (Hkv, M, D).
    Returns a dict of device tensors: out (H, Q, D), idx (H, Q, k_max) int32 (sentinel m_i),
    newpos_k, newpos_q, set_size, with want_scores scores (H, Q, M), and under rule "pq" usize
    and overflow (H, Q)."""
    return DecodePlan(q, k, v, tau, inv_freq, q_pos0, pos_scale, rope_scale, sm_scale, n_global, n_local,
                      k_max, pct_decode, causal, want_scores, inv_freq_c, pos_scale_c, rope_scale_c,
                      rule, block_n).run()


class PerQueryPrefillPlan:
    """The per-query prefill (perquery.py:905-924, prefill_mode="perquery"): every position P of
    the N prompt tokens selects its own set over the keys [0, P] by the per-query rule and attends
    it.  Runs as the batched decode path with Q = M = N, q_pos0 = 0, over groups of heads so that
    the per-query score rows (heads x N x N fp32) stay bounded; outputs and one workspace are
    allocated once and run() allocates nothing.

    The prompt runs in chunks of query_chunk positions: chunk [i0, i1) is a decode batch of
    i1 - i0 queries at positions i0 .. over the cache prefix [0, i1), so a chunk's selection
    workgroups size their key store by i1 rather than N (two of them fit a CU where one of N keys
    did) and its score rows take (i1 - i0) x i1 floats per head.  A query's scores, set and output
    do not depend on the chunking.  query_chunk=None runs the prompt as one batch.

    Outputs: out (H, N, D) in the input dtype; set_size, usize (H, N) int32 and overflow (H, N)
    bool per query.  The per-launch idx / newpos_q buffers are reused (newpos_k is not written: the
    per-query rule's positions are the slot indices); a chunk's per-query outputs land in staging
    buffers and are copied into place on the same stream."""

    def __init__(self, q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                 sm_scale=None, n_global=32, n_local=32, k_max=4096, heads_per_group=None,
                 score_bytes_budget=2 << 30, query_chunk=2048):
        qh = _heads_view(q)
        kh = _heads_view(k.to(qh.device))
        vh = _heads_view(v.to(qh.device))
        H, N, D = qh.shape
        Hkv = kh.shape[0]
        G = H // Hkv
        dev = qh.device
        qc = N if query_chunk is None else max(1, min(int(query_chunk), N))
        chunks = [(i0, min(N, i0 + qc)) for i0 in range(0, N, qc)]
        if heads_per_group is None:
            # whole kv groups, as many as the score budget allows for the largest chunk
            per_head = qc * N * 4
            heads_per_group = max(G, (score_bytes_budget // per_head) // G * G)
        hg = min(H, heads_per_group)
        if hg % G:
            raise ValueError(f"heads_per_group={hg} must be a multiple of the GQA group {G}")
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        tau = tau.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if tau.numel() == 1 and H > 1:
            tau = tau.expand(H).contiguous()
        self.device = dev
        self.out = {
            "out": torch.empty((H, N, D), dtype=qh.dtype, device=dev),
            "set_size": torch.empty((H, N), dtype=torch.int32, device=dev),
            "usize": torch.empty((H, N), dtype=torch.int32, device=dev),
            "overflow": torch.empty((H, N), dtype=torch.bool, device=dev),
        }
        self._idx = torch.empty((hg, qc, k_max), dtype=torch.int32, device=dev)
        self._npq = torch.empty((hg, qc), dtype=torch.float32, device=dev)
        whole = len(chunks) == 1
        if not whole:   # a chunk's (heads, queries) outputs are not a contiguous slice of (H, N)
            self._stage = {"out": torch.empty((hg, qc, D), dtype=qh.dtype, device=dev),
                           "set_size": torch.empty((hg, qc), dtype=torch.int32, device=dev),
                           "usize": torch.empty((hg, qc), dtype=torch.int32, device=dev),
                           "overflow": torch.empty((hg, qc), dtype=torch.bool, device=dev)}
        self._keep = (qh, kh, vh, tau)
        self.plans = []
        self._spans = []       # (h0, h1, i0, i1) of each plan
        ws = None
        for i0, i1 in chunks:
            for h0 in range(0, H, hg):
                h1 = min(H, h0 + hg)
                p = DecodePlan.__new__(DecodePlan)
                p.device = dev
                p._events = None
                a = p.args = DecodeArgsC()
                a.q = _ptr(qh[h0:h1, i0:])
                a.k, a.v = _ptr(kh[h0 // G:h1 // G]), _ptr(vh[h0 // G:h1 // G])
                a.q_head_stride, a.q_tok_stride = qh.stride(0), qh.stride(1)
                a.k_head_stride, a.k_tok_stride = kh.stride(0), kh.stride(1)
                a.v_head_stride, a.v_tok_stride = vh.stride(0), vh.stride(1)
                a.dtype = DTYPES[qh.dtype]
                a.H, a.Hkv, a.Q, a.M, a.D = h1 - h0, (h1 - h0) // G, i1 - i0, i1, D
                a.tau = _ptr(tau[h0:h1])
                a.inv_freq_a = _ptr(inv_freq_a)
                a.inv_freq_c = _ptr(inv_freq_c)
                a.pos_scale_a, a.rope_scale_a, a.sm_scale = float(pos_scale_a), float(rope_scale_a), float(sm_scale)
                a.pos_scale_c, a.rope_scale_c = 1.0, 1.0
                a.q_pos0, a.n_global, a.n_local, a.k_max = i0, int(n_global), int(n_local), int(k_max)
                a.pct_decode, a.causal, a.rule = 100.0, 0, RULES["pq"]
                dst = self.out if whole else self._stage
                a.out = _ptr(dst["out"][h0:h1] if whole else dst["out"])
                a.idx, a.newpos_k, a.newpos_q = _ptr(self._idx), None, _ptr(self._npq)
                for name in ("set_size", "usize", "overflow"):
                    setattr(a, name, _ptr(dst[name][h0:h1] if whole else dst[name]))
                n = lib().sta_decode_workspace_size(ctypes.byref(a))
                if n == 0:
                    _check(-1, "sta_decode_workspace_size")
                if ws is None or ws.numel() < n:
                    ws = torch.empty(n, dtype=torch.uint8, device=dev)
                self.plans.append(p)
                self._spans.append((h0, h1, i0, i1))
        for p in self.plans:
            p.args.workspace, p.args.workspace_bytes = _ptr(ws), ws.numel()
        self.workspace = ws
        self._keep = self._keep + (inv_freq_a, inv_freq_c)

    def run(self, events=None):
        """events: None or one list of 4 recorded events per head group (len(self.plans)),
        marking that group's scores, selection and attend."""
        staged = hasattr(self, "_stage")
        for i, p in enumerate(self.plans):
            p.args.stage_events = None
            if events is not None:
                p._events = (ctypes.c_void_p * 4)(*[e.cuda_event for e in events[i]])
                p.args.stage_events = ctypes.cast(p._events, ctypes.c_void_p)
            _check(lib().sta_decode_attention(ctypes.byref(p.args), _stream(self.device)), "sta_decode_attention")
            if staged:
                # the launch wrote (heads, queries[, D]) contiguously from the staging buffers' start
                h0, h1, i0, i1 = self._spans[i]
                for name, t in self._stage.items():
                    dst = self.out[name][h0:h1, i0:i1]
                    dst.copy_(t.view(-1)[:dst.numel()].view(dst.shape))
        return self.out


def perquery_prefill_attention(q, k, v, tau, inv_freq_a, inv_freq_c, pos_scale_a=1.0, rope_scale_a=1.0,
                               sm_scale=None, n_global=32, n_local=32, k_max=4096, heads_per_group=None,
                               query_chunk=2048):
    """Per-query prefill of (1, H, N, D) inputs; returns the PerQueryPrefillPlan's outputs."""
    ia = inv_freq_a.to(device=q.device, dtype=torch.float32).contiguous()
    ic = inv_freq_c.to(device=q.device, dtype=torch.float32).contiguous()
    return PerQueryPrefillPlan(q, k, v, tau, ia, ic, pos_scale_a, rope_scale_a, sm_scale, n_global, n_local,
                               k_max, heads_per_group, query_chunk=query_chunk).run()
