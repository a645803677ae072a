"""CPU checks of the C-ABI library: it loads, exports every entry point include/sta.h declares,
and rejects bad arguments with the documented error codes.  No call here reaches a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sta.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(sta_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "sta_shared_attention" in names and "sta_build_sets" in names
    assert len(names) >= 7


def test_library_exports_every_declared_symbol():
    import _sta_native as native
    lib = native.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert sorted(native.EXPORTS) == _declared()
    assert lib.sta_abi_version() == 5


def _args(**kw):
    import _sta_native as native
    a = native.ShareArgs()
    a.dtype, a.H, a.Hkv, a.N, a.D, a.tile, a.k_max = 1, 32, 32, 12288, 128, 64, 2048
    a.start_pct, a.n_global, a.n_local = 30, 32, 32
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_workspace_size_matches_layout():
    import _sta_native as native
    lib = native.lib()
    a = _args()
    n = lib.sta_shared_workspace_size(ctypes.byref(a))
    nt = 12288 // 64
    # q / k fragments (hi + lo bf16), per-row (||hi||, ||lo||) and per-head maxima of those, then
    # the screened pass 1's row maxima and per-workgroup flags
    screen = 32 * 12288 * 4 + 32 * (12288 // 256 + 1) * 4
    # the fp6 correction operands: e2m3 planes of [hi | x - hi] (1.5 D bytes per row), a scale
    # dword per lane (8 bytes per row), per row the two quantisation-error norms, per head their
    # maxima
    fp6 = 32 * 12288 * 128 * 3 // 2 + 32 * 12288 * 8 + 32 * 12288 * 8 + 32 * 8
    q = 32 * 12288 * 128 * 4 + 32 * 12288 * 8 + 32 * 8 + screen + fp6
    k = 32 * 12288 * 128 * 4 + 32 * 12288 * 8 + 32 * 8 + screen + fp6
    votes = 32 * nt * 12288             # byte votes, one row per tile
    trig = 12288 * (128 // 2) * 8       # the K rotation's (cos, sin) per key row (float2 per pair)
    assert n >= q + k + trig + votes and n < q + k + trig + votes + 4096


@pytest.mark.parametrize("field,value,code", [
    ("D", 96, -2), ("tile", 48, -2), ("Hkv", 5, -1), ("k_max", 0, -1), ("N", 0, -1),
    ("dtype", 7, -1), ("q_pos_base", -1, -1),
])
def test_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _args(**{field: value})
    assert lib.sta_shared_workspace_size(ctypes.byref(a)) == 0
    assert lib.sta_shared_attention(ctypes.byref(a), None) == code
    assert len(lib.sta_last_error()) > 0


def test_pq_long_rows_are_sized():
    """Rows past the selection's LDS (N = 100000) are supported: their rank keys are read from
    the workspace rows."""
    import _sta_native as native
    assert native.lib().sta_pq_workspace_size(ctypes.byref(_pq_args(N=100000))) > 0


def test_missing_pointers_are_rejected_before_any_launch():
    import _sta_native as native
    lib = native.lib()
    a = _args()
    assert lib.sta_shared_attention(ctypes.byref(a), None) == -1       # q is NULL
    assert b"NULL" in lib.sta_last_error()
    assert lib.sta_shared_attention(None, None) == -1


def test_product_path_refuses_cpu_tensors():
    import torch
    import shared_selection_triton_exact_2 as st
    q = torch.zeros(1, 2, 64, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        st.shared_pi_attention(q, q, q, torch.ones(2), torch.ones(32), tile=64)


def test_yarn_geometry_matches_transformers():
    """The YaRN frequencies of config 2 against transformers' own initialiser."""
    import torch
    from synthetic import yarn_inv_freq
    tr = pytest.importorskip("transformers")
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, head_dim=128,
                      max_position_embeddings=32768,
                      rope_parameters={"rope_type": "yarn", "rope_theta": 500000.0, "factor": 4.0,
                                       "original_max_position_embeddings": 8192,
                                       "beta_fast": 32.0, "beta_slow": 1.0})
    ref_f, ref_m = ROPE_INIT_FUNCTIONS["yarn"](cfg, "cpu")
    f, m = yarn_inv_freq(128, 500000.0, 4.0, 8192, 32.0, 1.0)
    assert torch.equal(f, ref_f.float())
    assert abs(m - ref_m) < 1e-12
    assert abs(m - 1.1386294361119891) < 1e-12


# ------------------------------------------------------------------------------------------------
# per-query variants and DCA: argument validation, no GPU
# ------------------------------------------------------------------------------------------------
def _pq_args(**kw):
    import _sta_native as native
    a = native.PqArgs()
    a.dtype, a.H, a.Hkv, a.N, a.D, a.tile, a.k_max = 1, 32, 32, 16384, 128, 32, 2048
    a.n_global, a.n_local, a.select_score = 32, 32, 2
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("tile", 64, -1), ("D", 80, -2), ("select_score", 5, -1), ("k_max", 60000, -2), ("k_max", 0, -1),
])
def test_pq_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _pq_args(**{field: value})
    assert lib.sta_pq_workspace_size(ctypes.byref(a)) == 0
    assert lib.sta_pq_attention(ctypes.byref(a), None) == code
    assert len(lib.sta_last_error()) > 0


def test_pq_forced_set_must_fit_k_max():
    """perquery.py:474-476: n_global + n_local + tile - 1 <= k_max, checked before any launch."""
    import _sta_native as native
    lib = native.lib()
    a = _pq_args(k_max=64)
    buf = ctypes.create_string_buffer(64)
    a.q = a.k = a.v = ctypes.cast(buf, ctypes.c_void_p)  # non-NULL, 16-byte aligned host memory
    a.q_tok_stride = a.k_tok_stride = a.v_tok_stride = 128
    a.tau = a.inv_freq_a = a.inv_freq_c = a.out = ctypes.cast(buf, ctypes.c_void_p)
    if ctypes.addressof(buf) % 16:
        pytest.skip("host buffer not 16-byte aligned")
    assert lib.sta_pq_attention(ctypes.byref(a), None) == -1
    assert b"forced set" in lib.sta_last_error()


def _stream_args(**kw):
    import _sta_native as native
    a = native.StreamArgsC()
    a.dtype, a.H, a.Hkv, a.N, a.D, a.tile, a.block_n = 1, 32, 32, 16384, 128, 32, 32
    a.n_global, a.n_local, a.pos_advance, a.use_skip = 32, 32, 0, 1
    a.sm_scale = 128 ** -0.5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("tile", 64, -1), ("q_pos_base", 3, -1), ("block_n", 16, -1), ("block_n", 128, -2),
    ("pos_advance", 2, -1), ("D", 96, -2), ("sm_scale", 0.0, -1), ("sm_scale", -0.1, -1),
    ("sm_scale", float("inf"), -1),
])
def test_pqstream_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _stream_args(**{field: value})
    assert lib.sta_pqstream_workspace_size(ctypes.byref(a)) == 0
    assert lib.sta_pqstream_attention(ctypes.byref(a), None) == code


def test_pqstream_workspace_size_matches_layout():
    import _sta_native as native
    lib = native.lib()
    n = lib.sta_pqstream_workspace_size(ctypes.byref(_stream_args()))
    N, H, D = 16384, 32, 128
    frags = 2 * (H * N * D * 4 + H * N * 8 + H * 8 + H * N * 4 + H * (N // 256 + 1) * 4)   # q/k fragments
    need = frags + H * (N // 32) * N * 4 + H * N * D * 2   # + keep bits, K~
    need += N * (D // 2) * 8                               # + the K rotation's (cos, sin) table
    assert need <= n < need + 8192


def _dca_args(**kw):
    import _sta_native as native
    a = native.DcaArgsC()
    a.dtype, a.H, a.Hkv, a.N, a.D = 1, 32, 32, 65536, 128
    a.chunk_size, a.pretrain_len, a.local_window, a.scale = 4096, 4096, 512, 128 ** -0.5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("local_window", 0, -1), ("local_window", 4096, -1), ("chunk_size", 4100, -2), ("D", 32, -2),
    ("pretrain_len", 0, -1), ("scale", 0.0, -1), ("scale", -0.1, -1), ("scale", float("inf"), -1),
])
def test_dca_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _dca_args(**{field: value})
    assert lib.sta_dca_workspace_size(ctypes.byref(a)) == 0
    assert lib.sta_dca_attention(ctypes.byref(a), None) == code


def test_dca_workspace_size_matches_layout():
    import _sta_native as native
    lib = native.lib()
    n = lib.sta_dca_workspace_size(ctypes.byref(_dca_args()))
    need = 32 * 65536 * 128 * 2 * 4          # rotated keys + three query variants, bf16
    need += (4096 + 1) * 64 * 8              # (cos, sin) float pairs for positions 0 .. chunk_size
    assert need <= n < need + 4096


def _decode_args(**kw):
    import _sta_native as native
    a = native.DecodeArgsC()
    a.dtype, a.H, a.Hkv, a.Q, a.M, a.D = 1, 32, 8, 1, 12288, 128
    a.q_pos0, a.n_global, a.n_local, a.k_max = 12287, 32, 32, 2048
    a.pos_scale_a, a.rope_scale_a, a.sm_scale, a.pct_decode = 1.0 / 3.0, 1.0, 0.0884, 100.0
    a.pos_scale_c, a.rope_scale_c = 1.0 / 3.0, 1.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("D", 96, -2), ("M", 0, -1), ("Q", 0, -1), ("q_pos0", 12288, -1), ("k_max", 0, -2),
    ("k_max", 70000, -2), ("rule", 3, -1), ("Hkv", 5, -1),
    ("n_local", -1, -2), ("dtype", 7, -1),
])
def test_decode_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _decode_args(**{field: value})
    assert lib.sta_decode_attention(ctypes.byref(a), None) == code
    assert lib.sta_decode_build_sets(ctypes.byref(a), None, None) == code


def test_decode_scores_take_any_position_and_need_a_workspace():
    import _sta_native as native
    lib = native.lib()
    a = _decode_args(q_pos0=50000)       # the scores alone: any query position
    assert lib.sta_decode_workspace_size(ctypes.byref(a)) > 0
    assert lib.sta_decode_scores(ctypes.byref(a), None, None) == -4      # no workspace
    assert lib.sta_decode_attention(ctypes.byref(a), None) == -1         # q_pos0 + Q > M


def test_decode_workspace_size_matches_layout():
    import _sta_native as native
    lib = native.lib()
    n = lib.sta_decode_workspace_size(ctypes.byref(_decode_args()))
    need = 32 * 128 * 4 + 32 * 12288 * 4 + 32 * 4 + 32 * 32 * 130 * 4    # qrot, scores, sizes, splits
    assert need <= n < need + 5 * 256
    # past the LDS key store (M > 35840) the selection keeps its keys in the workspace
    n2 = lib.sta_decode_workspace_size(ctypes.byref(_decode_args(M=40000, q_pos0=39999)))
    need2 = 32 * 128 * 4 + 32 * 40000 * 4 + 32 * 1024 * 40 * 4 + 32 * 4 + 32 * 32 * 130 * 4
    assert need2 <= n2 < need2 + 5 * 256


def _dca_decode_args(**kw):
    import _sta_native as native
    a = native.DcaDecodeArgsC()
    a.dtype, a.H, a.Hkv, a.M, a.D = 1, 32, 8, 5000, 128
    a.chunk_size, a.local_window, a.mscale, a.scale = 3072, 512, 1.0, 0.088
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_dca_decode_workspace_size():
    import _sta_native as native
    lib = native.lib()
    n = lib.sta_dca_decode_workspace_size(ctypes.byref(_dca_decode_args()))
    nb = (5000 + 255) // 256
    need = 32 * 3 * 128 * 4 + 32 * 5000 * 4 + 2 * 32 * nb * 4 + 32 * nb * 128 * 4
    assert need <= n < need + 5 * 256


@pytest.mark.parametrize("field,value,code", [
    ("D", 96, -2), ("Hkv", 5, -1), ("M", 0, -1), ("dtype", 7, -1), ("local_window", 0, -1),
    ("local_window", 3072, -1), ("mscale", 0.0, -1), ("mscale", float("inf"), -1), ("Hkv", 1, -2),
])
def test_dca_decode_invalid_arguments_are_rejected(field, value, code):
    import _sta_native as native
    lib = native.lib()
    a = _dca_decode_args(**{field: value})
    assert lib.sta_dca_decode_workspace_size(ctypes.byref(a)) == 0
    assert lib.sta_dca_decode(ctypes.byref(a), None) == code
    assert len(lib.sta_last_error()) > 0


def test_dca_rotate_keys_rejects_bad_arguments_before_any_launch():
    import _sta_native as native
    lib = native.lib()
    a = native.DcaRotateArgsC()
    a.dtype, a.heads, a.N, a.D, a.pos0 = 1, 8, 4, 128, 100
    a.chunk_size, a.local_window, a.mscale = 3072, 512, 1.0
    assert lib.sta_dca_rotate_keys(ctypes.byref(a), None) == -1            # inv_freq is NULL
    a.D = 80
    assert lib.sta_dca_rotate_keys(ctypes.byref(a), None) == -2
    a.D, a.mscale = 128, -1.0
    assert lib.sta_dca_rotate_keys(ctypes.byref(a), None) == -1
    assert lib.sta_dca_rotate_keys(None, None) == -1
