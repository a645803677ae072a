"""Reference e2m3 (OCP MX fp6) block encoding of the fp6 correction operands, for the tests.

Mirrors csrc/sta_fp6.h and the RoPE pre-kernel's fp6 layout (csrc/sta_score.hip): each row's
vector [hi | x - hi] is cut into 32-element blocks; block b gets the E8M0 exponent e = the
smallest with max|x| <= 7.5 * 2^e (clamped to [-126, 127]) and its elements are rounded to
nearest even on the e2m3 grid of x / 2^e (steps 1/8 below 2, 1/4 in [2, 4), 1/2 in [4, 7.5]).
"""
import numpy as np

# the 32 non-negative e2m3 values by code: exponent 0 = subnormal m/8, exponent k = 2^(k-1)(1+m/8)
E2M3_VALUES = np.array([m / 8.0 for m in range(8)] +
                       [(1 + m / 8.0) * 2.0 ** (k - 1) for k in (1, 2, 3) for m in range(8)], np.float64)


def block_exp(bm):
    """E8M0 exponent per block maximum (float32 array)."""
    bm = np.asarray(bm, np.float32)
    u = bm.view(np.uint32).astype(np.int64)
    E = (u >> 23) & 0xFF
    e = np.where((u & 0x7FFFFF) <= 0x700000, E - 129, E - 128)
    e = np.where(E == 0, -126, e)
    e = np.clip(e, -126, 127)
    return np.where(bm > 0, e, 0).astype(np.int64)


def encode(x, e):
    """x (float32) under exponent e (broadcastable) -> (6-bit codes, represented values)."""
    x = np.asarray(x, np.float32).astype(np.float64)
    y = x * np.exp2(-np.asarray(e, np.float64))          # exact: a power-of-two scaling
    a = np.abs(y)
    step = np.where(a < 2, 0.125, np.where(a < 4, 0.25, 0.5))
    n = np.rint(a / step)                                  # numpy rint: round half to even
    code = np.where(a < 2, n, np.where(a < 4, n + 8, n + 16)).astype(np.int64)
    neg = np.signbit(y)
    code = np.where(neg, code | 32, code)
    val = np.where(neg, -1.0, 1.0) * n * step * np.exp2(np.asarray(e, np.float64))
    return code, val


def decode(code, e):
    code = np.asarray(code, np.int64)
    v = E2M3_VALUES[code & 31] * np.exp2(np.asarray(e, np.float64))
    return np.where(code & 32, -v, v)
