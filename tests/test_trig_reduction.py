"""CPU: the attend-side sin/cos argument reduction (csrc/sta_device.h, fast_sincos).

The gather, decode-attend and stream kernels rotate keys / queries at the reference's fp32 angle
x = fl(pos * inv_freq) (shared_selection_triton_exact_2.py:199-207) and reduce it to revolutions,
t = x / (2 pi) - k, with 1 / (2 pi) split into two fp32 terms kH + kL:
    k = rint(fl(x * kH)),  t = fma(x, kH, -k),  t = fma(x, kL, t).
The constants are read from the header; the reduction is restated in float64 (every fma of two
fp32 operands is exact in float64 before its single fp32 rounding) and checked against the
float64 reduction of x itself over the angle range the configurations reach (|x| < 5000).
"""
import os
import re

import numpy as np

HDR = os.path.join(os.path.dirname(__file__), "..", "sparse-thresholded-attention_amd", "csrc", "sta_device.h")


def _consts():
    src = open(HDR).read()
    body = src[src.index("void fast_sincos"):]
    kh = float(re.search(r"kH = ([0-9.eE+-]+)f;", body).group(1))
    kl = float(re.search(r"kL = ([0-9.eE+-]+)f;", body).group(1))
    return np.float32(kh), np.float32(kl)


def _fma32(a, b, c):
    return np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def test_constants_split_one_over_two_pi():
    kh, kl = _consts()
    assert kh == np.float32(1.0 / (2.0 * np.pi))
    assert kl == np.float32(1.0 / (2.0 * np.pi) - np.float64(kh))
    assert abs(np.float64(kh) + np.float64(kl) - 1.0 / (2.0 * np.pi)) < 1e-16


def test_reduction_error_below_4e8_revolutions():
    kh, kl = _consts()
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-5000, 5000, 20000), rng.uniform(-1, 1, 2000),
                         np.float32(np.arange(0, 4096) * np.float32(0.3333333))]).astype(np.float32)
    worst = 0.0
    for x in xs:
        k = np.float32(np.rint(np.float32(x * kh)))
        t = _fma32(x, kh, -k)
        t = _fma32(x, kl, t)
        assert abs(t) <= 0.5 + 1e-6
        ref = np.float64(x) / (2.0 * np.pi)
        d = (np.float64(t) - (ref - np.rint(ref)) + 0.5) % 1.0 - 0.5
        worst = max(worst, abs(d))
    assert worst < 4e-8, worst
