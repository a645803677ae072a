"""CPU: the attend-side sin/cos argument reduction (csrc/sta_device.h, fast_sincos).

The gather, decode-attend and stream kernels rotate keys / queries at the reference's fp32 angle
x = fl(pos * inv_freq) (shared_selection_triton_exact_2.py:199-207) and reduce it to revolutions,
t = x / (2 pi) - k, with 1 / (2 pi) split into two fp32 terms kH + kL:
    k = rint(fl(x * kH)),  t = fma(x, kH, -k),  t = fma(x, kL, t).
The constants are read from the header; the reduction is restated in float64 (every fma of two
fp32 operands is exact in float64 before its single fp32 rounding) and checked against the
float64 reduction of x itself.  The bound is 4e-8 revolutions for |x| < 5000 and 6e-8 up to
|x| = 65536, the largest angle the configurations reach (YaRN and DCA at position scale 1 over
32k and 64k positions): there fl(x * kH) can round k to the neighbouring integer, |t| then
exceeds 0.5 slightly and its ulp doubles.
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


def _worst(xs, kh, kl):
    worst = 0.0
    for x in xs:
        k = np.float32(np.rint(np.float32(x * kh)))
        t = _fma32(x, kh, -k)
        t = _fma32(x, kl, t)
        # k = rint(fl(x kH)) may pick the neighbouring integer when x kH lies within the product's
        # rounding error of a half-integer, by less than an ulp of x kH (2^-10 below 16384
        # revolutions); the hardware sine / cosine are periodic in t, so only the error counts
        assert abs(t) <= 0.5 + 2.0 ** -10
        ref = np.float64(x) / (2.0 * np.pi)
        d = (np.float64(t) - (ref - np.rint(ref)) + 0.5) % 1.0 - 0.5
        worst = max(worst, abs(d))
    return worst


def test_reduction_error_below_4e8_revolutions():
    kh, kl = _consts()
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-5000, 5000, 20000), rng.uniform(-1, 1, 2000),
                         np.float32(np.arange(0, 4096) * np.float32(0.3333333))]).astype(np.float32)
    worst = _worst(xs, kh, kl)
    assert worst < 4e-8, worst


def test_reduction_error_below_6e8_revolutions_to_65536():
    kh, kl = _consts()
    rng = np.random.default_rng(1)
    # uniform samples over the whole range, the integer positions of the largest frequency
    # (inv_freq[0] = 1 at position scale 1) and the points where x * kH sits closest to a
    # half-integer, which are the ones where k can round the wrong way
    pos = np.arange(0, 65537, dtype=np.float32)
    frac = np.abs((pos.astype(np.float64) / (2 * np.pi)) % 1.0 - 0.5)
    near_half = pos[np.argsort(frac)[:4000]]
    xs = np.concatenate([rng.uniform(-65536, 65536, 30000), pos[::7], near_half,
                         -near_half]).astype(np.float32)
    worst = _worst(xs, kh, kl)
    assert worst < 6e-8, worst
