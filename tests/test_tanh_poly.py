"""The softcap tanh polynomials of csrc/fw_common.h against numpy's tanh.

The kernels use x (d0 + d1 x^2) for tanh(x) when every |x| of a wave's tile is
at most kTanhPoly3Bound, and x (c0 + c1 x^2 + c2 x^4) when it is at most
kTanhPolyBound.  This reads the constants from the source and checks the stated
bound (abs error < 2.5e-7) with the kernels' float32 evaluation order, plus
oddness and the tanh'(0) = 1 slope, over each polynomial's whole range.
"""

import os
import re

import numpy as np

SRC = os.path.join(os.path.dirname(__file__), "..", "flywheel-tpu_amd", "csrc", "fw_common.h")


def _constants():
    text = open(SRC).read()
    bound = float(re.search(r"kTanhPolyBound = ([0-9.eE+-]+)f", text).group(1))
    c = [float(re.search(rf"kTanhC{i} = ([0-9.eE+-]+)f", text).group(1)) for i in range(3)]
    return np.float32(bound), [np.float32(v) for v in c]


def _poly(x, c):
    x = x.astype(np.float32)
    x2 = x * x
    p = (x2 * c[2] + c[1]).astype(np.float32)  # fmaf(x2, c2, c1)
    p = (x2 * p + c[0]).astype(np.float32)      # fmaf(x2, p, c0)
    return x * p


def _constants3():
    text = open(SRC).read()
    bound = float(re.search(r"kTanhPoly3Bound = ([0-9.eE+-]+)f", text).group(1))
    d = [float(re.search(rf"kTanhD{i} = ([0-9.eE+-]+)f", text).group(1)) for i in range(2)]
    return np.float32(bound), [np.float32(v) for v in d]


def _poly3(x, d):
    x = x.astype(np.float32)
    return x * (x * x * d[1] + d[0]).astype(np.float32)  # x * fmaf(x*x, d1, d0)


def test_tanh_poly3_error_bound():
    bound, d = _constants3()
    assert bound < _constants()[0]
    x = np.linspace(-bound, bound, 600001, dtype=np.float32)
    err = np.abs(_poly3(x, d).astype(np.float64) - np.tanh(x.astype(np.float64)))
    assert err.max() < 2.5e-7
    np.testing.assert_array_equal(_poly3(-x, d), -_poly3(x, d))


def test_tanh_poly_error_bound():
    bound, c = _constants()
    x = np.linspace(-bound, bound, 600001, dtype=np.float32)
    err = np.abs(_poly(x, c).astype(np.float64) - np.tanh(x.astype(np.float64)))
    assert err.max() < 2.5e-7


def test_tanh_poly_odd_and_slope():
    bound, c = _constants()
    x = np.linspace(0, bound, 1001, dtype=np.float32)
    np.testing.assert_array_equal(_poly(-x, c), -_poly(x, c))
    assert abs(float(c[0]) - 1.0) < 1e-5  # tanh'(0) = 1
    assert _poly(np.zeros(1, np.float32), c)[0] == 0.0
