"""Pins oracle/rotary.py with closed forms and brute force (none re-types the
oracle's formula): identity at zero angle, complex multiplication, norm
preservation, interleaved = permuted halves, RoPE's relative-position score
property, and a loop restatement of the packed positions
(flywheel_tpu/softmax_attention/rotary.py:99-167, tests/softmax_attention/
util.py:103-146 for the reference test's own restatement)."""

import numpy as np
import pytest

from oracle import dtypes as T
from oracle import rotary as RO


def _rand(rng, shape):
    return T.bf16(rng.standard_normal(shape, dtype=np.float32))


@pytest.mark.parametrize("interleaved", [False, True])
def test_zero_angle_is_identity(interleaved):
    rng = np.random.default_rng(0)
    x = _rand(rng, (3, 40, 128))
    cos, sin = np.ones((50, 64), np.float32), np.zeros((50, 64), np.float32)
    y = RO.rotate(x, cos, sin, np.arange(40) + 5, interleaved)
    np.testing.assert_array_equal(y, x)


@pytest.mark.parametrize("d", [64, 96, 128, 192, 512])
def test_halves_pairing_is_complex_multiplication(d):
    rng = np.random.default_rng(1)
    hd = d // 2
    x = _rand(rng, (2, 33, d))
    ang = rng.random((40, hd)) * 2 * np.pi
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    pos = rng.integers(0, 40, 33)
    z = (x[..., :hd].astype(np.float64) + 1j * x[..., hd:]) * (
        cos[pos].astype(np.float64) + 1j * sin[pos])
    y = RO.rotate_f32(x, cos, sin, pos, False)
    np.testing.assert_allclose(y[..., :hd], z.real, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(y[..., hd:], z.imag, atol=2e-6, rtol=1e-5)
    # |rotated pair| == |pair| (rotation).
    np.testing.assert_allclose(np.hypot(y[..., :hd], y[..., hd:]),
                               np.hypot(x[..., :hd], x[..., hd:]), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("d", [64, 96, 128, 192, 512])
def test_interleaved_is_permuted_halves(d):
    rng = np.random.default_rng(2)
    hd = d // 2
    x = _rand(rng, (4, 17, d))
    ang = rng.random((30, hd)) * 2 * np.pi
    cos, sin = T.bf16(np.cos(ang)), T.bf16(np.sin(ang))
    pos = rng.integers(0, 30, 17)
    # dim 2i of the interleaved head is dim i of the halves head, 2i+1 is i+d/2.
    perm = np.empty(d, np.int64)
    perm[0::2], perm[1::2] = np.arange(hd), np.arange(hd) + hd
    yi = RO.rotate(x[..., perm], cos, sin, pos, True)
    yh = RO.rotate(x, cos, sin, pos, False)
    np.testing.assert_array_equal(yi, yh[..., perm])


@pytest.mark.parametrize("interleaved", [False, True])
def test_scores_depend_on_relative_position(interleaved):
    """<rope(q, m), rope(k, n)> is a function of m - n only."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    cos, sin = RO.rope_tables(200, 128)
    qs = RO.rotate_f32(np.broadcast_to(q, (200, 128)), cos, sin, np.arange(200), interleaved)
    ks = RO.rotate_f32(np.broadcast_to(k, (200, 128)), cos, sin, np.arange(200), interleaved)
    s = qs.astype(np.float64) @ ks.astype(np.float64).T
    for delta in (0, 3, 57):
        diag = np.diagonal(s, offset=-delta)
        np.testing.assert_allclose(diag, diag[0], atol=5e-4 * np.abs(diag).max() + 1e-4)
    assert abs(s[10, 10] - float(q.astype(np.float64) @ k)) < 1e-3


def test_packed_positions_match_loop():
    rng = np.random.default_rng(4)
    for _ in range(50):
        lens = rng.integers(0, 7, rng.integers(1, 6))
        cu = np.concatenate([[0], np.cumsum(lens)])
        total = int(cu[-1]) + int(rng.integers(0, 4))
        offs = rng.integers(0, 20, lens.shape[0])
        want = np.zeros(total, np.int64)
        for s in range(lens.shape[0]):
            for j in range(lens[s]):
                want[cu[s] + j] = offs[s] + j
        np.testing.assert_array_equal(RO.packed_positions(cu, total, offs), want)


def test_dense_positions_are_bottom_right():
    qp, kp = RO.dense_positions(3, 10)
    np.testing.assert_array_equal(qp, [7, 8, 9])
    np.testing.assert_array_equal(kp, np.arange(10))
    # One packed sequence places its rows like the dense layout.
    np.testing.assert_array_equal(RO.packed_positions([0, 3], 3, [7]), qp)
