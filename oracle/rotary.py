"""NumPy restatement of the reference's prefill RoPE (test infrastructure only).

Only tests, smoke() and the bench's CPU baseline use this module, as the
checker.  Follows flywheel_tpu/softmax_attention/rotary.py:99-167 (per-token
positions) and rotary.py:170-215 (rotate_tile: f32 rotation, one rounding).
Pinned in tests/test_oracle_rotary.py by: zero angle = identity, equality with
complex multiplication, norm preservation per pair, the interleaved pairing as
a permutation of the halves pairing, the relative-position property of RoPE
scores, and a loop restatement of the packed positions.
"""

import numpy as np

from oracle.dtypes import bf16


def dense_positions(seqlen_q, seqlen_k):
    """rotary.py:115-120: Q at seqlen_k - seqlen_q + i, K at i."""
    return np.arange(seqlen_q) + seqlen_k - seqlen_q, np.arange(seqlen_k)


def packed_positions(cu_seqlens, num_tokens, seq_offsets):
    """rotary.py:99-111: token t of sequence s (cu[s] <= t < cu[s+1], the last
    such s) sits at t - cu[s] + seq_offsets[s]; tokens past cu[-1] at 0."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    t = np.arange(num_tokens)
    seq = np.minimum(np.searchsorted(cu, t, side="right") - 1, cu.shape[0] - 2)
    seq = np.maximum(seq, 0)
    pos = t - cu[seq] + np.asarray(seq_offsets, dtype=np.int64)[seq]
    return np.where(t < cu[-1], pos, 0)


def rotate_f32(x, cos, sin, positions, interleaved):
    """rotary.py:170-215 before the final rounding.  x (..., T, D) f32 values,
    cos / sin (rows, D/2) f32 values, positions (T,).  Halves pairing: dims
    (i, i + D/2) with column i; interleaved: dims (2i, 2i+1) with column i.
    Each output is x_a * c - x_b * s or x_b * c + x_a * s in f32, each product
    and the sum rounded separately."""
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)[positions]
    s = np.asarray(sin, dtype=np.float32)[positions]
    half = x.shape[-1] // 2
    if interleaved:
        a, b = x[..., 0::2], x[..., 1::2]
    else:
        a, b = x[..., :half], x[..., half:]
    ya = (a * c).astype(np.float32) - (b * s).astype(np.float32)
    yb = (b * c).astype(np.float32) + (a * s).astype(np.float32)
    y = np.empty_like(x)
    if interleaved:
        y[..., 0::2], y[..., 1::2] = ya, yb
    else:
        y[..., :half], y[..., half:] = ya, yb
    return y


def rotate(x, cos, sin, positions, interleaved):
    """rotate_f32 rounded once to bf16 (values as f32)."""
    return bf16(rotate_f32(x, cos, sin, positions, interleaved))


def rope_tables(rows, head_dim, base=10000.0):
    """Standard RoPE tables cos / sin (rows, head_dim / 2) in f32: angle
    pos * base**(-2i / head_dim)."""
    inv = base ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
