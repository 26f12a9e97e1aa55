"""RoPE for prefill: table checks and the fw_rotary launch.

Restates the reference's prepare_rotary contract
(flywheel_tpu/softmax_attention/rotary.py:27-167) and the rotation of
rotate_tile (rotary.py:170-215): tables (seqlen_ro, head_dim / 2) in q's dtype
or float32, full-head rotation only, f32 arithmetic rounded once to bf16, K at
positions 0..len_k-1 and Q at len_k-len_q..len_k-1 of each sequence.  Q is
rotated by the prefill kernels as they load it (the fused path); K, when it is
rotated, goes to a fresh buffer (fw_rotary) which the kernel then reads.  q and
k themselves are never modified.
"""

import torch

from . import _native as N
from .inputs import as_tensor

ROTARY_DIM_MULTIPLE = 16


def check_tables(cos, sin, *, head_dim, dtype, rotate_k, interleaved, kv_len_bound):
    """`rotary.py:56-97`: (cos, sin) checked, or None without tables."""
    if type(interleaved) is not bool:
        raise ValueError("rotary_interleaved must be a static bool.")
    if type(rotate_k) is not bool:
        raise ValueError("rotary_k must be a static bool.")
    if (cos is None) != (sin is None):
        raise ValueError("rotary_cos and rotary_sin must be provided together.")
    if cos is None and not rotate_k:
        raise ValueError("rotary_k=False needs rotary_cos and rotary_sin.")
    if cos is None:
        return None
    cos, sin = as_tensor(cos), as_tensor(sin)
    if cos.ndim != 2 or tuple(sin.shape) != tuple(cos.shape):
        raise ValueError("rotary_cos and rotary_sin must have the same 2-D shape.")
    rotary_dim = 2 * cos.shape[1]
    if rotary_dim == 0 or rotary_dim % ROTARY_DIM_MULTIPLE:
        raise ValueError(f"rotary_dim must be positive and divisible by {ROTARY_DIM_MULTIPLE}.")
    if rotary_dim != head_dim:
        raise ValueError(f"rotary_dim ({rotary_dim}) must equal head_dim ({head_dim});"
                         " partial rotary is not supported.")
    if cos.dtype != sin.dtype or cos.dtype not in (dtype, torch.float32):
        raise ValueError("rotary_cos and rotary_sin must share Q's dtype or be float32.")
    if cos.shape[0] < kv_len_bound:
        raise ValueError("rotary table is shorter than the KV sequence bound.")
    return cos, sin


def check_packed_lengths(cu_q, k_lens, table_rows):
    """`rotary.py:122-147`: 0 <= len_q <= len_k <= table rows.  Checked here
    when the lengths are host tensors; device-resident lengths are the caller's
    contract (positions are then clamped into the table)."""
    if cu_q.is_cuda or k_lens.is_cuda:
        return
    q_lens = torch.diff(cu_q.to(torch.int64))
    k_lens = k_lens.to(torch.int64)
    if not bool(((q_lens >= 0) & (k_lens >= q_lens) & (k_lens <= table_rows)).all()):
        raise ValueError("RoPE requires 0 <= len_q <= len_k <= rotary table length.")


def set_q_rotary(p, tables, interleaved, device):
    """Fills the fused Q-RoPE fields of a PrefillParams (the prefill kernels
    rotate Q as they load it, at position i + kv_len - q_len of each row).
    Returns the device tables, to be kept alive until the launch is queued."""
    if tables is None:
        return None
    cos = tables[0].to(device).contiguous()
    sin = tables[1].to(device).contiguous()
    p.rotary_cos, p.rotary_sin = N.ptr(cos), N.ptr(sin)
    p.rotary_rows = cos.shape[0]
    p.rotary_f32 = int(cos.dtype == torch.float32)
    p.rotary_interleaved = int(interleaved)
    return cos, sin


def rotate(x, tables, interleaved, *, strides, batch_rows, nheads, ntokens, pos_offset=0,
           cu=None, kv_cu=None, kv_lens=None, num_active=None):
    """A rotated copy of the contiguous bf16 tensor x (same shape and strides).

    Element (b, h, t, :) sits at b*strides[0] + h*strides[1] + t*strides[2];
    its position is t + pos_offset, or for packed rows (cu given) its offset in
    its sequence plus kv_len - q_len (kv_len from kv_lens or kv_cu; 0 without
    either).
    """
    cos, sin = tables
    device = x.device
    cos = cos.to(device).contiguous()
    sin = sin.to(device).contiguous()
    y = torch.empty_like(x)
    p = N.RotaryParams()
    p.x, p.y, p.cos_table, p.sin_table = N.ptr(x), N.ptr(y), N.ptr(cos), N.ptr(sin)
    p.cu_seqlens, p.kv_cu, p.kv_lens = N.ptr(cu), N.ptr(kv_cu), N.ptr(kv_lens)
    p.num_active = N.ptr(num_active)
    p.x_stride_b, p.x_stride_h, p.x_stride_t = strides
    p.y_stride_b, p.y_stride_h, p.y_stride_t = strides
    p.batch_rows, p.nheads, p.ntokens = batch_rows, nheads, ntokens
    p.head_dim = 2 * cos.shape[1]
    p.table_rows = cos.shape[0]
    p.table_f32 = int(cos.dtype == torch.float32)
    p.interleaved = int(interleaved)
    p.pos_offset = pos_offset
    p.nseq = 0 if cu is None else cu.shape[0] - 1
    N.check(N.lib().fw_rotary(p, N.stream_of(x)))
    return y
