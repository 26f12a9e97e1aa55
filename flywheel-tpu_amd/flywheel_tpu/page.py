"""write_kv_cache_pages: host-sliced copy of new K/V rows into the merged
cache (reference flywheel_tpu/softmax_attention/page.py:32-73)."""

import torch

from . import _native as N
from .inputs import as_tensor
from .kv_layout import check_merged_kv_dtype, merged_cache_heads


def write_kv_cache_pages(k, v, kv_cache, slices, num_slices, *, interpret=False):
    """Copy new K/V rows into the merged interleaved cache, in place; returns
    the cache.

    k and v are (T, H, D) and kv_cache (P, S, merged_cache_heads(H), D) of one
    dtype.  slices is int32 (3, n) and num_slices int32 (1,): column
    j < num_slices[0] is (cache_row_start, new_row_start, length) over the flat
    (P * S) row view and k / v rows.
    """
    del interpret
    k, v, kv_cache = as_tensor(k), as_tensor(v), as_tensor(kv_cache)
    _, nheads_k, head_dim = k.shape
    check_merged_kv_dtype(kv_cache.dtype)
    if k.dtype != kv_cache.dtype or v.dtype != kv_cache.dtype:
        raise NotImplementedError(
            f"k, v and the cache must share one dtype; got {k.dtype}, {v.dtype}, {kv_cache.dtype}."
        )
    if tuple(v.shape) != tuple(k.shape) or (kv_cache.shape[2], kv_cache.shape[3]) != (
        merged_cache_heads(nheads_k, kv_cache.dtype), head_dim):
        raise ValueError(
            "k and v must be (T, H, D) of a (P, S, merged_cache_heads(H), D) cache; got"
            f" {tuple(k.shape)=}, {tuple(v.shape)=}, {tuple(kv_cache.shape)=}."
        )
    if head_dim % 128:
        raise ValueError(f"head_dim must be a multiple of 128; got {head_dim}.")
    slices = as_tensor(slices)
    if slices.ndim != 2 or slices.shape[0] != 3:
        raise ValueError(f"slices must be int32 (3, n); got {tuple(slices.shape)}.")
    N.require_device(k, v, kv_cache)
    dev = kv_cache.device
    sl = slices.to(device=dev, dtype=torch.int32).contiguous()
    ns = as_tensor(num_slices).reshape(-1)[:1].to(device=dev, dtype=torch.int32)
    k, v = k.contiguous(), v.contiguous()
    N.check(N.lib().fw_write_kv_cache_pages(
        N.ptr(k), N.ptr(v), N.ptr(kv_cache), N.ptr(sl), sl.shape[1], N.ptr(ns), k.shape[0],
        nheads_k, head_dim, kv_cache.shape[0] * kv_cache.shape[1], N.KV_DTYPES[kv_cache.dtype],
        N.stream_of(kv_cache)))
    return kv_cache
