"""Merged paged-cache layout and cache writes on raw codes (oracle only).

Cache codes are uint16 (bf16) or uint8 (fp8).  A merged pool is
(num_pages, page_size, cache_heads, head_dim); a token row holds each KV head's
K row then its V row, [k0, v0, k1, v1, ...], and an fp8 pool pads an odd KV
head count with one zero head (`flywheel_tpu/softmax_attention/kv_layout.py:
39-46, 67-70`; `tests/softmax_attention/util.py:40-59`).
"""

import numpy as np


def merged_cache_heads(nheads_k, itemsize):
    """`kv_layout.py:67-70`: 2 * nheads_k, fp8 rounded up to an even count."""
    heads_per_word = 2 // itemsize
    return 2 * (-(-nheads_k // heads_per_word) * heads_per_word)


def merge_kv_heads(k, v):
    """(..., Hk, D) K and V codes -> (..., cache_heads, D) merged rows
    (`util.py:40-51`)."""
    k = np.asarray(k)
    v = np.asarray(v)
    *lead, hk, d = k.shape
    ch = merged_cache_heads(hk, k.dtype.itemsize)
    out = np.zeros((*lead, ch, d), k.dtype)
    out[..., 0 : 2 * hk : 2, :] = k
    out[..., 1 : 2 * hk : 2, :] = v
    return out


def split_kv_heads(kv, nheads_k):
    """merge_kv_heads' inverse (`util.py:54-59`)."""
    kv = np.asarray(kv)
    return kv[..., 0 : 2 * nheads_k : 2, :], kv[..., 1 : 2 * nheads_k : 2, :]


def append_to_pages(pool, k_new, v_new, cu_seqlens, cache_seqlens, table, num_active=None):
    """A copy of pool with each active request's new rows written after its
    cache_seqlens (`test_paged.py:80-95`, `kernels/kv_append.py:116-184`).

    k_new / v_new (T, Hk, D) codes packed by cu_seqlens; table (B, pages_per_seq).
    Token t of request r goes to page table[r, pos // P], slot pos % P with
    pos = cache_seqlens[r] + t, as a whole merged row (pad head zero).  Requests
    >= num_active and packed rows past cu_seqlens[num_active] are not written.
    """
    pool = np.array(pool, copy=True)
    page_size = pool.shape[1]
    cu = np.asarray(cu_seqlens)
    lens = np.asarray(cache_seqlens)
    table = np.asarray(table)
    batch = len(cu) - 1 if num_active is None else int(num_active)
    merged = merge_kv_heads(k_new, v_new)
    for r in range(batch):
        start, end = int(cu[r]), int(cu[r + 1])
        pos = int(lens[r]) + np.arange(end - start)
        pool[table[r, pos // page_size], pos % page_size] = merged[start:end]
    return pool


def write_kv_cache_pages(k, v, cache, slices, num_slices):
    """`flywheel_tpu/softmax_attention/page.py:32-73`: for column j <
    num_slices of slices (3, n) = (cache_row_start, new_row_start, length),
    copy merged rows [new_row_start, +length) of k/v into flat cache rows
    [cache_row_start, +length).  Returns the updated copy."""
    cache = np.array(cache, copy=True)
    flat = cache.reshape(-1, *cache.shape[2:])
    merged = merge_kv_heads(k, v)
    slices = np.asarray(slices)
    for j in range(int(num_slices)):
        c0, n0, length = (int(x) for x in slices[:, j])
        flat[c0 : c0 + length] = merged[n0 : n0 + length]
    return flat.reshape(cache.shape)


def gather_rows(pages, table, lengths=None):
    """Each request's logical (max_pages * P, ...) view of a paged pool
    (`test_prefill.py:527-533`)."""
    table = np.asarray(table)
    b, n = table.shape
    rows = pages[table.reshape(-1)].reshape(b, n * pages.shape[1], *pages.shape[2:])
    return rows
