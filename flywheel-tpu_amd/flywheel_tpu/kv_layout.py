"""Merged paged-cache layout (reference flywheel_tpu/softmax_attention/
kv_layout.py:39-95): a token row is [k0, v0, k1, v1, ...]; an fp8 pool pads an
odd KV head count with one zero head."""

import torch

# Values the reference exports for its callers (config.py:40, :89; core/tpu.py:18):
# pages here need only be a multiple of 16 (the kernels walk 16-key sub-tiles);
# the block-size list and lane width keep the reference's values, and block sizes
# built from them are accepted (tiles are chosen by this backend).
PAGE_SIZE_MULTIPLE = 16
FWD_BLOCKS = (2048, 1024, 512, 256, 128)
NUM_LANES = 128

MERGED_KV_DTYPES = (torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2)


def check_merged_kv_dtype(dtype):
    if dtype not in MERGED_KV_DTYPES:
        raise NotImplementedError(
            "the merged KV cache holds bfloat16, float8_e4m3fn or float8_e5m2;"
            f" got {dtype}."
        )


def kv_heads_per_word(dtype):
    return 4 // (2 * dtype.itemsize) if dtype.itemsize == 1 else 1


def merged_cache_heads(num_kv_heads, dtype):
    """`kv_layout.py:67-70`."""
    per = 2 if dtype.itemsize == 1 else 1
    return 2 * (-(-num_kv_heads // per) * per)


def resolve_merged_kv_heads(cache_heads, dtype, nheads_k):
    """`kv_layout.py:73-95`."""
    check_merged_kv_dtype(dtype)
    if nheads_k is not None:
        num_kv_heads = int(nheads_k)
    elif dtype.itemsize == 1:
        raise ValueError(
            "an fp8 cache pads an odd nheads_k, so its head axis does not give"
            " the KV head count; pass nheads_k."
        )
    else:
        num_kv_heads = cache_heads // 2
    if merged_cache_heads(num_kv_heads, dtype) != cache_heads:
        raise ValueError(
            f"a merged {dtype} cache of {num_kv_heads} KV heads holds"
            f" {merged_cache_heads(num_kv_heads, dtype)} head rows per token;"
            f" got {cache_heads}."
        )
    return num_kv_heads


def merge_kv_heads(k, v):
    """(..., Hk, D) K and V -> (..., cache_heads, D) merged rows."""
    *lead, hk, d = k.shape
    ch = merged_cache_heads(hk, k.dtype)
    out = torch.zeros((*lead, ch, d), dtype=k.dtype, device=k.device)
    out[..., 0: 2 * hk: 2, :] = k
    out[..., 1: 2 * hk: 2, :] = v
    return out


def split_kv_heads(kv, nheads_k):
    return kv[..., 0: 2 * nheads_k: 2, :], kv[..., 1: 2 * nheads_k: 2, :]
