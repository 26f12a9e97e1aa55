"""flash_attn_with_kvcache: attention against a paged merged KV cache or a
contiguous K/V cache pair, with an optional append, on the gfx950 kernels.

Mirrors the reference's `flash_attn_with_kvcache`
(flywheel_tpu/softmax_attention/decode.py:175-625): same argument names,
order, defaults, routing and exception types.  Differences are in the
implementation only:

* the cache is a torch tensor updated in place in HBM and returned as the same
  object (the reference donates and rebinds, `decode.py:175-188`);
* page_size may be any multiple of 16 (the reference requires 128,
  `decode.py:364-368`, a TPU DMA constraint; attention and the cache write
  depend only on the logical (page, slot) mapping);
* single-token decode uses a split-K kernel with the append fused in; a folded
  verify window appends first, then runs the same kernel
  (`decode.py:469-478, 521-541`); any other multi-token or packed call appends
  and then runs the paged varlen prefill kernel (`decode.py:56-172`).
"""

import torch

from . import _native as N
from . import rotary as R
from .inputs import (
    as_tensor,
    check_common_kwargs,
    check_paged_window,
    check_sinks,
    descale_scalar,
    effective_window,
    int32_device,
    resolve_scale,
    set_descales,
)
from .kv_layout import resolve_merged_kv_heads

# `decode.py` MAX_FOLDED_QUERY_ROWS: a verify window folds into the decode
# kernel's query rows while seqlen_q * (nheads // nheads_k) stays within it.
MAX_FOLDED_QUERY_ROWS = 128


def _num_active_tensor(num_active, batch, device):
    if num_active is None:
        return None
    t = as_tensor(num_active) if not isinstance(num_active, int) else None
    if t is None:
        if not 0 <= num_active <= batch:
            raise ValueError(f"num_active must be in [0, {batch}]; got {num_active}.")
        return torch.tensor([num_active], dtype=torch.int32, device=device)
    if t.numel() != 1 or t.is_floating_point():
        raise ValueError(f"num_active must be one integer; got {tuple(t.shape)} {t.dtype}.")
    return t.reshape(1).to(device=device, dtype=torch.int32)


def append_ragged(kv_cache, k, v, cu_seqlens, cache_seqlens, block_table, num_active, nheads_k,
                  batch=None):
    """Packed new tokens k, v (total, nheads_k, head_dim) after each active
    request's cache_seqlens (kernels/kv_append.py:116-184); in place.
    cu_seqlens None: total // batch tokens per request."""
    total, _, head_dim = k.shape
    if cu_seqlens is not None:
        batch = cu_seqlens.shape[0] - 1
    N.check(N.lib().fw_append_ragged(
        N.ptr(kv_cache), N.ptr(k), N.ptr(v), N.ptr(cu_seqlens), N.ptr(cache_seqlens),
        N.ptr(block_table), N.ptr(num_active), batch, total, nheads_k, head_dim,
        kv_cache.shape[1], kv_cache.shape[0], block_table.shape[1],
        N.KV_DTYPES[kv_cache.dtype], N.stream_of(kv_cache)))


def decode_params(q, kv_cache, k_new, v_new, cache_seqlens, block_table, num_active, sinks, *,
                  nheads_k, softmax_scale, softcap, causal, window_left, k_descale, v_descale,
                  seqlen_add=0, return_lse=False, num_splits=0, v_cache=None):
    """A filled fw_decode_params (no workspace yet) and the tensors it points
    at: returns (params, out, lse | None, keep), keep holding every tensor the
    launch reads that the caller does not already hold."""
    batch, seqlen_q, nheads, head_dim = q.shape
    out = torch.empty_like(q)
    lse = (torch.empty((batch, nheads, seqlen_q), dtype=torch.float32, device=q.device)
           if return_lse else None)
    p = N.DecodeParams()
    p.q, p.kv_cache, p.k_new, p.v_new = N.ptr(q), N.ptr(kv_cache), N.ptr(k_new), N.ptr(v_new)
    p.v_cache = N.ptr(v_cache)
    p.cache_seqlens, p.block_table = N.ptr(cache_seqlens), N.ptr(block_table)
    p.num_active, p.sinks, p.out, p.lse = N.ptr(num_active), N.ptr(sinks), N.ptr(out), N.ptr(lse)
    p.batch, p.seqlen_q, p.nheads, p.nheads_k, p.head_dim = batch, seqlen_q, nheads, nheads_k, head_dim
    p.page_size, p.num_pages, p.max_pages = kv_cache.shape[1], kv_cache.shape[0], block_table.shape[1]
    p.kv_dtype = N.KV_DTYPES[kv_cache.dtype]
    p.seqlen_add = seqlen_add
    p.softmax_scale, p.softcap = softmax_scale, softcap
    p.causal, p.window_left = int(causal), window_left
    keep = set_descales(p, k_descale, v_descale)
    p.num_splits = num_splits
    return p, out, lse, keep


def paged_decode(q, kv_cache, k_new, v_new, cache_seqlens, block_table, num_active, sinks, **kw):
    """The split-K decode kernel (kernels/decode.py:463-1915) over a merged
    pool, or with v_cache over the contiguous (batch_cache, capacity, nheads_k,
    head_dim) K/V pair, block_table then being cache_batch_idx as (batch, 1).

    q (batch, seqlen_q, nheads, head_dim) bf16; keyword arguments as
    decode_params.  Returns (out, lse|None)."""
    p, out, lse, keep = decode_params(q, kv_cache, k_new, v_new, cache_seqlens, block_table,
                                      num_active, sinks, **kw)
    lib = N.lib()
    nbytes = lib.fw_paged_decode_workspace_bytes(p)
    if nbytes == 0:
        N.check(lib.fw_paged_decode(p, None))  # raises the validation error
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = N.ptr(ws), nbytes
    N.check(lib.fw_paged_decode(p, N.stream_of(q)))
    del keep
    return out, lse


def paged_prefill(q, kv_cache, cu_seqlens_q, seqused_k, block_table, num_active, sinks, *,
                  nheads_k, softmax_scale, softcap, causal, window_size, k_descale, v_descale,
                  max_seqlen_q, return_lse, token_major_q, q_rotary=None,
                  seqused_excludes_q=False, k_new=None, v_new=None):
    """The paged varlen forward (kernels/fwd_paged.py:1351-1491).

    q is (total_q, nheads, D) when token_major_q, else head-major
    (nheads, total_q, D); out has q's layout; lse is (nheads, total_q).
    q_rotary: None or (tables, interleaved) for the fused Q RoPE.
    seqused_excludes_q: seqused_k holds the lengths before the q rows were
    appended (the kernel adds each sequence's q length).  k_new / v_new
    (total_q, nheads_k, D) in the pool's dtype: rows appended after seqused_k
    first, in the launch that builds the schedule (needs seqused_excludes_q)."""
    if token_major_q:
        total_q, nheads, head_dim = q.shape
        qs_h, qs_t = head_dim, nheads * head_dim
    else:
        nheads, total_q, head_dim = q.shape
        qs_h, qs_t = total_q * head_dim, head_dim
    out = torch.empty_like(q)
    lse = (torch.empty((nheads, total_q), dtype=torch.float32, device=q.device)
           if return_lse else None)
    left, right = effective_window(causal, window_size)
    p = N.PrefillParams()
    p.kv_mode = N.FW_KV_PAGED
    p.q, p.out, p.lse, p.k, p.v = N.ptr(q), N.ptr(out), N.ptr(lse), N.ptr(kv_cache), None
    p.cu_seqlens_q, p.seqused_k, p.block_table = N.ptr(cu_seqlens_q), N.ptr(seqused_k), N.ptr(block_table)
    p.num_active, p.sinks = N.ptr(num_active), N.ptr(sinks)
    p.q_stride_b, p.q_stride_h, p.q_stride_t = 0, qs_h, qs_t
    p.o_stride_b, p.o_stride_h, p.o_stride_t = 0, qs_h, qs_t
    p.lse_stride_b, p.lse_stride_h = 0, total_q
    p.batch, p.nheads, p.nheads_k, p.head_dim = cu_seqlens_q.shape[0] - 1, nheads, nheads_k, head_dim
    p.seqlen_q, p.seqlen_k, p.max_seqlen_q = total_q, 0, max_seqlen_q
    p.page_size, p.num_pages, p.max_pages = kv_cache.shape[1], kv_cache.shape[0], block_table.shape[1]
    p.kv_dtype = N.KV_DTYPES[kv_cache.dtype]
    p.softmax_scale, p.softcap = softmax_scale, softcap
    p.causal, p.window_left, p.window_right = int(causal), left, right
    keep_d = set_descales(p, k_descale, v_descale)
    p.seqused_k_excludes_q = int(seqused_excludes_q)
    p.k_new, p.v_new = N.ptr(k_new), N.ptr(v_new)
    keep = None if q_rotary is None else R.set_q_rotary(p, *q_rotary, q.device)
    lib = N.lib()
    nbytes = lib.fw_prefill_workspace_bytes(p)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = N.ptr(ws), ws.numel()
    N.check(lib.fw_prefill(p, N.stream_of(q)))
    del keep, keep_d
    return out, lse


def flash_attn_with_kvcache(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    *,
    cache_seqlens,
    cache_batch_idx=None,
    block_table=None,
    num_active=None,
    cu_seqlens_q=None,
    max_seqlen_q=None,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    return_softmax_lse=False,
    interpret=False,
    k_descale=None,
    v_descale=None,
    nheads_k=None,
    learnable_sink=None,
):
    """Attention against a KV cache, with optional append.

    Same contract as the reference (`softmax_attention/decode.py:189-285`):
    q (batch, seqlen_q, nheads, head_dim) or packed (total_q, nheads, head_dim)
    with cu_seqlens_q / max_seqlen_q; k_cache the merged
    (num_pages, page_size, cache_heads, head_dim) pool with v_cache=None and
    block_table (batch, max_pages_per_seq), or (single-token decode) separate
    (batch_cache, capacity, nheads_k, head_dim) k_cache / v_cache with
    cache_batch_idx; new k / v appended after each row's cache_seqlens.
    Returns (out, [lse,] kv_cache) or (out, [lse,] k_cache, v_cache), the
    caches updated in place.
    `interpret` is accepted and ignored (there is no interpreter here).
    """
    del interpret
    window_size = check_common_kwargs(window_size, softcap=softcap)
    q = as_tensor(q)
    k_cache = as_tensor(k_cache)
    v_cache = as_tensor(v_cache)
    k = as_tensor(k)
    v = as_tensor(v)
    is_ragged = cu_seqlens_q is not None
    if is_ragged:
        cu_seqlens_q = as_tensor(cu_seqlens_q)
        if cu_seqlens_q.ndim != 1 or cu_seqlens_q.shape[0] < 2 or cu_seqlens_q.is_floating_point():
            raise ValueError("cu_seqlens_q must be a 1-D integer array of batch + 1 boundaries.")
        if q.ndim != 3:
            raise ValueError("With cu_seqlens_q, q must be (total_q, nheads, head_dim).")
        if type(max_seqlen_q) is not int or max_seqlen_q <= 0:
            raise ValueError(
                "With cu_seqlens_q, max_seqlen_q must be a positive static python int,"
                f" the longest request's query length; got {max_seqlen_q!r}."
            )
        batch = cu_seqlens_q.shape[0] - 1
        nheads, head_dim = q.shape[-2:]
        seqlen_q = None
    elif max_seqlen_q is not None:
        raise ValueError(
            "max_seqlen_q is only for a packed q with cu_seqlens_q; a (batch, seqlen_q,"
            f" nheads, head_dim) q takes seqlen_q from its shape; got {max_seqlen_q=}."
        )
    elif q.ndim != 4:
        raise ValueError(f"q must be (batch, seqlen_q, nheads, head_dim); got {tuple(q.shape)=}.")
    else:
        batch, seqlen_q, nheads, head_dim = q.shape
        if batch <= 0 or seqlen_q <= 0:
            raise ValueError("batch and seqlen_q must be positive.")
    is_extend = is_ragged or seqlen_q != 1
    is_paged = block_table is not None
    if is_extend and not is_paged:
        raise NotImplementedError(
            "Multi-token and packed KV-cache attention needs the paged merged cache"
            " (block_table); the contiguous K/V pair serves single-token decode only."
        )
    if is_paged:
        if v_cache is not None:
            raise ValueError(
                "With block_table, pass one merged (num_pages, page_size, cache_heads,"
                " head_dim) cache as k_cache and v_cache=None; separate paged K and V"
                " caches are not supported."
            )
        if cache_batch_idx is not None:
            raise ValueError(
                "block_table and cache_batch_idx are mutually exclusive: the block table"
                " already maps each query row to its pages."
            )
        if k_cache.ndim != 4:
            raise ValueError(
                "With block_table, k_cache must be (num_pages, page_size, cache_heads,"
                f" head_dim), the KV heads' K and V rows interleaved; got {tuple(k_cache.shape)=}."
            )
        if nheads_k is None and k is not None:
            nheads_k = k.shape[-2]
        nheads_k = resolve_merged_kv_heads(k_cache.shape[2], k_cache.dtype, nheads_k)
        page_size = k_cache.shape[1]
        if page_size % 16:
            raise ValueError(f"page_size (k_cache.shape[1]) must be a multiple of 16; got {page_size}.")
        block_table = as_tensor(block_table)
        if block_table.is_floating_point() or block_table.dtype == torch.bool:
            raise ValueError(f"block_table must be an integer array; got {block_table.dtype}.")
        if block_table.ndim != 2 or block_table.shape[0] != batch:
            raise ValueError(
                f"block_table must be (batch={batch}, max_pages_per_seq); got {tuple(block_table.shape)}."
            )
    else:
        if v_cache is None:
            raise ValueError(
                "Without block_table, k_cache and v_cache must be separate (batch_cache,"
                " capacity, nheads_k, head_dim) caches; got v_cache=None (a merged cache"
                " must be paged)."
            )
        if k_cache.ndim != 4 or tuple(v_cache.shape) != tuple(k_cache.shape):
            raise ValueError(
                "k_cache and v_cache must share the shape (batch_cache, capacity, nheads_k,"
                f" head_dim); got {tuple(k_cache.shape)=}, {tuple(v_cache.shape)=}."
            )
        if nheads_k is not None and nheads_k != k_cache.shape[2]:
            raise ValueError(f"{nheads_k=} must match the contiguous caches' {k_cache.shape[2]}.")
        nheads_k = k_cache.shape[2]
        # the reference's decode tiles need whole 128-key blocks of capacity
        # (decode.py:219-220, kernels/decode.py:2006-2011)
        if k_cache.shape[1] <= 0 or k_cache.shape[1] % 128:
            raise ValueError(
                f"capacity (k_cache.shape[1]) must be a positive multiple of 128; got {k_cache.shape[1]}."
            )
    if k_cache.shape[3] != head_dim:
        raise ValueError(f"cache head_dim {k_cache.shape[3]} must match q's {head_dim}.")
    if nheads_k <= 0 or nheads <= 0 or nheads % nheads_k:
        raise ValueError(f"{nheads=} must be a multiple of {nheads_k=}.")
    has_new = k is not None
    if has_new != (v is not None):
        raise ValueError("k and v must be passed together, or both left out.")
    cache_operands = (k_cache,) if is_paged else (k_cache, v_cache)
    kv_operands = (*cache_operands, k, v) if has_new else cache_operands
    if (q.dtype != torch.bfloat16 or any(t.dtype != k_cache.dtype for t in kv_operands)
            or (not is_paged and k_cache.dtype != torch.bfloat16)):
        raise NotImplementedError(
            "q must be bfloat16 and the KV operands share one dtype, bfloat16 or (paged"
            f" pool) float8_e4m3fn / float8_e5m2; got q {q.dtype}, KV"
            f" {tuple(str(t.dtype) for t in kv_operands)}."
        )
    k_descale = descale_scalar(k_descale, "k_descale", q.device)
    v_descale = descale_scalar(v_descale, "v_descale", q.device)
    expected_new_shape = (*q.shape[:-2], nheads_k, head_dim)
    if has_new and (tuple(k.shape) != expected_new_shape or tuple(v.shape) != expected_new_shape):
        raise ValueError(
            f"k and v must be {expected_new_shape} (matching q's token layout); got"
            f" {tuple(k.shape)=}, {tuple(v.shape)=}."
        )
    if not isinstance(cache_seqlens, int):
        cs_shape = tuple(as_tensor(cache_seqlens).shape)
        if cs_shape not in ((), (batch,)):
            raise ValueError(
                f"cache_seqlens must be a scalar or ({batch},) int array; got {cs_shape}."
            )
    if cache_batch_idx is not None:
        idx_shape = tuple(as_tensor(cache_batch_idx).shape)
        if idx_shape != (batch,):
            raise ValueError(f"cache_batch_idx must be a scalar or ({batch},) int array; got {idx_shape}.")
    device = q.device
    N.require_device(q, k_cache, v_cache, k, v)
    if isinstance(cache_seqlens, int):
        row_cache_seqlens = torch.full((batch,), cache_seqlens, dtype=torch.int32, device=device)
    else:
        row_cache_seqlens = int32_device(cache_seqlens, device, "cache_seqlens")
        if row_cache_seqlens.ndim == 0:
            row_cache_seqlens = row_cache_seqlens.expand(batch).contiguous()
        if tuple(row_cache_seqlens.shape) != (batch,):
            raise ValueError(
                f"cache_seqlens must be a scalar or ({batch},) int array; got"
                f" {tuple(row_cache_seqlens.shape)}."
            )
    softmax_scale = resolve_scale(softmax_scale, head_dim)
    sinks = check_sinks(learnable_sink, nheads, device)
    left, _ = effective_window(causal, window_size)
    if is_extend:
        check_paged_window(causal, window_size)
        is_folded = (not is_ragged and left == -1
                     and seqlen_q * (nheads // nheads_k) <= MAX_FOLDED_QUERY_ROWS)
    else:
        is_folded = False
    if is_paged:
        table = block_table.to(device=device, dtype=torch.int32).contiguous()
    elif cache_batch_idx is None:
        table = torch.arange(batch, dtype=torch.int32, device=device).reshape(batch, 1)
    else:
        table = int32_device(cache_batch_idx, device, "cache_batch_idx").reshape(batch, 1).contiguous()
    num_active_t = _num_active_tensor(num_active, batch, device)
    q = q.contiguous()
    if has_new:
        k = k.contiguous()
        v = v.contiguous()
    if is_extend and not is_folded:
        # chunked / packed prefill: append, then the paged varlen kernel
        if is_ragged:
            cu = cu_seqlens_q.to(device=device, dtype=torch.int32).contiguous()
            packed_max = max_seqlen_q
        else:
            cu = torch.arange(batch + 1, dtype=torch.int32, device=device) * seqlen_q
            packed_max = seqlen_q
        packed_q = q.reshape(-1, nheads, head_dim)
        # with new tokens the kv length of a row is its cache length plus its
        # q rows (the kernel adds them), and the rows are appended in the
        # launch that builds the schedule (fw_append_ragged's rule)
        out, lse = paged_prefill(
            packed_q, k_cache, cu, row_cache_seqlens, table, num_active_t, sinks,
            nheads_k=nheads_k, softmax_scale=softmax_scale, softcap=float(softcap),
            causal=causal, window_size=window_size, k_descale=k_descale, v_descale=v_descale,
            max_seqlen_q=packed_max, return_lse=return_softmax_lse, token_major_q=True,
            seqused_excludes_q=has_new,
            k_new=k.reshape(-1, nheads_k, head_dim) if has_new else None,
            v_new=v.reshape(-1, nheads_k, head_dim) if has_new else None)
        out = out.reshape(q.shape)
        if return_softmax_lse:
            if not is_ragged:
                lse = lse.reshape(nheads, batch, seqlen_q).permute(1, 0, 2).contiguous()
            return out, lse, k_cache
        return out, k_cache

    # single-token decode (append fused) or folded verify window
    seqlen_add = 0
    k_new = v_new = None
    if has_new and is_folded:
        # cu_seqlens None: seqlen_q tokens per row
        append_ragged(k_cache, k.reshape(-1, nheads_k, head_dim), v.reshape(-1, nheads_k, head_dim),
                      None, row_cache_seqlens, table, num_active_t, nheads_k, batch=batch)
        seqlen_add = seqlen_q
    elif has_new:
        k_new = k.reshape(batch, nheads_k, head_dim)
        v_new = v.reshape(batch, nheads_k, head_dim)
    causal_eff = bool(causal) or window_size[1] == 0
    out, lse = paged_decode(
        q, k_cache, k_new, v_new, row_cache_seqlens, table, num_active_t, sinks,
        nheads_k=nheads_k, softmax_scale=softmax_scale, softcap=float(softcap),
        causal=causal_eff, window_left=left, k_descale=k_descale, v_descale=v_descale,
        seqlen_add=seqlen_add, return_lse=return_softmax_lse,
        v_cache=None if is_paged else v_cache)
    if return_softmax_lse:
        return (out, lse, *cache_operands)
    return (out, *cache_operands)
