"""flash_attn_func and flash_attn_varlen_func on the gfx950 MFMA kernel.

Mirrors the reference's API layer (flywheel_tpu/softmax_attention/
prefill.py:62-341, 437-661, 664-963): argument names, order, defaults,
layouts (head-major (B, H, S, D) / (H, total, D), token-major with head_dim,
heads_outer_fold), bottom-right causal / window alignment and exception types.
Every layout is addressed in place through strides; nothing is padded or
transposed.  Sequence lengths need not be multiples of 128 (the reference's
padding rule, prefill.py:176-194, is a TPU tiling constraint).
"""

import torch

from . import _native as N
from .decode import paged_prefill, _num_active_tensor
from .inputs import (
    as_tensor,
    check_common_kwargs,
    check_paged_window,
    check_sinks,
    descale_scalar,
    effective_window,
    int32_device,
    resolve_scale,
)
from .kv_layout import resolve_merged_kv_heads
from . import backward as B
from . import rotary as R

# prefill.py:940-950: the varlen kernels have no backward.
_VARLEN_FORWARD_ONLY = "flash_attn_varlen_func is forward-only; backward is unsupported."


def _check_bf16(*ts):
    if not all(t.dtype == torch.bfloat16 for t in ts):
        raise NotImplementedError(
            f"Only bfloat16 is supported; got {tuple(str(t.dtype) for t in ts)}."
        )


def _split_token_major(x, head_dim):
    """(…, S, nheads * head_dim) -> nheads."""
    if x.shape[-1] % head_dim:
        raise ValueError(f"head_dim {head_dim} must divide the fused width {x.shape[-1]}.")
    return x.shape[-1] // head_dim


def _run_prefill(mode, q, k, v, out, lse, *, qs, ks, vs, os_, ls, batch, nheads, nheads_k,
                 head_dim, seqlen_q, seqlen_k, causal, window_size, softmax_scale, softcap,
                 sinks, cu_q=None, cu_k=None, max_seqlen_q=0, q_rotary=None, head_dim_v=0):
    left, right = effective_window(causal, window_size)
    p = N.PrefillParams()
    p.kv_mode = mode
    p.q, p.out, p.lse, p.k, p.v = N.ptr(q), N.ptr(out), N.ptr(lse), N.ptr(k), N.ptr(v)
    p.cu_seqlens_q, p.cu_seqlens_k, p.sinks = N.ptr(cu_q), N.ptr(cu_k), N.ptr(sinks)
    p.q_stride_b, p.q_stride_h, p.q_stride_t = qs
    p.k_stride_b, p.k_stride_h, p.k_stride_t = ks
    p.v_stride_b, p.v_stride_h, p.v_stride_t = vs
    p.o_stride_b, p.o_stride_h, p.o_stride_t = os_
    p.lse_stride_b, p.lse_stride_h = ls
    p.batch, p.nheads, p.nheads_k, p.head_dim = batch, nheads, nheads_k, head_dim
    p.head_dim_v = head_dim_v
    p.seqlen_q, p.seqlen_k, p.max_seqlen_q = seqlen_q, seqlen_k, max_seqlen_q
    p.kv_dtype = N.FW_BF16
    p.softmax_scale, p.softcap = softmax_scale, float(softcap)
    p.causal, p.window_left, p.window_right = int(causal), left, right
    p.k_descale, p.v_descale = 1.0, 1.0
    keep = None if q_rotary is None else R.set_q_rotary(p, *q_rotary, q.device)
    lib = N.lib()
    nbytes = lib.fw_prefill_workspace_bytes(p)
    ws = None
    if nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        p.workspace, p.workspace_bytes = N.ptr(ws), nbytes
    N.check(lib.fw_prefill(p, N.stream_of(q)))
    del keep


def flash_attn_func(
    q,
    k,
    v,
    dropout_p=0.0,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    attention_chunk=None,
    softcap=0.0,
    alibi_slopes=None,
    deterministic=False,
    return_attn_probs=False,
    return_softmax_lse=False,
    interpret=False,
    head_dim=None,
    token_major=False,
    *,
    rotary_cos=None,
    rotary_sin=None,
    rotary_interleaved=False,
    rotary_k=True,
    heads_outer_fold=False,
    learnable_sink=None,
):
    """flash_attn.flash_attn_func, `prefill.py:62-341`.

    Head-major: q (batch, nheads, seqlen_q, d), k (batch, nheads_k, seqlen_k,
    d), v (batch, nheads_k, seqlen_k, dv), out (batch, nheads, seqlen_q, dv);
    token-major (token_major=True): (batch, seqlen, nheads * head_dim) with
    head_dim given (v's head dim from its width); heads_outer_fold: (nheads,
    batch, seqlen, d).  d / dv: 64/64, 96/96, 128/128, 192/192, 256/256,
    384/384, 512/512, 128/256, 256/128, 192/128, 64/256 or 64/512
    (inputs.py:154-207; token-major 64 is the reference's paired form: MHA
    with an even head count, inputs.py:106-147).  causal is bottom-right aligned: query i sees key j iff
    j <= i + seqlen_k - seqlen_q.  Rows with no reachable key return out 0 and
    lse -inf (or the sink).  lse (batch, nheads, seqlen_q) f32.

    rotary_cos / rotary_sin: (seqlen_ro >= seqlen_k, d / 2) tables in q's dtype
    or float32; K is rotated at positions 0..seqlen_k-1, Q at seqlen_k -
    seqlen_q + i (rotary_k=False: Q only), in f32 with one rounding to bf16
    (rotary.py:27-215).  Gradients (torch.autograd) cover MHA / GQA / MQA with
    a causal or full mask; window_size, softcap, RoPE, heads_outer_fold and
    learnable_sink run forward and raise NotImplementedError when a gradient
    is requested (autograd.py:27-109).
    """
    del interpret
    window_size = check_common_kwargs(
        window_size, dropout_p=dropout_p, softcap=softcap, alibi_slopes=alibi_slopes,
        deterministic=deterministic, return_attn_probs=return_attn_probs)
    if attention_chunk is not None:
        raise NotImplementedError("attention_chunk is not implemented.")
    if type(heads_outer_fold) is not bool:
        raise TypeError("heads_outer_fold must be a bool.")
    has_rotary = rotary_cos is not None or rotary_sin is not None
    if heads_outer_fold and (token_major or return_softmax_lse or (has_rotary and rotary_k)):
        raise NotImplementedError(
            "heads_outer_fold is a forward-only head-major layout; it supports fused RoPE"
            " only as Q-only rotation (rotary_k=False) and no return_softmax_lse."
        )
    q, k, v = as_tensor(q), as_tensor(k), as_tensor(v)
    if token_major:
        if head_dim is None:
            raise ValueError(
                "token-major (fused head_dim) inputs require head_dim=; the fused width"
                f" alone cannot determine the head split (got {tuple(q.shape)=})."
            )
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise ValueError(f"q/k/v ranks must be 3; got {q.shape=}, {k.shape=}, {v.shape=}.")
        if type(head_dim) is not int:
            raise ValueError(f"head_dim must be a static python int; got {head_dim!r}.")
        if head_dim <= 0 or (head_dim % 128 and head_dim != 64):
            raise ValueError("token-major inputs require head_dim % 128 == 0 or head_dim == 64"
                             f" (paired); got {head_dim}.")
        batch, seqlen_q = q.shape[:2]
        seqlen_k = k.shape[1]
        nheads = _split_token_major(q, head_dim)
        nheads_k = _split_token_major(k, head_dim)
        if v.shape[:2] != k.shape[:2] or v.shape[-1] % nheads_k:
            raise ValueError(f"v fused width {v.shape[-1]} must be a multiple of nheads_k"
                             f" {nheads_k}; got {tuple(v.shape)=}, {tuple(k.shape)=}.")
        dv = v.shape[-1] // nheads_k
        if dv % 128 and dv != 64:
            raise ValueError("token-major requires head_dim_v % 128 == 0 or head_dim_v == 64"
                             f" (paired); got {dv}.")
        if head_dim % 128 or dv % 128:
            if dv != head_dim:
                raise NotImplementedError("token-major d64 requires head_dim_v == head_dim;"
                                          f" got {head_dim} vs {dv}.")
            if nheads_k != nheads:
                raise NotImplementedError("token-major d64 is MHA-only; pass 4-D head-major"
                                          " inputs instead.")
            if nheads % 2:
                raise ValueError(f"token-major d64 requires an even head count; got {nheads}.")
        d = head_dim
        qs = (seqlen_q * nheads * d, d, nheads * d)
        ks = (seqlen_k * nheads_k * d, d, nheads_k * d)
        vs = (seqlen_k * nheads_k * dv, dv, nheads_k * dv)
        os_ = (seqlen_q * nheads * dv, dv, nheads * dv)
        out_shape = (batch, seqlen_q, nheads * dv)
    else:
        if head_dim is not None:
            raise ValueError("head_dim is only meaningful for token-major inputs.")
        if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
            raise ValueError(
                f"q/k/v must be 4-D head-major; got {tuple(q.shape)=}, {tuple(k.shape)=},"
                f" {tuple(v.shape)=}."
            )
        if q.shape[-1] != k.shape[-1]:
            raise ValueError(f"Incompatible shapes: {tuple(q.shape)=} vs {tuple(k.shape)=}.")
        # v may differ from k in head_dim only (inputs.py:201-207)
        if k.shape[:-1] != v.shape[:-1]:
            raise ValueError(f"k and v must share every axis but head_dim; got"
                             f" {tuple(k.shape)=}, {tuple(v.shape)=}.")
        dv = v.shape[-1]
        if heads_outer_fold:
            nheads, batch, seqlen_q, d = q.shape
            nheads_k, _, seqlen_k, _ = k.shape
            qs = (seqlen_q * d, batch * seqlen_q * d, d)
            ks = (seqlen_k * d, batch * seqlen_k * d, d)
            vs = (seqlen_k * dv, batch * seqlen_k * dv, dv)
            os_ = (seqlen_q * dv, batch * seqlen_q * dv, dv)
            out_shape = (nheads, batch, seqlen_q, dv)
            kb = k.shape[1]
        else:
            batch, nheads, seqlen_q, d = q.shape
            _, nheads_k, seqlen_k, _ = k.shape
            qs = (nheads * seqlen_q * d, seqlen_q * d, d)
            ks = (nheads_k * seqlen_k * d, seqlen_k * d, d)
            vs = (nheads_k * seqlen_k * dv, seqlen_k * dv, dv)
            os_ = (nheads * seqlen_q * dv, seqlen_q * dv, dv)
            out_shape = (batch, nheads, seqlen_q, dv)
            kb = k.shape[0]
        if kb != batch:
            raise ValueError(f"Incompatible shapes: {tuple(q.shape)=} vs {tuple(k.shape)=}.")
    if nheads_k <= 0 or nheads % nheads_k:
        raise ValueError(f"{nheads=} must be a multiple of {nheads_k=}.")
    tables = R.check_tables(rotary_cos, rotary_sin, head_dim=d, dtype=q.dtype,
                            rotate_k=rotary_k, interleaved=rotary_interleaved,
                            kv_len_bound=seqlen_k)
    if tables is not None and seqlen_q > seqlen_k:
        raise ValueError("RoPE prefill requires seqlen_q <= seqlen_k.")
    _check_bf16(q, k, v)
    N.require_device(q, k, v)
    grad = B.needs_grad(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    softmax_scale = resolve_scale(softmax_scale, d)
    sinks = check_sinks(learnable_sink, nheads, q.device)
    lse_shape = (batch, nheads, seqlen_q)

    def run(q, k, v, with_lse):
        if tables is not None and rotary_k:
            # rotary.py:118-120: K at i; Q (at seqlen_k - seqlen_q + i) is
            # rotated by the kernel as it loads it.
            k = R.rotate(k, tables, rotary_interleaved, strides=ks, batch_rows=batch,
                         nheads=nheads_k, ntokens=seqlen_k)
        out = q.new_empty(out_shape)
        lse = torch.empty(lse_shape, dtype=torch.float32, device=q.device) if with_lse else None
        _run_prefill(N.FW_KV_DENSE, q, k, v, out, lse, qs=qs, ks=ks, vs=vs, os_=os_,
                     ls=(nheads * seqlen_q, seqlen_q), batch=batch, nheads=nheads,
                     nheads_k=nheads_k, head_dim=d, seqlen_q=seqlen_q, seqlen_k=seqlen_k,
                     causal=causal, window_size=window_size, softmax_scale=softmax_scale,
                     softcap=softcap, sinks=sinks,
                     q_rotary=None if tables is None else (tables, rotary_interleaved),
                     head_dim_v=dv)
        return out, lse

    if not grad:
        out, lse = run(q, k, v, return_softmax_lse)
    else:
        # prefill.py:250-297 and variant.py:365-384: which configurations have
        # a backward; the others raise when a gradient is requested.
        reason = None
        if heads_outer_fold or tables is not None or sinks is not None:
            what = ("Fused RoPE" if tables is not None else
                    "heads_outer_fold" if heads_outer_fold else "learnable_sink")
            reason = f"{what} is forward-only; backward is unsupported."
        else:
            unsupported = ("window_size" if window_size != (-1, -1) else
                           "softcap" if softcap != 0.0 else
                           f"head_dim {d} / head_dim_v {dv}" if B.bwd_widths(d, dv) is None
                           else None)
            if unsupported:
                reason = (f"The backward kernel does not support {unsupported}; that"
                          " configuration is forward-only.")
        spec = {
            "run": lambda q, k, v: run(q, k, v, True),
            "forward_only": reason,
            "geometry": dict(qs=qs, ks=ks, vs=vs, os_=os_, ls=(nheads * seqlen_q, seqlen_q),
                             batch=batch, nheads=nheads, nheads_k=nheads_k, seqlen_q=seqlen_q,
                             seqlen_k=seqlen_k, softmax_scale=softmax_scale, causal=causal,
                             head_dim=d, head_dim_v=dv),
        }
        out, lse = B.FlashAttnFunction.apply(q, k, v, spec)
    if return_softmax_lse:
        return out, lse
    return out


def flash_attn_varlen_func(
    q,
    k,
    v,
    cu_seqlens_q,
    cu_seqlens_k,
    max_seqlen_q,
    max_seqlen_k,
    dropout_p=0.0,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    alibi_slopes=None,
    deterministic=False,
    return_attn_probs=False,
    return_softmax_lse=False,
    interpret=False,
    head_dim=None,
    token_major=False,
    block_sizes=None,
    *,
    rotary_cos=None,
    rotary_sin=None,
    rotary_interleaved=False,
    rotary_k=True,
    block_table=None,
    seqused_k=None,
    num_active=None,
    k_descale=None,
    v_descale=None,
    nheads_k=None,
    learnable_sink=None,
    guard_replay_unroll=1,
):
    """flash_attn.flash_attn_varlen_func for packed sequences, `prefill.py:664-963`.

    Packed K/V: q (nheads, total_q, d), k (nheads_k, total_k, d), v
    (nheads_k, total_k, dv), out (nheads, total_q, dv), with cu_seqlens_q /
    cu_seqlens_k (token-major: (total, nheads * head_dim)).
    Paged KV cache (block_table given, read-only): k is the merged pool, v None,
    cu_seqlens_k None, seqused_k (batch,) each sequence's kv length.  Padding q
    rows return out 0, lse -inf; lse is (nheads, total_q).  block_sizes and
    guard_replay_unroll are accepted for compatibility (tiles are chosen by
    this backend).  RoPE tables as in flash_attn_func, positions per sequence
    (Q at len_k - len_q + i); a paged cache takes rotary_k=False.  No backward:
    a gradient request raises NotImplementedError (prefill.py:940-950).
    """
    del interpret
    window_size = check_common_kwargs(
        window_size, dropout_p=dropout_p, softcap=softcap, alibi_slopes=alibi_slopes,
        deterministic=deterministic, return_attn_probs=return_attn_probs)
    if block_sizes is not None:
        bs = tuple(block_sizes)
        if len(bs) != 4 or not all(type(b) is int and b > 0 for b in bs):
            raise ValueError(
                "block_sizes must be 4 positive ints (block_q, block_kv, block_q_compute,"
                f" block_kv_compute); got {bs!r}."
            )
        if bs[0] % 128 or bs[1] % 128:
            raise ValueError(f"block_q and block_kv must be multiples of 128; got {bs!r}.")
    for name, bound in (("max_seqlen_q", max_seqlen_q), ("max_seqlen_k", max_seqlen_k)):
        if isinstance(bound, torch.Tensor):
            bound = int(bound)
        if int(bound) <= 0:
            raise ValueError(f"{name} must be positive; got {bound}.")
    q = as_tensor(q)
    k = as_tensor(k)
    v = as_tensor(v)
    if block_table is not None:
        if guard_replay_unroll != 1:
            raise ValueError(
                "guard_replay_unroll applies to packed K/V; a paged KV cache always"
                " unrolls its replay."
            )
        if token_major:
            raise NotImplementedError(
                "a paged KV cache takes head-major q (nheads, total_q, headdim);"
                " token_major=True is not supported."
            )
        if head_dim is not None:
            raise ValueError("head_dim is only meaningful for token-major inputs; a paged call"
                             " takes head-major q.")
        if cu_seqlens_k is not None:
            raise ValueError("with block_table, pass cu_seqlens_k=None: seqused_k gives each"
                             " sequence's kv length.")
        if v is not None:
            raise ValueError("with block_table, pass one merged (num_pages, page_size,"
                             " cache_heads, headdim) cache as k and v=None; separate paged K"
                             " and V caches are not supported.")
        if seqused_k is None:
            raise ValueError("block_table needs seqused_k, the (batch,) kv length of each"
                             " sequence (its new tokens included).")
        if rotary_cos is not None and rotary_k:
            raise NotImplementedError(
                "a paged KV cache holds K already rotated; pass rotary_k=False to rotate Q"
                " only.")
        if q.ndim != 3:
            raise ValueError(f"with block_table, q must be (nheads, total_q, headdim); got"
                             f" {tuple(q.shape)=}.")
        cu = as_tensor(cu_seqlens_q)
        if cu.ndim != 1 or cu.shape[0] < 2 or cu.is_floating_point():
            raise ValueError("cu_seqlens_q must be a 1-D integer array of batch + 1 boundaries;"
                             f" got {tuple(cu.shape)} {cu.dtype}.")
        batch = cu.shape[0] - 1
        if not cu.is_cuda and int(cu[0]) != 0:
            raise ValueError(f"with block_table, cu_seqlens_q must start at 0; got"
                             f" cu_seqlens_q[0]={int(cu[0])}.")
        if isinstance(num_active, int) and not 0 <= num_active <= batch:
            raise ValueError(f"num_active must be in [0, {batch}]; got {num_active}.")
        check_paged_window(causal, window_size)
        if k.ndim != 4:
            raise ValueError(f"k must be the merged (num_pages, page_size, cache_heads, head_dim)"
                             f" pool; got {tuple(k.shape)}.")
        nheads, total_q, d = q.shape
        nkv = resolve_merged_kv_heads(k.shape[2], k.dtype, nheads_k)
        if k.shape[3] != d:
            raise ValueError(f"cache head_dim {k.shape[3]} must match q's {d}.")
        if nheads % nkv:
            raise ValueError(f"{nheads=} must be a multiple of nheads_k={nkv}.")
        if k.shape[1] % 16:
            raise ValueError(f"page_size must be a multiple of 16; got {k.shape[1]}.")
        if q.dtype != torch.bfloat16:
            raise NotImplementedError(f"q must be bfloat16; got {q.dtype}.")
        tables = R.check_tables(rotary_cos, rotary_sin, head_dim=d, dtype=q.dtype,
                                rotate_k=rotary_k, interleaved=rotary_interleaved,
                                kv_len_bound=int(max_seqlen_k))
        if tables is not None and (num_active is None or isinstance(num_active, int)):
            cu_h, used_h = cu, as_tensor(seqused_k)
            if isinstance(num_active, int) and not (cu.is_cuda or used_h.is_cuda):
                # prefill.py:570-577: inactive sequences hold no rows, kv length 0.
                cu_h = torch.where(torch.arange(batch + 1) <= num_active, cu, cu[num_active])
                used_h = torch.where(torch.arange(batch) < num_active, used_h, 0)
            R.check_packed_lengths(cu_h, used_h, tables[0].shape[0])
        N.require_device(q, k)
        device = q.device
        bt = as_tensor(block_table)
        if bt.ndim != 2 or bt.shape[0] != batch or bt.is_floating_point():
            raise ValueError(f"block_table must be (batch={batch}, max_pages) int; got"
                             f" {tuple(bt.shape)} {bt.dtype}.")
        cu_dev = int32_device(cu, device, "cu_seqlens_q")
        used_dev = int32_device(seqused_k, device, "seqused_k", (batch,))
        active = _num_active_tensor(num_active, batch, device)
        q = q.contiguous()
        sinks = check_sinks(learnable_sink, nheads, device)
        bt_dev = bt.to(device=device, dtype=torch.int32).contiguous()
        kd = descale_scalar(k_descale, "k_descale", device)
        vd = descale_scalar(v_descale, "v_descale", device)

        def run_paged(q, k, unused_v):
            return paged_prefill(
                q, k, cu_dev, used_dev, bt_dev, active, sinks,
                nheads_k=nkv, softmax_scale=resolve_scale(softmax_scale, d),
                softcap=float(softcap), causal=causal, window_size=window_size,
                k_descale=kd, v_descale=vd, max_seqlen_q=int(max_seqlen_q),
                return_lse=return_softmax_lse, token_major_q=False,
                q_rotary=None if tables is None else (tables, rotary_interleaved))

        if B.needs_grad(q, k):
            out, lse = B.forward_only(run_paged, _VARLEN_FORWARD_ONLY, q, k, None)
        else:
            out, lse = run_paged(q, k, None)
        return (out, lse) if return_softmax_lse else out
    if seqused_k is not None or num_active is not None:
        raise ValueError("seqused_k and num_active describe a paged KV cache and need"
                         " block_table; packed K/V takes cu_seqlens_k.")
    if any(x is not None for x in (k_descale, v_descale, nheads_k)):
        raise ValueError("k_descale, v_descale and nheads_k describe an fp8 paged pool and need"
                         " block_table; packed K/V is bf16.")
    cu_q = as_tensor(cu_seqlens_q)
    cu_k = as_tensor(cu_seqlens_k)
    if cu_q.ndim != 1 or tuple(cu_q.shape) != tuple(cu_k.shape):
        raise ValueError("cu_seqlens_q and cu_seqlens_k must be equal-shaped 1-D arrays; got"
                         f" {tuple(cu_q.shape)=}, {tuple(cu_k.shape)=}.")
    batch = cu_q.shape[0] - 1
    if token_major:
        if head_dim is None:
            raise ValueError("token-major (fused head_dim) inputs require head_dim=.")
        if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
            raise ValueError(f"token-major packed q/k/v must be 2-D; got {q.shape=}.")
        total_q, total_k = q.shape[0], k.shape[0]
        nheads = _split_token_major(q, head_dim)
        nkv = _split_token_major(k, head_dim)
        if v.shape[0] != total_k or v.shape[-1] % nkv:
            raise ValueError(f"v fused width {v.shape[-1]} must be a multiple of nheads_k {nkv};"
                             f" got {tuple(v.shape)=}, {tuple(k.shape)=}.")
        d, dv = head_dim, v.shape[-1] // nkv
        qs = (0, d, nheads * d)
        ks = (0, d, nkv * d)
        vs = (0, dv, nkv * dv)
        os_ = (0, dv, nheads * dv)
        out_shape = (total_q, nheads * dv)
    else:
        if head_dim is not None:
            raise ValueError("head_dim is only meaningful for token-major inputs.")
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise ValueError(f"q/k/v must be (heads, total, d); got {q.shape=}, {k.shape=}.")
        nheads, total_q, d = q.shape
        nkv, total_k, _ = k.shape
        if q.shape[-1] != k.shape[-1] or k.shape[:-1] != v.shape[:-1]:
            raise ValueError("k and v must share every axis but head_dim, and q and k their"
                             f" head_dim; got {tuple(q.shape)=}, {tuple(k.shape)=}, {tuple(v.shape)=}.")
        dv = v.shape[-1]
        qs = (0, total_q * d, d)
        ks = (0, total_k * d, d)
        vs = (0, total_k * dv, dv)
        os_ = (0, total_q * dv, dv)
        out_shape = (nheads, total_q, dv)
    if nkv <= 0 or nheads % nkv:
        raise ValueError(f"{nheads=} must be a multiple of nheads_k={nkv}.")
    tables = R.check_tables(rotary_cos, rotary_sin, head_dim=d, dtype=q.dtype,
                            rotate_k=rotary_k, interleaved=rotary_interleaved,
                            kv_len_bound=int(max_seqlen_k))
    if tables is not None:
        R.check_packed_lengths(cu_q, torch.diff(cu_k.to(torch.int64)), tables[0].shape[0])
    _check_bf16(q, k, v)
    N.require_device(q, k, v)
    device = q.device
    grad = B.needs_grad(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    cu_q_dev = int32_device(cu_q, device, "cu_seqlens_q")
    cu_k_dev = int32_device(cu_k, device, "cu_seqlens_k")
    if tables is not None and rotary_k:
        # rotary.py:148-156: K at local; Q (at len_k - len_q + local) is rotated
        # by the kernel as it loads it.
        k = R.rotate(k, tables, rotary_interleaved, strides=ks, batch_rows=1,
                     nheads=nkv, ntokens=total_k, cu=cu_k_dev)
    sinks = check_sinks(learnable_sink, nheads, device)

    def run_packed(q, k, v):
        out = q.new_empty(out_shape)
        lse = (torch.empty((nheads, total_q), dtype=torch.float32, device=device)
               if return_softmax_lse else None)
        _run_prefill(N.FW_KV_VARLEN, q, k, v, out, lse, qs=qs, ks=ks, vs=vs, os_=os_,
                     ls=(0, total_q), batch=batch, nheads=nheads, nheads_k=nkv, head_dim=d,
                     seqlen_q=total_q, seqlen_k=total_k, causal=causal,
                     window_size=window_size, softmax_scale=resolve_scale(softmax_scale, d),
                     softcap=softcap, sinks=sinks, cu_q=cu_q_dev, cu_k=cu_k_dev,
                     max_seqlen_q=int(max_seqlen_q),
                     q_rotary=None if tables is None else (tables, rotary_interleaved),
                     head_dim_v=dv)
        return out, lse

    if grad:
        out, lse = B.forward_only(run_packed, _VARLEN_FORWARD_ONLY, q, k, v)
    else:
        out, lse = run_packed(q, k, v)
    if return_softmax_lse:
        return out, lse
    return out


def _flash_attn_func_pcp_causal_offset(
    q,
    k,
    v,
    causal_offset,
    *,
    softmax_scale=None,
    return_softmax_lse=False,
    heads_outer_fold=False,
    interpret=False,
):
    """Dense causal forward with a device-side Q-position offset (reference
    prefill.py:344-434, the context-parallel caller's internal entry): query i
    sees keys 0 .. causal_offset + i.  q/k/v are head-major (1, nheads, seqlen,
    headdim), or (nheads, 1, seqlen, headdim) with heads_outer_fold; bf16; the
    caller guarantees 0 <= offset and offset + q_len <= kv_len.

    Runs the packed-varlen kernel on one sequence whose key count is
    offset + q_len, computed on the device (no host read of the offset): its
    bottom-right causal alignment then puts query i at key offset + i, and the
    keys past offset + q_len, which no query sees, are never read."""
    del interpret
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("runtime-offset attention requires 4-D head-major Q/K/V.")
    batch_axis, head_axis = (1, 0) if heads_outer_fold else (0, 1)
    batch, nheads = q.shape[batch_axis], q.shape[head_axis]
    q_len, head_dim = q.shape[2], q.shape[3]
    if batch != 1 or k.shape[batch_axis] != 1 or v.shape[batch_axis] != 1:
        raise ValueError("runtime-offset attention requires batch_size == 1.")
    if tuple(k.shape) != tuple(v.shape) or k.shape[3] != head_dim:
        raise ValueError("K/V must share shape and Q/K head dimensions must match.")
    nkv, kv_len = k.shape[head_axis], k.shape[2]
    if nheads % nkv:
        raise ValueError("Q heads must be divisible by KV heads.")
    if q_len <= 0 or kv_len < q_len:
        raise ValueError("runtime-offset attention requires a positive Q length, a positive KV"
                         " length, and kv_len >= q_len.")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise NotImplementedError("runtime-offset attention supports bf16 only.")
    off = as_tensor(causal_offset)
    if off.numel() != 1 or off.is_floating_point() or off.dtype == torch.bool:
        raise ValueError("causal_offset must be one integer scalar.")
    N.require_device(q, k, v)
    device = q.device
    d = head_dim
    # (1, H, S, D) and (H, 1, S, D) are both (H, S, D) in memory
    qp, kp, vp = (t.contiguous().reshape(t.shape[head_axis], t.shape[2], d) for t in (q, k, v))
    off_dev = off.reshape(1).to(device=device, dtype=torch.int32)
    cu_q = torch.tensor([0, q_len], dtype=torch.int32, device=device)
    cu_k = torch.cat([torch.zeros(1, dtype=torch.int32, device=device), off_dev + q_len])
    out = qp.new_empty((nheads, q_len, d))
    lse = (torch.empty((nheads, q_len), dtype=torch.float32, device=device)
           if return_softmax_lse else None)
    _run_prefill(N.FW_KV_VARLEN, qp, kp, vp, out, lse, qs=(0, q_len * d, d),
                 ks=(0, kv_len * d, d), vs=(0, kv_len * d, d), os_=(0, q_len * d, d),
                 ls=(0, q_len), batch=1, nheads=nheads, nheads_k=nkv, head_dim=d,
                 seqlen_q=q_len, seqlen_k=kv_len, causal=True, window_size=(-1, -1),
                 softmax_scale=resolve_scale(softmax_scale, d), softcap=0.0, sinks=None,
                 cu_q=cu_q, cu_k=cu_k, max_seqlen_q=q_len)
    out = out.reshape(q.shape)
    if return_softmax_lse:
        return out, lse.reshape(1, nheads, q_len)  # (batch, nheads, q_len) either way
    return out
