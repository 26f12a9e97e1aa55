"""Gradients of flash_attn_func through the gfx950 backward kernels.

Mirrors the reference's differentiation rules (flywheel_tpu/softmax_attention/
autograd.py:27-109): the dense MHA / GQA / MQA forward with a causal or full
mask has a backward (flash_attn_bwd, kernels/bwd.py:463); every other
configuration runs its forward and raises NotImplementedError, naming the
feature, only when a gradient is requested.  The kernels take head dims
128/128, 128/256, 128/512, 256/128 and 256/256 (q and k / v and out); the
reference's other backward pairs (64/64, 64/256, 64/512, 96/96, 192/128,
192/192, test_prefill.py:205-208,285-333) run through them on zero-padded
operands (attn_bwd_padded).  lse carries no gradient of its own.
"""

import torch

from . import _native as N


def bwd_widths(d, dv):
    """(head_dim, head_dim_v) the backward kernels run for head dims d / dv
    (zero-padded up to them), or None when no kernel takes the pair."""
    dq_w = 128 if d <= 128 else 256 if d <= 256 else None
    dv_w = 128 if dv <= 128 else 256 if dv <= 256 else 512 if dv <= 512 else None
    if dq_w is None or dv_w is None or (dq_w, dv_w) == (256, 512):
        return None
    return dq_w, dv_w


def attn_bwd(q, k, v, out, dout, lse, *, qs, ks, vs, os_, ls, batch, nheads, nheads_k,
             seqlen_q, seqlen_k, softmax_scale, causal, head_dim=128, head_dim_v=None):
    """fw_attn_bwd: (dq, dk, dv) laid out like q, k, v (all contiguous), at
    head dims the kernels take (128/128, 128/256, 128/512, 256/128, 256/256)."""
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    p = N.AttnBwdParams()
    p.q, p.k, p.v, p.out, p.dout, p.lse = (N.ptr(t) for t in (q, k, v, out, dout, lse))
    p.dq, p.dk, p.dv = N.ptr(dq), N.ptr(dk), N.ptr(dv)
    p.q_stride_b, p.q_stride_h, p.q_stride_t = qs
    p.k_stride_b, p.k_stride_h, p.k_stride_t = ks
    p.v_stride_b, p.v_stride_h, p.v_stride_t = vs
    p.o_stride_b, p.o_stride_h, p.o_stride_t = os_
    p.lse_stride_b, p.lse_stride_h = ls
    p.batch, p.nheads, p.nheads_k = batch, nheads, nheads_k
    p.head_dim, p.head_dim_v = head_dim, head_dim if head_dim_v is None else head_dim_v
    p.seqlen_q, p.seqlen_k = seqlen_q, seqlen_k
    p.softmax_scale, p.causal = softmax_scale, int(causal)
    lib = N.lib()
    nbytes = lib.fw_attn_bwd_workspace_bytes(p)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = N.ptr(ws), ws.numel()
    N.check(lib.fw_attn_bwd(p, N.stream_of(q)))
    return dq, dk, dv


def _pad_heads(x, d, width):
    """x (contiguous, head dim d innermost) as (rows, width) with each
    d-vector zero-padded to width."""
    return torch.nn.functional.pad(x.reshape(-1, d), (0, width - d))


def attn_bwd_padded(q, k, v, out, dout, lse, *, head_dim, head_dim_v, qs, ks, vs, os_,
                    **geometry):
    """The backward at head dims the kernels do not take directly (64, 96,
    192, and head_dim_v 64 .. 512) through the next kernel widths
    (bwd_widths): every d-vector of q and k is zero-padded to head_dim's width
    and every dv-vector of v, out and dout to head_dim_v's.  The scores, the
    softmax (the scale stays the caller's) and rowsum(dout * out) are unchanged
    by the zero dims, and the padded columns of dq, dk and dv come out zero,
    so the leading columns are the gradients.  The strides of contiguous
    head-dim-innermost layouts scale by width / head dim."""
    d, dv = head_dim, head_dim_v
    dq_w, dv_w = bwd_widths(d, dv)
    pq, pk = _pad_heads(q, d, dq_w), _pad_heads(k, d, dq_w)
    pv, po, pdo = (_pad_heads(t, dv, dv_w) for t in (v, out, dout))
    scale = lambda st, hd, w: tuple(x // hd * w for x in st)
    dq, dk, dvv = attn_bwd(pq, pk, pv, po, pdo, lse, qs=scale(qs, d, dq_w), ks=scale(ks, d, dq_w),
                           vs=scale(vs, dv, dv_w), os_=scale(os_, dv, dv_w), head_dim=dq_w,
                           head_dim_v=dv_w, **geometry)
    return (dq[:, :d].reshape(q.shape), dk[:, :d].reshape(k.shape),
            dvv[:, :dv].reshape(v.shape))


class FlashAttnFunction(torch.autograd.Function):
    """forward(q, k, v, spec) -> (out, lse); spec holds the launch closure, the
    geometry for the backward and, for forward-only configurations, the
    message the backward raises (autograd.py:75-109, variant.py:365-384)."""

    @staticmethod
    def forward(ctx, q, k, v, spec):
        out, lse = spec["run"](q, k, v)
        ctx.spec = spec
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, unused_dlse):
        spec = ctx.spec
        if spec["forward_only"]:
            raise NotImplementedError(spec["forward_only"])
        q, k, v, out, lse = ctx.saved_tensors
        g = dict(spec["geometry"])
        d, dv = g["head_dim"], g["head_dim_v"]
        if bwd_widths(d, dv) == (d, dv):
            dq, dk, dv_ = attn_bwd(q, k, v, out, dout.contiguous(), lse, **g)
        else:
            dq, dk, dv_ = attn_bwd_padded(q, k, v, out, dout.contiguous(), lse, **g)
        return dq, dk, dv_, None


class ForwardOnlyFunction(torch.autograd.Function):
    """A forward with no backward: the gradient request raises the message
    (autograd.py:75-109, forward_only_attn).  holder carries the launch
    closure in and lse (not differentiable) out."""

    @staticmethod
    def forward(ctx, q, k, v, holder):
        out, holder["lse"] = holder["run"](q, k, v)
        ctx.msg = holder["msg"]
        return out

    @staticmethod
    def backward(ctx, unused_dout):
        raise NotImplementedError(ctx.msg)


def forward_only(run, msg, q, k, v):
    """(out, lse) of run(q, k, v) as an autograd node whose backward raises."""
    holder = {"run": run, "msg": msg}
    out = ForwardOnlyFunction.apply(q, k, v, holder)
    return out, holder["lse"]


def needs_grad(*tensors):
    return torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)
