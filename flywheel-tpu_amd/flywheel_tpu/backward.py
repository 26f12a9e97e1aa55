"""Gradients of flash_attn_func through the gfx950 backward kernels.

Mirrors the reference's differentiation rules (flywheel_tpu/softmax_attention/
autograd.py:27-109): the dense MHA / GQA / MQA forward with a causal or full
mask has a backward (flash_attn_bwd, kernels/bwd.py:463); every other
configuration runs its forward and raises NotImplementedError, naming the
feature, only when a gradient is requested.  Head dims 64 and 96 go through the
head-dim-128 kernels on zero-padded operands (attn_bwd_padded); 192, 256 and
head_dim_v != head_dim are forward-only.  lse carries no gradient of its own.
"""

import torch

from . import _native as N


def attn_bwd(q, k, v, out, dout, lse, *, qs, ks, ls, batch, nheads, nheads_k, seqlen_q,
             seqlen_k, softmax_scale, causal):
    """fw_attn_bwd: (dq, dk, dv) laid out like q, k, v (all contiguous)."""
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    p = N.AttnBwdParams()
    p.q, p.k, p.v, p.out, p.dout, p.lse = (N.ptr(t) for t in (q, k, v, out, dout, lse))
    p.dq, p.dk, p.dv = N.ptr(dq), N.ptr(dk), N.ptr(dv)
    p.q_stride_b, p.q_stride_h, p.q_stride_t = qs
    p.k_stride_b, p.k_stride_h, p.k_stride_t = ks
    p.v_stride_b, p.v_stride_h, p.v_stride_t = ks
    p.lse_stride_b, p.lse_stride_h = ls
    p.batch, p.nheads, p.nheads_k, p.head_dim = batch, nheads, nheads_k, 128
    p.seqlen_q, p.seqlen_k = seqlen_q, seqlen_k
    p.softmax_scale, p.causal = softmax_scale, int(causal)
    lib = N.lib()
    nbytes = lib.fw_attn_bwd_workspace_bytes(p)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = N.ptr(ws), ws.numel()
    N.check(lib.fw_attn_bwd(p, N.stream_of(q)))
    return dq, dk, dv


def _pad_heads(x, d):
    """x (contiguous, head dim d innermost) as (rows, 128) with each d-vector
    zero-padded to 128."""
    return torch.nn.functional.pad(x.reshape(-1, d), (0, 128 - d))


def attn_bwd_padded(q, k, v, out, dout, lse, *, head_dim, qs, ks, **geometry):
    """The backward at a head dim below 128 (q, k and v share it) through the
    head-dim-128 kernels: every d-vector of q, k, v, out and dout is
    zero-padded to 128.  The scores, the softmax (the scale stays the caller's)
    and rowsum(dout * out) are unchanged by the zero dims, and the padded
    columns of dq, dk and dv come out zero, so the first d columns are the
    gradients.  The strides of contiguous d-innermost layouts scale by 128 / d."""
    d = head_dim
    padded = [_pad_heads(t, d) for t in (q, k, v, out, dout)]
    scale = lambda st: tuple(x // d * 128 for x in st)
    dq, dk, dv = attn_bwd(*padded[:3], padded[3], padded[4], lse, qs=scale(qs), ks=scale(ks),
                          **geometry)
    return tuple(g[:, :d].reshape(t.shape) for g, t in ((dq, q), (dk, k), (dv, v)))


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
        d = g.pop("head_dim", 128)
        if d == 128:
            dq, dk, dv = attn_bwd(q, k, v, out, dout.contiguous(), lse, **g)
        else:
            dq, dk, dv = attn_bwd_padded(q, k, v, out, dout.contiguous(), lse, head_dim=d, **g)
        return dq, dk, dv, None


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
