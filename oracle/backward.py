"""NumPy restatement of the dense attention backward (test infrastructure only).

Only tests, smoke() and the bench's CPU baseline use this module, as the
checker.  Follows the recurrences of flash_attn_bwd
(flywheel_tpu/softmax_attention/bwd_pipeline.py:401-570, kernels/bwd.py:685-720):
p from the forward's scores and lse, delta = rowsum(dout * out),
ds = p (dp - delta), dq = scale ds k, dk = scale ds^T q, dv = p^T dout, with
GQA heads summed into their KV head.  Pinned in tests/test_oracle_backward.py
against torch.autograd through a float64 attention (a library routine's own
backward) on MHA, GQA, MQA, causal with seqlen_q != seqlen_k and full masks.
"""

import math

import numpy as np

from oracle.dtypes import bf16

LOG2E = math.log2(math.e)


def attention_bwd_ref(q, k, v, dout, *, causal=False, softmax_scale=None,
                      round_scaled_q=False, bf16_intermediates=False):
    """(dq, dk, dv) of attention_ref's out for the upstream gradient dout.

    q, dout (B, Sq, H, D); k, v (B, Sk, Hk, D); float32 values.  causal is
    bottom-right aligned (query i sees key j iff j <= i + Sk - Sq).
    round_scaled_q forms the scores from bf16(q * scale * log2 e) as the
    forward kernels do (bwd_pipeline.py:418-427), so p is the forward's own
    softmax.  bf16_intermediates rounds out, p, dp and ds to bf16 where a bf16
    computation would hold them, and the gradients themselves (a bf16
    computation returns bf16 gradients): the coarse reference of the
    reference's tolerance rule, test_prefill.py:301-333.  Rows with no visible key have
    p = 0.  Returns float32 arrays shaped like q, k, v.
    """
    q, k, v, dout = (np.asarray(x, np.float64) for x in (q, k, v, dout))
    batch, sq, nheads, d = q.shape
    sk, nkv = k.shape[1], k.shape[2]
    group = nheads // nkv
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else float(softmax_scale)
    rnd = (lambda x: bf16(x).astype(np.float64)) if bf16_intermediates else (lambda x: x)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    visible = np.ones((sq, sk), bool)
    if causal:
        visible = np.arange(sk)[None, :] <= np.arange(sq)[:, None] + (sk - sq)
    seen = visible.any(axis=1, keepdims=True)
    for b in range(batch):
        for h in range(nheads):
            hk = h // group
            qh, kh, vh, doh = q[b, :, h], k[b, :, hk], v[b, :, hk], dout[b, :, h]
            if round_scaled_q:
                qs = bf16((qh * scale * LOG2E).astype(np.float32)).astype(np.float64)
                s = (qs @ kh.T) / LOG2E  # natural-log logits
            else:
                s = (qh @ kh.T) * scale
            s = np.where(visible, s, -np.inf)
            m = np.where(seen, s.max(axis=1, keepdims=True), 0.0)
            e = np.where(visible, np.exp(s - m), 0.0)
            p = e / np.where(seen, e.sum(axis=1, keepdims=True), 1.0)
            out = rnd(p @ vh)
            p = rnd(p)
            dv[b, :, hk] += p.T @ doh
            dp = rnd(doh @ vh.T)
            delta = (doh * out).sum(axis=1, keepdims=True)
            ds = rnd(p * (dp - delta))
            dq[b, :, h] = scale * (ds @ kh)
            dk[b, :, hk] += scale * (ds.T @ qh)
    grads = tuple(x.astype(np.float32) for x in (dq, dk, dv))
    return tuple(bf16(x) for x in grads) if bf16_intermediates else grads
