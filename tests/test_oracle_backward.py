"""Pins oracle/backward.py against torch.autograd through a float64 attention
(torch's own backward of softmax, matmul and repeat_interleave), for the
shapes the reference's backward covers (test_prefill.py:285-333: MHA, GQA /
MQA, causal with seqlen_q != seqlen_k, full masks)."""

import math

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import dtypes as T


def torch_grads(q, k, v, dout, causal):
    q, k, v = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    sq, h, sk, hk = q.shape[1], q.shape[2], k.shape[1], k.shape[2]
    kk = k.repeat_interleave(h // hk, dim=2)
    vv = v.repeat_interleave(h // hk, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, kk) / math.sqrt(q.shape[-1])
    if causal:
        vis = torch.arange(sk)[None, :] <= torch.arange(sq)[:, None] + (sk - sq)
        s = s.masked_fill(~vis, -torch.inf)
        seen = vis.any(dim=1)[None, None, :, None]
    else:
        seen = torch.ones(1, 1, sq, 1, dtype=torch.bool)
    p = torch.where(seen, torch.softmax(torch.where(seen, s, torch.zeros_like(s)), -1), 0.0)
    out = torch.einsum("bhqk,bkhd->bqhd", p, vv)
    out.backward(torch.tensor(dout, dtype=torch.float64))
    return q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("h,hk,sq,sk,causal", [
    (4, 4, 37, 37, True), (4, 2, 20, 45, True), (6, 1, 33, 17, True), (4, 2, 30, 30, False),
    (2, 2, 9, 64, False)])
def test_backward_matches_torch_autograd(h, hk, sq, sk, causal):
    rng = np.random.default_rng(5)
    q = T.bf16(rng.standard_normal((2, sq, h, 64), dtype=np.float32))
    k = T.bf16(rng.standard_normal((2, sk, hk, 64), dtype=np.float32))
    v = T.bf16(rng.standard_normal((2, sk, hk, 64), dtype=np.float32))
    do = T.bf16(rng.standard_normal((2, sq, h, 64), dtype=np.float32))
    ours = B.attention_bwd_ref(q, k, v, do, causal=causal)
    theirs = torch_grads(q, k, v, do, causal)
    for a, b_ in zip(ours, theirs):
        np.testing.assert_allclose(a, b_, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("d,dv,h,hk,causal", [(48, 16, 4, 2, True), (16, 64, 2, 1, False),
                                                (32, 128, 3, 3, True)])
def test_backward_head_dim_v_matches_torch_autograd(d, dv, h, hk, causal):
    """head_dim_v != head_dim (the reference's 192/128 and 64/256, 64/512
    pairs, test_prefill.py:205-208), at small sizes: the scale stays
    1/sqrt(head_dim)."""
    rng = np.random.default_rng(7)
    q = T.bf16(rng.standard_normal((1, 21, h, d), dtype=np.float32))
    k = T.bf16(rng.standard_normal((1, 26, hk, d), dtype=np.float32))
    v = T.bf16(rng.standard_normal((1, 26, hk, dv), dtype=np.float32))
    do = T.bf16(rng.standard_normal((1, 21, h, dv), dtype=np.float32))
    ours = B.attention_bwd_ref(q, k, v, do, causal=causal)
    theirs = torch_grads(q, k, v, do, causal)
    for a, b_ in zip(ours, theirs):
        assert a.shape == b_.shape
        np.testing.assert_allclose(a, b_, rtol=1e-5, atol=1e-5)


def test_rounding_variants_stay_close():
    """round_scaled_q and bf16_intermediates perturb at bf16 precision only."""
    rng = np.random.default_rng(6)
    q, k, v, do = (T.bf16(rng.standard_normal((1, 40, 2, 64), dtype=np.float32)) for _ in range(4))
    exact = B.attention_bwd_ref(q, k, v, do, causal=True)
    for kw in ({"round_scaled_q": True}, {"bf16_intermediates": True}):
        approx = B.attention_bwd_ref(q, k, v, do, causal=True, **kw)
        for a, b_ in zip(approx, exact):
            assert np.abs(a - b_).max() < 0.05 * np.abs(b_).max()
            assert np.abs(a - b_).max() > 0  # the variant does change something
