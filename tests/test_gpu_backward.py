"""GPU parity of the dense backward (flash_attn_func under torch.autograd)
against oracle/backward.py, with the reference's tolerance rule
(test_prefill.py:301-333): max |grad - ref| <= 3 * max |bf16_ref - ref| + atol,
where ref is the float64 backward from the forward's rounded scaled q and
bf16_ref rounds out, p, dp and ds to bf16 as a bf16 computation would."""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func
from oracle import backward as OB
from tests.gpu_util import DEV, announce, randn, to_dev_bf16

pytestmark = pytest.mark.gpu


def head_major(x):  # (B, S, H, D) <-> (B, H, S, D)
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


def check_grads(got, q, k, v, do, causal, what):
    ref = OB.attention_bwd_ref(q, k, v, do, causal=causal, round_scaled_q=True)
    coarse = OB.attention_bwd_ref(q, k, v, do, causal=causal, round_scaled_q=True,
                                  bf16_intermediates=True)
    for name, g, r, c in zip(("dq", "dk", "dv"), got, ref, coarse):
        err = np.abs(g - r).max()
        bound = 3 * np.abs(c - r).max() + 2 * np.abs(r + 0.3 - 0.3 - r).max() + 1e-4
        print(f"{what} {name}: max err {err:.3e} bound {bound:.3e} |ref| {np.abs(r).max():.3e}")
        assert err <= bound, f"{what} {name}: {err} > {bound}"


def run(q, k, v, do, causal, token_major=False):
    b, sq, h, d = q.shape
    hk = k.shape[2]
    if token_major:
        tens = [to_dev_bf16(x.reshape(x.shape[0], x.shape[1], -1)).requires_grad_() for x in (q, k, v)]
        out = flash_attn_func(*tens, causal=causal, token_major=True, head_dim=d)
        out.backward(to_dev_bf16(do.reshape(b, sq, -1)))
        torch.cuda.synchronize()
        return [t.grad.float().cpu().numpy().reshape(x.shape) for t, x in zip(tens, (q, k, v))]
    tens = [to_dev_bf16(head_major(x)).requires_grad_() for x in (q, k, v)]
    out = flash_attn_func(*tens, causal=causal)
    out.backward(to_dev_bf16(head_major(do)))
    torch.cuda.synchronize()
    return [head_major(t.grad.float().cpu().numpy()) for t in tens]


@pytest.mark.parametrize(
    "b,h,hk,sq,sk,causal",
    [
        (1, 4, 4, 128, 128, True),
        (2, 4, 2, 200, 333, True),
        (1, 4, 1, 333, 200, True),   # leading rows see no key
        (1, 8, 2, 300, 300, False),
        (1, 2, 2, 64, 1000, False),
        (1, 16, 2, 520, 520, True),  # query heads of a KV head split over workgroups
    ],
)
def test_flash_attn_func_backward(b, h, hk, sq, sk, causal):
    what = f"bwd b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
    announce(what)
    rng = np.random.default_rng(60)
    q, k, v = randn(rng, (b, sq, h, 128)), randn(rng, (b, sk, hk, 128)), randn(rng, (b, sk, hk, 128))
    do = randn(rng, (b, sq, h, 128))
    check_grads(run(q, k, v, do, causal), q, k, v, do, causal, what)


@pytest.mark.parametrize("b,h,hk,sq,sk,causal", [(2, 4, 2, 200, 333, True), (1, 4, 1, 333, 200, True),
                                                (1, 8, 2, 300, 300, False), (1, 16, 2, 520, 520, True)])
def test_backward_recompute_path(b, h, hk, sq, sk, causal, monkeypatch):
    """The recomputing dk / dv kernel (the path above the stored planes'
    size limit), selected with FW_BWD_STORED=0."""
    monkeypatch.setenv("FW_BWD_STORED", "0")
    what = f"bwd recompute b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
    announce(what)
    rng = np.random.default_rng(61)
    q, k, v = randn(rng, (b, sq, h, 128)), randn(rng, (b, sk, hk, 128)), randn(rng, (b, sk, hk, 128))
    do = randn(rng, (b, sq, h, 128))
    check_grads(run(q, k, v, do, causal), q, k, v, do, causal, what)


def test_backward_token_major_and_repeat():
    announce("bwd token-major, bitwise repeat")
    rng = np.random.default_rng(61)
    q, k, v = randn(rng, (2, 150, 4, 128)), randn(rng, (2, 150, 2, 128)), randn(rng, (2, 150, 2, 128))
    do = randn(rng, (2, 150, 4, 128))
    g1 = run(q, k, v, do, True, token_major=True)
    check_grads(g1, q, k, v, do, True, "token-major")
    g2 = run(q, k, v, do, True, token_major=True)
    for a, b_ in zip(g1, g2):
        np.testing.assert_array_equal(a, b_)


def test_backward_forward_only_configurations_raise():
    """autograd.py:75-109, variant.py:365-384: the forward runs, the backward
    names the unsupported feature."""
    announce("bwd forward-only raises")
    rng = np.random.default_rng(62)
    x = lambda *s: to_dev_bf16(randn(rng, s)).requires_grad_()
    q, k, v = x(1, 2, 64, 128), x(1, 2, 64, 128), x(1, 2, 64, 128)
    for kw, msg in ((dict(window_size=(8, 0)), "window_size"), (dict(softcap=5.0), "softcap"),
                    (dict(learnable_sink=torch.zeros(2, device=DEV)), "learnable_sink")):
        out = flash_attn_func(q, k, v, causal=True, **kw)
        with pytest.raises(NotImplementedError, match=msg):
            out.sum().backward()
    # no gradient requested: the same calls run as plain forwards
    with torch.no_grad():
        flash_attn_func(q, k, v, causal=True, window_size=(8, 0))


def test_varlen_is_forward_only():
    """prefill.py:940-950: flash_attn_varlen_func (packed and paged) runs its
    forward and raises when a gradient is requested."""
    announce("varlen forward-only")
    from flywheel_tpu import flash_attn_varlen_func
    rng = np.random.default_rng(63)
    q = to_dev_bf16(randn(rng, (4, 40, 128))).requires_grad_()
    k = to_dev_bf16(randn(rng, (2, 40, 128))).requires_grad_()
    v = to_dev_bf16(randn(rng, (2, 40, 128)))
    cu = torch.tensor([0, 15, 40], dtype=torch.int32, device=DEV)
    out = flash_attn_varlen_func(q, k, v, cu, cu, 25, 25, causal=True)
    with pytest.raises(NotImplementedError, match="forward-only"):
        out.sum().backward()
    with torch.no_grad():
        ref = flash_attn_varlen_func(q, k, v, cu, cu, 25, 25, causal=True)
    torch.testing.assert_close(out.detach(), ref, rtol=0, atol=0)
    pool = torch.zeros(4, 16, 4, 128, dtype=torch.bfloat16, device=DEV)
    table = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    out = flash_attn_varlen_func(q, pool, None, cu, None, 25, 32, causal=True, block_table=table,
                                 seqused_k=torch.tensor([20, 30], dtype=torch.int32, device=DEV))
    with pytest.raises(NotImplementedError, match="forward-only"):
        out.sum().backward()


@pytest.mark.parametrize("d", [64, 96])
@pytest.mark.parametrize("b,h,hk,sq,sk,causal", [(2, 4, 2, 200, 333, True), (1, 4, 4, 150, 300, False),
                                                 (1, 4, 1, 333, 200, True)])
def test_backward_small_head_dims(d, b, h, hk, sq, sk, causal):
    """Head dims 64 and 96 (the reference's compiled set, test_prefill.py:52,
    285-333) through the head-dim-128 kernels on zero-padded operands."""
    what = f"bwd d{d} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
    announce(what)
    rng = np.random.default_rng(63 + d)
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, d))
    do = randn(rng, (b, sq, h, d))
    check_grads(run(q, k, v, do, causal), q, k, v, do, causal, what)


def test_backward_token_major_d64():
    """The reference's paired token-major d64 form (MHA, even head count)."""
    announce("bwd token-major d64")
    rng = np.random.default_rng(65)
    q, k, v = randn(rng, (2, 140, 4, 64)), randn(rng, (2, 140, 4, 64)), randn(rng, (2, 140, 4, 64))
    do = randn(rng, (2, 140, 4, 64))
    check_grads(run(q, k, v, do, True, token_major=True), q, k, v, do, True, "token-major d64")


WIDE_PAIRS = [(192, 192), (192, 128), (256, 256), (64, 256), (64, 512), (128, 256), (256, 128)]


@pytest.mark.parametrize("d,dv", WIDE_PAIRS)
@pytest.mark.parametrize("b,h,hk,sq,sk,causal", [(2, 4, 2, 200, 333, True), (1, 4, 4, 150, 300, False),
                                                 (1, 4, 1, 333, 200, True),
                                                 (1, 16, 2, 260, 260, True)])
def test_backward_wide_head_dims(d, dv, b, h, hk, sq, sk, causal):
    """The reference's backward pairs above head dim 128 and with head_dim_v
    != head_dim (test_prefill.py:205-208,285-333: 192/128, 192/192, 256/256,
    64/256, 64/512), plus 128/256 and 256/128: the wide kernels, one
    launch per 128-dim chunk of the gradients; the last shape splits a KV
    head's query heads over workgroups (f32 partials at both widths)."""
    what = f"bwd d{d}/{dv} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
    announce(what)
    rng = np.random.default_rng(70 + d + dv)
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, dv))
    do = randn(rng, (b, sq, h, dv))
    check_grads(run(q, k, v, do, causal), q, k, v, do, causal, what)


def test_backward_wide_token_major():
    """Token-major (fused head) layout at 256/128 and 256/256 (token-major
    head dims are multiples of 128, prefill.py:150)."""
    for d, dv in ((256, 128), (256, 256)):
        what = f"bwd token-major d{d}/{dv}"
        announce(what)
        rng = np.random.default_rng(80 + d)
        q, k, v = randn(rng, (2, 150, 4, d)), randn(rng, (2, 150, 2, d)), randn(rng, (2, 150, 2, dv))
        do = randn(rng, (2, 150, 4, dv))
        check_grads(run(q, k, v, do, True, token_major=True), q, k, v, do, True, what)


@pytest.mark.parametrize("d,dv,msg", [(384, 384, "head_dim 384"), (512, 512, "head_dim 512")])
def test_backward_large_head_dims_are_forward_only(d, dv, msg):
    announce(f"bwd d{d}/{dv} forward-only")
    rng = np.random.default_rng(66)
    x = lambda *s: to_dev_bf16(randn(rng, s)).requires_grad_()
    out = flash_attn_func(x(1, 2, 64, d), x(1, 2, 64, d), x(1, 2, 64, dv), causal=True)
    with pytest.raises(NotImplementedError, match=msg):
        out.sum().backward()


@pytest.mark.parametrize("d", [64, 96, 128, 192, 256, 384, 512])
def test_forward_backward_bitwise_repeat_head_dims(d):
    """test_prefill.py:827-875's race check at each head dim: repeated calls
    on the same inputs are bitwise equal (out, and dq / dk / dv where the
    backward exists)."""
    announce(f"repeat d{d}")
    rng = np.random.default_rng(67)
    grad = d <= 256  # a backward exists
    b, h, s = 2, 4, 384
    q, k, v, do = (to_dev_bf16(randn(rng, (b, h, s, d))) for _ in range(4))

    def once():
        ts = [t.detach().clone().requires_grad_(grad) for t in (q, k, v)]
        out = flash_attn_func(*ts, causal=True)
        if grad:
            out.backward(do)
        torch.cuda.synchronize()
        return [out.detach()] + ([t.grad for t in ts] if grad else [])

    ref = once()
    for _ in range(10):
        for a, b_ in zip(once(), ref):
            assert torch.equal(a, b_)


def test_stored_path_matches_recompute_at_c2_shape(monkeypatch):
    """At BASELINE C2's shape (1 x 32/4 heads x 4096, causal) the stored path
    (the P plane, 16 key blocks of 256, 128 query tiles, heads split 8 ways)
    against the recomputing kernels (parity-tested above).  dq is the same
    computation; dk's dS is formed from the stored bf16 P, so it differs by
    bf16 rounding (measured 0.45% of max |dk|); an indexing error in the
    plane would differ by O(1)."""
    announce("bwd stored vs recompute at C2 shape")
    gen = torch.Generator(device=DEV).manual_seed(7)
    b, h, hk, s, d = 1, 32, 4, 4096, 128
    q, k, v, do = (torch.randn((b, n, s, d), generator=gen, device=DEV, dtype=torch.bfloat16)
                   for n in (h, hk, hk, h))

    def grads():
        t = [x.clone().requires_grad_() for x in (q, k, v)]
        flash_attn_func(*t, causal=True).backward(do)
        torch.cuda.synchronize()
        return [x.grad.float() for x in t]

    stored = grads()
    monkeypatch.setenv("FW_BWD_STORED", "0")
    recompute = grads()
    for name, a, r in zip(("dq", "dk", "dv"), stored, recompute):
        err = (a - r).abs().max().item()
        scale = r.abs().max().item()
        print(f"C2 {name}: max |stored - recompute| {err:.3e}, max |grad| {scale:.3e}")
        assert torch.isfinite(a).all()
        assert err <= 1e-2 * scale, (name, err, scale)


@pytest.mark.parametrize("seed", range(24))
def test_backward_random_shapes(seed):
    """Seeded random shapes through the 128/128 backward (the stored path:
    P plane blocks of 32 rows x 64 keys, 256-key dk/dv workgroups, head
    chunks): lengths that are multiples of none of 32, 64, 256, seqlen_q
    above and below seqlen_k, MHA / GQA / MQA, batch 1-2, causal or full,
    head-major or token-major; against the float64 oracle under the
    reference's 3x rule."""
    rng = np.random.default_rng(1000 + seed)
    b = int(rng.integers(1, 3))
    hk = int(rng.choice([1, 2, 4]))
    h = hk * int(rng.choice([1, 2, 4]))
    sq = int(rng.integers(1, 600))
    sk = int(rng.integers(1, 600))
    causal = bool(rng.integers(0, 2))
    token_major = bool(rng.integers(0, 2))
    what = (f"bwd random seed={seed} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
            f" token_major={token_major}")
    announce(what)
    q, k, v = randn(rng, (b, sq, h, 128)), randn(rng, (b, sk, hk, 128)), randn(rng, (b, sk, hk, 128))
    do = randn(rng, (b, sq, h, 128))
    check_grads(run(q, k, v, do, causal, token_major=token_major), q, k, v, do, causal, what)


@pytest.mark.parametrize("d", [192, 256])
@pytest.mark.parametrize("b,h,hk,sq,sk,causal", [(2, 4, 2, 200, 333, True), (1, 4, 1, 333, 200, True),
                                                 (1, 16, 2, 260, 260, True)])
def test_backward_wide_recompute_path(d, b, h, hk, sq, sk, causal, monkeypatch):
    """At head dims 192/192 and 256/256 the stored path (P and dS planes)
    runs by default; FW_BWD_STORED=0 selects the recomputing wide kernels,
    the path above the planes' size limit."""
    monkeypatch.setenv("FW_BWD_STORED", "0")
    what = f"bwd recompute d{d} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
    announce(what)
    rng = np.random.default_rng(62 + d)
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, d))
    do = randn(rng, (b, sq, h, d))
    check_grads(run(q, k, v, do, causal), q, k, v, do, causal, what)


@pytest.mark.parametrize("seed", range(12))
def test_backward_random_shapes_d256(seed):
    """Seeded random shapes through the 256/256 stored path (the dq kernel
    writes P and dS; 128-key dk/dv workgroups read them, with key halves
    and head chunks): lengths that are multiples of none of 32, 64, 128, 256,
    MHA / GQA / MQA, causal or full, head-major or token-major; against the
    float64 oracle under the reference's 3x rule."""
    rng = np.random.default_rng(2000 + seed)
    b = int(rng.integers(1, 3))
    hk = int(rng.choice([1, 2, 4]))
    h = hk * int(rng.choice([1, 2, 4]))
    sq = int(rng.integers(1, 400))
    sk = int(rng.integers(1, 400))
    causal = bool(rng.integers(0, 2))
    token_major = bool(rng.integers(0, 2))
    what = (f"bwd d256 random seed={seed} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal}"
            f" token_major={token_major}")
    announce(what)
    q, k, v = randn(rng, (b, sq, h, 256)), randn(rng, (b, sk, hk, 256)), randn(rng, (b, sk, hk, 256))
    do = randn(rng, (b, sq, h, 256))
    check_grads(run(q, k, v, do, causal, token_major=token_major), q, k, v, do, causal, what)


def test_stored_path_matches_recompute_at_c2_shape_d256(monkeypatch):
    """C2's shape at head dim 256 (1 x 32/4 heads x 4096, causal): the stored
    path (P and dS planes, 32 key blocks of 128, heads split over
    workgroups) against the recomputing wide kernels.  dq is the same
    computation; dk and dv read the bf16-rounded dS and P, so they differ by
    bf16 rounding; an indexing error in a plane would differ by O(1)."""
    announce("bwd d256 stored vs recompute at C2 shape")
    gen = torch.Generator(device=DEV).manual_seed(8)
    b, h, hk, s, d = 1, 32, 4, 4096, 256
    q, k, v, do = (torch.randn((b, n, s, d), generator=gen, device=DEV, dtype=torch.bfloat16)
                   for n in (h, hk, hk, h))

    def grads():
        t = [x.clone().requires_grad_() for x in (q, k, v)]
        flash_attn_func(*t, causal=True).backward(do)
        torch.cuda.synchronize()
        return [x.grad.float() for x in t]

    stored = grads()
    monkeypatch.setenv("FW_BWD_STORED", "0")
    recompute = grads()
    for name, a, r in zip(("dq", "dk", "dv"), stored, recompute):
        err = (a - r).abs().max().item()
        scale = r.abs().max().item()
        print(f"C2 d256 {name}: max |stored - recompute| {err:.3e}, max |grad| {scale:.3e}")
        assert torch.isfinite(a).all()
        assert err <= 1e-2 * scale, (name, err, scale)
