"""GPU parity of the MFMA prefill kernel (dense, packed varlen, paged varlen,
and chunked prefill through flash_attn_with_kvcache) against the oracle."""

import math

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from oracle import attention as A
from oracle import paged as P
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, codes_of,
                            dev_from_codes, randn, to_dev_bf16)

pytestmark = pytest.mark.gpu


def head_major(x):  # (B, S, H, D) -> (B, H, S, D)
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


@pytest.mark.parametrize(
    "b,h,hk,sq,sk,causal,window,softcap,sinks",
    [
        (1, 8, 2, 512, 512, True, (-1, -1), 0.0, False),
        (2, 4, 4, 200, 333, True, (-1, -1), 0.0, False),
        (1, 4, 1, 333, 200, True, (-1, -1), 0.0, False),  # leading rows see nothing
        (1, 8, 2, 300, 300, False, (-1, -1), 0.0, False),
        (2, 4, 2, 257, 257, False, (64, 17), 0.0, False),
        (1, 4, 2, 384, 384, True, (100, -1), 30.0, False),
        # softcap tanh paths (N(0,1) scores, |s| < 6): exact (|s/5| > 0.3 somewhere in every
        # tile), degree-5 polynomial (0.12 < max |s/20| <= 0.3), degree-3 (max |s/50| <= 0.12)
        (1, 4, 1, 512, 512, True, (-1, -1), 5.0, False),
        (1, 4, 1, 512, 512, True, (-1, -1), 20.0, False),
        (1, 4, 1, 512, 512, True, (-1, -1), 50.0, False),
        (1, 4, 2, 130, 130, True, (-1, -1), 0.0, True),
        # head packing: 3 (one head per workgroup), 6 (two), 16 (8 per workgroup, two
        # workgroups per KV head) query heads per KV head
        (1, 6, 2, 300, 300, True, (-1, -1), 0.0, False),
        (2, 12, 2, 200, 260, True, (40, -1), 0.0, True),
        (1, 16, 1, 100, 400, True, (-1, -1), 50.0, False),
        (1, 16, 2, 77, 77, False, (-1, -1), 0.0, False),
    ],
)
def test_flash_attn_func(b, h, hk, sq, sk, causal, window, softcap, sinks):
    announce(f"dense b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal} window={window} softcap={softcap}")
    rng = np.random.default_rng(10)
    q, k, v = randn(rng, (b, sq, h, 128)), randn(rng, (b, sk, hk, 128)), randn(rng, (b, sk, hk, 128))
    s = rng.standard_normal(h).astype(np.float32) if sinks else None
    out, lse = flash_attn_func(
        to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)), to_dev_bf16(head_major(v)),
        causal=causal, window_size=window, softcap=softcap, return_softmax_lse=True,
        learnable_sink=None if s is None else torch.tensor(s, device=DEV))
    torch.cuda.synchronize()
    ro, rl = A.attention_ref(q, k, v, causal=causal, window_size=window, softcap=softcap, sinks=s,
                             round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)


def test_flash_attn_func_layouts():
    """token_major and heads_outer_fold address the same math in place."""
    announce("dense layouts")
    rng = np.random.default_rng(11)
    b, h, hk, s, d = 2, 4, 2, 160, 128
    q, k, v = randn(rng, (b, s, h, d)), randn(rng, (b, s, hk, d)), randn(rng, (b, s, hk, d))
    ro, _ = A.attention_ref(q, k, v, causal=True, round_scaled_q=True)
    out = flash_attn_func(to_dev_bf16(q.reshape(b, s, h * d)), to_dev_bf16(k.reshape(b, s, hk * d)),
                          to_dev_bf16(v.reshape(b, s, hk * d)), causal=True, head_dim=d,
                          token_major=True)
    assert_close(out.float().cpu().numpy().reshape(b, s, h, d), ro)
    hof = lambda x: np.ascontiguousarray(x.transpose(2, 0, 1, 3))  # (H, B, S, D)
    out = flash_attn_func(to_dev_bf16(hof(q)), to_dev_bf16(hof(k)), to_dev_bf16(hof(v)),
                          causal=True, heads_outer_fold=True)
    assert_close(out.float().cpu().numpy(), hof(ro))


def test_flash_attn_func_c2_full_size():
    """BASELINE config 2 at full size; the oracle checks 4 of the 32 heads."""
    announce("dense C2 1x32/4x4096")
    rng = np.random.default_rng(12)
    q, k, v = randn(rng, (1, 4096, 32, 128)), randn(rng, (1, 4096, 4, 128)), randn(rng, (1, 4096, 4, 128))
    out, lse = flash_attn_func(to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)),
                               to_dev_bf16(head_major(v)), causal=True, return_softmax_lse=True)
    torch.cuda.synchronize()
    heads = [0, 9, 18, 31]  # query head h reads KV head h // 8
    outs = out.float().cpu().numpy()
    lses = lse.cpu().numpy()
    for hh in heads:
        ro, rl = A.attention_ref(q[:, :, [hh]], k[:, :, [hh // 8]], v[:, :, [hh // 8]], causal=True,
                                 round_scaled_q=True)
        assert_close(outs[:, hh], ro[:, :, 0], what=f"head {hh}")
        assert_lse(lses[:, [hh]], rl)


@pytest.mark.parametrize("b,h,hk,sq,sk,causal,window,softcap,sinks", [
    (1, 32, 4, 4096, 4096, True, (-1, -1), 0.0, False),     # C2
    (1, 32, 4, 4096, 4096, False, (-1, -1), 0.0, False),
    (1, 32, 4, 4096, 4096, True, (1000, 0), 0.0, True),
    (1, 32, 4, 4096, 4096, True, (-1, -1), 30.0, False),
    (1, 32, 4, 4096, 6000, True, (-1, -1), 0.0, False),     # keys past the queries
    (2, 32, 32, 4096, 4096, True, (-1, -1), 0.0, False),    # MHA: XCD-aware head groups
])
@pytest.mark.parametrize("d", [128, 256])
def test_pair_kernel_matches_one_tile_kernel(d, b, h, hk, sq, sk, causal, window, softcap, sinks,
                                             monkeypatch):
    """Dense grids whose q tiles pair up and whose half still covers every CU
    run fw_prefill_pp_pair_kernel / fw_prefill_d256_pair_kernel (a heavy q
    tile, then its mirror of the same head group, per workgroup);
    FW_PREFILL_PAIR=0 runs one q tile per workgroup.  Both compute every tile the same way: bitwise equal out and
    lse, and the C2 full-size test above checks the pair kernel against the
    oracle."""
    announce(f"pair kernel d{d} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal} window={window}"
             f" softcap={softcap} sinks={sinks}")
    gen = torch.Generator(device=DEV).manual_seed(21)
    q = torch.randn((b, h, sq, d), generator=gen, device=DEV, dtype=torch.bfloat16)
    k = torch.randn((b, hk, sk, d), generator=gen, device=DEV, dtype=torch.bfloat16)
    v = torch.randn((b, hk, sk, d), generator=gen, device=DEV, dtype=torch.bfloat16)
    kw = dict(causal=causal, window_size=window, softcap=softcap, return_softmax_lse=True)
    if sinks:
        kw["learnable_sink"] = torch.randn((h,), generator=gen, device=DEV, dtype=torch.float32)
    out_p, lse_p = flash_attn_func(q, k, v, **kw)
    monkeypatch.setenv("FW_PREFILL_PAIR", "0")
    out_1, lse_1 = flash_attn_func(q, k, v, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(out_p.float()).all()
    assert torch.equal(out_p, out_1)
    assert torch.equal(lse_p, lse_1)


@pytest.mark.parametrize("causal,window,softcap", [(True, (-1, -1), 0.0), (False, (-1, -1), 0.0),
                                                   (True, (50, -1), 20.0)])
def test_flash_attn_varlen_packed(causal, window, softcap):
    announce(f"varlen packed causal={causal} window={window}")
    rng = np.random.default_rng(13)
    qlens, klens = [5, 130, 1, 300], [9, 130, 40, 512]
    h, hk, d = 8, 2, 128
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    pad = 7
    q = randn(rng, (h, cu_q[-1] + pad, d))
    k = randn(rng, (hk, cu_k[-1] + 3, d))
    v = randn(rng, (hk, cu_k[-1] + 3, d))
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), torch.tensor(cu_q, device=DEV),
        torch.tensor(cu_k, device=DEV), max(qlens), max(klens), causal=causal, window_size=window,
        softcap=softcap, return_softmax_lse=True)
    torch.cuda.synchronize()
    outs, lses = out.float().cpu().numpy(), lse.cpu().numpy()
    for s in range(4):
        qs = q[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2)[None]
        ks = k[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        vs = v[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        ro, rl = A.attention_ref(qs, ks, vs, causal=causal, window_size=window, softcap=softcap,
                                 round_scaled_q=True)
        got = outs[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2)
        rows_ok = np.isfinite(rl[0]).all(axis=0)  # rows with no visible key are unspecified
        assert_close(got[rows_ok], ro[0][rows_ok], what=f"seq {s}")
        assert_lse(lses[:, cu_q[s]:cu_q[s + 1]][:, rows_ok], rl[0][:, rows_ok])
    assert not outs[:, cu_q[-1]:].any()
    assert np.isneginf(lses[:, cu_q[-1]:]).all()


@pytest.mark.parametrize("nseq", [300, 2100])
def test_flash_attn_varlen_many_sequences(nseq):
    """Many short packed sequences: the tile schedule orders up to 2048 q tiles
    by cost (300) and keeps the sequence order beyond that (2100)."""
    announce(f"varlen packed many sequences n={nseq}")
    rng = np.random.default_rng(15)
    qlens = rng.integers(1, 5, nseq)
    qlens[::97] = 300  # a few multi-tile sequences among the short ones
    klens = qlens + rng.integers(0, 40, nseq)
    h, hk, d = 2, 1, 128
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn(rng, (h, cu_q[-1], d))
    k = randn(rng, (hk, cu_k[-1], d))
    v = randn(rng, (hk, cu_k[-1], d))
    out = flash_attn_varlen_func(
        to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), torch.tensor(cu_q, device=DEV),
        torch.tensor(cu_k, device=DEV), int(qlens.max()), int(klens.max()), causal=True)
    torch.cuda.synchronize()
    outs = out.float().cpu().numpy()
    for s in range(nseq):
        qs = q[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2)[None]
        ks = k[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        vs = v[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        ro, _ = A.attention_ref(qs, ks, vs, causal=True, round_scaled_q=True)
        assert_close(outs[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2), ro[0], what=f"seq {s}")


@pytest.mark.parametrize("dtype", ["bf16", "e4m3", "e5m2"])
@pytest.mark.parametrize("h,hk", [(4, 2), (8, 1), (16, 2), (6, 3)])
def test_paged_varlen_read_only(dtype, h, hk):
    """flash_attn_varlen_func(block_table=...) over a merged pool; reference
    edge case random_ragged_case lengths (3, 0, 5) on prefixes (127, 0, 251).
    Heads: 2 or 8 query heads per KV head (one workgroup serves 2 or 8), and
    an odd KV head count (the fp8 pool's zero pad head)."""
    announce(f"paged varlen {dtype} h{h}/{hk}")
    rng = np.random.default_rng(14)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (0.5, 2.0)
    qlens = [3, 0, 5, 200]
    prefix = [127, 0, 251, 1000]
    totals = np.array(qlens) + np.array(prefix)
    case = PagedCase(rng, batch=4, nheads=h, nheads_k=hk, lengths=totals, new_tokens=[0] * 4,
                     dtype=dt, k_descale=ks, v_descale=vs)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1] + 7, h, 128))
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
        torch.tensor(cu, device=DEV), None, max(qlens), int(totals.max()), causal=True,
        return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), k_descale=ks,
        v_descale=vs, nheads_k=hk)
    torch.cuda.synchronize()
    kp, vp = case.kv_pages(case.pool_codes)
    ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=True, k_descale=ks,
                                v_descale=vs, round_scaled_q=True)
    assert_close(out.float().cpu().numpy().transpose(1, 0, 2), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
def test_chunked_prefill_kvcache(dtype):
    """BASELINE config 4's call at reduced size: packed chunks appended to the
    paged cache then attended causally with a sliding window and softcap;
    num_active leaves the last request out."""
    announce(f"chunked prefill {dtype}")
    rng = np.random.default_rng(15)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (1.5, 0.7)
    chunks = [256, 700, 1, 129, 64]
    prior = [0, 3000, 17, 999, 50]
    case = PagedCase(rng, batch=5, nheads=8, nheads_k=2, lengths=prior, new_tokens=chunks,
                     dtype=dt, k_descale=ks, v_descale=vs)
    cu = case.cu
    q = randn(rng, (cu[-1] + 5, 8, 128))
    k_dev = dev_from_codes(np.concatenate([case.k_codes, np.zeros((5, 2, 128), case.k_codes.dtype)]), dt)
    v_dev = dev_from_codes(np.concatenate([case.v_codes, np.zeros((5, 2, 128), case.v_codes.dtype)]), dt)
    pool = case.pool()
    out, lse, pool2 = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, k_dev, v_dev,
        cache_seqlens=torch.tensor(prior, dtype=torch.int32, device=DEV),
        block_table=torch.tensor(case.table, device=DEV),
        cu_seqlens_q=torch.tensor(cu, device=DEV), max_seqlen_q=max(chunks), causal=True,
        window_size=(4095 // 8, 0), softcap=50.0, return_softmax_lse=True, num_active=4,
        k_descale=ks, v_descale=vs)
    torch.cuda.synchronize()
    assert pool2 is pool
    exp_pool = case.expected_pool(num_active=4)
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    kp, vp = case.kv_pages(exp_pool)
    totals = case.lengths + case.new_tokens
    ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=True,
                                window_left=4095 // 8, softcap=50.0, k_descale=ks, v_descale=vs,
                                round_scaled_q=True, num_active=4)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
    assert not out[cu[4]:].float().abs().sum().item()


def test_prefill_bitwise_repeat():
    """test_prefill.py:827-875's race check: repeats are bitwise equal."""
    announce("dense repeat")
    rng = np.random.default_rng(16)
    q = to_dev_bf16(randn(rng, (1, 8, 1024, 128)))
    k = to_dev_bf16(randn(rng, (1, 2, 1024, 128)))
    v = to_dev_bf16(randn(rng, (1, 2, 1024, 128)))
    ref = flash_attn_func(q, k, v, causal=True)
    for _ in range(20):
        assert torch.equal(flash_attn_func(q, k, v, causal=True), ref)


# ---------------------------------------------------------------- head_dim 256
# The reference benchmarks and accepts head_dim 256 (multiples of 128,
# inputs.py:100-140, fwd_paged.py:1186); its published shapes are d256
# (docs/v7x.md:49-60, 157-169).


# Head dims of q/k and v: the d256 kernel, the register-staged kernel at 64, 96
# and 192 and with head_dim_v != head_dim (inputs.py:193-207); the reference's
# compiled set (test_prefill.py:52,205-208), 384 and 512 (multiples of 128,
# inputs.py:100-140) plus 128/256 and 256/128.  A head_dim_v above 256 runs as
# launches over chunks of v and out.
HEAD_DIMS = [(256, 256), (64, 64), (128, 256), (256, 128), (96, 96), (192, 192), (192, 128),
             (64, 256), (64, 512), (384, 384), (512, 512)]


@pytest.mark.parametrize("d,dv", HEAD_DIMS)
@pytest.mark.parametrize(
    "b,h,hk,sq,sk,causal,window,softcap",
    [
        (1, 8, 2, 512, 512, True, (-1, -1), 0.0),
        (2, 4, 4, 200, 333, True, (-1, -1), 0.0),
        (1, 4, 1, 333, 200, True, (-1, -1), 0.0),
        (1, 4, 2, 257, 257, False, (64, 17), 0.0),
        (1, 8, 1, 384, 384, True, (100, -1), 30.0),
    ],
)
def test_flash_attn_func_head_dims(d, dv, b, h, hk, sq, sk, causal, window, softcap):
    announce(f"dense d{d}/{dv} b{b} h{h}/{hk} sq{sq} sk{sk} causal={causal} window={window}")
    rng = np.random.default_rng(70)
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, dv))
    out, lse = flash_attn_func(
        to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)), to_dev_bf16(head_major(v)),
        causal=causal, window_size=window, softcap=softcap, return_softmax_lse=True)
    torch.cuda.synchronize()
    ro, rl = A.attention_ref(q, k, v, causal=causal, window_size=window, softcap=softcap,
                             round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("jump", [40.0, 600.0])
def test_flash_attn_func_anchor_rescale(d, jump):
    """The slow path of the static anchor (new row maximum, O and l rescaled)
    taken twice per row: keys in thirds score 0, J/2 and J (log2 units), values
    1, 2, 3.  J = 40 rescales by 2^-20 twice (the rescale must reach every O
    register: one left unscaled moves out by ~1); J = 600 underflows the
    factor to 0 (as the reference's anchor-change test,
    test_regression.py:1035-1063).  Out is ~3 in closed form."""
    announce(f"dense d{d} anchor rescale jump {jump}")
    sk, sq, h = 768, 256, 2
    y = jump / (math.sqrt(d) * A.LOG2E)  # q = 1: score(log2) = y * sqrt(d) * log2(e)
    q = np.ones((1, sq, h, d), np.float32)
    k = np.zeros((1, sk, 1, d), np.float32)
    v = np.ones((1, sk, 1, d), np.float32)
    k[:, 256:512], k[:, 512:] = y / 2, y
    v[:, 256:512], v[:, 512:] = 2.0, 3.0
    q, k, v = (np.asarray(torch.tensor(x).to(torch.bfloat16).float()) for x in (q, k, v))
    out, lse = flash_attn_func(to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)),
                               to_dev_bf16(head_major(v)), return_softmax_lse=True)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    np.testing.assert_allclose(o, 3.0, atol=2e-2)
    ro, rl = A.attention_ref(q, k, v, round_scaled_q=True)
    assert_close(o, head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("d,dv", HEAD_DIMS)
def test_flash_attn_func_head_dims_sinks(d, dv):
    """learnable_sink through the d256 and register-staged kernels (rows that
    see no key return the sink-only result: out 0, lse = the sink)."""
    announce(f"dense d{d}/{dv} sinks")
    rng = np.random.default_rng(74)
    b, h, hk, sq, sk = 1, 8, 2, 200, 150
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, dv))
    sinks = rng.standard_normal(h).astype(np.float32)
    out, lse = flash_attn_func(
        to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)), to_dev_bf16(head_major(v)),
        causal=True, return_softmax_lse=True, learnable_sink=torch.tensor(sinks, device=DEV))
    torch.cuda.synchronize()
    ro, rl = A.attention_ref(q, k, v, causal=True, sinks=sinks, round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)


def test_flash_attn_func_token_major_paired_d64():
    """Token-major head_dim 64 (the reference's paired form: MHA, even head
    count, inputs.py:106-147)."""
    announce("dense token-major d64")
    rng = np.random.default_rng(73)
    b, h, s, d = 2, 6, 300, 64
    q, k, v = randn(rng, (b, s, h, d)), randn(rng, (b, s, h, d)), randn(rng, (b, s, h, d))
    out = flash_attn_func(to_dev_bf16(q.reshape(b, s, h * d)), to_dev_bf16(k.reshape(b, s, h * d)),
                          to_dev_bf16(v.reshape(b, s, h * d)), causal=True, head_dim=d,
                          token_major=True)
    torch.cuda.synchronize()
    ro, _ = A.attention_ref(q, k, v, causal=True, round_scaled_q=True)
    assert_close(out.float().cpu().numpy().reshape(b, s, h, d), ro)


@pytest.mark.parametrize("d,dv", HEAD_DIMS)
def test_flash_attn_varlen_head_dims(d, dv):
    announce(f"varlen packed d{d}/{dv}")
    rng = np.random.default_rng(71)
    qlens, klens = [1, 130, 77, 256], [1, 200, 77, 300]
    h, hk = 4, 2
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn(rng, (h, cu_q[-1] + 5, d))
    k = randn(rng, (hk, cu_k[-1], d))
    v = randn(rng, (hk, cu_k[-1], dv))
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), torch.tensor(cu_q, device=DEV),
        torch.tensor(cu_k, device=DEV), max(qlens), max(klens), causal=True,
        return_softmax_lse=True)
    torch.cuda.synchronize()
    outs, lses = out.float().cpu().numpy(), lse.cpu().numpy()
    for s in range(4):
        qs = q[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2)[None]
        ks = k[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        vs = v[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        ro, rl = A.attention_ref(qs, ks, vs, causal=True, round_scaled_q=True)
        assert_close(outs[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2), ro[0], what=f"seq {s}")
        assert_lse(lses[:, cu_q[s]:cu_q[s + 1]], rl[0])
    assert not outs[:, cu_q[-1]:].any()


@pytest.mark.parametrize("hd", [256, 64, 384, 512])
@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
def test_chunked_prefill_kvcache_head_dims(dtype, hd):
    """The chunked-prefill call (append + paged varlen, window, softcap,
    num_active) at head_dim 256, 64, 384 and 512 (the reference's paged
    prefill takes any multiple of 128 shared by q and the pool,
    kernels/fwd_paged.py:1186-1190)."""
    announce(f"chunked prefill d{hd} {dtype}")
    rng = np.random.default_rng(72)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (1.5, 0.7)
    chunks = [256, 300, 1, 129]
    prior = [0, 1000, 17, 500]
    case = PagedCase(rng, batch=4, nheads=8, nheads_k=2, lengths=prior, new_tokens=chunks,
                     head_dim=hd, dtype=dt, k_descale=ks, v_descale=vs)
    cu = case.cu
    q = randn(rng, (cu[-1], 8, hd))
    pool = case.pool()
    out, lse, pool2 = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, dev_from_codes(case.k_codes, dt),
        dev_from_codes(case.v_codes, dt),
        cache_seqlens=torch.tensor(prior, dtype=torch.int32, device=DEV),
        block_table=torch.tensor(case.table, device=DEV),
        cu_seqlens_q=torch.tensor(cu, device=DEV), max_seqlen_q=max(chunks), causal=True,
        window_size=(400, 0), softcap=30.0, return_softmax_lse=True, num_active=3,
        k_descale=ks, v_descale=vs)
    torch.cuda.synchronize()
    assert pool2 is pool
    exp_pool = case.expected_pool(num_active=3)
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    kp, vp = case.kv_pages(exp_pool)
    totals = case.lengths + case.new_tokens
    ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=True, window_left=400,
                                softcap=30.0, k_descale=ks, v_descale=vs, round_scaled_q=True,
                                num_active=3)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("hd", [384, 512])
@pytest.mark.parametrize("dtype", ["bf16", "e4m3", "e5m2"])
def test_paged_varlen_read_only_wide_heads(dtype, hd):
    """flash_attn_varlen_func(block_table=...) over a merged pool at head dims
    384 and 512 (launched as 128-dim chunks of V, each chunk reading its dims
    of the merged row's V head): random_ragged_case's (3, 0, 5) on prefixes
    (127, 0, 251), plus a longer request, with an odd KV head count."""
    announce(f"paged varlen d{hd} {dtype}")
    rng = np.random.default_rng(91 + hd)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (0.5, 2.0)
    h, hk = 6, 3
    qlens = [3, 0, 5, 300]
    prefix = [127, 0, 251, 700]
    totals = np.array(qlens) + np.array(prefix)
    case = PagedCase(rng, batch=4, nheads=h, nheads_k=hk, lengths=totals, new_tokens=[0] * 4,
                     dtype=dt, k_descale=ks, v_descale=vs, head_dim=hd)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1] + 7, h, hd))
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
        torch.tensor(cu, device=DEV), None, max(qlens), int(totals.max()), causal=True,
        window_size=(200, 0), softcap=20.0,
        return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), k_descale=ks,
        v_descale=vs, nheads_k=hk)
    torch.cuda.synchronize()
    kp, vp = case.kv_pages(case.pool_codes)
    ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=True, window_left=200,
                                softcap=20.0, k_descale=ks, v_descale=vs, round_scaled_q=True)
    got = out.float().cpu().numpy().transpose(1, 0, 2)
    assert_close(got[:cu[-1]], ro[:cu[-1]], fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy()[:, :cu[-1]], rl[:, :cu[-1]])
    assert not got[cu[-1]:].any()


@pytest.mark.parametrize("dtype,window,softcap,sinks", [
    ("bf16", -1, 0.0, False), ("bf16", 1000, 30.0, True), ("e4m3", -1, 50.0, False),
    ("bf16", 300, 0.0, True)])
def test_key_split_slots(dtype, window, softcap, sinks):
    """Few heavy q tiles over long prior contexts: the schedule splits the
    heaviest slots in two along their keys (fewer workgroups than CUs), each
    half stores an (m, l, O) partial and the second to finish merges them.
    Windows leave rows with no key in one half; sinks fold in after the
    merge."""
    announce(f"key split {dtype} window {window} softcap {softcap} sinks {sinks}")
    rng = np.random.default_rng(400 + window)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (0.8, 1.25)
    h, hk = 32, 8
    qlens = [300, 100, 64]
    prefix = [4000, 700, 2500]
    totals = np.array(qlens) + np.array(prefix)
    case = PagedCase(rng, batch=3, nheads=h, nheads_k=hk, lengths=totals, new_tokens=[0] * 3,
                     dtype=dt, k_descale=ks, v_descale=vs)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1], h, 128))
    sk = rng.standard_normal(h).astype(np.float32) if sinks else None
    w2 = (window, 0) if window >= 0 else (-1, -1)
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
        torch.tensor(cu, device=DEV), None, max(qlens), int(totals.max()), causal=True,
        window_size=w2, softcap=softcap, return_softmax_lse=True,
        block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), k_descale=ks,
        v_descale=vs, nheads_k=hk, learnable_sink=None if sk is None else torch.tensor(sk, device=DEV))
    torch.cuda.synchronize()
    kp, vp = case.kv_pages(case.pool_codes)
    ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=True,
                                window_left=None if window < 0 else window, softcap=softcap,
                                sinks=sk, k_descale=ks, v_descale=vs, round_scaled_q=True)
    assert_close(out.float().cpu().numpy().transpose(1, 0, 2), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
    # the same call again: the arrival counters start from zero every call
    out2 = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
        torch.tensor(cu, device=DEV), None, max(qlens), int(totals.max()), causal=True,
        window_size=w2, softcap=softcap, block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), k_descale=ks,
        v_descale=vs, nheads_k=hk, learnable_sink=None if sk is None else torch.tensor(sk, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_key_split_packed_varlen():
    """The packed-varlen (non-paged) mode of the same kernel with split slots."""
    announce("key split packed varlen")
    rng = np.random.default_rng(410)
    h, hk, d = 16, 4, 128
    ql = np.array([256, 70]); kl = np.array([3000, 1500])
    cu_q = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(kl)]).astype(np.int32)
    q, k, v = randn(rng, (h, cu_q[-1], d)), randn(rng, (hk, cu_k[-1], d)), randn(rng, (hk, cu_k[-1], d))
    out, lse = flash_attn_varlen_func(to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v),
                                      torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV),
                                      int(ql.max()), int(kl.max()), causal=True,
                                      return_softmax_lse=True)
    torch.cuda.synchronize()
    outs, lses = out.float().cpu().numpy(), lse.cpu().numpy()
    for s in range(2):
        qs_ = q[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2)[None]
        ks_ = k[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        vs_ = v[:, cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2)[None]
        ro, rl = A.attention_ref(qs_, ks_, vs_, causal=True, round_scaled_q=True)
        assert_close(outs[:, cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2), ro[0], what=f"seq {s}")
        assert_lse(lses[:, cu_q[s]:cu_q[s + 1]], rl[0])


@pytest.mark.parametrize("h,hk,q_len,kv_len,offset,fold", [
    (8, 2, 300, 1000, 0, False), (8, 2, 300, 1000, 700, False), (4, 4, 129, 700, 333, True),
    (16, 2, 1024, 4096, 2048, False)])
def test_runtime_causal_offset(h, hk, q_len, kv_len, offset, fold):
    """The dense forward with a device-side causal offset (reference
    prefill.py:344-434): query i sees keys 0 .. offset + i; against the oracle
    on the first offset + q_len keys with bottom-right causal alignment."""
    from flywheel_tpu.prefill import _flash_attn_func_pcp_causal_offset
    announce(f"runtime causal offset h{h}/{hk} q{q_len} kv{kv_len} off{offset} fold{fold}")
    rng = np.random.default_rng(500 + offset)
    q, k, v = randn(rng, (1, q_len, h, 128)), randn(rng, (1, kv_len, hk, 128)), randn(rng, (1, kv_len, hk, 128))
    hm = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))
    dev = [to_dev_bf16(hm(x)) for x in (q, k, v)]
    if fold:
        dev = [t.transpose(0, 1).contiguous() for t in dev]
    out, lse = _flash_attn_func_pcp_causal_offset(
        *dev, torch.tensor(offset, dtype=torch.int32, device=DEV), return_softmax_lse=True,
        heads_outer_fold=fold)
    torch.cuda.synchronize()
    if fold:
        out = out.transpose(0, 1)
    assert lse.shape == (1, h, q_len)
    n = offset + q_len
    ro, rl = A.attention_ref(q, k[:, :n], v[:, :n], causal=True, round_scaled_q=True)
    assert_close(out.float().cpu().numpy().transpose(0, 2, 1, 3), ro)
    assert_lse(lse.cpu().numpy(), rl)
