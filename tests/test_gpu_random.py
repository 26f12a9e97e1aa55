"""Randomised GPU parity of every prefill and decode path against the oracle
(head_dim 128, and 64 and 256 in a second set of draws):
dense (GQA ratios, any lengths, causal / windows / softcap / sinks / RoPE),
packed varlen (empty sequences, padding rows), paged varlen over bf16 / e4m3 /
e5m2 pools (page sizes 16-64, descales) and paged decode with the fused append
(1-4 new tokens).  Fixed seeds; each case states its configuration."""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from oracle import attention as A
from oracle import rotary as RO
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, dev_from_codes,
                            randn, to_dev_bf16)

pytestmark = pytest.mark.gpu


def hm(x): return np.ascontiguousarray(x.transpose(0, 2, 1, 3))
def run(name, fn):
    announce(name)
    fn()


def one_case(seed, kind, d=128):
    rng = np.random.default_rng(seed)
    hk = int(rng.choice([1, 2, 4])); G = int(rng.choice([1, 2, 4, 8])); h = hk * G
    causal = bool(rng.integers(0, 2))
    window = (-1, -1)
    if rng.random() < 0.3:
        window = (int(rng.integers(0, 300)), -1 if not causal and rng.random() < 0.5 else 0)
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    sinks = rng.standard_normal(h).astype(np.float32) if rng.random() < 0.2 else None
    if kind == 0:
        b = int(rng.integers(1, 3)); sq = int(rng.integers(1, 700)); sk = int(rng.integers(1, 700))
        rope = rng.random() < 0.25 and softcap == 0.0
        if rope and sq > sk: sq = sk
        name = f"dense d{d} b{b} h{h}/{hk} sq{sq} sk{sk} c{causal} w{window} sc{softcap} sink{sinks is not None} rope{rope}"
        def f():
            q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, d))
            kw = {}
            qr, kr = q, k
            if rope:
                ang = rng.random((sk + 3, d // 2)) * 6.283
                cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
                kw = dict(rotary_cos=torch.tensor(cos, device=DEV), rotary_sin=torch.tensor(sin, device=DEV))
                qp, kp = RO.dense_positions(sq, sk)
                qr = RO.rotate(q.transpose(0, 2, 1, 3), cos, sin, qp, False).transpose(0, 2, 1, 3)
                kr = RO.rotate(k.transpose(0, 2, 1, 3), cos, sin, kp, False).transpose(0, 2, 1, 3)
            out, lse = flash_attn_func(to_dev_bf16(hm(q)), to_dev_bf16(hm(k)), to_dev_bf16(hm(v)), causal=causal,
                                       window_size=window, softcap=softcap, return_softmax_lse=True,
                                       learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV), **kw)
            torch.cuda.synchronize()
            ro, rl = A.attention_ref(qr, kr, v, causal=causal, window_size=window, softcap=softcap, sinks=sinks, round_scaled_q=True)
            assert_close(out.float().cpu().numpy(), hm(ro), what=name)
            assert_lse(lse.cpu().numpy(), rl)
        run(name, f)
    elif kind == 1:
        nseq = int(rng.integers(1, 6))
        ql = rng.integers(0, 300, nseq); kl = ql + rng.integers(0, 300, nseq)
        if not causal: kl = np.maximum(kl, 1)
        name = f"varlen d{d} h{h}/{hk} ql{ql.tolist()} kl{kl.tolist()} c{causal} w{window} sc{softcap}"
        def f():
            cu_q = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
            cu_k = np.concatenate([[0], np.cumsum(kl)]).astype(np.int32)
            pad = int(rng.integers(0, 9))
            q = randn(rng, (h, cu_q[-1] + pad, d)); k = randn(rng, (hk, max(cu_k[-1], 1), d)); v = randn(rng, (hk, max(cu_k[-1], 1), d))
            out, lse = flash_attn_varlen_func(to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), torch.tensor(cu_q, device=DEV),
                                              torch.tensor(cu_k, device=DEV), max(int(ql.max()), 1), max(int(kl.max()), 1),
                                              causal=causal, window_size=window, softcap=softcap, return_softmax_lse=True,
                                              learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
            torch.cuda.synchronize()
            outs, lses = out.float().cpu().numpy(), lse.cpu().numpy()
            for s in range(nseq):
                if ql[s] == 0: continue
                qs_ = q[:, cu_q[s]:cu_q[s+1]].transpose(1, 0, 2)[None]
                ks_ = k[:, cu_k[s]:cu_k[s+1]].transpose(1, 0, 2)[None]
                vs_ = v[:, cu_k[s]:cu_k[s+1]].transpose(1, 0, 2)[None]
                ro, rl = A.attention_ref(qs_, ks_, vs_, causal=causal, window_size=window, softcap=softcap, sinks=sinks, round_scaled_q=True)
                got = outs[:, cu_q[s]:cu_q[s+1]].transpose(1, 0, 2)
                ok = np.isfinite(rl[0]).all(axis=0) if sinks is None else np.ones(ql[s], bool)
                assert_close(got[ok], ro[0][ok], what=f"{name} seq{s}")
            assert not outs[:, cu_q[-1]:].any()
        run(name, f)
    elif kind == 2:
        nseq = int(rng.integers(1, 5))
        dt_name = str(rng.choice(["bf16", "e4m3", "e5m2"]))
        dt = torch.bfloat16 if dt_name == "bf16" else FP8[dt_name]
        ql = rng.integers(0, 200, nseq); pre = rng.integers(0, 800, nseq)
        page = int(rng.choice([16, 32, 64]))
        ks_, vs_ = (1.0, 1.0) if dt_name == "bf16" else (float(rng.uniform(0.5, 2)), float(rng.uniform(0.5, 2)))
        w2 = (window[0], 0) if window[0] >= 0 else (-1, -1)
        name = f"paged d{d} {dt_name} P{page} h{h}/{hk} ql{ql.tolist()} pre{pre.tolist()} c{causal} w{w2} sc{softcap}"
        def f():
            totals = ql + pre
            case = PagedCase(rng, batch=nseq, nheads=h, nheads_k=hk, lengths=totals, new_tokens=[0] * nseq,
                             dtype=dt, k_descale=ks_, v_descale=vs_, page_size=page, head_dim=d)
            cu = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
            q = randn(rng, (cu[-1] + 3, h, d))
            out, lse = flash_attn_varlen_func(
                to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
                torch.tensor(cu, device=DEV), None, max(int(ql.max()), 1), int(max(totals.max(), 1)), causal=causal,
                window_size=w2, softcap=softcap, return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
                seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), k_descale=ks_, v_descale=vs_, nheads_k=hk,
                learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
            torch.cuda.synchronize()
            kp, vp = case.kv_pages(case.pool_codes)
            ro, rl = A.ragged_reference(q, kp, vp, cu, totals, case.table, causal=causal or w2[1] == 0,
                                        window_left=None if w2[0] < 0 else w2[0], softcap=softcap, sinks=sinks,
                                        k_descale=ks_, v_descale=vs_, round_scaled_q=True)
            got = out.float().cpu().numpy().transpose(1, 0, 2)
            ok = np.isfinite(rl).all(axis=0) if sinks is None else np.ones(q.shape[0], bool)
            assert_close(got[ok], ro[ok], fp8=dt_name != "bf16", what=name)
        run(name, f)
    else:
        bsz = int(rng.integers(1, 9)); lens = rng.integers(0, 3000, bsz)
        dt_name = str(rng.choice(["bf16", "e4m3"]))
        dt = torch.bfloat16 if dt_name == "bf16" else FP8[dt_name]
        nq = int(rng.choice([1, 1, 2, 4]))
        w2 = window if not (nq > 1 and window[1] > 0) else (window[0], 0)
        name = f"decode d{d} {dt_name} b{bsz} h{h}/{hk} nq{nq} lens{lens.tolist()} c{causal} w{w2} sc{softcap}"
        def f():
            case = PagedCase(rng, batch=bsz, nheads=h, nheads_k=hk, lengths=lens, new_tokens=[nq] * bsz, dtype=dt,
                             k_descale=1.0, v_descale=1.0, head_dim=d)
            q = randn(rng, (bsz, nq, h, d))
            shape = (bsz, nq, hk, d)
            res = flash_attn_with_kvcache(to_dev_bf16(q), case.pool(), None,
                                          dev_from_codes(case.k_codes.reshape(shape), dt), dev_from_codes(case.v_codes.reshape(shape), dt),
                                          cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=DEV),
                                          block_table=torch.tensor(case.table, device=DEV), causal=causal, window_size=w2,
                                          softcap=softcap, return_softmax_lse=True, nheads_k=hk,
                                          learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
            torch.cuda.synchronize()
            out, lse = res[0], res[1]
            pool_after = case.expected_pool()
            krows, vrows = case.rows(pool_after)
            ro, rl = A.kvcache_reference(q, krows, vrows, lens + nq, causal=causal, window_size=w2, softcap=softcap,
                                         sinks=sinks, k_descale=1.0, v_descale=1.0)
            assert_close(out.float().cpu().numpy(), ro, fp8=dt_name != "bf16", what=name)
        run(name, f)


KINDS = ("dense", "varlen", "paged", "decode")


@pytest.mark.parametrize("kind", range(4), ids=KINDS)
@pytest.mark.parametrize("seed", range(20))
def test_random_case(kind, seed):
    one_case(1000 * kind + seed, kind)


@pytest.mark.parametrize("kind", range(4), ids=KINDS)
@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("d", [64, 256])
def test_random_case_head_dims(d, kind, seed):
    """The same draws at head_dim 64 (register-staged prefill kernel, decode)
    and 256 (the head_dim-256 prefill kernel over bf16 and fp8 pools, decode)."""
    one_case(5000 + 100 * d + 1000 * kind + seed, kind, d)


@pytest.mark.parametrize("kind", range(2), ids=KINDS[:2])
@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("d", [96, 192, 384, 512])
def test_random_case_dense_head_dims(d, kind, seed):
    """Dense and packed-varlen draws (with RoPE, windows, softcap, sinks) at
    the head dims only those paths take: 96, 192 (register-staged kernel),
    384 and 512 (head_dim_v in 128-dim launches)."""
    one_case(9000 + 100 * d + 1000 * kind + seed, kind, d)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("d", [384, 512])
def test_random_case_paged_wide_heads(d, seed):
    """Paged varlen draws (bf16 / e4m3 / e5m2 pools, page sizes 16-64,
    windows, softcap, sinks) at head dims 384 and 512."""
    one_case(20000 + 100 * d + seed, 2, d)
