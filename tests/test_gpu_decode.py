"""GPU parity of flash_attn_with_kvcache's decode paths (single token with the
fused append, folded verify window) against the NumPy oracle."""

import math

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_with_kvcache
from flywheel_tpu.decode import paged_decode
from oracle import attention as A
from oracle import dtypes as T
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, codes_of,
                            randn, to_dev_bf16)

pytestmark = pytest.mark.gpu

# test_decode_packed.py:44 PREFIXES at capacity 1024
PREFIXES = (0, 300, 1, 1022, 255, 256, 511, 700)


def run_decode(case, q, *, append=True, causal=False, window=(-1, -1), softcap=0.0, sinks=None,
               num_active=None, return_lse=True):
    pool = case.pool()
    kw = {}
    if append:
        shape = (case.batch, q.shape[1], case.nheads_k, case.head_dim)
        from tests.gpu_util import dev_from_codes
        kw["k"] = dev_from_codes(case.k_codes.reshape(shape), case.dtype)
        kw["v"] = dev_from_codes(case.v_codes.reshape(shape), case.dtype)
    res = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, **kw,
        cache_seqlens=torch.tensor(case.lengths, dtype=torch.int32, device=DEV),
        block_table=torch.tensor(case.table, device=DEV), causal=causal, window_size=window,
        softcap=softcap, return_softmax_lse=return_lse, nheads_k=case.nheads_k,
        k_descale=case.k_descale, v_descale=case.v_descale, num_active=num_active,
        learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
    torch.cuda.synchronize()
    assert res[-1] is pool
    return res


def oracle(case, q, pool_codes, *, append=True, causal=False, window=(-1, -1), softcap=0.0,
           sinks=None):
    krows, vrows = case.rows(pool_codes)
    totals = case.lengths + (case.new_tokens if append else 0)
    return A.kvcache_reference(q, krows, vrows, totals, causal=causal, window_size=window,
                               softcap=softcap, sinks=sinks, k_descale=case.k_descale,
                               v_descale=case.v_descale)


@pytest.mark.parametrize("append", [True, False])
def test_decode_bf16_prefixes(append):
    announce(f"decode bf16 PREFIXES append={append}")
    rng = np.random.default_rng(0)
    b = len(PREFIXES)
    case = PagedCase(rng, batch=b, nheads=8, nheads_k=2, lengths=PREFIXES,
                     new_tokens=[1 if append else 0] * b, max_pages=1024 // 16 + 1)
    q = randn(rng, (b, 1, 8, 128))
    out, lse, pool = run_decode(case, q, append=append)
    exp_pool = case.expected_pool() if append else case.pool_codes
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool, append=append)
    nonempty = (case.lengths + (1 if append else 0)) > 0
    assert_close(out.float().cpu().numpy()[nonempty], ro[nonempty])
    assert_lse(lse.cpu().numpy(), rl)


def test_decode_c3_shape_small_batch():
    """C3's geometry (32 q / 8 KV heads, page 16) at batch 6, contexts up to 32K."""
    announce("decode C3 geometry batch 6")
    rng = np.random.default_rng(1)
    lengths = [1024, 32767, 5000, 17, 16, 20000]
    case = PagedCase(rng, batch=6, nheads=32, nheads_k=8, lengths=lengths, new_tokens=[1] * 6)
    q = randn(rng, (6, 1, 32, 128))
    out, lse, pool = run_decode(case, q)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool)
    assert_close(out.float().cpu().numpy(), ro)
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("window,softcap,with_sinks", [((100, -1), 0.0, False), ((-1, -1), 15.0, False),
                                                       ((37, 0), 50.0, True), ((-1, -1), 0.0, True)])
def test_decode_window_softcap_sinks(window, softcap, with_sinks):
    announce(f"decode window={window} softcap={softcap} sinks={with_sinks}")
    rng = np.random.default_rng(2)
    lengths = [0, 5, 129, 700, 2047]
    case = PagedCase(rng, batch=5, nheads=8, nheads_k=2, lengths=lengths, new_tokens=[1] * 5)
    q = randn(rng, (5, 1, 8, 128))
    sinks = rng.standard_normal(8).astype(np.float32) * 2 if with_sinks else None
    if with_sinks:
        sinks[1] = -np.inf
    out, lse, pool = run_decode(case, q, window=window, softcap=softcap, sinks=sinks)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool, window=window, softcap=softcap, sinks=sinks)
    assert_close(out.float().cpu().numpy(), ro)
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("hk", [8, 3])
def test_decode_fp8(fmt, hk):
    announce(f"decode fp8 {fmt} hk={hk}")
    rng = np.random.default_rng(3)
    lengths = [4096, 33, 1000, 7]
    ks, vs = 0.75, 1.5
    case = PagedCase(rng, batch=4, nheads=4 * hk, nheads_k=hk, lengths=lengths, new_tokens=[1] * 4,
                     dtype=FP8[fmt], k_descale=ks, v_descale=vs)
    q = randn(rng, (4, 1, 4 * hk, 128))
    out, lse, pool = run_decode(case, q)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool)
    assert_close(out.float().cpu().numpy(), ro, fp8=True)
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
def test_folded_verify_window(dtype):
    """C5's shape of call: 4 query tokens per row, causal, appended first."""
    announce(f"verify window {dtype}")
    rng = np.random.default_rng(4)
    lengths = [4096, 100, 9000, 3]
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (1.25, 0.6)
    case = PagedCase(rng, batch=4, nheads=32, nheads_k=8, lengths=lengths, new_tokens=[4] * 4,
                     dtype=dt, k_descale=ks, v_descale=vs)
    q = randn(rng, (4, 4, 32, 128))
    out, lse, pool = run_decode(case, q, causal=True)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool, causal=True)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("dtype,sq,nheads,splits", [
    ("bf16", 3, 8, 0), ("e4m3", 16, 8, 0), ("bf16", 20, 24, 0), ("bf16", 5, 8, 300),
    ("e4m3", 7, 8, 300)])
def test_verify_window_boundaries(dtype, sq, nheads, splits):
    """Folded verify windows of 3 to 20 tokens whose new keys straddle a
    32-key tile (L0 % 32 = 30, 31) and, with 300 key ranges, the boundary
    between two workgroups' ranges (every range a few tiles); the whole pool,
    appended rows included, bit-exact."""
    announce(f"verify window boundaries {dtype} sq={sq} heads={nheads} splits={splits}")
    rng = np.random.default_rng(40 + sq)
    lengths = [30, 62, 1000, 0, 95, 4127]
    b = len(lengths)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (1.25, 0.6)
    case = PagedCase(rng, batch=b, nheads=nheads, nheads_k=8 if nheads == 8 else 4, lengths=lengths,
                     new_tokens=[sq] * b, dtype=dt, k_descale=ks, v_descale=vs)
    q = randn(rng, (b, sq, nheads, 128))
    if splits:
        # the API's two launches, the decode one with `splits` key ranges
        from flywheel_tpu.decode import append_ragged
        from tests.gpu_util import dev_from_codes
        pool = case.pool()
        shape = (b * sq, case.nheads_k, 128)
        lens = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
        table = torch.tensor(case.table, device=DEV)
        append_ragged(pool, dev_from_codes(case.k_codes.reshape(shape), case.dtype),
                      dev_from_codes(case.v_codes.reshape(shape), case.dtype), None, lens, table,
                      None, case.nheads_k, batch=b)
        out, lse = paged_decode(
            to_dev_bf16(q), pool, None, None, lens, table, None, None, nheads_k=case.nheads_k,
            softmax_scale=128 ** -0.5, softcap=0.0, causal=True, window_left=-1,
            k_descale=case.k_descale, v_descale=case.v_descale, seqlen_add=sq, return_lse=True,
            num_splits=splits)
        torch.cuda.synchronize()
    else:
        out, lse, pool = run_decode(case, q, causal=True)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool, causal=True)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)


def test_num_active_rows_skipped():
    announce("decode num_active=2")
    rng = np.random.default_rng(5)
    case = PagedCase(rng, batch=4, nheads=8, nheads_k=2, lengths=[10, 20, 30, 40], new_tokens=[1] * 4)
    q = randn(rng, (4, 1, 8, 128))
    out, lse, pool = run_decode(case, q, num_active=2)
    exp_pool = case.expected_pool(num_active=2)
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool)
    assert_close(out.float().cpu().numpy()[:2], ro[:2])
    assert_lse(lse.cpu().numpy()[:2], rl[:2])


def test_anchor_change_known_answer():
    """test_regression.py:1035-1063 on a paged pool: keys 0 then 16 (D=128, so
    the second half scores 256 higher), values 1 then 3 -> out = 3."""
    announce("decode anchor known answer")
    cap, h, d, page = 4096, 2, 128, 16
    pages = cap // page
    pool = torch.zeros((pages, page, 2 * h, d), dtype=torch.bfloat16, device=DEV)
    half = pages // 2
    pool[:half, :, 1::2] = 1.0
    pool[half:, :, 0::2] = 16.0
    pool[half:, :, 1::2] = 3.0
    table = torch.arange(pages, dtype=torch.int32, device=DEV)[None]
    q = torch.ones((1, 1, h, d), dtype=torch.bfloat16, device=DEV)
    out, lse, _ = flash_attn_with_kvcache(q, pool, None, cache_seqlens=cap, block_table=table,
                                          return_softmax_lse=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), 3.0, atol=1e-2)
    qs = float(np.asarray(T.bf16(np.float32(1 / math.sqrt(d) * A.LOG2E))).reshape(-1)[0])
    expect = 128 * 16 * qs * math.log(2) + math.log(cap // 2)
    np.testing.assert_allclose(lse.cpu().numpy(), expect, rtol=1e-5)


def test_split_k_invariance_and_determinism():
    """Cutting the keys into many more ranges (so every row spans several
    segments, some one tile long) must agree with the default; repeats are
    bitwise equal (the reference's race test, test_prefill.py:827-875)."""
    announce("decode split invariance")
    rng = np.random.default_rng(6)
    case = PagedCase(rng, batch=3, nheads=8, nheads_k=2, lengths=[3000, 77, 1500], new_tokens=[0] * 3)
    q = to_dev_bf16(randn(rng, (3, 1, 8, 128)))
    pool = case.pool()
    lens = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
    table = torch.tensor(case.table, device=DEV)
    kw = dict(nheads_k=2, softmax_scale=1 / math.sqrt(128), softcap=0.0, causal=False,
              window_left=-1, k_descale=1.0, v_descale=1.0, return_lse=True)
    o1, l1 = paged_decode(q, pool, None, None, lens, table, None, None, num_splits=150, **kw)
    o2, l2 = paged_decode(q, pool, None, None, lens, table, None, None, **kw)
    torch.cuda.synchronize()
    assert_close(o1.float().cpu().numpy(), o2.float().cpu().numpy())
    np.testing.assert_allclose(l1.cpu().numpy(), l2.cpu().numpy(), atol=1e-4)
    for _ in range(20):
        o3, l3 = paged_decode(q, pool, None, None, lens, table, None, None, **kw)
        assert torch.equal(o3, o2) and torch.equal(l3, l2)


# ---------------------------------------------------------------- contiguous K/V cache pair
def run_contig(rng, *, batch, batch_cache, nheads, nheads_k, capacity, lengths, append,
               batch_idx=None, window=(-1, -1), softcap=0.0, sinks=None, num_active=None):
    """One single-token step over separate (batch_cache, capacity, nheads_k, 128)
    K/V caches (decode.py:383-403); returns (out, lse, expected k/v codes, oracle
    out, oracle lse)."""
    from tests.gpu_util import dev_from_codes, random_codes
    shape = (batch_cache, capacity, nheads_k, 128)
    kc, vc = random_codes(rng, shape, torch.bfloat16), random_codes(rng, shape, torch.bfloat16)
    q = randn(rng, (batch, 1, nheads, 128))
    lengths = np.asarray(lengths, np.int32)
    idx = np.arange(batch, dtype=np.int32) if batch_idx is None else np.asarray(batch_idx, np.int32)
    kw = {}
    exp_k, exp_v = kc.copy(), vc.copy()
    if append:
        kn = random_codes(rng, (batch, 1, nheads_k, 128), torch.bfloat16)
        vn = random_codes(rng, (batch, 1, nheads_k, 128), torch.bfloat16)
        kw["k"], kw["v"] = dev_from_codes(kn, torch.bfloat16), dev_from_codes(vn, torch.bfloat16)
        live = batch if num_active is None else num_active
        for r in range(live):
            exp_k[idx[r], lengths[r]] = kn[r, 0]
            exp_v[idx[r], lengths[r]] = vn[r, 0]
    k_dev, v_dev = dev_from_codes(kc, torch.bfloat16), dev_from_codes(vc, torch.bfloat16)
    res = flash_attn_with_kvcache(
        to_dev_bf16(q), k_dev, v_dev, **kw,
        cache_seqlens=torch.tensor(lengths, device=DEV),
        cache_batch_idx=None if batch_idx is None else torch.tensor(idx, device=DEV),
        window_size=window, softcap=softcap, return_softmax_lse=True, num_active=num_active,
        learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
    torch.cuda.synchronize()
    out, lse, k_out, v_out = res
    assert k_out is k_dev and v_out is v_dev
    np.testing.assert_array_equal(codes_of(k_out), exp_k)
    np.testing.assert_array_equal(codes_of(v_out), exp_v)
    totals = lengths + (1 if append else 0)
    ro, rl = A.decode_reference(q, T.bf16_to_f32(exp_k), T.bf16_to_f32(exp_v), totals,
                                cache_batch_idx=idx, window_size=window, softcap=softcap,
                                sinks=sinks)
    return out.float().cpu().numpy(), lse.cpu().numpy(), ro, rl, totals


@pytest.mark.parametrize("append", [True, False])
@pytest.mark.parametrize("with_idx", [True, False])
def test_contiguous_cache_decode(append, with_idx):
    announce(f"contiguous decode append={append} batch_idx={with_idx}")
    rng = np.random.default_rng(7)
    lengths = [3, 517, 1799, 2047] if append else [1, 517, 2048, 1000]
    idx = rng.permutation(6)[:4] if with_idx else None
    out, lse, ro, rl, _ = run_contig(rng, batch=4, batch_cache=6 if with_idx else 4, nheads=8,
                                     nheads_k=2, capacity=2048, lengths=lengths, append=append,
                                     batch_idx=idx)
    assert_close(out, ro)
    assert_lse(lse, rl)


def test_contiguous_cache_boundary_append_window():
    """test_regression.py:1065-1112: a 255-key window over 512 / 1799 cached keys
    in cache rows 2 and 0, the append landing on position 1799."""
    announce("contiguous decode boundary append, window 255")
    rng = np.random.default_rng(91)
    out, lse, ro, rl, _ = run_contig(rng, batch=2, batch_cache=3, nheads=4, nheads_k=2,
                                     capacity=2048, lengths=[512, 1799], append=True,
                                     batch_idx=[2, 0], window=(255, 0))
    assert_close(out, ro)
    assert_lse(lse, rl)


@pytest.mark.parametrize("window", [(-1, -1), (255, 0)])
@pytest.mark.parametrize("nheads,nheads_k", [(8, 1), (8, 2)])
def test_contiguous_cache_sinks(window, nheads, nheads_k):
    """test_regression.py:1148-1180: the empty row attends only its sink
    (out 0, lse = sink)."""
    announce(f"contiguous decode sinks window={window} h{nheads}/{nheads_k}")
    rng = np.random.default_rng(29)
    sinks = rng.uniform(-2.0, 8.0, nheads).astype(np.float32)
    out, lse, ro, rl, _ = run_contig(rng, batch=3, batch_cache=3, nheads=nheads, nheads_k=nheads_k,
                                     capacity=1024, lengths=[0, 517, 1024], append=False,
                                     window=window, sinks=sinks)
    assert_close(out, ro)
    assert_lse(lse, rl)
    np.testing.assert_allclose(lse[0], np.broadcast_to(sinks[:, None], lse[0].shape), atol=1e-5)
    assert np.abs(out[0]).max() == 0.0


def test_contiguous_cache_num_active_softcap():
    announce("contiguous decode num_active=2 softcap")
    rng = np.random.default_rng(8)
    out, lse, ro, rl, _ = run_contig(rng, batch=4, batch_cache=4, nheads=16, nheads_k=4,
                                     capacity=1024, lengths=[10, 1000, 30, 40], append=True,
                                     softcap=30.0, num_active=2)
    assert_close(out[:2], ro[:2])
    assert_lse(lse[:2], rl[:2])


@pytest.mark.parametrize("hd", [256, 64])
@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
@pytest.mark.parametrize("seqlen_q", [1, 4])
def test_decode_head_dims(dtype, seqlen_q, hd):
    """head_dim 256 and 64 (the reference's DECODE_HEAD_DIMS, traits.py:50):
    single token with the fused append, and a causal 4-token verify window."""
    announce(f"decode d{hd} {dtype} seqlen_q={seqlen_q}")
    rng = np.random.default_rng(60)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    ks, vs = (1.0, 1.0) if dtype == "bf16" else (0.8, 1.3)
    lengths = [0, 17, 1000, 5000, 129]
    b = len(lengths)
    case = PagedCase(rng, batch=b, nheads=16, nheads_k=4, lengths=lengths,
                     new_tokens=[seqlen_q] * b, head_dim=hd, dtype=dt, k_descale=ks, v_descale=vs)
    q = randn(rng, (b, seqlen_q, 16, hd))
    out, lse, pool = run_decode(case, q, causal=seqlen_q > 1)
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    ro, rl = oracle(case, q, exp_pool, causal=seqlen_q > 1)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
