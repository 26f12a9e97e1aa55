"""GPU counterparts of the reference's regression tests
(tests/softmax_attention/test_regression.py, and the packed-cache cases of
test_paged.py) that pin behaviour rather than a TPU compile detail: scale
arguments given as 0-d arrays, sinks far above the scores, -inf sinks, padding
rows with sinks, a contiguous cache appended step after step, block tables that
change between calls, rows ending around block boundaries of a padded table,
read-only rows over empty caches, a shared prefix page, an allocation of
padding rows only, and the static anchor overtaken by a later tile (by ~500
log2 units, and on the last live tile).  Each compares the HIP path with the NumPy oracle (or with
the same call without the feature, where the reference does)."""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from oracle import attention as A
from oracle import dtypes as T
from tests.gpu_util import (DEV, PagedCase, announce, assert_close, assert_lse, codes_of,
                            dev_from_codes, random_codes, randn, to_dev_bf16)

pytestmark = pytest.mark.gpu


def head_major(x):  # (B, S, H, D) <-> (B, H, S, D)
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


def packed(rng, seqlens, h, hk, d):
    cu = np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32)
    return cu, randn(rng, (cu[-1], h, d)), randn(rng, (cu[-1], hk, d)), randn(rng, (cu[-1], hk, d))


def heads_first(x):  # (T, H, D) -> (H, T, D)
    return np.ascontiguousarray(x.transpose(1, 0, 2))


@pytest.mark.parametrize("entry", ["dense", "varlen"])
@pytest.mark.parametrize("array_type", ["numpy", "torch"])
def test_array_softmax_scale(entry, array_type):
    """test_regression.py:235-270: a concrete 0-d array scale gives the result
    of the float it holds, bit for bit."""
    announce(f"array softmax_scale {entry} {array_type}")
    rng = np.random.default_rng(120)
    d = 128
    scale = np.asarray(np.float32(1.0) / np.sqrt(np.float32(d)))
    arr = scale if array_type == "numpy" else torch.tensor(scale)
    seqlens = [100, 156]
    cu, q, k, v = packed(rng, seqlens, 2, 2, d)

    def attend(softmax_scale):
        if entry == "dense":
            return flash_attn_func(to_dev_bf16(head_major(q[None])), to_dev_bf16(head_major(k[None])),
                                   to_dev_bf16(head_major(v[None])), causal=True,
                                   softmax_scale=softmax_scale)
        c = torch.tensor(cu, device=DEV)
        return flash_attn_varlen_func(to_dev_bf16(heads_first(q)), to_dev_bf16(heads_first(k)),
                                      to_dev_bf16(heads_first(v)), c, c, max(seqlens), max(seqlens),
                                      causal=True, softmax_scale=softmax_scale)

    want = attend(float(scale))
    got = attend(arr)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def _contig_decode(q, k_cache, v_cache, lens, sinks=None):
    res = flash_attn_with_kvcache(
        to_dev_bf16(q), to_dev_bf16(k_cache), to_dev_bf16(v_cache),
        cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=DEV), return_softmax_lse=True,
        learnable_sink=None if sinks is None else torch.tensor(sinks, device=DEV))
    torch.cuda.synchronize()
    return res[0].float().cpu().numpy(), res[1].cpu().numpy()


@pytest.mark.parametrize("entry", ["dense", "varlen", "decode"])
def test_sinks_far_above_the_scores(entry):
    """test_regression.py:608-670: q = -2.5 against k = +2.5 scores about
    -70.7 at d 128, so sinks of 20 and 40 sit far above the anchor; lse must
    stay finite and out / lse match the oracle."""
    announce(f"sinks far above the scores: {entry}")
    rng = np.random.default_rng(121)
    sinks = np.array([20.0, 40.0, 20.0, 40.0], np.float32)
    h, hk, d = 4, 2, 128
    if entry == "decode":
        cap = 256
        q = np.full((2, 1, h, d), -2.5, np.float32)
        kc = np.full((2, cap, hk, d), 2.5, np.float32)
        vc = T.bf16_to_f32(random_codes(rng, (2, cap, hk, d), torch.bfloat16))
        lens = np.array([100, 256], np.int32)
        out, lse = _contig_decode(q, kc, vc, lens, sinks)
        ro, rl = A.decode_reference(q, kc, vc, lens, cache_batch_idx=np.arange(2), sinks=sinks)
    else:
        s = 256
        q = np.full((1, s, h, d), -2.5, np.float32)
        k = np.full((1, s, hk, d), 2.5, np.float32)
        v = randn(rng, (1, s, hk, d))
        ro, rl = A.attention_ref(q, k, v, causal=True, sinks=sinks, round_scaled_q=True)
        if entry == "dense":
            o, l = flash_attn_func(to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)),
                                   to_dev_bf16(head_major(v)), causal=True, return_softmax_lse=True,
                                   learnable_sink=torch.tensor(sinks, device=DEV))
            torch.cuda.synchronize()
            out, lse = head_major(o.float().cpu().numpy()), l.cpu().numpy()
        else:
            c = torch.tensor([0, s], dtype=torch.int32, device=DEV)
            o, l = flash_attn_varlen_func(to_dev_bf16(heads_first(q[0])), to_dev_bf16(heads_first(k[0])),
                                          to_dev_bf16(heads_first(v[0])), c, c, s, s, causal=True,
                                          return_softmax_lse=True,
                                          learnable_sink=torch.tensor(sinks, device=DEV))
            torch.cuda.synchronize()
            out = o.float().cpu().numpy().transpose(1, 0, 2)[None]
            lse = l.cpu().numpy()[None]
    assert np.isfinite(lse).all()
    assert_close(out, ro)
    assert_lse(lse, rl)


@pytest.mark.parametrize("entry", ["varlen", "decode"])
def test_minus_inf_sinks_are_no_sink(entry):
    """test_regression.py:672-735: a -inf sink adds nothing (the head matches
    the call without sinks); a row with no key returns out 0 and lse -inf
    under a -inf sink and lse = sink under a finite one, never NaN."""
    announce(f"-inf sinks: {entry}")
    rng = np.random.default_rng(122)
    sinks = np.array([-np.inf, 2.0, -np.inf, 4.0], np.float32)
    none_heads, sink_heads = np.array([0, 2]), np.array([1, 3])
    h, hk, d = 4, 2, 128
    if entry == "decode":
        cap = 256
        q = randn(rng, (2, 1, h, d))
        kc = T.bf16_to_f32(random_codes(rng, (2, cap, hk, d), torch.bfloat16))
        vc = T.bf16_to_f32(random_codes(rng, (2, cap, hk, d), torch.bfloat16))
        lens = np.array([0, 200], np.int32)
        out, lse = _contig_decode(q, kc, vc, lens, sinks)
        plain_out, plain_lse = _contig_decode(q, kc, vc, lens)
        # (B, 1, H, D) -> (H, B, D); lse (B, H, 1) -> (H, B)
        out, plain_out = out[:, 0].swapaxes(0, 1), plain_out[:, 0].swapaxes(0, 1)
        lse, plain_lse = lse[..., 0].T, plain_lse[..., 0].T
        empty, keyed = np.array([0]), np.array([1])
    else:
        q = randn(rng, (128, h, d))
        k, v = randn(rng, (80, hk, d)), randn(rng, (80, hk, d))
        cu_q = torch.tensor([0, 64, 128], dtype=torch.int32, device=DEV)
        cu_k = torch.tensor([0, 16, 80], dtype=torch.int32, device=DEV)
        args = (to_dev_bf16(heads_first(q)), to_dev_bf16(heads_first(k)), to_dev_bf16(heads_first(v)),
                cu_q, cu_k, 64, 64)
        o, l = flash_attn_varlen_func(*args, causal=True, return_softmax_lse=True,
                                      learnable_sink=torch.tensor(sinks, device=DEV))
        po, pl = flash_attn_varlen_func(*args, causal=True, return_softmax_lse=True)
        torch.cuda.synchronize()
        out, plain_out = o.float().cpu().numpy(), po.float().cpu().numpy()  # (H, T, D)
        lse, plain_lse = l.cpu().numpy(), pl.cpu().numpy()
        # causal rows end on their bottom-right diagonal: the first 48 rows of
        # the 64-row query against 16 keys see no key
        empty, keyed = np.arange(48), np.arange(48, 128)
    assert not np.isnan(out).any() and not np.isnan(lse).any()
    assert np.all(out[:, empty] == 0)
    assert np.all(lse[np.ix_(none_heads, empty)] == -np.inf)
    np.testing.assert_allclose(lse[np.ix_(sink_heads, empty)],
                               np.broadcast_to(sinks[sink_heads, None], (2, len(empty))))
    np.testing.assert_allclose(out[np.ix_(none_heads, keyed)], plain_out[np.ix_(none_heads, keyed)],
                               atol=1e-2)
    np.testing.assert_allclose(lse[np.ix_(none_heads, keyed)], plain_lse[np.ix_(none_heads, keyed)],
                               atol=1e-3)


def test_varlen_padding_rows_ignore_sinks():
    """test_regression.py:863-887: padding rows past cu_seqlens[-1] keep out 0
    and lse -inf with sinks, even when their q is NaN."""
    announce("varlen padding rows with sinks and NaN q")
    rng = np.random.default_rng(123)
    seqlens = [17, 40]
    cu, q, k, v = packed(rng, seqlens, 4, 2, 128)
    q = np.concatenate([q, np.full((23, 4, 128), np.nan, np.float32)])
    k = np.concatenate([k, randn(rng, (23, 2, 128))])
    v = np.concatenate([v, randn(rng, (23, 2, 128))])
    c = torch.tensor(cu, device=DEV)
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(heads_first(q)), to_dev_bf16(heads_first(k)), to_dev_bf16(heads_first(v)), c, c,
        40, 40, causal=True, return_softmax_lse=True,
        learnable_sink=torch.tensor(rng.standard_normal(4).astype(np.float32), device=DEV))
    torch.cuda.synchronize()
    out, lse = out.float().cpu().numpy(), lse.cpu().numpy()
    assert np.all(out[:, 57:] == 0)
    assert np.all(lse[:, 57:] == -np.inf)
    assert np.isfinite(out[:, :57]).all()


@pytest.mark.parametrize("nheads,nheads_k,d", [(8, 1, 128), (6, 1, 256), (8, 2, 128)])
def test_contiguous_cache_appends_step_after_step(nheads, nheads_k, d):
    """test_regression.py:1185-1230: each step's append lands on the cache the
    previous step returned; positions cross the cache's first rows and end at
    its last slot."""
    announce(f"contiguous append step after step h{nheads}/{nheads_k} d{d}")
    rng = np.random.default_rng(124)
    batch, cap = 2, 256
    positions = [*range(0, 12), *range(cap - 8, cap)]
    kc = random_codes(rng, (batch, cap, nheads_k, d), torch.bfloat16)
    vc = random_codes(rng, (batch, cap, nheads_k, d), torch.bfloat16)
    kc[:, positions] = 0
    vc[:, positions] = 0
    q = randn(rng, (batch, 1, nheads, d))
    k_dev, v_dev = dev_from_codes(kc, torch.bfloat16), dev_from_codes(vc, torch.bfloat16)
    exp_k, exp_v = kc.copy(), vc.copy()
    rows = np.arange(batch)
    for pos in positions:
        kn = random_codes(rng, (batch, 1, nheads_k, d), torch.bfloat16)
        vn = random_codes(rng, (batch, 1, nheads_k, d), torch.bfloat16)
        lens = np.full(batch, pos, np.int32)
        out, lse, k_dev, v_dev = flash_attn_with_kvcache(
            to_dev_bf16(q), k_dev, v_dev, dev_from_codes(kn, torch.bfloat16),
            dev_from_codes(vn, torch.bfloat16), cache_seqlens=torch.tensor(lens, device=DEV),
            return_softmax_lse=True)
        torch.cuda.synchronize()
        exp_k[rows, pos], exp_v[rows, pos] = kn[:, 0], vn[:, 0]
        np.testing.assert_array_equal(codes_of(k_dev), exp_k)
        np.testing.assert_array_equal(codes_of(v_dev), exp_v)
        ro, rl = A.decode_reference(q, T.bf16_to_f32(exp_k), T.bf16_to_f32(exp_v), lens + 1,
                                    cache_batch_idx=rows)
        assert_close(out.float().cpu().numpy(), ro, what=f"position {pos}")
        assert_lse(lse.cpu().numpy(), rl)


def test_block_table_changes_between_calls():
    """test_regression.py:1233-1270: the table and lengths are runtime
    operands; each append lands where its call's table says, and nothing else
    in the pool changes."""
    announce("paged append under two block tables")
    batch, page, heads, d = 2, 128, 2, 128
    pool = torch.zeros((4, page, 2 * heads, d), dtype=torch.bfloat16, device=DEV)
    q = torch.ones((batch, 1, heads, d), dtype=torch.bfloat16, device=DEV)
    k = torch.ones((batch, 1, heads, d), dtype=torch.bfloat16, device=DEV)
    v = torch.full_like(k, 2.0)
    calls = [(np.array([[0, 1], [2, 3]], np.int32), np.array([0, 129], np.int32)),
             (np.array([[3, 2], [1, 0]], np.int32), np.array([130, 5], np.int32))]
    for table, lens in calls:
        _, pool = flash_attn_with_kvcache(q, pool, None, k, v,
                                          cache_seqlens=torch.tensor(lens, device=DEV),
                                          block_table=torch.tensor(table, device=DEV))
        torch.cuda.synchronize()
        p = pool.float().cpu().numpy()
        for r in range(batch):
            slot = p[table[r, lens[r] // page], lens[r] % page]
            np.testing.assert_array_equal(slot[0::2], 1.0)
            np.testing.assert_array_equal(slot[1::2], 2.0)
    assert float(pool.float().abs().sum()) == 4 * heads * d * (1.0 + 2.0)


def test_rows_around_block_boundaries_of_a_padded_table():
    """test_regression.py:1272-1310: 9 pages of 128 tokens per row, rows ending
    inside the first 1024 keys, on 1024, one past it and on the last real
    page; append then attend, against the oracle."""
    announce("paged decode, rows around 1024-key boundaries")
    rng = np.random.default_rng(125)
    lens = np.array([129, 1023, 1024, 1151], np.int32)
    case = PagedCase(rng, batch=4, nheads=4, nheads_k=2, lengths=lens, new_tokens=[1] * 4,
                     page_size=128, max_pages=9)
    q = randn(rng, (4, 1, 4, 128))
    shape = (4, 1, 2, 128)
    out, lse, pool = flash_attn_with_kvcache(
        to_dev_bf16(q), case.pool(), None, dev_from_codes(case.k_codes.reshape(shape), torch.bfloat16),
        dev_from_codes(case.v_codes.reshape(shape), torch.bfloat16),
        cache_seqlens=torch.tensor(lens, device=DEV), block_table=torch.tensor(case.table, device=DEV),
        return_softmax_lse=True)
    torch.cuda.synchronize()
    after = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), after)
    krows, vrows = case.rows(after)
    ro, rl = A.kvcache_reference(q, krows, vrows, lens + 1)
    assert_close(out.float().cpu().numpy(), ro)
    assert_lse(lse.cpu().numpy(), rl)


def _extend(case, q, cu, prefix, *, causal, append, max_q):
    """flash_attn_with_kvcache over the case's pool with a packed q: append the
    case's new rows (k / v padded like q) or read only."""
    kw = {}
    if append:
        pad = q.shape[0] - case.k_codes.shape[0]
        z = np.zeros((pad,) + case.k_codes.shape[1:], case.k_codes.dtype)
        kw = dict(k=dev_from_codes(np.concatenate([case.k_codes, z]), case.dtype),
                  v=dev_from_codes(np.concatenate([case.v_codes, z]), case.dtype))
    pool = case.pool()
    out, lse, pool2 = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, cache_seqlens=torch.tensor(prefix, dtype=torch.int32, device=DEV),
        block_table=torch.tensor(case.table, device=DEV), cu_seqlens_q=torch.tensor(cu, device=DEV),
        max_seqlen_q=max_q, causal=causal, return_softmax_lse=True, **kw)
    torch.cuda.synchronize()
    assert pool2 is pool
    return out.float().cpu().numpy(), lse.cpu().numpy(), codes_of(pool)


def test_read_only_empty_cache_between_cached_requests():
    """test_paged.py:483-495: read-only packed rows over empty caches (they
    see no key and are not checked) between requests with cached keys."""
    announce("read-only packed rows, empty caches between cached requests")
    rng = np.random.default_rng(126)
    qlens, prefix = np.array([4, 3, 9, 2]), np.array([0, 130, 0, 5])
    case = PagedCase(rng, batch=4, nheads=4, nheads_k=2, lengths=prefix, new_tokens=[0] * 4,
                     page_size=128)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1] + 5, 4, 128))
    out, lse, pool = _extend(case, q, cu, prefix, causal=False, append=False, max_q=9)
    np.testing.assert_array_equal(pool, case.pool_codes)
    kp, vp = case.kv_pages(case.pool_codes)
    ro, rl = A.ragged_reference(q, kp, vp, cu, prefix, case.table, causal=False,
                                round_scaled_q=True)
    for s in (1, 3):
        rows = slice(cu[s], cu[s + 1])
        assert_close(out[rows], ro[rows], what=f"request {s}")
        assert_lse(lse[:, rows], rl[:, rows])
    assert not np.abs(out[cu[-1]:]).any()


def test_shared_read_only_prefix_and_private_append_pages():
    """test_paged.py:498-510: two requests share their first page (a 128-token
    prefix) and append to private pages."""
    announce("shared prefix page, private append pages")
    rng = np.random.default_rng(127)
    qlens, prefix = np.array([2, 7]), np.array([128, 128])
    case = PagedCase(rng, batch=2, nheads=4, nheads_k=2, lengths=prefix, new_tokens=qlens,
                     page_size=128)
    case.table[1, 0] = case.table[0, 0]
    q = randn(rng, (int(qlens.sum()), 4, 128))
    out, lse, pool = _extend(case, q, case.cu, prefix, causal=True, append=True, max_q=7)
    after = case.expected_pool()
    np.testing.assert_array_equal(pool, after)
    kp, vp = case.kv_pages(after)
    ro, rl = A.ragged_reference(q, kp, vp, case.cu, prefix + qlens, case.table, causal=True,
                                round_scaled_q=True)
    assert_close(out, ro)
    assert_lse(lse, rl)


@pytest.mark.parametrize("append", [False, True])
def test_empty_packed_allocation(append):
    """test_paged.py:512-525: every request has zero q rows, so the buffer
    holds packed padding only: out 0, lse -inf, the pool unchanged."""
    announce(f"empty packed allocation append={append}")
    rng = np.random.default_rng(128)
    case = PagedCase(rng, batch=2, nheads=4, nheads_k=2, lengths=[0, 0], new_tokens=[0, 0],
                     page_size=128)
    q = randn(rng, (8, 4, 128))
    out, lse, pool = _extend(case, q, case.cu, np.array([0, 0]), causal=True, append=append,
                             max_q=1)
    np.testing.assert_array_equal(pool, case.pool_codes)
    assert not np.abs(out).any()
    assert np.all(lse == -np.inf)


def _merged_pool(kp, vp):
    """(pages, page, Hk, D) K and V values -> the merged bf16 pool [k0, v0, ...]."""
    pages, page, hk, d = kp.shape
    m = np.empty((pages, page, 2 * hk, d), np.float32)
    m[:, :, 0::2], m[:, :, 1::2] = kp, vp
    return to_dev_bf16(m)


def test_later_block_raises_anchor_paged():
    """test_paged.py:667-689: cached keys jump from 0 to 32 at position 1024,
    so later tiles score hundreds of log2 units above the anchor the first
    ones set; the kernel must rescale instead of overflowing (out ~ 3)."""
    announce("paged chunk: a later block raises the anchor by ~500 log2 units")
    rng = np.random.default_rng(129)
    page, hk, h, d, prefix, qlen = 128, 2, 4, 128, 2048, 64
    table = rng.permutation(32).astype(np.int32)[None]
    kp = np.zeros((32, page, hk, d), np.float32)
    vp = np.ones((32, page, hk, d), np.float32)
    late = table[0, 1024 // page:]
    kp[late], vp[late] = 32.0, 3.0
    q = np.ones((qlen, h, d), np.float32)
    kn, vn = np.full((qlen, hk, d), 32.0, np.float32), np.full((qlen, hk, d), 3.0, np.float32)
    out, pool = flash_attn_with_kvcache(
        to_dev_bf16(q), _merged_pool(kp, vp), None, to_dev_bf16(kn), to_dev_bf16(vn),
        cache_seqlens=torch.tensor([prefix], dtype=torch.int32, device=DEV),
        block_table=torch.tensor(table, device=DEV),
        cu_seqlens_q=torch.tensor([0, qlen], dtype=torch.int32, device=DEV), max_seqlen_q=qlen,
        causal=True)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.isfinite(o).all()
    np.testing.assert_allclose(o, 3.0, atol=2e-2)
    ro, _ = A.ragged_reference(q, kp, vp, np.array([0, qlen]), np.array([prefix + qlen]), table,
                               causal=True, round_scaled_q=True)
    assert_close(o, ro)


def test_overflow_guard_at_the_last_live_kv_tile():
    """test_paged.py:978-1010: keys [0, 512) score 0 and keys [512, 600) about
    200 nats; rows past 512 anchor on the first tiles and overflow on the last
    live one (600 tokens appended to an empty 16-page pool, causal)."""
    announce("paged chunk: overflow on the last live kv tile")
    length, hk, h, d, pages, page = 600, 2, 4, 128, 16, 128
    mag = np.sqrt(200.0 * np.sqrt(d))
    q = np.zeros((length, h, d), np.float32)
    q[:, :, 0] = mag
    k = np.zeros((length, hk, d), np.float32)
    k[512:, :, 0] = mag
    v = np.where(np.arange(length)[:, None, None] < 512, 1.0, 3.0) * np.ones((length, hk, d), np.float32)
    q, k, v = (T.bf16(x) for x in (q, k, v))
    table = np.arange(pages, dtype=np.int32)[None]
    zeros = np.zeros((pages, page, hk, d), np.float32)
    out, lse, pool = flash_attn_with_kvcache(
        to_dev_bf16(q), _merged_pool(zeros, zeros), None, to_dev_bf16(k), to_dev_bf16(v),
        cache_seqlens=torch.tensor([0], dtype=torch.int32, device=DEV),
        block_table=torch.tensor(table, device=DEV),
        cu_seqlens_q=torch.tensor([0, length], dtype=torch.int32, device=DEV),
        max_seqlen_q=length, causal=True, return_softmax_lse=True)
    torch.cuda.synchronize()
    kp, vp = zeros.copy(), zeros.copy()
    kp.reshape(-1, hk, d)[:length], vp.reshape(-1, hk, d)[:length] = k, v
    o = out.float().cpu().numpy()
    assert np.isfinite(o).all()
    ro, rl = A.ragged_reference(q, kp, vp, np.array([0, length]), np.array([length]), table,
                                causal=True, round_scaled_q=True)
    assert_close(o, ro)
    assert_lse(lse.cpu().numpy(), rl)
