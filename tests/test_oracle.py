"""Pins the NumPy oracle against library routines, brute force and closed
forms (none of these re-types the oracle's own formula)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import dtypes as T
from oracle import paged as P


def randn(rng, shape):
    return T.bf16(rng.standard_normal(shape, dtype=np.float32))


# ---------------------------------------------------------------- dtypes


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, 1.0, 65504.0, 3.4e38, 1e-40], np.float32),
    ]).astype(np.float32)
    ours = T.bf16_round(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


@pytest.mark.parametrize("fmt,tdt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_fp8_tables_match_torch(fmt, tdt):
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    theirs = codes.view(tdt).to(torch.float32).numpy()
    ours = T.fp8_decode(np.arange(256, dtype=np.uint8), fmt)
    np.testing.assert_array_equal(np.isnan(ours), np.isnan(theirs))
    fin = ~np.isnan(ours)
    np.testing.assert_array_equal(ours[fin], theirs[fin])


@pytest.mark.parametrize("fmt,tdt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_fp8_encode_matches_torch(fmt, tdt):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200000) * 4).astype(np.float32)
    x = np.concatenate([x, T.fp8_decode(np.arange(256, dtype=np.uint8), fmt)])
    x = x[np.isfinite(x) & (np.abs(x) < 440)]
    # also exact midpoints between neighbouring codes (ties to even)
    vals = np.unique(np.abs(T.fp8_decode(np.arange(127, dtype=np.uint8), fmt)))
    vals = vals[np.isfinite(vals)]
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    ours = T.fp8_encode(x, fmt)
    theirs = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


# ---------------------------------------------------------------- layout


@pytest.mark.parametrize("hk,dt", [(1, np.uint16), (3, np.uint16), (1, np.uint8), (3, np.uint8), (8, np.uint8)])
def test_merge_kv_heads_layout(hk, dt):
    rng = np.random.default_rng(2)
    k = rng.integers(1, 200, (5, hk, 16)).astype(dt)
    v = rng.integers(1, 200, (5, hk, 16)).astype(dt)
    m = P.merge_kv_heads(k, v)
    itemsize = np.dtype(dt).itemsize
    assert m.shape[-2] == (2 * hk if itemsize == 2 else 2 * (hk + hk % 2))
    for h in range(hk):
        np.testing.assert_array_equal(m[:, 2 * h], k[:, h])
        np.testing.assert_array_equal(m[:, 2 * h + 1], v[:, h])
    if m.shape[-2] > 2 * hk:
        assert not m[:, 2 * hk:].any()
    k2, v2 = P.split_kv_heads(m, hk)
    np.testing.assert_array_equal(k2, k)
    np.testing.assert_array_equal(v2, v)


def test_append_to_pages_addresses_and_untouched_bytes():
    rng = np.random.default_rng(3)
    page, hk, d = 16, 2, 8
    lengths = [3, 0, 5]
    prefixes = [27, 0, 13]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    table = rng.permutation(3 * 4).reshape(3, 4)
    pool = rng.integers(0, 65535, (12, page, 2 * hk, d)).astype(np.uint16)
    k = rng.integers(0, 65535, (cu[-1] + 2, hk, d)).astype(np.uint16)
    v = rng.integers(0, 65535, (cu[-1] + 2, hk, d)).astype(np.uint16)
    new = P.append_to_pages(pool, k, v, cu, prefixes, table)
    touched = np.zeros(pool.shape[:2], bool)
    for r in range(3):
        for t in range(lengths[r]):
            pos = prefixes[r] + t
            pg, slot = table[r, pos // page], pos % page
            touched[pg, slot] = True
            row = new[pg, slot]
            np.testing.assert_array_equal(row[0::2], k[cu[r] + t])
            np.testing.assert_array_equal(row[1::2], v[cu[r] + t])
    np.testing.assert_array_equal(new[~touched], pool[~touched])
    # num_active=1 only writes request 0
    new1 = P.append_to_pages(pool, k, v, cu, prefixes, table, num_active=1)
    assert (new1 != pool).any(axis=(2, 3)).sum() == lengths[0]


def test_write_kv_cache_pages_known_pieces():
    # The fixed pieces of test_page.py:33-69 at page 128: a page tail, a whole
    # page and a page head, out of token order.
    rng = np.random.default_rng(0)
    page, d, hk = 128, 16, 3
    cache = rng.integers(0, 255, (6, page, P.merged_cache_heads(hk, 1), d)).astype(np.uint8)
    k = rng.integers(0, 255, (300, hk, d)).astype(np.uint8)
    v = rng.integers(0, 255, (300, hk, d)).astype(np.uint8)
    pieces = [(4 * page + 100, 0, 28), (1 * page, 28, 128), (3 * page, 156, 100)]
    slices = np.zeros((3, 8), np.int32)
    for j, pc in enumerate(pieces):
        slices[:, j] = pc
    out = P.write_kv_cache_pages(k, v, cache, slices, 3).reshape(-1, 8, d)
    flat = cache.reshape(-1, 8, d)
    untouched = np.ones(len(flat), bool)
    for c0, n0, ln in pieces:
        for i in range(ln):
            np.testing.assert_array_equal(out[c0 + i, 0:6:2], k[n0 + i])
            np.testing.assert_array_equal(out[c0 + i, 1:6:2], v[n0 + i])
            assert not out[c0 + i, 6:].any()
            untouched[c0 + i] = False
    np.testing.assert_array_equal(out[untouched], flat[untouched])


# ---------------------------------------------------------------- attention


def brute_force(q, k, v, causal, window, softcap, sinks, scale):
    """Per-element pure-Python attention on one (Sq, H, D) / (Sk, Hk, D) row."""
    sq, h, d = q.shape
    sk, hk, _ = k.shape
    out = np.zeros((sq, h, d))
    lse = np.full((h, sq), -np.inf)
    for hh in range(h):
        kh = hh // (h // hk)
        for i in range(sq):
            diag = i + sk - sq
            logits = []
            for j in range(sk):
                if causal and j > diag:
                    continue
                if window[1] >= 0 and j > diag + window[1]:
                    continue
                if window[0] >= 0 and j < diag - window[0]:
                    continue
                s = sum(float(q[i, hh, x]) * float(k[j, kh, x]) for x in range(d)) * scale
                if softcap:
                    s = math.tanh(s / softcap) * softcap
                logits.append((j, s))
            terms = [s for _, s in logits] + ([float(sinks[hh])] if sinks is not None else [])
            if not logits and sinks is None:
                continue
            m = max(terms)
            z = sum(math.exp(t - m) for t in terms)
            lse[hh, i] = m + math.log(z)
            for j, s in logits:
                out[i, hh] += math.exp(s - m) / z * v[j, kh].astype(np.float64)
    return out, lse


@pytest.mark.parametrize(
    "sq,sk,causal,window,softcap,sinks",
    [
        (5, 5, True, (-1, -1), 0.0, False),
        (3, 7, True, (-1, -1), 0.0, False),
        (7, 3, True, (-1, -1), 0.0, False),  # leading rows see nothing
        (6, 6, False, (2, 1), 0.0, False),
        (6, 9, True, (3, -1), 5.0, False),
        (4, 6, True, (-1, -1), 0.0, True),
    ],
)
def test_attention_ref_brute_force(sq, sk, causal, window, softcap, sinks):
    rng = np.random.default_rng(4)
    q = randn(rng, (1, sq, 4, 8))
    k = randn(rng, (1, sk, 2, 8))
    v = randn(rng, (1, sk, 2, 8))
    s = rng.standard_normal(4).astype(np.float32) if sinks else None
    out, lse = A.attention_ref(q, k, v, causal=causal, window_size=window, softcap=softcap, sinks=s)
    bo, bl = brute_force(q[0], k[0], v[0], causal, window, softcap, s, 1 / math.sqrt(8))
    np.testing.assert_allclose(out[0], bo, atol=2e-5, rtol=1e-4)
    np.testing.assert_array_equal(np.isneginf(lse[0]), np.isneginf(bl))
    fin = np.isfinite(bl)
    np.testing.assert_allclose(lse[0][fin], bl[fin], atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("d,dv", [(96, 96), (192, 128), (64, 256), (384, 384), (512, 512)])
def test_attention_ref_head_dims_match_torch_sdpa(d, dv):
    """The oracle at the prefill head-dim pairs the kernels take, including
    head_dim_v != head_dim, against torch's float64 SDPA (bottom-right causal
    with Sq < Sk)."""
    rng = np.random.default_rng(9)
    sq, sk = 24, 40
    q = randn(rng, (1, sq, 4, d))
    k = randn(rng, (1, sk, 2, d))
    v = randn(rng, (1, sk, 2, dv))
    out, lse = A.attention_ref(q, k, v, causal=True)
    tq, tk, tv = (torch.from_numpy(x).permute(0, 2, 1, 3).double() for x in (q, k, v))
    tk, tv = tk.repeat_interleave(2, dim=1), tv.repeat_interleave(2, dim=1)
    mask = torch.arange(sk)[None, :] <= torch.arange(sq)[:, None] + (sk - sq)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask)
    np.testing.assert_allclose(out, ref.permute(0, 2, 1, 3).numpy(), atol=2e-5)
    scores = (tq @ tk.transpose(-1, -2)) / math.sqrt(d)
    want = torch.logsumexp(scores.masked_fill(~mask, -math.inf), dim=-1)
    np.testing.assert_allclose(lse, want.numpy(), atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_ref_matches_torch_sdpa(causal):
    rng = np.random.default_rng(5)
    q = randn(rng, (2, 64, 8, 32))
    k = randn(rng, (2, 64, 2, 32))
    v = randn(rng, (2, 64, 2, 32))
    out, lse = A.attention_ref(q, k, v, causal=causal)
    tq, tk, tv = (torch.from_numpy(x).permute(0, 2, 1, 3).double() for x in (q, k, v))
    tk = tk.repeat_interleave(4, dim=1)
    tv = tv.repeat_interleave(4, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal)
    np.testing.assert_allclose(out, ref.permute(0, 2, 1, 3).numpy(), atol=2e-5)
    scores = (tq @ tk.transpose(-1, -2)) / math.sqrt(32)
    if causal:
        scores = scores.masked_fill(torch.ones(64, 64, dtype=torch.bool).triu(1), -math.inf)
    np.testing.assert_allclose(lse, torch.logsumexp(scores, -1).numpy(), atol=2e-5)


def test_closed_forms():
    rng = np.random.default_rng(6)
    # one visible key (first row, causal, square): out = v0, lse = score
    q = randn(rng, (1, 4, 2, 16))
    k = randn(rng, (1, 4, 2, 16))
    v = randn(rng, (1, 4, 2, 16))
    out, lse = A.attention_ref(q, k, v, causal=True)
    np.testing.assert_allclose(out[0, 0], v[0, 0], atol=1e-6)
    np.testing.assert_allclose(lse[0, :, 0], (q[0, 0] * k[0, 0]).sum(-1) / 4.0, atol=1e-5)
    # identical keys: out = mean of the visible V
    k_same = np.broadcast_to(k[:, :1], k.shape).copy()
    out, lse = A.attention_ref(q, k_same, v, causal=False)
    np.testing.assert_allclose(out[0, 2], np.broadcast_to(v[0].mean(0), (2, 16)), atol=1e-5)
    # window >= context is plain causal; softcap -> inf is no softcap; -inf sink
    big = A.attention_ref(q, k, v, causal=True, window_size=(100, -1))
    plain = A.attention_ref(q, k, v, causal=True)
    np.testing.assert_array_equal(big[0], plain[0])
    capped = A.attention_ref(q, k, v, causal=True, softcap=1e7)
    np.testing.assert_allclose(capped[0], plain[0], atol=1e-5)
    sunk = A.attention_ref(q, k, v, causal=True, sinks=np.full(2, -np.inf, np.float32))
    np.testing.assert_allclose(sunk[0], plain[0], atol=1e-6)
    np.testing.assert_allclose(sunk[1], plain[1], atol=1e-6)


def test_anchor_known_answer():
    # test_regression.py:1035-1063: q = ones (D=64), keys 0 then 32, values 1
    # then 3: the second half's scores are 256 above the first, so out = 3.
    cap, h, d = 4096, 2, 64
    q = np.ones((1, 1, h, d), np.float32)
    kc = np.concatenate([np.zeros((1, cap // 2, h, d)), np.full((1, cap // 2, h, d), 32.0)], 1).astype(np.float32)
    vc = np.concatenate([np.ones((1, cap // 2, h, d)), np.full((1, cap // 2, h, d), 3.0)], 1).astype(np.float32)
    out, lse = A.decode_reference(q, kc, vc, np.array([cap]), round_scaled_q=False)
    np.testing.assert_allclose(out, 3.0, atol=1e-6)
    # lse = 256 + ln(2048) (the first half contributes exp(-256) ~ 0)
    np.testing.assert_allclose(lse, 256 + math.log(cap // 2), rtol=1e-5)


def test_kvcache_reference_matches_attention_ref():
    """The decode/verify-window oracle (q pre-rounded) against attention_ref
    (different code path: bottom-right masks on key padding)."""
    rng = np.random.default_rng(7)
    b, sq, h, hk, d, cap = 3, 4, 8, 2, 32, 40
    q = randn(rng, (b, sq, h, d))
    kc = randn(rng, (b, cap, hk, d))
    vc = randn(rng, (b, cap, hk, d))
    lens = np.array([40, 9, 4])
    for causal in (False, True):
        out, lse = A.kvcache_reference(q, kc, vc, lens, causal=causal, round_scaled_q=False)
        ro, rl = A.attention_ref(q, kc, vc, causal=causal, key_lengths=lens)
        np.testing.assert_allclose(out, ro, atol=2e-5)
        np.testing.assert_allclose(lse, rl, atol=2e-5)
    # rounding the scaled q moves results by at most bf16 noise
    out_r, _ = A.kvcache_reference(q, kc, vc, lens, causal=True)
    np.testing.assert_allclose(out_r, ro, atol=2e-2)


def test_ragged_reference_matches_attention_ref():
    rng = np.random.default_rng(8)
    page, hk, h, d = 16, 2, 4, 32
    qlens = [3, 0, 5, 17]
    prefix = [27, 0, 13, 40]
    cu = np.concatenate([[0], np.cumsum(qlens)])
    tot = np.array(qlens) + np.array(prefix)
    pps = 4
    table = rng.permutation(4 * pps).reshape(4, pps)
    kp = randn(rng, (4 * pps, page, hk, d))
    vp = randn(rng, (4 * pps, page, hk, d))
    q = randn(rng, (cu[-1] + 3, h, d))
    for causal, wl, sc in ((True, None, 0.0), (True, 7, 30.0), (False, None, 0.0)):
        out, lse = A.ragged_reference(q, kp, vp, cu, tot, table, causal=causal, window_left=wl, softcap=sc)
        assert not out[cu[-1]:].any() and np.isneginf(lse[:, cu[-1]:]).all()
        krows = P.gather_rows(kp, table)
        vrows = P.gather_rows(vp, table)
        for s in range(4):
            if qlens[s] == 0:
                continue
            ro, rl = A.attention_ref(
                q[None, cu[s]:cu[s + 1]], krows[s:s + 1, :tot[s]], vrows[s:s + 1, :tot[s]],
                causal=causal, window_size=(-1 if wl is None else wl, -1), softcap=sc)
            np.testing.assert_allclose(out[cu[s]:cu[s + 1]], ro[0], atol=2e-5)
            np.testing.assert_allclose(lse[:, cu[s]:cu[s + 1]], rl[0], atol=2e-5)


def brute_force_rounded(q, k, v, causal, window, softcap, scale, k_descale=1.0, v_descale=1.0):
    """brute_force with the kernels' q convention, element by element in
    float64: q is multiplied by the fused factor (scale * k_descale / softcap,
    or scale * k_descale * log2 e), rounded to bf16 (torch's cast), and the
    score in natural units is tanh(q_s . k) * softcap, or (q_s . k) * ln 2."""
    fac = np.float32(scale * k_descale / softcap if softcap else scale * k_descale * math.log2(math.e))
    qs = torch.from_numpy(np.ascontiguousarray(q * fac, np.float32)).to(torch.bfloat16).double().numpy()
    sq, h, d = q.shape
    sk, hk, _ = k.shape
    out = np.zeros((sq, h, d))
    lse = np.full((h, sq), -np.inf)
    for hh in range(h):
        kh = hh // (h // hk)
        for i in range(sq):
            diag = i + sk - sq
            logits = []
            for j in range(sk):
                if causal and j > diag:
                    continue
                if window[0] >= 0 and j < diag - window[0]:
                    continue
                dot = sum(float(qs[i, hh, x]) * float(k[j, kh, x]) for x in range(d))
                s = math.tanh(dot) * softcap if softcap else dot * math.log(2.0)
                logits.append((j, s))
            if not logits:
                continue
            m = max(s for _, s in logits)
            z = sum(math.exp(s - m) for _, s in logits)
            lse[hh, i] = m + math.log(z)
            for j, s in logits:
                out[i, hh] += math.exp(s - m) / z * v[j, kh].astype(np.float64) * v_descale
    return out, lse


@pytest.mark.parametrize("softcap,window,causal", [(5.0, (-1, -1), True), (30.0, (3, -1), True),
                                                   (0.0, (2, -1), True), (2.0, (-1, -1), False)])
def test_rounded_q_softcap_branches_brute_force(softcap, window, causal):
    """The rounded-q branches of attention_ref, kvcache_reference and
    ragged_reference (with softcap and descales) against brute force."""
    rng = np.random.default_rng(9)
    sq, sk, h, hk, d = 4, 11, 4, 2, 16
    q = randn(rng, (1, sq, h, d)) * 3
    k = randn(rng, (1, sk, hk, d))
    v = randn(rng, (1, sk, hk, d))
    scale = 1 / math.sqrt(d)
    bo, bl = brute_force_rounded(q[0], k[0], v[0], causal, window, softcap, scale)
    out, lse = A.attention_ref(q, k, v, causal=causal, window_size=window, softcap=softcap,
                               round_scaled_q=True)
    np.testing.assert_allclose(out[0], bo, atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(lse[0], bl, atol=2e-5, rtol=1e-5)
    kd, vd = 0.75, 1.5
    bo, bl = brute_force_rounded(q[0], k[0], v[0], causal, window, softcap, scale, kd, vd)
    out, lse = A.kvcache_reference(q, k, v, np.array([sk]), causal=causal, window_size=window,
                                   softcap=softcap, k_descale=kd, v_descale=vd)
    np.testing.assert_allclose(out[0], bo, atol=4e-5, rtol=1e-4)
    np.testing.assert_allclose(lse[0], bl, atol=2e-5, rtol=1e-5)
    if causal:  # the paged varlen oracle: k / v as one page of sk keys
        out, lse = A.ragged_reference(q[0], k, v, np.array([0, sq]), np.array([sk]),
                                      np.zeros((1, 1), np.int64), causal=True,
                                      window_left=None if window[0] < 0 else window[0],
                                      softcap=softcap, k_descale=kd, v_descale=vd,
                                      round_scaled_q=True)
        np.testing.assert_allclose(out, bo, atol=4e-5, rtol=1e-4)
        np.testing.assert_allclose(lse, bl, atol=2e-5, rtol=1e-5)
