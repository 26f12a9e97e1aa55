"""GPU tests of the path's robustness rules:

* cache slots past a row's length may hold anything (NaN included): they are
  never used (the reference zeroes / keeps finite the slots past seqused_k,
  kernels/fwd_paged.py:285-290, kernels/decode.py:836; its test
  tests/softmax_attention/test_paged.py:465 pads with NaN);
* a block-table entry outside [0, num_pages) is never dereferenced: writes to
  it are dropped and its keys read as zero K and V rows;
* k_descale / v_descale given as device tensors are read on the device: the
  result equals the Python-float call bit for bit, and the call needs no host
  synchronisation (it can be captured into a graph).
"""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_varlen_func, flash_attn_with_kvcache
from oracle import attention as A
from oracle import paged as P
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, codes_of,
                            dev_from_codes, randn, to_dev_bf16)

pytestmark = pytest.mark.gpu

NAN_CODE = {torch.bfloat16: 0x7FC0, torch.float8_e4m3fn: 0x7F, torch.float8_e5m2: 0x7F}


def poison_unused_slots(case, used):
    """Every slot at a logical position >= used[r] of row r, and every page no
    row maps, gets the dtype's NaN code."""
    codes = case.pool_codes
    page = case.page_size
    mapped = np.zeros(codes.shape[0], bool)
    for r in range(case.batch):
        n_pages = -(-int(used[r]) // page) if used[r] else 0
        row_pages = case.table[r, :max(n_pages, 1)]
        mapped[row_pages[:n_pages]] = True
        if used[r] % page:
            codes[case.table[r, n_pages - 1], used[r] % page:] = NAN_CODE[case.dtype]
    codes[~mapped] = NAN_CODE[case.dtype]


def clean_rows(krows, vrows, totals):
    """The oracle's gathered rows with the (never visible) poisoned slots set
    to 0, so its masked products stay finite."""
    krows, vrows = krows.copy(), vrows.copy()
    for r, t in enumerate(totals):
        krows[r, t:] = 0
        vrows[r, t:] = 0
    return krows, vrows


@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
@pytest.mark.parametrize("append", [True, False])
def test_decode_ignores_nan_in_unused_slots(dtype, append):
    announce(f"decode NaN-filled unused slots {dtype} append={append}")
    rng = np.random.default_rng(40)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    lengths = [0, 5, 16, 17, 1000, 4095]
    new = [1 if append else 0] * len(lengths)
    case = PagedCase(rng, batch=len(lengths), nheads=16, nheads_k=4, lengths=lengths,
                     new_tokens=new, dtype=dt, k_descale=1.25, v_descale=0.75, extra_pages=4)
    totals = case.lengths + case.new_tokens
    # the slot the append writes is poisoned too: the kernel must read the
    # new token from k / v, never from the slot it is writing
    poison_unused_slots(case, case.lengths)
    q = randn(rng, (case.batch, 1, 16, 128))
    kw = {}
    if append:
        kw = dict(k=dev_from_codes(case.k_codes.reshape(case.batch, 1, 4, 128), dt),
                  v=dev_from_codes(case.v_codes.reshape(case.batch, 1, 4, 128), dt))
    pool = case.pool()
    out, lse, _ = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, **kw, cache_seqlens=torch.tensor(lengths, device=DEV),
        block_table=torch.tensor(case.table, device=DEV), return_softmax_lse=True,
        k_descale=1.25, v_descale=0.75, nheads_k=4)
    torch.cuda.synchronize()
    exp_pool = case.expected_pool() if append else case.pool_codes
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    krows, vrows = clean_rows(*case.rows(exp_pool), totals)
    ro, rl = A.kvcache_reference(q, krows, vrows, totals, k_descale=1.25, v_descale=0.75)
    nonempty = totals > 0
    assert_close(out.float().cpu().numpy()[nonempty], ro[nonempty], fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("hd", [128, 256])
@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
def test_verify_window_and_chunked_prefill_ignore_nan(dtype, hd):
    """The folded verify window (decode kernel after an append) and the paged
    varlen prefill kernels (the ping-pong kernel at head_dim 128, the d256
    kernel at 256; bf16 and fp8 pools) over a pool whose unused slots hold
    NaN."""
    announce(f"verify window + chunked prefill NaN slots {dtype} d{hd}")
    rng = np.random.default_rng(41)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    lengths = [3, 100, 700, 2047]
    case = PagedCase(rng, batch=4, nheads=32, nheads_k=8, lengths=lengths, new_tokens=[4] * 4,
                     head_dim=hd, dtype=dt, k_descale=0.5, v_descale=2.0, extra_pages=2)
    poison_unused_slots(case, case.lengths)
    totals = case.lengths + 4
    q = randn(rng, (4, 4, 32, hd))
    pool = case.pool()
    out, lse, _ = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, dev_from_codes(case.k_codes.reshape(4, 4, 8, hd), dt),
        dev_from_codes(case.v_codes.reshape(4, 4, 8, hd), dt),
        cache_seqlens=torch.tensor(lengths, device=DEV), causal=True,
        block_table=torch.tensor(case.table, device=DEV), return_softmax_lse=True,
        k_descale=0.5, v_descale=2.0)
    torch.cuda.synchronize()
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    krows, vrows = clean_rows(*case.rows(exp_pool), totals)
    ro, rl = A.kvcache_reference(q, krows, vrows, totals, causal=True, k_descale=0.5, v_descale=2.0)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
    # the same pool read by the paged varlen kernel: 300 query rows per
    # sequence on top of the appended lengths
    qlens = np.array([1, 100, 77, 300])
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    qp = randn(rng, (int(cu[-1]), 32, hd))
    used = totals  # kv lengths: the appended lengths
    out2, lse2 = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(qp.transpose(1, 0, 2))), pool, None,
        torch.tensor(cu, device=DEV), None, int(qlens.max()), int(used.max()), causal=True,
        return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(used, dtype=torch.int32, device=DEV), k_descale=0.5,
        v_descale=2.0, nheads_k=8)
    torch.cuda.synchronize()
    kp, vp = case.kv_pages(exp_pool)
    kp, vp = np.nan_to_num(kp, nan=0.0), np.nan_to_num(vp, nan=0.0)
    ro2, rl2 = A.ragged_reference(qp, kp, vp, cu, used, case.table, causal=True, k_descale=0.5,
                                  v_descale=2.0, round_scaled_q=True)
    assert_close(out2.float().cpu().numpy().transpose(1, 0, 2), ro2, fp8=dtype != "bf16")
    assert_lse(lse2.cpu().numpy(), rl2)


@pytest.mark.parametrize("hd", [128, 256])
@pytest.mark.parametrize("dtype", ["bf16", "e4m3"])
@pytest.mark.parametrize("bad_id", [-1, 1 << 30])
def test_invalid_page_ids_read_as_zero_rows(dtype, bad_id, hd):
    """Decode (with the fused append), the folded verify window and the paged
    varlen prefill over a table with out-of-range entries: nothing is read or
    written through them, and their keys act as zero K and V rows.  Expected:
    the oracle over the same table with those entries pointing at a page of
    zeros."""
    announce(f"invalid page ids {dtype} id={bad_id} d{hd}")
    rng = np.random.default_rng(42)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    lengths = [64, 700, 333, 1500]
    case = PagedCase(rng, batch=4, nheads=8, nheads_k=2, lengths=lengths, new_tokens=[1] * 4,
                     head_dim=hd, dtype=dt, extra_pages=2)
    poison_unused_slots(case, case.lengths)
    bad = {0: [1], 1: [0, 5, 6, 30], 2: [19], 3: [92]}  # full pages before each row's append page
    table = case.table.copy()
    for r, idx in bad.items():
        table[r, idx] = bad_id
    q = randn(rng, (4, 1, 8, hd))
    pool = case.pool()
    kn = dev_from_codes(case.k_codes.reshape(4, 1, 2, hd), dt)
    vn = dev_from_codes(case.v_codes.reshape(4, 1, 2, hd), dt)
    out, lse, _ = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, kn, vn, cache_seqlens=torch.tensor(lengths, device=DEV),
        block_table=torch.tensor(table, device=DEV), return_softmax_lse=True)
    torch.cuda.synchronize()
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(codes_of(pool), exp_pool)
    totals = case.lengths + 1
    kp, vp = case.kv_pages(exp_pool)
    zero = kp.shape[0]  # an extra all-zero page stands for every invalid id
    kp = np.concatenate([np.nan_to_num(kp, nan=0.0), np.zeros_like(kp[:1])])
    vp = np.concatenate([np.nan_to_num(vp, nan=0.0), np.zeros_like(vp[:1])])
    ztab = np.where((table < 0) | (table >= zero), zero, table)
    krows, vrows = clean_rows(P.gather_rows(kp, ztab), P.gather_rows(vp, ztab), totals)
    ro, rl = A.kvcache_reference(q, krows, vrows, totals)
    assert_close(out.float().cpu().numpy(), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
    # paged varlen prefill over the same table, causal with a window
    qlens = np.array([5, 300, 1, 64])
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    qp = randn(rng, (int(cu[-1]), 8, hd))
    out2, lse2 = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(qp.transpose(1, 0, 2))), pool, None,
        torch.tensor(cu, device=DEV), None, int(qlens.max()), int(totals.max()), causal=True,
        window_size=(200, 0), return_softmax_lse=True, block_table=torch.tensor(table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), nheads_k=2)
    torch.cuda.synchronize()
    ro2, rl2 = A.ragged_reference(qp, kp, vp, cu, totals, ztab, causal=True, window_left=200,
                                  round_scaled_q=True)
    assert_close(out2.float().cpu().numpy().transpose(1, 0, 2), ro2, fp8=dtype != "bf16")
    assert_lse(lse2.cpu().numpy(), rl2)


def _fp8_verify_case(rng):
    lengths = [40, 3000, 17, 999]
    case = PagedCase(rng, batch=4, nheads=32, nheads_k=8, lengths=lengths, new_tokens=[4] * 4,
                     dtype=torch.float8_e4m3fn, k_descale=0.6, v_descale=1.7)
    q = to_dev_bf16(randn(rng, (4, 4, 32, 128)))
    k = dev_from_codes(case.k_codes.reshape(4, 4, 8, 128), case.dtype)
    v = dev_from_codes(case.v_codes.reshape(4, 4, 8, 128), case.dtype)
    return case, q, k, v, torch.tensor(lengths, dtype=torch.int32, device=DEV)


def test_device_descales_equal_float_descales():
    announce("device-tensor descales, decode + paged prefill")
    rng = np.random.default_rng(43)
    case, q, k, v, lens = _fp8_verify_case(rng)
    table = torch.tensor(case.table, device=DEV)
    results = []
    for kd, vd in ((0.6, 1.7), (torch.tensor(0.6, device=DEV), torch.tensor([1.7], device=DEV))):
        pool = case.pool()
        out, lse, _ = flash_attn_with_kvcache(q, pool, None, k, v, cache_seqlens=lens,
                                              block_table=table, causal=True, k_descale=kd,
                                              v_descale=vd, return_softmax_lse=True)
        qp = q.reshape(16, 32, 128).transpose(0, 1).contiguous()
        cu = torch.tensor([0, 4, 8, 12, 16], dtype=torch.int32, device=DEV)
        out2 = flash_attn_varlen_func(qp, pool, None, cu, None, 4, 4000, causal=True,
                                      block_table=table, seqused_k=lens + 4, k_descale=kd,
                                      v_descale=vd, nheads_k=8)
        torch.cuda.synchronize()
        results.append((out, lse, out2, codes_of(pool)))
    for a, b in zip(*results):
        if isinstance(a, np.ndarray):
            np.testing.assert_array_equal(a, b)
        else:
            assert torch.equal(a, b)
    # and the float path matches the oracle
    exp_pool = case.expected_pool()
    np.testing.assert_array_equal(results[0][3], exp_pool)
    krows, vrows = case.rows(exp_pool)
    ro, rl = A.kvcache_reference(q.float().cpu().numpy(), krows, vrows, case.lengths + 4,
                                 causal=True, k_descale=0.6, v_descale=1.7)
    assert_close(results[0][0].float().cpu().numpy(), ro, fp8=True)


def test_decode_with_device_descales_captures_into_a_graph():
    """No host synchronisation inside the call: it is captured into a CUDA
    graph; every replay (with eager work and synchronisation between them)
    equals the eager result."""
    announce("graph capture of fp8 decode with device descales")
    rng = np.random.default_rng(44)
    case, q, k, v, lens = _fp8_verify_case(rng)
    table = torch.tensor(case.table, device=DEV)
    kd = torch.tensor([0.6], device=DEV)
    vd = torch.tensor([1.7], device=DEV)
    q1 = q[:, :1].contiguous()
    k1, v1 = k[:, :1].contiguous(), v[:, :1].contiguous()
    pool = case.pool()
    step = lambda: flash_attn_with_kvcache(q1, pool, None, k1, v1, cache_seqlens=lens,
                                           block_table=table, k_descale=kd, v_descale=vd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = step()[0].clone()  # the append is idempotent: same slot, same row
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()[0]
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        _ = (q1.float() * 2).sum().item()  # eager work between replays
    got = codes_of(pool)
    # one token appended per row at cache_seqlens
    cu = np.arange(5, dtype=np.int32)
    exp_pool = P.append_to_pages(case.pool_codes, case.k_codes.reshape(4, 4, 8, 128)[:, 0],
                                 case.v_codes.reshape(4, 4, 8, 128)[:, 0], cu, case.lengths,
                                 case.table)
    np.testing.assert_array_equal(got, exp_pool)
