"""GPU parity at the full size of BASELINE configs C3, C4 (bf16 and over an e4m3
pool) and C5: the exact
seeded draws bench.py times (bench.inputs_c3 / inputs_c4 / inputs_c5; shapes
from the reference's scenario generator, benchmarks/softmax_attention/
kvcache_scenarios.py:313-329,682).

Each test runs the HIP path once at full size, then checks
  * the whole KV pool bit-exact against oracle.paged.append_to_pages applied to
    a host copy of the pool taken before the call (every appended row, and
    every other byte unchanged);
  * out (and lse) against the NumPy oracle on every row / request (about a
    minute of host time in all), with the north_star tolerance: bf16 max-abs
    2e-2 and mean-abs 2e-3, fp8 caches 5e-2.
"""

import numpy as np
import pytest
import torch

import bench
from flywheel_tpu import flash_attn_with_kvcache
from oracle import attention as A
from oracle import paged as P
from tests.gpu_util import announce, assert_close, assert_lse, codes_of, values_of_codes

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(400)]

DEV = torch.device("cuda:0")


def seq_rows(pool_codes, table_row, length, hk, dtype):
    """(length, Hk, D) K and V stored values (f32) of one sequence, in
    logical order, from a host copy of the pool's codes."""
    page = pool_codes.shape[1]
    pos = np.arange(length)
    rows = pool_codes[table_row[pos // page], pos % page]  # (L, CH, D)
    k, v = P.split_kv_heads(rows, hk)
    return values_of_codes(k, dtype), values_of_codes(v, dtype)


def new_rows_codes(t):
    """(T, Hk, D) codes of a new-token tensor."""
    return codes_of(t.reshape(-1, t.shape[-2], t.shape[-1]))


def test_c3_full_size():
    """C3: B=64, 32 q / 8 KV heads, page 16, ctx U[1K, 32K], fused append."""
    announce("C3 full size: decode bf16 B=64 ctx<=32K with fused append")
    x = bench.inputs_c3(DEV)
    lengths, hk = x["lengths"], x["hk"]
    before = codes_of(x["pool"])
    out, lse, pool = flash_attn_with_kvcache(
        x["q"], x["pool"], None, x["kn"], x["vn"], cache_seqlens=x["lens"],
        block_table=x["table"], return_softmax_lse=True)
    torch.cuda.synchronize()
    assert pool is x["pool"]
    after = codes_of(pool)
    b = x["b"]
    cu = np.arange(b + 1, dtype=np.int32)
    expected = P.append_to_pages(before, new_rows_codes(x["kn"]), new_rows_codes(x["vn"]), cu,
                                 lengths, x["table_np"])
    del before
    np.testing.assert_array_equal(after, expected)
    del expected
    rows = range(b)  # every row: stream-K cuts each at different range boundaries
    q = x["q"].float().cpu().numpy()
    o = out.float().cpu().numpy()
    ls = lse.cpu().numpy()
    for r in rows:
        total = int(lengths[r]) + 1
        k, v = seq_rows(after, x["table_np"][r], total, hk, torch.bfloat16)
        ro, rl = A.kvcache_reference(q[r:r + 1], k[None], v[None], np.array([total]))
        assert_close(o[r:r + 1], ro, what=f"row {r} (len {total})")
        assert_lse(ls[r:r + 1], rl)


def test_c4_full_size():
    """C4: 8 requests, chunks U[256, 2K] over prior U[0, 16K], 32/8 heads,
    window (4095, 0), softcap 50, causal; append then attend."""
    announce("C4 full size: chunked prefill window 4095 softcap 50")
    x = bench.inputs_c4(DEV)
    hk, window = x["hk"], x["window"]
    chunks, prior = x["chunks"], x["prior"]
    before = codes_of(x["pool"])
    out, lse, pool = flash_attn_with_kvcache(
        x["q"], x["pool"], None, x["kn"], x["vn"], cache_seqlens=x["lens"], block_table=x["tab"],
        cu_seqlens_q=x["cu"], max_seqlen_q=int(chunks.max()), causal=True,
        window_size=(window - 1, 0), softcap=50.0, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert pool is x["pool"]
    after = codes_of(pool)
    cu = x["cu"].cpu().numpy()
    expected = P.append_to_pages(before, new_rows_codes(x["kn"]), new_rows_codes(x["vn"]), cu,
                                 prior, x["table_np"])
    del before
    np.testing.assert_array_equal(after, expected)
    del expected
    q = x["q"].float().cpu().numpy()
    o = out.float().cpu().numpy()
    ls = lse.cpu().numpy()
    for s in range(x["n"]):  # every request
        total = int(prior[s] + chunks[s])
        k, v = seq_rows(after, x["table_np"][s], total, hk, torch.bfloat16)
        rows = slice(int(cu[s]), int(cu[s + 1]))
        ro, rl = A.ragged_reference(q[rows], k[None], v[None], np.array([0, chunks[s]]),
                                    np.array([total]), np.zeros((1, 1), np.int64), causal=True,
                                    window_left=window - 1, softcap=50.0, round_scaled_q=True)
        assert_close(o[rows], ro, what=f"request {s} (prior {prior[s]}, chunk {chunks[s]})")
        assert_lse(ls[:, rows], rl)


def test_c4_fp8_full_size():
    """C4's draw over an e4m3 pool (descales 0.8 / 1.25; bench.py's c4fp8):
    the fp8 rows widened into LDS by the ping-pong kernel, at full size."""
    announce("C4 full size over an e4m3 pool")
    x = bench.inputs_c4(DEV, fp8=True)
    hk, window = x["hk"], x["window"]
    chunks, prior = x["chunks"], x["prior"]
    kd, vd = x["extra"]["k_descale"], x["extra"]["v_descale"]
    before = codes_of(x["pool"])
    out, lse, pool = flash_attn_with_kvcache(
        x["q"], x["pool"], None, x["kn"], x["vn"], cache_seqlens=x["lens"], block_table=x["tab"],
        cu_seqlens_q=x["cu"], max_seqlen_q=int(chunks.max()), causal=True,
        window_size=(window - 1, 0), softcap=50.0, k_descale=kd, v_descale=vd,
        return_softmax_lse=True)
    torch.cuda.synchronize()
    assert pool is x["pool"]
    after = codes_of(pool)
    cu = x["cu"].cpu().numpy()
    expected = P.append_to_pages(before, new_rows_codes(x["kn"]), new_rows_codes(x["vn"]), cu,
                                 prior, x["table_np"])
    del before
    np.testing.assert_array_equal(after, expected)
    del expected
    q = x["q"].float().cpu().numpy()
    o = out.float().cpu().numpy()
    ls = lse.cpu().numpy()
    for s in range(x["n"]):  # every request
        total = int(prior[s] + chunks[s])
        k, v = seq_rows(after, x["table_np"][s], total, hk, torch.float8_e4m3fn)
        rows = slice(int(cu[s]), int(cu[s + 1]))
        ro, rl = A.ragged_reference(q[rows], k[None], v[None], np.array([0, chunks[s]]),
                                    np.array([total]), np.zeros((1, 1), np.int64), causal=True,
                                    window_left=window - 1, softcap=50.0, k_descale=kd,
                                    v_descale=vd, round_scaled_q=True)
        assert_close(o[rows], ro, fp8=True, what=f"request {s} (prior {prior[s]}, chunk {chunks[s]})")
        assert_lse(ls[:, rows], rl)


def test_c5_full_size():
    """C5: e4m3 pool, B=128, ctx U[4K, 64K], 4-token causal verify window,
    descales U[0.5, 2]."""
    announce("C5 full size: fp8 e4m3 verify window B=128 ctx<=64K")
    x = bench.inputs_c5(DEV)
    lengths, hk, sq = x["lengths"], x["hk"], x["sq"]
    kd, vd = x["k_descale"], x["v_descale"]
    before = codes_of(x["pool"])
    out, lse, pool = flash_attn_with_kvcache(
        x["q"], x["pool"], None, x["kn"], x["vn"], cache_seqlens=x["lens"], block_table=x["table"],
        causal=True, k_descale=kd, v_descale=vd, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert pool is x["pool"]
    after = codes_of(pool)
    b = x["b"]
    cu = (np.arange(b + 1) * sq).astype(np.int32)
    expected = P.append_to_pages(before, new_rows_codes(x["kn"]), new_rows_codes(x["vn"]), cu,
                                 lengths, x["table_np"])
    del before
    np.testing.assert_array_equal(after, expected)
    del expected
    rows = range(b)  # every row
    q = x["q"].float().cpu().numpy()
    o = out.float().cpu().numpy()
    ls = lse.cpu().numpy()
    for r in rows:
        total = int(lengths[r]) + sq
        k, v = seq_rows(after, x["table_np"][r], total, hk, torch.float8_e4m3fn)
        ro, rl = A.kvcache_reference(q[r:r + 1], k[None], v[None], np.array([total]), causal=True,
                                     k_descale=kd, v_descale=vd)
        assert_close(o[r:r + 1], ro, fp8=True, what=f"row {r} (len {total})")
        assert_lse(ls[r:r + 1], rl)
