"""GPU parity of paged decode at serving batch sizes: more rows than the
decode kernel's resident workgroups (256 at head_dim 128), so one workgroup's
stream-K range spans many rows, rows with no key sit between live ones, and
the row walk crosses many 64-row passes.

Shapes follow the reference's ragged draws (`test_paged.py:43-77`): many short
rows (0-64 cached tokens) mixed with long ones (1-3000), some rows past
`num_active` (never appended; out 0, lse -inf), the fused append on and off,
bf16 and e4m3 pools, 1 and 4 query tokens.  Every live row is compared with
the NumPy oracle (`kvcache_reference`, after `decode_reference`,
`test_regression.py:901-961`), and the whole pool bit-exact with the oracle's
append."""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_with_kvcache
from oracle import attention as A
from oracle import paged as P
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, codes_of,
                            dev_from_codes, randn, to_dev_bf16)

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(300)]

CHUNK = 64  # oracle rows per pass (bounds the host's gathered K/V)


def serving_lengths(rng, batch):
    """80 % short rows (0-64 cached tokens), 20 % long (1-3000), shuffled."""
    short = rng.integers(0, 65, batch)
    long_ = rng.integers(1, 3001, batch)
    return np.where(rng.random(batch) < 0.8, short, long_)


CASES = [
    # batch, nheads, nheads_k, dtype, query tokens, fused append, num_active
    (300, 32, 8, "bf16", 1, True, 300),
    (300, 32, 8, "e4m3", 4, True, 281),
    (300, 32, 4, "bf16", 4, False, 300),
    (1024, 32, 8, "bf16", 1, True, 1000),
    (1024, 32, 8, "e4m3", 1, False, 1024),
    (1024, 16, 2, "bf16", 4, True, 1024),
]


@pytest.mark.parametrize("batch,h,hk,dt_name,nq,append,num_active", CASES,
                         ids=[f"b{c[0]}-{c[1]}/{c[2]}-{c[3]}-nq{c[4]}-app{int(c[5])}-na{c[6]}"
                              for c in CASES])
def test_serving_batch(batch, h, hk, dt_name, nq, append, num_active):
    announce(f"serving decode b{batch} h{h}/{hk} {dt_name} nq{nq} append={append}"
             f" num_active={num_active}")
    rng = np.random.default_rng(batch * 7 + h + hk + nq + int(append))
    dt = torch.bfloat16 if dt_name == "bf16" else FP8[dt_name]
    kd, vd = (1.0, 1.0) if dt_name == "bf16" else (0.75, 1.5)
    lengths = serving_lengths(rng, batch)
    if not append:  # the query tokens' own keys must already be cached
        lengths = np.maximum(lengths, nq)
    d = 128
    case = PagedCase(rng, batch=batch, nheads=h, nheads_k=hk, lengths=lengths,
                     new_tokens=[nq if append else 0] * batch, dtype=dt, k_descale=kd,
                     v_descale=vd, head_dim=d)
    q = randn(rng, (batch, nq, h, d))
    pool = case.pool()
    kw = {}
    if append:
        shape = (batch, nq, hk, d)
        kw = dict(k=dev_from_codes(case.k_codes.reshape(shape), dt),
                  v=dev_from_codes(case.v_codes.reshape(shape), dt))
    na = None if num_active == batch else num_active
    out, lse, pool_out = flash_attn_with_kvcache(
        to_dev_bf16(q), pool, None, **kw,
        cache_seqlens=torch.tensor(lengths, dtype=torch.int32, device=DEV),
        block_table=torch.tensor(case.table, device=DEV), causal=True,
        return_softmax_lse=True, nheads_k=hk, k_descale=kd, v_descale=vd, num_active=na)
    torch.cuda.synchronize()
    assert pool_out is pool
    after = codes_of(pool)
    expected = case.expected_pool(num_active=na) if append else case.pool_codes
    np.testing.assert_array_equal(after, expected)
    o = out.float().cpu().numpy()
    ls = lse.cpu().numpy()
    totals = lengths + (nq if append else 0)
    kp, vp = case.kv_pages(after)
    fp8 = dt_name != "bf16"
    for r0 in range(0, num_active, CHUNK):
        r1 = min(r0 + CHUNK, num_active)
        tab = case.table[r0:r1]
        need = max(1, -(-int(totals[r0:r1].max()) // case.page_size))
        krows = P.gather_rows(kp, tab[:, :need])
        vrows = P.gather_rows(vp, tab[:, :need])
        ro, rl = A.kvcache_reference(q[r0:r1], krows, vrows, totals[r0:r1], causal=True,
                                     k_descale=kd, v_descale=vd)
        assert_close(o[r0:r1], ro, fp8=fp8, what=f"rows {r0}..{r1 - 1}")
        assert_lse(ls[r0:r1], rl)
    # rows past num_active: nothing appended (checked above), out 0, lse -inf
    assert not o[num_active:].any()
    assert np.isneginf(ls[num_active:]).all()
