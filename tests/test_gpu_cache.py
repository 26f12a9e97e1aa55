"""GPU bit-exactness of the cache writers: the ragged append and
write_kv_cache_pages (test_page.py:33-69's fixed pieces)."""

import numpy as np
import pytest
import torch

from flywheel_tpu import write_kv_cache_pages
from flywheel_tpu.decode import append_ragged
from oracle import paged as P
from tests.gpu_util import DEV, FP8, PagedCase, announce, codes_of, dev_from_codes, random_codes

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, **FP8}


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("hk", [1, 3, 8])
def test_append_ragged_bit_exact(dtype, hk):
    announce(f"append {dtype} hk={hk}")
    rng = np.random.default_rng(20)
    dt = DTYPES[dtype]
    lengths = [0, 15, 16, 300, 1]
    new = [17, 1, 0, 40, 33]
    case = PagedCase(rng, batch=5, nheads=hk, nheads_k=hk, lengths=lengths, new_tokens=new, dtype=dt)
    pool = case.pool()
    pad = 3  # packed padding rows past cu[-1] are never written
    k = dev_from_codes(np.concatenate([case.k_codes, random_codes(rng, (pad, hk, 128), dt)]), dt)
    v = dev_from_codes(np.concatenate([case.v_codes, random_codes(rng, (pad, hk, 128), dt)]), dt)
    for num_active in (None, 3):
        p = pool.clone()
        na = None if num_active is None else torch.tensor([num_active], dtype=torch.int32, device=DEV)
        append_ragged(p, k, v, torch.tensor(case.cu, device=DEV),
                      torch.tensor(case.lengths, dtype=torch.int32, device=DEV),
                      torch.tensor(case.table, device=DEV), na, hk)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(codes_of(p), case.expected_pool(num_active))


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("hk", [1, 2, 3, 8])
def test_write_kv_cache_pages(dtype, hk):
    announce(f"write pages {dtype} hk={hk}")
    rng = np.random.default_rng(0)
    dt = DTYPES[dtype]
    num_pages, page_size, d = 6, 128, 128
    ch = P.merged_cache_heads(hk, dt.itemsize)
    cache_codes = random_codes(rng, (num_pages, page_size, ch, d), dt)
    k_codes = random_codes(rng, (300, hk, d), dt)
    v_codes = random_codes(rng, (300, hk, d), dt)
    pieces = [(4 * page_size + 100, 0, 28), (1 * page_size, 28, 128), (3 * page_size, 156, 100)]
    slices = np.zeros((3, 8), np.int32)
    for j, pc in enumerate(pieces):
        slices[:, j] = pc
    expected = P.write_kv_cache_pages(k_codes, v_codes, cache_codes, slices, len(pieces))
    cache = dev_from_codes(cache_codes, dt)
    out = write_kv_cache_pages(dev_from_codes(k_codes, dt), dev_from_codes(v_codes, dt), cache,
                               torch.tensor(slices, device=DEV),
                               torch.tensor([len(pieces)], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert out is cache
    np.testing.assert_array_equal(codes_of(out), expected)
