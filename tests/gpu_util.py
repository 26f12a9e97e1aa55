"""Shared helpers of the GPU parity tests: seeded inputs, oracle adapters and
the tolerance contract (bf16 out: max-abs 2e-2, mean-abs 2e-3; fp8 caches:
max-abs 5e-2; cache writes bit-exact)."""

import numpy as np
import torch

from oracle import attention as A
from oracle import dtypes as T
from oracle import paged as P

DEV = "cuda"
BF16_MAX, BF16_MEAN = 2e-2, 2e-3
FP8_MAX, FP8_MEAN = 5e-2, 5e-3
LSE_ATOL, LSE_RTOL = 4e-3, 2e-3

FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def announce(msg):
    print(f"[case] {msg}", flush=True)


def randn(rng, shape, scale=1.0):
    """float32 N(0, 1) from a numpy Generator rounded to bf16 (util.py:32-37)."""
    return T.bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def to_dev_bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).to(DEV)


def codes_of(t):
    """Raw codes of a device tensor as numpy (uint16 bf16 / uint8 fp8)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.uint8).numpy()


def values_of_codes(codes, dtype):
    if dtype == torch.bfloat16:
        return T.bf16_to_f32(codes)
    fmt = "e4m3" if dtype == torch.float8_e4m3fn else "e5m2"
    return T.fp8_decode(codes, fmt)


def dev_from_codes(codes, dtype):
    if dtype == torch.bfloat16:
        return torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(codes.view(np.uint8)).view(dtype).to(DEV)


def f32(t):
    return t.detach().float().cpu().numpy()


def random_codes(rng, shape, dtype, descale=1.0):
    """Stored codes of N(0,1)/descale in the cache dtype."""
    x = rng.standard_normal(shape, dtype=np.float32) / np.float32(descale)
    if dtype == torch.bfloat16:
        return T.bf16_round(x)
    fmt = "e4m3" if dtype == torch.float8_e4m3fn else "e5m2"
    return T.fp8_encode(x, fmt)


def assert_close(out, ref, fp8=False, what="out", valid=None):
    out = np.asarray(out, np.float32)
    ref = np.asarray(ref, np.float32)
    if valid is not None:
        out, ref = out[valid], ref[valid]
    err = np.abs(out - ref)
    mx, mean = float(err.max(initial=0.0)), float(err.mean()) if err.size else 0.0
    lim_max, lim_mean = (FP8_MAX, FP8_MEAN) if fp8 else (BF16_MAX, BF16_MEAN)
    assert np.isfinite(out).all(), f"{what}: non-finite values"
    assert mx <= lim_max and mean <= lim_mean, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"


def assert_lse(lse, ref):
    lse = np.asarray(lse, np.float32)
    ref = np.asarray(ref, np.float32)
    np.testing.assert_array_equal(np.isneginf(lse), np.isneginf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(lse[fin], ref[fin], rtol=LSE_RTOL, atol=LSE_ATOL)


class PagedCase:
    """A merged paged pool, its block table and the seeded new tokens."""

    def __init__(self, rng, *, batch, nheads, nheads_k, lengths, new_tokens, page_size=16,
                 head_dim=128, dtype=torch.bfloat16, k_descale=1.0, v_descale=1.0,
                 extra_pages=3, max_pages=None):
        self.batch, self.nheads, self.nheads_k = batch, nheads, nheads_k
        self.page_size, self.head_dim, self.dtype = page_size, head_dim, dtype
        self.lengths = np.asarray(lengths, np.int64)
        self.new_tokens = np.asarray(new_tokens, np.int64)
        need = [-(-(int(l) + int(n)) // page_size) for l, n in zip(self.lengths, self.new_tokens)]
        self.max_pages = max(max(need), 1) if max_pages is None else max_pages
        num_pages = sum(max(x, 1) for x in need) + extra_pages
        perm = rng.permutation(num_pages)
        table = np.zeros((batch, self.max_pages), np.int32)
        pos = 0
        for r in range(batch):
            cnt = max(need[r], 1)
            table[r, :cnt] = perm[pos:pos + cnt]
            pos += cnt
        self.table = table
        ch = P.merged_cache_heads(nheads_k, dtype.itemsize)
        self.pool_codes = random_codes(rng, (num_pages, page_size, ch, head_dim), dtype)
        if ch > 2 * nheads_k:  # the pad head of an fp8 pool holds zeros
            self.pool_codes[:, :, 2 * nheads_k:] = 0
        total_new = int(self.new_tokens.sum())
        self.k_codes = random_codes(rng, (total_new, nheads_k, head_dim), dtype, k_descale)
        self.v_codes = random_codes(rng, (total_new, nheads_k, head_dim), dtype, v_descale)
        self.cu = np.concatenate([[0], np.cumsum(self.new_tokens)]).astype(np.int32)
        self.k_descale, self.v_descale = k_descale, v_descale

    def pool(self):
        return dev_from_codes(self.pool_codes, self.dtype)

    def expected_pool(self, num_active=None):
        return P.append_to_pages(self.pool_codes, self.k_codes, self.v_codes, self.cu,
                                 self.lengths, self.table, num_active)

    def kv_pages(self, pool_codes):
        """(K pages, V pages) stored values as f32."""
        kc, vc = P.split_kv_heads(pool_codes, self.nheads_k)
        return values_of_codes(kc, self.dtype), values_of_codes(vc, self.dtype)

    def rows(self, pool_codes):
        kp, vp = self.kv_pages(pool_codes)
        return P.gather_rows(kp, self.table), P.gather_rows(vp, self.table)
