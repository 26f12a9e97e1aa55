"""The HIP path on the committed golden fixtures' inputs reproduces their
expected outputs: cache codes bit-exact, out / lse within the tolerance
contract (bf16 2e-2 max-abs / 2e-3 mean-abs, fp8 5e-2)."""

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func, flash_attn_with_kvcache, write_kv_cache_pages
from tests.golden import make_golden as G
from tests.gpu_util import DEV, FP8, announce, assert_close, assert_lse, codes_of, dev_from_codes

pytestmark = pytest.mark.gpu


def head_major(x):
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


def bf16_dev(codes):
    return dev_from_codes(np.ascontiguousarray(codes), torch.bfloat16)


@pytest.mark.parametrize("name", ["prefill_causal_gqa", "prefill_window_softcap"])
def test_golden_prefill(name):
    announce(f"golden {name}")
    f = G.load(name)
    out, lse = flash_attn_func(bf16_dev(head_major(f["q"])), bf16_dev(head_major(f["k"])),
                               bf16_dev(head_major(f["v"])), causal=bool(f["causal"]),
                               window_size=tuple(int(x) for x in f["window"]),
                               softcap=float(f["softcap"]), return_softmax_lse=True)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), head_major(f["out"]))
    assert_lse(lse.cpu().numpy(), f["lse"])


@pytest.mark.parametrize("name", ["decode_append_bf16", "decode_fp8_verify"])
def test_golden_decode(name):
    announce(f"golden {name}")
    f = G.load(name)
    fmt = str(f["fmt"])
    dt = torch.bfloat16 if fmt == "bf16" else FP8[fmt]
    b, sq = f["q"].shape[:2]
    hk = f["k_new"].shape[1]
    pool = dev_from_codes(f["pool"], dt)
    shape = (b, sq, hk, 128)
    out, lse, pool_out = flash_attn_with_kvcache(
        bf16_dev(f["q"]), pool, None, dev_from_codes(f["k_new"].reshape(shape), dt),
        dev_from_codes(f["v_new"].reshape(shape), dt),
        cache_seqlens=torch.tensor(f["lengths"], device=DEV), block_table=torch.tensor(f["table"], device=DEV),
        causal=bool(f["causal"]), return_softmax_lse=True, nheads_k=hk,
        k_descale=float(f["k_descale"]), v_descale=float(f["v_descale"]))
    torch.cuda.synchronize()
    assert pool_out is pool
    np.testing.assert_array_equal(codes_of(pool_out), f["exp_pool"])
    assert_close(out.float().cpu().numpy(), f["out"], fp8=fmt != "bf16")
    assert_lse(lse.cpu().numpy(), f["lse"])


def test_golden_write_pages():
    announce("golden write_pages_bf16")
    f = G.load("write_pages_bf16")
    cache = bf16_dev(f["cache"])
    out = write_kv_cache_pages(bf16_dev(f["k"]), bf16_dev(f["v"]), cache, torch.tensor(f["slices"], device=DEV),
                               torch.tensor([int(f["num_slices"])], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert out is cache
    np.testing.assert_array_equal(codes_of(out), f["exp_cache"])
