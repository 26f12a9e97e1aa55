"""fw_paged_decode_noalloc (the workspace-free decode entry point) called
through the C-ABI, against fw_paged_decode with a workspace on the same
inputs: two calls in a row, the second with a smaller input, each within the
bf16 tolerance (max-abs 2e-2, mean-abs 2e-3) of the workspace entry point
(the same kernels, so in practice bit-equal), the KV pool bit-exact, and out
and lse against the NumPy oracle (kvcache_reference) themselves."""

import numpy as np
import pytest
import torch

from flywheel_tpu import _native as N
from flywheel_tpu.decode import decode_params, paged_decode
from oracle import attention as A
from tests.gpu_util import (DEV, PagedCase, announce, assert_close, assert_lse, codes_of,
                            dev_from_codes, randn, to_dev_bf16)

pytestmark = pytest.mark.gpu


def _case(seed, batch, max_len):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, max_len, batch)
    case = PagedCase(rng, batch=batch, nheads=32, nheads_k=8, lengths=lengths,
                     new_tokens=[1] * batch)
    qh = randn(rng, (batch, 1, 32, 128))
    q = to_dev_bf16(qh)
    case.q_host = qh
    kn = dev_from_codes(case.k_codes.reshape(batch, 8, 128), torch.bfloat16)
    vn = dev_from_codes(case.v_codes.reshape(batch, 8, 128), torch.bfloat16)
    return case, q, kn, vn


def _kw(case):
    return dict(nheads_k=8, softmax_scale=128 ** -0.5, softcap=0.0, causal=False, window_left=-1,
                k_descale=1.0, v_descale=1.0, return_lse=True)


def _run_noalloc(case, q, kn, vn):
    pool = case.pool()
    lens = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
    table = torch.tensor(case.table, device=DEV)
    p, out, lse, keep = decode_params(q, pool, kn, vn, lens, table, None, None, **_kw(case))
    lib = N.lib()
    need = lib.fw_paged_decode_workspace_bytes(p)
    assert 0 < need <= N.FW_DECODE_SCRATCH_BYTES
    p.workspace, p.workspace_bytes = None, 0  # ignored by the no-alloc entry point
    N.check(lib.fw_paged_decode_noalloc(p, N.stream_of(q)))
    torch.cuda.synchronize()
    del keep
    return out, lse, pool


def _run_workspace(case, q, kn, vn):
    pool = case.pool()
    lens = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
    table = torch.tensor(case.table, device=DEV)
    out, lse = paged_decode(q, pool, kn, vn, lens, table, None, None, **_kw(case))
    torch.cuda.synchronize()
    return out, lse, pool


def test_noalloc_decode_matches_workspace_decode_twice():
    big = _case(50, batch=48, max_len=20000)
    small = _case(51, batch=5, max_len=3000)
    for name, (case, q, kn, vn) in (("large", big), ("smaller", small)):
        announce(f"no-alloc decode, {name} call (batch {case.batch})")
        out_n, lse_n, pool_n = _run_noalloc(case, q, kn, vn)
        out_w, lse_w, pool_w = _run_workspace(case, q, kn, vn)
        np.testing.assert_array_equal(codes_of(pool_n), codes_of(pool_w))
        np.testing.assert_array_equal(codes_of(pool_n), case.expected_pool())
        assert_close(out_n.float().cpu().numpy(), out_w.float().cpu().numpy(),
                     what=f"{name} out")
        np.testing.assert_allclose(lse_n.cpu().numpy(), lse_w.cpu().numpy(), rtol=2e-3, atol=4e-3)
        krows, vrows = case.rows(case.expected_pool())
        ro, rl = A.kvcache_reference(case.q_host, krows, vrows, case.lengths + 1)
        assert_close(out_n.float().cpu().numpy(), ro, what=f"{name} out vs oracle")
        assert_lse(lse_n.cpu().numpy(), rl)


def test_noalloc_rejects_a_call_beyond_its_scratch():
    """Partials scale with (key ranges + rows) x KV heads x query rows: a batch
    of 4096 rows with a 4-token verify window needs far more than the static
    scratch, and the call is refused before anything is launched."""
    announce("no-alloc decode, oversized call rejected")
    case, q, kn, vn = _case(52, batch=4, max_len=100)
    pool = case.pool()
    lens = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
    table = torch.tensor(case.table, device=DEV)
    p, out, lse, keep = decode_params(q, pool, None, None, lens, table, None, None, **_kw(case))
    p.batch, p.seqlen_q = 4096, 4  # only the sizes matter: it is rejected unlaunched
    lib = N.lib()
    assert lib.fw_paged_decode_workspace_bytes(p) > N.FW_DECODE_SCRATCH_BYTES
    assert lib.fw_paged_decode_noalloc(p, N.stream_of(q)) == N.FW_ERR_VALUE
    assert b"FW_DECODE_SCRATCH_BYTES" in lib.fw_last_error()
