"""GPU parity of RoPE prefill: fw_rotary bit-exact against oracle/rotary.py
through the C-ABI, and flash_attn_func / flash_attn_varlen_func (packed and
paged, Q only) with rotary tables against the oracle's rotate-then-attend
(tests/softmax_attention/test_prefill.py:222-236, test_paged.py:410-470)."""

import math

import numpy as np
import pytest
import torch

from flywheel_tpu import flash_attn_func, flash_attn_varlen_func
from flywheel_tpu import rotary as R
from oracle import attention as A
from oracle import dtypes as T
from oracle import rotary as RO
from tests.gpu_util import (DEV, FP8, PagedCase, announce, assert_close, assert_lse, codes_of,
                            randn, to_dev_bf16)

pytestmark = pytest.mark.gpu


def tables(rng, rows, f32, d=128):
    ang = rng.random((rows, d // 2)) * 2 * math.pi
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    if not f32:
        cos, sin = T.bf16(cos), T.bf16(sin)
    dt = torch.float32 if f32 else torch.bfloat16
    return (cos, sin), (torch.tensor(cos, dtype=dt, device=DEV), torch.tensor(sin, dtype=dt, device=DEV))


def head_major(x):  # (B, S, H, D) -> (B, H, S, D)
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("f32", [False, True])
def test_rotate_rows_bitexact(interleaved, f32):
    """Dense head-major rows at t + offset, then packed rows with kv bases."""
    announce(f"fw_rotary interleaved={interleaved} f32={f32}")
    rng = np.random.default_rng(40)
    (cos, sin), tab = tables(rng, 300, f32)
    x = randn(rng, (2, 3, 129, 128), scale=3.0)
    y = R.rotate(to_dev_bf16(x), tab, interleaved, strides=(3 * 129 * 128, 129 * 128, 128),
                 batch_rows=2, nheads=3, ntokens=129, pos_offset=100)
    want = RO.rotate(x, cos, sin, np.arange(129) + 100, interleaved)
    np.testing.assert_array_equal(codes_of(y), T.bf16_round(want))
    # Packed token-major rows: (total, H * D), a zero-length sequence, pad rows.
    cu_q = np.array([0, 5, 5, 40, 41], np.int32)
    cu_k = np.array([0, 9, 12, 60, 300], np.int32)
    total = 45
    x = randn(rng, (total, 2, 128))
    y = R.rotate(to_dev_bf16(x.reshape(total, 256)), tab, interleaved, strides=(0, 128, 256),
                 batch_rows=1, nheads=2, ntokens=total, cu=torch.tensor(cu_q, device=DEV),
                 kv_cu=torch.tensor(cu_k, device=DEV))
    pos = RO.packed_positions(cu_q, total, np.diff(cu_k) - np.diff(cu_q))
    want = RO.rotate(x.transpose(1, 0, 2), cos, sin, pos, interleaved).transpose(1, 0, 2)
    np.testing.assert_array_equal(codes_of(y).reshape(total, 2, 128), T.bf16_round(want))
    # kv lengths given directly and two of four sequences active.
    used = np.array([9, 3, 60, 299], np.int32)
    y = R.rotate(to_dev_bf16(x.reshape(total, 256)), tab, interleaved, strides=(0, 128, 256),
                 batch_rows=1, nheads=2, ntokens=total, cu=torch.tensor(cu_q, device=DEV),
                 kv_lens=torch.tensor(used, device=DEV),
                 num_active=torch.tensor([2], dtype=torch.int32, device=DEV))
    cu_pin = np.minimum(cu_q, cu_q[2])
    pos = RO.packed_positions(cu_pin, total, np.where(np.arange(4) < 2, used, 0) - np.diff(cu_pin))
    want = RO.rotate(x.transpose(1, 0, 2), cos, sin, pos, interleaved).transpose(1, 0, 2)
    np.testing.assert_array_equal(codes_of(y).reshape(total, 2, 128), T.bf16_round(want))


@pytest.mark.parametrize(
    "b,h,hk,sq,sk,causal,interleaved,rotary_k,f32",
    [
        (2, 6, 2, 128, 256, True, False, True, False),
        (1, 4, 1, 77, 300, True, True, True, True),
        (2, 4, 4, 200, 200, False, False, False, True),
        (1, 8, 2, 512, 512, True, True, True, False),
    ],
)
def test_flash_attn_func_rotary(b, h, hk, sq, sk, causal, interleaved, rotary_k, f32):
    announce(f"dense rotary b{b} h{h}/{hk} sq{sq} sk{sk} il={interleaved} rk={rotary_k}")
    rng = np.random.default_rng(41)
    q, k, v = randn(rng, (b, sq, h, 128)), randn(rng, (b, sk, hk, 128)), randn(rng, (b, sk, hk, 128))
    (cos, sin), (tc, ts) = tables(rng, sk + 5, f32)
    qpos, kpos = RO.dense_positions(sq, sk)
    qr = RO.rotate(q.transpose(0, 2, 1, 3), cos, sin, qpos, interleaved).transpose(0, 2, 1, 3)
    kr = RO.rotate(k.transpose(0, 2, 1, 3), cos, sin, kpos, interleaved).transpose(0, 2, 1, 3)
    if not rotary_k:
        kr = k
    qd, kd = to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k))
    out, lse = flash_attn_func(qd, kd, to_dev_bf16(head_major(v)), causal=causal,
                               return_softmax_lse=True, rotary_cos=tc, rotary_sin=ts,
                               rotary_interleaved=interleaved, rotary_k=rotary_k)
    torch.cuda.synchronize()
    ro, rl = A.attention_ref(qr, kr, v, causal=causal, round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)
    # the caller's q and k are not modified
    np.testing.assert_array_equal(qd.float().cpu().numpy(), head_major(q))
    np.testing.assert_array_equal(kd.float().cpu().numpy(), head_major(k))


def test_flash_attn_func_rotary_heads_outer_fold():
    announce("dense rotary heads_outer_fold")
    rng = np.random.default_rng(42)
    b, h, hk, s = 2, 4, 2, 140
    q, k, v = randn(rng, (b, s, h, 128)), randn(rng, (b, s, hk, 128)), randn(rng, (b, s, hk, 128))
    (cos, sin), (tc, ts) = tables(rng, s, True)
    qr = RO.rotate(q.transpose(0, 2, 1, 3), cos, sin, np.arange(s), False).transpose(0, 2, 1, 3)
    hof = lambda x: np.ascontiguousarray(x.transpose(2, 0, 1, 3))
    out = flash_attn_func(to_dev_bf16(hof(q)), to_dev_bf16(hof(k)), to_dev_bf16(hof(v)),
                          causal=True, heads_outer_fold=True, rotary_cos=tc, rotary_sin=ts,
                          rotary_k=False)
    ro, _ = A.attention_ref(qr, k, v, causal=True, round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), hof(ro))


@pytest.mark.parametrize("interleaved,token_major", [(False, False), (True, True)])
def test_flash_attn_varlen_rotary(interleaved, token_major):
    announce(f"varlen rotary il={interleaved} tm={token_major}")
    rng = np.random.default_rng(43)
    qlens, klens = [5, 130, 0, 40], [9, 130, 7, 512]
    h, hk, d = 4, 2, 128
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn(rng, (cu_q[-1] + 3, h, d))
    k, v = randn(rng, (cu_k[-1], hk, d)), randn(rng, (cu_k[-1], hk, d))
    (cos, sin), (tc, ts) = tables(rng, 600, False)
    if token_major:
        args = [to_dev_bf16(x.reshape(x.shape[0], -1)) for x in (q, k, v)]
        kw = dict(token_major=True, head_dim=d)
    else:
        args = [to_dev_bf16(np.ascontiguousarray(x.transpose(1, 0, 2))) for x in (q, k, v)]
        kw = {}
    out = flash_attn_varlen_func(*args, torch.tensor(cu_q, device=DEV),
                                 torch.tensor(cu_k, device=DEV), max(qlens), max(klens),
                                 causal=True, rotary_cos=tc, rotary_sin=ts,
                                 rotary_interleaved=interleaved, **kw)
    torch.cuda.synchronize()
    outs = out.float().cpu().numpy()
    outs = outs.reshape(outs.shape[0], h, d) if token_major else outs.transpose(1, 0, 2)
    for s in range(4):
        if qlens[s] == 0:
            continue
        qpos, kpos = RO.dense_positions(qlens[s], klens[s])
        qs = RO.rotate(q[cu_q[s]:cu_q[s + 1]].transpose(1, 0, 2), cos, sin, qpos, interleaved)
        ks = RO.rotate(k[cu_k[s]:cu_k[s + 1]].transpose(1, 0, 2), cos, sin, kpos, interleaved)
        ro, _ = A.attention_ref(qs.transpose(1, 0, 2)[None], ks.transpose(1, 0, 2)[None],
                                v[cu_k[s]:cu_k[s + 1]][None], causal=True, round_scaled_q=True)
        assert_close(outs[cu_q[s]:cu_q[s + 1]], ro[0], what=f"seq {s}")


@pytest.mark.parametrize("interleaved", [False, True])
def test_paged_rotary_q_at_cache_positions(interleaved):
    """Reference test_paged.py:410-470: Q only, token t of a request at
    seqused_k - len_q + t; f32 tables; lengths (3, 1, 130) on prefixes
    (127, 0, 251); then num_active=2."""
    announce(f"paged rotary il={interleaved}")
    rng = np.random.default_rng(44)
    qlens, prefix = [3, 1, 130], [127, 0, 251]
    totals = np.array(qlens) + np.array(prefix)
    case = PagedCase(rng, batch=3, nheads=6, nheads_k=3, lengths=totals, new_tokens=[0] * 3)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1] + 5, 6, 128))
    (cos, sin), (tc, ts) = tables(rng, 400, True)
    kp, vp = case.kv_pages(case.pool_codes)
    for num_active in (None, 2):
        out, lse = flash_attn_varlen_func(
            to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
            torch.tensor(cu, device=DEV), None, max(qlens), 400, causal=True,
            return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
            seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), rotary_cos=tc,
            rotary_sin=ts, rotary_interleaved=interleaved, rotary_k=False, num_active=num_active)
        torch.cuda.synchronize()
        pos = RO.packed_positions(cu, q.shape[0], np.array(prefix))
        qr = RO.rotate(q.transpose(1, 0, 2), cos, sin, pos, interleaved).transpose(1, 0, 2)
        ro, rl = A.ragged_reference(qr, kp, vp, cu, totals, case.table, causal=True,
                                    round_scaled_q=True, num_active=num_active)
        assert_close(out.float().cpu().numpy().transpose(1, 0, 2), ro, what=f"active={num_active}")
        assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("d", [64, 96, 192, 256, 384, 512])
@pytest.mark.parametrize("interleaved", [False, True])
def test_rotate_rows_bitexact_head_dims(d, interleaved):
    """fw_rotary at head_dims other than 128 (tables of d/2 columns): dense rows at
    t + offset and packed rows with kv bases, bit-exact."""
    announce(f"fw_rotary d{d} interleaved={interleaved}")
    rng = np.random.default_rng(45 + d)
    (cos, sin), tab = tables(rng, 300, f32=interleaved, d=d)  # bf16 and f32 tables both run
    x = randn(rng, (2, 3, 65, d), scale=3.0)
    y = R.rotate(to_dev_bf16(x), tab, interleaved, strides=(3 * 65 * d, 65 * d, d),
                 batch_rows=2, nheads=3, ntokens=65, pos_offset=200)
    want = RO.rotate(x, cos, sin, np.arange(65) + 200, interleaved)
    np.testing.assert_array_equal(codes_of(y), T.bf16_round(want))
    cu_q = np.array([0, 5, 5, 40], np.int32)
    cu_k = np.array([0, 9, 12, 290], np.int32)
    total = 43
    x = randn(rng, (total, 2, d))
    y = R.rotate(to_dev_bf16(x.reshape(total, 2 * d)), tab, interleaved, strides=(0, d, 2 * d),
                 batch_rows=1, nheads=2, ntokens=total, cu=torch.tensor(cu_q, device=DEV),
                 kv_cu=torch.tensor(cu_k, device=DEV))
    pos = RO.packed_positions(cu_q, total, np.diff(cu_k) - np.diff(cu_q))
    want = RO.rotate(x.transpose(1, 0, 2), cos, sin, pos, interleaved).transpose(1, 0, 2)
    np.testing.assert_array_equal(codes_of(y).reshape(total, 2, d), T.bf16_round(want))


@pytest.mark.parametrize("d", [64, 96, 192, 256, 512])
@pytest.mark.parametrize("interleaved,rotary_k,f32", [(False, True, False), (True, True, True),
                                                      (False, False, True)])
def test_flash_attn_func_rotary_head_dims(d, interleaved, rotary_k, f32):
    """Fused Q RoPE in the register-staged (64, 96, 192) and head_dim-256
    kernels, K through fw_rotary: against rotate-then-attend."""
    announce(f"dense rotary d{d} il={interleaved} rk={rotary_k} f32={f32}")
    rng = np.random.default_rng(46 + d)
    b, h, hk, sq, sk = 1, 8, 2, 190, 333
    q, k, v = randn(rng, (b, sq, h, d)), randn(rng, (b, sk, hk, d)), randn(rng, (b, sk, hk, d))
    (cos, sin), (tc, ts) = tables(rng, sk + 2, f32, d)
    qpos, kpos = RO.dense_positions(sq, sk)
    qr = RO.rotate(q.transpose(0, 2, 1, 3), cos, sin, qpos, interleaved).transpose(0, 2, 1, 3)
    kr = RO.rotate(k.transpose(0, 2, 1, 3), cos, sin, kpos, interleaved).transpose(0, 2, 1, 3)
    if not rotary_k:
        kr = k
    out, lse = flash_attn_func(to_dev_bf16(head_major(q)), to_dev_bf16(head_major(k)),
                               to_dev_bf16(head_major(v)), causal=True, return_softmax_lse=True,
                               rotary_cos=tc, rotary_sin=ts, rotary_interleaved=interleaved,
                               rotary_k=rotary_k)
    torch.cuda.synchronize()
    ro, rl = A.attention_ref(qr, kr, v, causal=True, round_scaled_q=True)
    assert_close(out.float().cpu().numpy(), head_major(ro))
    assert_lse(lse.cpu().numpy(), rl)


@pytest.mark.parametrize("d,dtype", [(64, "bf16"), (256, "bf16"), (256, "e4m3")])
def test_paged_rotary_head_dims(d, dtype):
    """Paged prefill with Q RoPE at head_dim 64 and 256 (bf16 and an e4m3
    pool): Q only, at seqused_k - len_q + t."""
    announce(f"paged rotary d{d} {dtype}")
    rng = np.random.default_rng(47 + d)
    dt = torch.bfloat16 if dtype == "bf16" else FP8[dtype]
    kd, vd = (1.0, 1.0) if dtype == "bf16" else (0.75, 1.5)
    qlens, prefix = [3, 70, 130], [127, 0, 200]
    totals = np.array(qlens) + np.array(prefix)
    case = PagedCase(rng, batch=3, nheads=8, nheads_k=2, lengths=totals, new_tokens=[0] * 3,
                     head_dim=d, dtype=dt, k_descale=kd, v_descale=vd)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = randn(rng, (cu[-1] + 2, 8, d))
    (cos, sin), (tc, ts) = tables(rng, 400, True, d)
    kp, vp = case.kv_pages(case.pool_codes)
    out, lse = flash_attn_varlen_func(
        to_dev_bf16(np.ascontiguousarray(q.transpose(1, 0, 2))), case.pool(), None,
        torch.tensor(cu, device=DEV), None, max(qlens), 400, causal=True,
        return_softmax_lse=True, block_table=torch.tensor(case.table, device=DEV),
        seqused_k=torch.tensor(totals, dtype=torch.int32, device=DEV), rotary_cos=tc,
        rotary_sin=ts, rotary_k=False, k_descale=kd, v_descale=vd, nheads_k=2)
    torch.cuda.synchronize()
    pos = RO.packed_positions(cu, q.shape[0], np.array(prefix))
    qr = RO.rotate(q.transpose(1, 0, 2), cos, sin, pos, False).transpose(1, 0, 2)
    ro, rl = A.ragged_reference(qr, kp, vp, cu, totals, case.table, causal=True,
                                k_descale=kd, v_descale=vd, round_scaled_q=True)
    assert_close(out.float().cpu().numpy().transpose(1, 0, 2), ro, fp8=dtype != "bf16")
    assert_lse(lse.cpu().numpy(), rl)
