"""Host-side checks that need no GPU: the C-ABI library exports what
include/flywheel_hip.h declares, its argument validation returns the
documented status codes, and the Python API raises the reference's exception
types (flywheel_tpu/softmax_attention/inputs.py:218-251, decode.py:286-435,
prefill.py:437-963) before anything is launched."""

import ctypes
import os
import re

import pytest
import torch

import flywheel_tpu
from flywheel_tpu import _native as N
from flywheel_tpu import (flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache,
                          write_kv_cache_pages)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flywheel_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fw_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    names = declared_functions()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), f"{name} is declared but not exported"
    assert set(names) == set(N.SIGNATURES), "ctypes bindings and header disagree"
    assert lib.fw_abi_version() == 6


def test_struct_layouts_match_header_fields():
    text = open(HEADER).read()
    for struct, cls in (("fw_decode_params", N.DecodeParams), ("fw_prefill_params", N.PrefillParams),
                        ("fw_rotary_params", N.RotaryParams),
                        ("fw_attn_bwd_params", N.AttnBwdParams)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            names = decl.split()[-1] if "," not in decl else decl
            for part in re.split(r",", decl):
                m = re.search(r"\**([A-Za-z_0-9]+)\s*$", part.strip())
                fields.append(m.group(1))
        assert fields == [f[0] for f in cls._fields_], struct


STRUCTS = (("fw_decode_params", N.DecodeParams), ("fw_prefill_params", N.PrefillParams),
           ("fw_rotary_params", N.RotaryParams), ("fw_attn_bwd_params", N.AttnBwdParams))


def test_struct_offsets_and_widths_match_c(tmp_path):
    """Every field's offset and width, and each struct's size, as the C
    compiler lays out include/flywheel_hip.h, against the ctypes mirror: an
    int32 / int64 / size_t / pointer mismatch moves an offset or a width."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"',
             "int main(void) {"]
    for struct, cls in STRUCTS:
        lines.append(f'printf("{struct} sizeof %zu %zu\\n", sizeof({struct}), (size_t)0);')
        for name, _ in cls._fields_:
            lines.append(f'printf("{struct} {name} %zu %zu\\n", offsetof({struct}, {name}),'
                         f' sizeof((({struct} *)0)->{name}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c99", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        struct, name, off, size = line.split()
        got[(struct, name)] = (int(off), int(size))
    for struct, cls in STRUCTS:
        assert got[(struct, "sizeof")][0] == ctypes.sizeof(cls), struct
        for name, _ in cls._fields_:
            f = getattr(cls, name)
            assert got[(struct, name)] == (f.offset, f.size), f"{struct}.{name}"


def test_capi_validation_status_codes():
    lib = N.lib()
    p = N.DecodeParams()
    p.batch, p.seqlen_q, p.nheads, p.nheads_k, p.head_dim = 2, 1, 8, 2, 96
    p.page_size, p.max_pages, p.num_pages = 16, 4, 8
    assert lib.fw_paged_decode_workspace_bytes(p) == 0
    assert lib.fw_paged_decode(p, None) == N.FW_ERR_NOT_IMPLEMENTED
    assert b"head_dim" in lib.fw_last_error()
    p.head_dim, p.page_size = 128, 24
    assert lib.fw_paged_decode(p, None) == N.FW_ERR_VALUE
    p.page_size, p.nheads = 16, 7
    assert lib.fw_paged_decode(p, None) == N.FW_ERR_VALUE
    p.nheads = 8
    assert lib.fw_paged_decode_workspace_bytes(p) > 0
    assert lib.fw_paged_decode(p, None) == N.FW_ERR_VALUE  # no workspace
    q = N.PrefillParams()
    q.kv_mode, q.head_dim, q.nheads, q.nheads_k = N.FW_KV_DENSE, 160, 4, 2
    assert lib.fw_prefill(q, None) == N.FW_ERR_NOT_IMPLEMENTED
    q.head_dim, q.head_dim_v = 64, 128  # d64 takes head_dim_v 64, 256 or 512
    assert lib.fw_prefill(q, None) == N.FW_ERR_NOT_IMPLEMENTED
    for d, dv in ((96, 96), (192, 192), (192, 128), (64, 256), (64, 512), (384, 384), (512, 512)):
        q.head_dim, q.head_dim_v = d, dv
        assert lib.fw_prefill(q, None) == N.FW_ERR_VALUE  # supported dims; no tensors
    q.head_dim, q.head_dim_v, q.kv_mode = 96, 0, N.FW_KV_PAGED  # pools: 64, 128, 256
    assert lib.fw_prefill(q, None) == N.FW_ERR_NOT_IMPLEMENTED
    q.kv_mode = N.FW_KV_DENSE
    q.head_dim, q.head_dim_v, q.kv_mode = 128, 256, N.FW_KV_PAGED  # one head dim in a pool
    assert lib.fw_prefill(q, None) == N.FW_ERR_VALUE
    q.kv_mode, q.head_dim_v = N.FW_KV_DENSE, 0
    q.head_dim, q.kv_dtype = 128, N.FW_FP8_E4M3
    assert lib.fw_prefill(q, None) == N.FW_ERR_NOT_IMPLEMENTED  # fp8 only for a paged pool
    # the checks run before any launch, so these stand-in addresses are never read
    fake = ctypes.c_void_p(0x1000)
    q.head_dim, q.kv_dtype, q.batch, q.seqlen_q, q.seqlen_k = 128, N.FW_BF16, 1, 8, 8
    q.q = q.out = q.k = fake
    assert lib.fw_prefill(q, None) == N.FW_ERR_VALUE  # dense without v
    assert b"needs v" in lib.fw_last_error()
    q.kv_mode, q.cu_seqlens_q, q.workspace, q.workspace_bytes = N.FW_KV_PAGED, fake, fake, 1 << 40
    q.seqused_k, q.block_table, q.num_pages, q.max_pages = fake, fake, 4, 4
    for page in (12, 20, 24):  # key groups of 8 and 16 rows would straddle pages
        q.page_size = page
        assert lib.fw_prefill(q, None) == N.FW_ERR_VALUE
        assert b"multiple of 16" in lib.fw_last_error()
    q.kv_mode = N.FW_KV_DENSE
    assert lib.fw_append_ragged(None, None, None, None, None, None, None, 1, 0, 2, 128, 16, 1, 1,
                                7, None) == N.FW_ERR_NOT_IMPLEMENTED
    bw = N.AttnBwdParams()
    bw.head_dim, bw.nheads, bw.nheads_k, bw.batch, bw.seqlen_q, bw.seqlen_k = 64, 4, 2, 1, 8, 8
    assert lib.fw_attn_bwd(bw, None) == N.FW_ERR_NOT_IMPLEMENTED
    for d, dv in ((192, 0), (256, 512), (128, 384)):  # kernels: 128 or 256 / 128, 256 or 512
        bw.head_dim, bw.head_dim_v = d, dv
        assert lib.fw_attn_bwd(bw, None) == N.FW_ERR_NOT_IMPLEMENTED
    bw.head_dim, bw.head_dim_v = 256, 128
    assert lib.fw_attn_bwd(bw, None) == N.FW_ERR_VALUE  # supported; no tensors
    assert lib.fw_attn_bwd_workspace_bytes(bw) >= 2 * 4 * 8 * 4
    bw.head_dim_v = 0
    bw.head_dim, bw.nheads = 128, 3
    assert lib.fw_attn_bwd(bw, None) == N.FW_ERR_VALUE  # heads not a multiple of nheads_k
    bw.nheads = 4
    assert lib.fw_attn_bwd(bw, None) == N.FW_ERR_VALUE  # no tensors, no workspace
    assert lib.fw_attn_bwd_workspace_bytes(bw) >= 2 * 4 * 8 * 4  # row statistics
    bw.nheads, bw.nheads_k, bw.seqlen_k = 16, 2, 520  # few key tiles: heads split, partials
    assert lib.fw_attn_bwd_workspace_bytes(bw) > 2 * 2 * 520 * 128 * 4
    r = N.RotaryParams()
    r.head_dim, r.table_rows = 160, 8
    assert lib.fw_rotary(r, None) == N.FW_ERR_NOT_IMPLEMENTED  # head dims 64 .. 512
    for d in (64, 96, 128, 192, 256, 384, 512):
        r.head_dim = d
        assert lib.fw_rotary(r, None) == N.FW_ERR_VALUE  # no buffers


def test_backward_workspace_planes(monkeypatch):
    """The stored backward's planes in fw_attn_bwd_workspace_bytes: bf16 P
    (and dS at 256/256) of B x H x roundup(Sq, 128) x roundup(Sk, 256), kept
    while the planes fit in 8 GiB and one head's share in 4 GiB (the dq
    kernel's 32-bit store offsets); otherwise, at other head-dim pairs and
    with FW_BWD_STORED=0 the recomputing kernels run and the workspace holds
    no plane."""
    lib = N.lib()
    GiB = 1 << 30

    def ws(d, dv, h, s, batch=1):
        bw = N.AttnBwdParams()
        bw.head_dim, bw.head_dim_v, bw.nheads, bw.nheads_k = d, dv, h, h
        bw.batch, bw.seqlen_q, bw.seqlen_k = batch, s, s
        return lib.fw_attn_bwd_workspace_bytes(bw)

    def plane(h, s, batch=1):
        return batch * h * (-(-s // 128) * 128) * (-(-s // 256) * 256) * 2

    assert ws(128, 128, 1, 32768) >= plane(1, 32768)          # one 2 GiB plane
    assert ws(256, 256, 1, 32768) >= 2 * plane(1, 32768)      # P and dS
    assert ws(256, 256, 2, 32768) >= 2 * plane(2, 32768)      # 8 GiB in all: kept
    assert ws(256, 256, 3, 32768) < GiB                       # 12 GiB: recompute
    assert ws(128, 128, 5, 32768) < GiB                       # 10 GiB: recompute
    assert plane(1, 46341) >= 4 * GiB and ws(128, 128, 1, 46341) < GiB  # one head >= 4 GiB
    assert ws(256, 128, 1, 32768) < GiB                       # wide pair: no plane
    monkeypatch.setenv("FW_BWD_STORED", "0")
    assert ws(128, 128, 1, 32768) < GiB
    assert ws(256, 256, 1, 32768) < GiB


def bf(*shape):
    return torch.zeros(shape, dtype=torch.bfloat16)


def test_flash_attn_func_errors():
    q, k = bf(1, 4, 8, 128), bf(1, 2, 8, 128)
    with pytest.raises(NotImplementedError):
        flash_attn_func(q, k, k, dropout_p=0.1)
    with pytest.raises(NotImplementedError):
        flash_attn_func(q, k, k, alibi_slopes=torch.zeros(4))
    with pytest.raises(NotImplementedError):
        flash_attn_func(q, k, k, deterministic=True)
    with pytest.raises(NotImplementedError):
        flash_attn_func(q, k, k, return_attn_probs=True)
    with pytest.raises(NotImplementedError):
        flash_attn_func(q, k, k, attention_chunk=64)
    with pytest.raises(ValueError):
        flash_attn_func(q, k, k, window_size=(-2, 0))
    with pytest.raises(ValueError):
        flash_attn_func(q, k, k, softcap=-1.0)
    with pytest.raises(ValueError):
        flash_attn_func(q, bf(1, 3, 8, 128), bf(1, 3, 8, 128))
    with pytest.raises(NotImplementedError):
        flash_attn_func(q.float(), k.float(), k.float())
    with pytest.raises(ValueError):
        flash_attn_func(bf(1, 8, 512), bf(1, 8, 256), bf(1, 8, 256), token_major=True)
    # inputs.py:106-147: token-major head dims, the paired d64 form
    with pytest.raises(ValueError, match="head_dim % 128"):
        flash_attn_func(bf(1, 8, 384), bf(1, 8, 384), bf(1, 8, 384), token_major=True, head_dim=96)
    with pytest.raises(NotImplementedError, match="MHA"):
        flash_attn_func(bf(1, 8, 256), bf(1, 8, 128), bf(1, 8, 128), token_major=True, head_dim=64)
    with pytest.raises(NotImplementedError, match="head_dim_v == head_dim"):
        flash_attn_func(bf(1, 8, 256), bf(1, 8, 256), bf(1, 8, 512), token_major=True, head_dim=64)
    with pytest.raises(ValueError, match="even head count"):
        flash_attn_func(bf(1, 8, 192), bf(1, 8, 192), bf(1, 8, 192), token_major=True, head_dim=64)
    # inputs.py:193-207: v differs from k in head_dim only
    with pytest.raises(ValueError, match="every axis but head_dim"):
        flash_attn_func(q, k, bf(1, 2, 9, 128))
    with pytest.raises(TypeError):
        flash_attn_func(q, k, k, heads_outer_fold=1)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_func(q, k, k, causal=True)


def test_rotary_argument_errors():
    """rotary.py:56-97, 113-114; prefill.py:480-485 (paged K arrives rotated)."""
    q, k = bf(1, 4, 8, 128), bf(1, 2, 16, 128)
    tab = torch.zeros(16, 64)
    with pytest.raises(ValueError, match="together"):
        flash_attn_func(q, k, k, rotary_cos=tab)
    with pytest.raises(ValueError, match="rotary_k=False needs"):
        flash_attn_func(q, k, k, rotary_k=False)
    with pytest.raises(ValueError, match="static bool"):
        flash_attn_func(q, k, k, rotary_cos=tab, rotary_sin=tab, rotary_interleaved=1)
    with pytest.raises(ValueError, match="partial rotary"):
        flash_attn_func(q, k, k, rotary_cos=tab[:, :32], rotary_sin=tab[:, :32])
    with pytest.raises(ValueError, match="divisible by 16"):
        flash_attn_func(q, k, k, rotary_cos=tab[:, :4], rotary_sin=tab[:, :4])
    with pytest.raises(ValueError, match="dtype"):
        flash_attn_func(q, k, k, rotary_cos=tab.double(), rotary_sin=tab.double())
    with pytest.raises(ValueError, match="shorter"):
        flash_attn_func(q, k, k, rotary_cos=tab[:15], rotary_sin=tab[:15])
    with pytest.raises(ValueError, match="seqlen_q <= seqlen_k"):
        flash_attn_func(bf(1, 4, 20, 128), k, k, rotary_cos=tab, rotary_sin=tab)
    with pytest.raises(NotImplementedError, match="heads_outer_fold"):
        flash_attn_func(bf(4, 1, 8, 128), bf(2, 1, 16, 128), bf(2, 1, 16, 128),
                        heads_outer_fold=True, rotary_cos=tab, rotary_sin=tab)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_func(q, k, k, rotary_cos=tab, rotary_sin=tab.to(torch.float32))
    qp, kp = bf(4, 10, 128), bf(2, 10, 128)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    with pytest.raises(ValueError, match="len_q <= len_k"):  # second sequence: 6 q rows, 2 keys
        flash_attn_varlen_func(qp, kp, kp, cu, torch.tensor([0, 8, 10], dtype=torch.int32), 6, 8,
                               rotary_cos=tab, rotary_sin=tab)
    with pytest.raises(ValueError, match="shorter"):
        flash_attn_varlen_func(qp, kp, kp, cu, cu, 6, 17, rotary_cos=tab, rotary_sin=tab)
    pool, table = bf(8, 16, 4, 128), torch.zeros(2, 4, dtype=torch.int32)
    with pytest.raises(NotImplementedError, match="rotary_k=False"):
        flash_attn_varlen_func(qp, pool, None, cu, None, 6, 16, block_table=table,
                               seqused_k=torch.tensor([4, 6]), rotary_cos=tab, rotary_sin=tab)
    with pytest.raises(ValueError, match="len_q <= len_k"):
        flash_attn_varlen_func(qp, pool, None, cu, None, 6, 16, block_table=table,
                               seqused_k=torch.tensor([4, 5]), rotary_cos=tab, rotary_sin=tab,
                               rotary_k=False)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_varlen_func(qp, pool, None, cu, None, 6, 16, block_table=table,
                               seqused_k=torch.tensor([4, 6]), rotary_cos=tab, rotary_sin=tab,
                               rotary_k=False, num_active=1)


def test_flash_attn_varlen_func_errors():
    q, k = bf(4, 10, 128), bf(2, 10, 128)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q, k, k, cu, cu[:2], 6, 6)
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q, k, k, cu, cu, 0, 6)
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q, k, k, cu, cu, 6, 6, seqused_k=torch.tensor([4, 6]))
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q, k, k, cu, cu, 6, 6, block_sizes=(100, 128, 1, 1))
    pool = bf(8, 16, 4, 128)
    table = torch.zeros(2, 4, dtype=torch.int32)
    with pytest.raises(ValueError):  # v must be None with a block table
        flash_attn_varlen_func(q, pool, pool, cu, None, 6, 64, block_table=table,
                               seqused_k=torch.tensor([4, 6]))
    with pytest.raises(ValueError):  # seqused_k required
        flash_attn_varlen_func(q, pool, None, cu, None, 6, 64, block_table=table)
    with pytest.raises(NotImplementedError):  # window right bound must be -1 or 0
        flash_attn_varlen_func(q, pool, None, cu, None, 6, 64, block_table=table,
                               seqused_k=torch.tensor([4, 6]), window_size=(-1, 3))
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q, pool, None, cu, None, 6, 64, block_table=table,
                               seqused_k=torch.tensor([4, 6]), num_active=3)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_varlen_func(q, pool, None, cu, None, 6, 64, block_table=table,
                               seqused_k=torch.tensor([4, 6]))


def test_flash_attn_with_kvcache_errors():
    pool = bf(8, 16, 4, 128)
    table = torch.zeros(2, 4, dtype=torch.int32)
    q = bf(2, 1, 4, 128)
    kw = dict(cache_seqlens=torch.tensor([3, 5], dtype=torch.int32), block_table=table)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, pool, pool, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, pool, None, cache_batch_idx=torch.tensor([0, 1]), **kw)
    with pytest.raises(ValueError):  # page size not a multiple of 16
        flash_attn_with_kvcache(q, bf(8, 24, 4, 128), None, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, pool, None, max_seqlen_q=1, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(bf(5, 4, 128), pool, None, cu_seqlens_q=torch.tensor([0, 2, 5]),
                                **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, pool, None, bf(2, 1, 2, 128), None, **kw)
    with pytest.raises(NotImplementedError):
        flash_attn_with_kvcache(q.float(), pool, None, **kw)
    with pytest.raises(NotImplementedError):  # multi-token call needs the paged cache
        flash_attn_with_kvcache(bf(2, 3, 4, 128), bf(2, 64, 2, 128), bf(2, 64, 2, 128),
                                cache_seqlens=3)
    with pytest.raises(ValueError):  # an fp8 pool needs nheads_k
        flash_attn_with_kvcache(q, pool.to(torch.float8_e4m3fn), None, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, pool, None, cache_seqlens=torch.tensor([1, 2, 3]),
                                block_table=table)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_with_kvcache(q, pool, None, **kw)


def test_contiguous_cache_errors():
    """decode.py:383-403 conditions for the contiguous K/V pair."""
    kc = bf(3, 256, 2, 128)
    q = bf(2, 1, 4, 128)
    kw = dict(cache_seqlens=torch.tensor([3, 5], dtype=torch.int32))
    with pytest.raises(ValueError):  # a merged cache must be paged
        flash_attn_with_kvcache(q, kc, None, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, kc, bf(3, 128, 2, 128), **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, kc, kc, nheads_k=1, **kw)
    with pytest.raises(ValueError):  # capacity a multiple of 128
        flash_attn_with_kvcache(q, bf(3, 200, 2, 128), bf(3, 200, 2, 128), **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, kc, kc, cache_batch_idx=torch.tensor([0, 1, 2]), **kw)
    with pytest.raises(NotImplementedError):  # fp8 only in a paged pool
        f8 = kc.to(torch.float8_e4m3fn)
        flash_attn_with_kvcache(q, f8, f8, **kw)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, kc, kc, bf(2, 1, 2, 128), None, **kw)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attn_with_kvcache(q, kc, kc, bf(2, 1, 2, 128), bf(2, 1, 2, 128),
                                cache_batch_idx=torch.tensor([2, 0]), **kw)


def test_write_kv_cache_pages_errors():
    cache = bf(6, 128, 4, 128)
    k = bf(10, 2, 128)
    slices = torch.zeros(3, 4, dtype=torch.int32)
    with pytest.raises(ValueError):
        write_kv_cache_pages(bf(10, 3, 128), bf(10, 3, 128), cache, slices, torch.tensor([1]))
    with pytest.raises(NotImplementedError):
        write_kv_cache_pages(k.float(), k.float(), cache, slices, torch.tensor([1]))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        write_kv_cache_pages(k, k, cache, slices, torch.tensor([1]))


def test_package_surface():
    assert set(flywheel_tpu.__all__) >= {"flash_attn_func", "flash_attn_varlen_func",
                                         "flash_attn_with_kvcache"}


def test_internal_exports_warn():
    """flywheel_tpu/__init__.py:35-60: the names tpu-inference reads, each
    access a FutureWarning; anything else an AttributeError."""
    with pytest.warns(FutureWarning):
        assert flywheel_tpu.PAGE_SIZE_MULTIPLE == 16
    with pytest.warns(FutureWarning):
        assert flywheel_tpu.FWD_BLOCKS[-1] % 128 == 0
    with pytest.warns(FutureWarning):
        assert flywheel_tpu.NUM_LANES == 128
    with pytest.warns(FutureWarning):
        mch = flywheel_tpu.merged_cache_heads
    assert mch(8, torch.bfloat16) == 16 and mch(3, torch.float8_e4m3fn) == 8
    with pytest.raises(AttributeError):
        flywheel_tpu.not_an_export


def test_runtime_causal_offset_errors():
    """_flash_attn_func_pcp_causal_offset's checks (reference prefill.py:362-400),
    raised before anything touches a device."""
    from flywheel_tpu.prefill import _flash_attn_func_pcp_causal_offset as f
    q, k = bf(1, 4, 64, 128), bf(1, 2, 128, 128)
    with pytest.raises(ValueError, match="4-D"):
        f(bf(4, 64, 128), k, k, 0)
    with pytest.raises(ValueError, match="batch_size == 1"):
        f(bf(2, 4, 64, 128), bf(2, 2, 128, 128), bf(2, 2, 128, 128), 0)
    with pytest.raises(ValueError, match="kv_len >= q_len"):
        f(bf(1, 4, 256, 128), k, k, 0)
    with pytest.raises(ValueError, match="divisible"):
        f(bf(1, 3, 64, 128), k, k, 0)
    with pytest.raises(ValueError, match="one integer scalar"):
        f(q, k, k, torch.tensor([1.5]))
    with pytest.raises(NotImplementedError, match="bf16"):
        f(q.float(), k.float(), k.float(), 0)
