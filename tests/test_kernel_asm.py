"""Checks on the gfx950 assembly of every kernel source (CPU; needs hipcc).

Each source is compiled for the device only (-S) with the library's own flags,
and the assembly is checked for properties the kernels rely on but no parity
test can see:
  * no packed-FP32 VALU forms (v_pk_add_f32 / v_pk_mul_f32 / v_pk_fma_f32):
    the build disables them and no kernel writes them by hand;
  * no scalar-memory writes of any kind (stores, atomics, cache write-back):
    every store in the library is a vector store;
  * paged prefill: the block-table entry that the ping-pong kernel fetches
    with an inline-asm `s_load_dword` one slot ahead is not read (or copied)
    before the next `s_waitcnt lgkmcnt(0)`.  The compiler does not know the
    load is in flight, so a copy it inserted before that wait would read a
    stale page id.
"""

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flywheel-tpu_amd")
sys.path.insert(0, PKG)
import build as B  # noqa: E402

pytestmark = pytest.mark.skipif(not shutil.which(B.HIPCC) and not os.path.exists(B.HIPCC),
                                reason="hipcc not available")


def _asm(src, out_dir):
    out = os.path.join(out_dir, os.path.splitext(src)[0] + ".s")
    flags = [f for f in B.FLAGS if f != "-fPIC"]
    cmd = [B.HIPCC, *flags, "--cuda-device-only", "-S", os.path.join(B.CSRC, src), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return src, open(out).read()


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("asm"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=5) as pool:
        return dict(pool.map(lambda s: _asm(s, d), B.SOURCES))


def _functions(text):
    """(name, body) of every kernel in an assembly file."""
    for m in re.finditer(r"^(_Z\w+):", text, re.M):
        end = text.find(".Lfunc_end", m.end())
        yield m.group(1), text[m.end():end]


def test_no_packed_fp32(asm):
    for src, text in asm.items():
        hits = re.findall(r"\bv_pk_(?:add|mul|fma)_f32\b", text)
        assert not hits, (src, hits[:3])


def test_no_scalar_memory_writes(asm):
    pat = re.compile(r"^\s+(s_(?:buffer_)?store\w*|s_(?:buffer_)?atomic\w*|s_scratch_store\w*|"
                     r"s_dcache_wb\w*|s_dcache_discard\w*)\b", re.M)
    for src, text in asm.items():
        hits = pat.findall(text)
        assert not hits, (src, hits[:3])


def test_paged_table_load_used_after_wait(asm):
    text = asm["fw_prefill.hip"]
    kernels = [(n, b) for n, b in _functions(text) if n.startswith("_ZN2fw20fw_prefill_pp_kernelILi2")]
    assert kernels, "no paged ping-pong kernel in the assembly"
    for name, body in kernels:
        lines = body.split("\n")
        loads = 0
        for k, line in enumerate(lines):
            m = re.match(r"\s+s_load_dword (s\d+), s\[\d+:\d+\], 0x0\s*$", line)
            if not m:
                continue
            loads += 1
            reg = re.compile(r"\b" + m.group(1) + r"\b")
            for later in lines[k + 1:]:
                if "s_waitcnt" in later and "lgkmcnt(0)" in later:
                    break
                assert not reg.search(later), (name, line.strip(), later.strip())
        assert loads > 0, name
