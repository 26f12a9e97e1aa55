"""Writes the golden fixtures of this directory from the NumPy oracle.

    python tests/golden/make_golden.py          # (re)write every fixture
    python tests/golden/make_golden.py --check  # compare against the files

Each fixture holds seeded inputs (raw bf16 / fp8 codes) and the oracle's
expected outputs: cache codes (compared bit-exactly) and attention out / lse
(compared within the tolerance contract).  tests/test_golden.py pins the
oracle to these files on the CPU; tests/test_gpu_golden.py runs the HIP path
on the same inputs and compares with the stored outputs.
"""

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attention as A  # noqa: E402
from oracle import dtypes as T  # noqa: E402
from oracle import paged as P  # noqa: E402


def _bf16_codes(rng, shape, scale=1.0):
    return T.bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def _pool(rng, lengths, new, page, hk, d, fmt=None, descale=1.0, extra=2):
    need = [-(-(int(l) + int(n)) // page) for l, n in zip(lengths, new)]
    npages = sum(max(x, 1) for x in need) + extra
    perm = rng.permutation(npages)
    table = np.zeros((len(lengths), max(max(need), 1)), np.int32)
    pos = 0
    for r, c in enumerate(need):
        c = max(c, 1)
        table[r, :c] = perm[pos:pos + c]
        pos += c
    ch = P.merged_cache_heads(hk, 1 if fmt else 2)

    def codes(shape):
        x = rng.standard_normal(shape, dtype=np.float32) / np.float32(descale)
        return T.fp8_encode(x, fmt) if fmt else T.bf16_round(x)

    pool = codes((npages, page, ch, d))
    if ch > 2 * hk:
        pool[:, :, 2 * hk:] = 0
    tot = int(np.sum(new))
    return pool, table, codes((tot, hk, d)), codes((tot, hk, d))


def _values(codes, fmt):
    return T.fp8_decode(codes, fmt) if fmt else T.bf16_to_f32(codes)


def prefill_case(seed, b, h, hk, s, causal, window, softcap):
    rng = np.random.default_rng(seed)
    q, k, v = (_bf16_codes(rng, (b, s, x, 128)) for x in (h, hk, hk))
    ro, rl = A.attention_ref(T.bf16_to_f32(q), T.bf16_to_f32(k), T.bf16_to_f32(v), causal=causal,
                             window_size=window, softcap=softcap, round_scaled_q=True)
    return dict(q=q, k=k, v=v, out=ro.astype(np.float32), lse=rl.astype(np.float32),
                causal=np.int32(causal), window=np.asarray(window, np.int32),
                softcap=np.float32(softcap))


def decode_case(seed, lengths, sq, h, hk, fmt=None, k_descale=1.0, v_descale=1.0, causal=False):
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, np.int64)
    b, page, d = len(lengths), 16, 128
    new = np.full(b, sq, np.int64)
    pool, table, kn, vn = _pool(rng, lengths, new, page, hk, d, fmt, k_descale)
    q = _bf16_codes(rng, (b, sq, h, d))
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    exp_pool = P.append_to_pages(pool, kn, vn, cu, lengths, table)
    kc, vc = P.split_kv_heads(exp_pool, hk)
    krows = P.gather_rows(_values(kc, fmt), table)
    vrows = P.gather_rows(_values(vc, fmt), table)
    ro, rl = A.kvcache_reference(T.bf16_to_f32(q), krows, vrows, lengths + new, causal=causal,
                                 k_descale=k_descale, v_descale=v_descale)
    return dict(pool=pool, table=table, lengths=lengths.astype(np.int32), q=q, k_new=kn, v_new=vn,
                k_descale=np.float32(k_descale), v_descale=np.float32(v_descale),
                causal=np.int32(causal), fmt=np.asarray(fmt or "bf16"),
                exp_pool=exp_pool, out=ro.astype(np.float32), lse=rl.astype(np.float32))


def write_pages_case(seed, hk):
    rng = np.random.default_rng(seed)
    num_pages, page, d = 4, 32, 128
    ch = P.merged_cache_heads(hk, 2)
    cache = _bf16_codes(rng, (num_pages, page, ch, d))
    k, v = _bf16_codes(rng, (60, hk, d)), _bf16_codes(rng, (60, hk, d))
    pieces = [(2 * page + 20, 0, 9), (page, 9, 32), (3 * page + 5, 41, 19)]
    slices = np.zeros((3, 4), np.int32)
    for j, pc in enumerate(pieces):
        slices[:, j] = pc
    exp = P.write_kv_cache_pages(k, v, cache, slices, len(pieces))
    return dict(k=k, v=v, cache=cache, slices=slices, num_slices=np.int32(len(pieces)), exp_cache=exp)


CASES = {
    "prefill_causal_gqa": lambda: prefill_case(101, 1, 4, 2, 96, True, (-1, -1), 0.0),
    "prefill_window_softcap": lambda: prefill_case(102, 1, 2, 1, 100, True, (31, 0), 30.0),
    "decode_append_bf16": lambda: decode_case(103, [40, 0, 100], 1, 8, 2),
    "decode_fp8_verify": lambda: decode_case(104, [70, 33], 4, 8, 2, "e4m3", 0.75, 1.5, causal=True),
    "write_pages_bf16": lambda: write_pages_case(105, 3),
}


def path(name):
    return os.path.join(HERE, name + ".npz")


def load(name):
    with np.load(path(name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args()
    for name, make in CASES.items():
        data = make()
        if args.check:
            ref = load(name)
            for k, val in data.items():
                np.testing.assert_array_equal(np.asarray(val), ref[k], err_msg=f"{name}:{k}")
            print("ok", name)
        else:
            np.savez_compressed(path(name), **data)
            print("wrote", path(name), os.path.getsize(path(name)))


if __name__ == "__main__":
    main()
