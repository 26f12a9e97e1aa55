"""Bit-level bf16 / fp8 conversions in NumPy (oracle only).

bf16 values are held as uint16 codes, fp8 values as uint8 codes.  The
reference's dtypes are jnp.bfloat16 and OCP float8_e4m3fn / float8_e5m2
(`flywheel_tpu/softmax_attention/kv_layout.py:30-34`); the conversions here are
restated from the formats' published definitions (round to nearest even).
"""

import numpy as np

FP8_FORMATS = {
    # name: (exponent bits, mantissa bits, bias, has_inf)
    "e4m3": (4, 3, 7, False),
    "e5m2": (5, 2, 15, True),
}


def bf16_round(x):
    """float32 -> bf16 code (uint16), round to nearest even; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounding = 0x7FFF + ((bits >> 16) & 1)
    out = ((bits + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    out[nan] = 0x7FC0
    return out


def bf16_to_f32(code):
    code = np.asarray(code, dtype=np.uint16)
    return (code.astype(np.uint32) << 16).view(np.float32)


def bf16(x):
    """x rounded through bf16, returned as float32."""
    return bf16_to_f32(bf16_round(x))


def _fp8_table(fmt):
    ebits, mbits, bias, has_inf = FP8_FORMATS[fmt]
    codes = np.arange(256, dtype=np.uint32)
    sign = np.where(codes >> 7, -1.0, 1.0)
    exp = (codes >> mbits) & ((1 << ebits) - 1)
    man = codes & ((1 << mbits) - 1)
    sub = man / (1 << mbits) * 2.0 ** (1 - bias)
    nor = (1 + man / (1 << mbits)) * 2.0 ** (exp.astype(np.float64) - bias)
    val = sign * np.where(exp == 0, sub, nor)
    emax = (1 << ebits) - 1
    if has_inf:  # IEEE-like: top exponent is inf / NaN
        val = np.where((exp == emax) & (man == 0), sign * np.inf, val)
        val = np.where((exp == emax) & (man != 0), np.nan, val)
    else:  # e4m3fn: only S.1111.111 is NaN, no inf
        val = np.where((exp == emax) & (man == (1 << mbits) - 1), np.nan, val)
    return val.astype(np.float32)


FP8_TABLES = {fmt: _fp8_table(fmt) for fmt in FP8_FORMATS}


def fp8_decode(code, fmt):
    return FP8_TABLES[fmt][np.asarray(code, dtype=np.uint8)]


def fp8_encode(x, fmt):
    """float32 -> fp8 code, round to nearest even over the finite codes.

    Values beyond the largest finite magnitude map to NaN for e4m3 and inf for
    e5m2 (torch's non-saturating cast); the hot path's inputs never reach it.
    """
    x = np.asarray(x, dtype=np.float32)
    table = FP8_TABLES[fmt].astype(np.float64)
    pos_codes = np.arange(128)
    finite = np.isfinite(table[:128])
    vals = table[:128][finite]
    codes = pos_codes[finite]
    order = np.argsort(vals)
    vals, codes = vals[order], codes[order]
    mag = np.abs(x.astype(np.float64))
    idx = np.clip(np.searchsorted(vals, mag), 1, len(vals) - 1)
    lo, hi = vals[idx - 1], vals[idx]
    pick_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & (codes[idx] % 2 == 0))
    out = np.where(pick_hi, codes[idx], codes[idx - 1]).astype(np.uint8)
    top = vals[-1]
    half_ulp = (vals[-1] - vals[-2]) / 2
    over = mag >= top + half_ulp
    if fmt == "e4m3":
        out = np.where(over, 0x7F, out)
    else:
        out = np.where(over, 0x7C, out)
    out = np.where(np.isnan(x), 0x7F, out).astype(np.uint8)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    return (out | sign).astype(np.uint8)
