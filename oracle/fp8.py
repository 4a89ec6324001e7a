"""OCP FP8 e4m3fn codec in numpy (oracle; test infrastructure only).

Restates the FP8 storage cast of fastserve kv/quant.py:44-45 (`x.clamp(±448).to(torch.float8_e4m3fn)`)
and the E4M3 round-to-nearest-even of quant/formats.py:39-52: sign bit, 4 exponent bits (bias 7), 3
mantissa bits, subnormals at multiples of 2^-9, no infinities, 0x7F / 0xFF NaN, largest finite 448.
A magnitude that rounds past 448 (|x| > 464) has no finite code and becomes NaN, as in the torch cast.
"""

from __future__ import annotations

import numpy as np

MAX = 448.0
NAN_CODE = 0x7F


def decode_table() -> np.ndarray:
    """float32 [256]: the value of every code (NaN for 0x7F and 0xFF)."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = sign * m * 2.0**-9
        else:
            out[code] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out.astype(np.float32)


_TABLE = decode_table()


def decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values."""
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray) -> np.ndarray:
    """float32 values -> uint8 codes, round to nearest even; NaN (and anything rounding past 448) -> NaN code."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = (np.signbit(x).astype(np.uint8)) << 7
    codes = np.zeros(x.shape, dtype=np.int64)

    sub = a < 2.0**-6  # subnormal range (and zero): multiples of 2^-9, code = the multiple (8 = 2^-6, normal)
    codes[sub] = np.rint(a[sub] / 2.0**-9).astype(np.int64)

    norm = ~sub & np.isfinite(a)
    mant, exp = np.frexp(a[norm])  # a = mant * 2^exp, mant in [0.5, 1)
    e = exp.astype(np.int64) - 1  # a in [2^e, 2^(e+1))
    r = np.rint(a[norm] / np.exp2(e - 3)).astype(np.int64)  # in [8, 16]; rint ties to even
    carry = r == 16
    e = np.where(carry, e + 1, e)
    r = np.where(carry, 8, r)
    field = e + 7
    c = (field << 3) | (r - 8)
    c = np.where((field > 15) | (c > 0x7E), NAN_CODE, c)
    codes[norm] = c

    codes[~np.isfinite(a)] = NAN_CODE
    return (codes.astype(np.uint8) | sign).astype(np.uint8)


def representable_values() -> np.ndarray:
    """Every finite value, sorted, zero once (quant/formats.py:55-68): 253 values."""
    vals = _TABLE[np.isfinite(_TABLE)].astype(np.float64)
    return np.unique(vals).astype(np.float32)
