"""OCP float8 e4m3fn codec restated from the format definition (numpy, CPU only).

Test infrastructure only (see ``oracle/__init__.py``).

Format (OCP 8-bit FP spec, E4M3): 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits,
no infinities, NaN = S.1111.111 (0x7f / 0xff), max finite 448 = 1.75 * 2^8, min normal
2^-6, subnormals m * 2^-9.  Rounding for encode: round-to-nearest, ties to the code with
an even mantissa LSB.  Out-of-range handling follows torch's ``to(float8_e4m3fn)`` (values
that round above 448 become NaN; 448 < |v| <= 464 round to 448) -- the reference always
clamps to [-448, 448] before the cast (``tilert/models/deepseek_v3_2/refs/kernel.py:193``),
so only the in-range branch is on the hot path.

This is deliberately NOT the bit-manipulation method the HIP kernels use: it decodes all
256 codes, sorts the finite magnitudes and picks the nearest neighbour, so the two
implementations can pin each other.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def decode_table() -> np.ndarray:
    """float64 value of every code 0..255 (NaN for 0x7f/0xff)."""
    out = np.empty(256, dtype=np.float64)
    for c in range(256):
        sign = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = sign * m * 2.0**-9
        else:
            out[c] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_DEC = decode_table()
# finite non-negative codes 0x00..0x7e in increasing magnitude order
_POS_CODES = np.arange(0x7F, dtype=np.int64)
_POS_VALS = _DEC[:0x7F]
assert np.all(np.diff(_POS_VALS) > 0)


def decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values."""
    return _DEC[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def encode(v: np.ndarray) -> np.ndarray:
    """float32 -> uint8 e4m3fn codes, RNE, torch-compatible overflow (NaN past 464)."""
    v = np.asarray(v, dtype=np.float32).astype(np.float64)
    sign = np.signbit(v)
    a = np.abs(v)
    nan = np.isnan(a)
    a_ = np.where(nan, 0.0, a)
    # neighbours: lo = largest representable <= a, hi = next one up
    idx_hi = np.searchsorted(_POS_VALS, a_, side="left")  # first >= a
    idx_hi = np.minimum(idx_hi, 0x7E)
    exact = _POS_VALS[idx_hi] == a_
    idx_lo = np.where(exact, idx_hi, np.maximum(idx_hi - 1, 0))
    lo = _POS_VALS[idx_lo]
    hi = _POS_VALS[idx_hi]
    d_lo = a_ - lo
    d_hi = hi - a_
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (idx_hi % 2 == 0) & ~exact)
    code = np.where(pick_hi, idx_hi, idx_lo)
    # above the largest finite value: the next code up would be 480 (not representable);
    # the midpoint 464 ties to even (448, mantissa 110), anything beyond is NaN
    over = a_ > E4M3_MAX
    code = np.where(over & (a_ <= 464.0), 0x7E, code)
    code = np.where((over & (a_ > 464.0)) | nan, 0x7F, code)
    code = code | np.where(sign, 0x80, 0)
    return code.astype(np.uint8)
