"""Independent fp32 -> e4m3fn encoder (test infrastructure only).

Built from the OCP 8-bit floating point specification (E4M3: bias 7, no
infinities, S.1111.111 is NaN, largest finite 448) as an explicit table of
the 256 code values and a nearest-value search with ties to the even code.
It shares no arithmetic with torch's cast or with the kernels' bit-twiddling
encoder, so agreement between the three pins all of them.
"""

from __future__ import annotations

import numpy as np


def code_values() -> np.ndarray:
    """float64 value of every code 0..255 (NaN for the two NaN codes)."""
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        sign = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = sign * m * 2.0 ** -9
        else:
            vals[c] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


_POS = code_values()[:0x7F]  # codes 0x00..0x7E: 0 .. 448, increasing


def encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even encode of float32 values.

    Magnitudes above 464 (the midpoint between 448 and the NaN slot at 480),
    infinities and NaN give the NaN code with the input's sign, as the OCP
    saturation-free conversion does."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x.astype(np.float64))
    sign = np.signbit(x).astype(np.uint8) << 7
    idx = np.searchsorted(_POS, a, side="left")        # _POS[idx-1] < a <= _POS[idx]
    idx = np.clip(idx, 1, len(_POS) - 1)
    lo, hi = _POS[idx - 1], _POS[idx]
    d_lo, d_hi = a - lo, hi - a
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (idx % 2 == 0))
    code = np.where(take_hi, idx, idx - 1).astype(np.uint8)
    code = np.where(a == 0.0, 0, code).astype(np.uint8)
    big = (a > 448.0)
    code = np.where(big & (a <= 464.0), 0x7E, code)     # 464 ties to 448 (even)
    code = np.where((a > 464.0) | np.isnan(a), 0x7F, code).astype(np.uint8)
    return code | sign
