"""Closed-form (integer / numpy) restatement of the two FP8 casts and of the
power-of-two scale rule.  TEST INFRASTRUCTURE ONLY.

These functions do not call torch's float8 casts or ``torch.log2``; they are
the independent second opinion that pins the torch-CPU oracle in
``oracle/fp8_mlp.py`` (which follows the reference literally, e.g.
``(w * q).clamp(-448, 448).to(torch.float8_e4m3fn)`` at spark-gpt
``train.py:952``).

* ``cast_e4m3`` / ``cast_e5m2``: OCP FP8 round-to-nearest-even by searching the
  table of every finite code; a tie goes to the code with an even mantissa.
  NaN maps to 0x7F with the input's sign bit, as ``torch.float8_e4m3fn`` /
  ``float8_e5m2`` do.  Inputs must already be clamped to the format's finite
  range (the reference always clamps first: ``train.py:952, 968, 1013-1014,
  1091-1092, 1172``).
* ``floor_log2_cr``: floor(log2(r)) where log2 is the *correctly rounded* fp32
  logarithm, decided with exact rational/Decimal arithmetic.  The reference
  rule ``exp2(floor(log2(fmax / amax)))`` (``train.py:944, 951``) is evaluated
  in fp32, so when r lies a few ulps below a power of two the rounded log2 can
  be the integer above and the floor then lands one binade higher than the
  exact floor.  ``band_table`` lists, per integer K, how many fp32 ulps below
  2^K that still happens.
"""
from __future__ import annotations

from decimal import Decimal, getcontext
from functools import lru_cache

import numpy as np

getcontext().prec = 60

# (exponent bias, mantissa bits, max finite value, NaN code) per format
_FORMATS = {
    "e4m3": (7, 3, 448.0),
    "e5m2": (15, 2, 57344.0),
}


def _code_values(fmt: str) -> tuple[np.ndarray, np.ndarray]:
    """All non-negative finite codes of ``fmt`` and their exact values (sorted)."""
    bias, mbits, fmax = _FORMATS[fmt]
    codes, vals = [], []
    for c in range(128):
        e = c >> mbits
        m = c & ((1 << mbits) - 1)
        if e == 0:
            v = m * 2.0 ** (1 - bias - mbits)
        else:
            v = (1 + m / (1 << mbits)) * 2.0 ** (e - bias)
        if v > fmax:  # e4m3fn: 0x7F is NaN; e5m2: 0x7C.. are inf/NaN
            continue
        codes.append(c)
        vals.append(v)
    return np.array(codes, dtype=np.uint8), np.array(vals, dtype=np.float64)


def _cast(x: np.ndarray, fmt: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    codes, vals = _code_values(fmt)
    a = np.abs(x.astype(np.float64))
    nan = np.isnan(a)
    a = np.where(nan, 0.0, a)
    if np.any(a > vals[-1]):
        raise ValueError("closed-form cast expects clamped input")
    hi = np.searchsorted(vals, a, side="left")  # vals[hi] >= a
    hi = np.minimum(hi, len(vals) - 1)
    lo = np.maximum(hi - 1, 0)
    exact = vals[hi] == a
    d_lo = a - vals[lo]
    d_hi = vals[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((codes[hi] & 1) == 0))
    idx = np.where(exact | pick_hi, hi, lo)
    out = codes[idx].astype(np.uint8)
    sign = (x.view(np.uint32) >> 31).astype(np.uint8)
    out = np.where(nan, np.uint8(0x7F), out)
    return (out | (sign << 7)).astype(np.uint8)


def cast_e4m3(x: np.ndarray) -> np.ndarray:
    """Bytes of OCP e4m3fn(x), RNE, for |x| <= 448 (or NaN)."""
    return _cast(x, "e4m3")


def cast_e5m2(x: np.ndarray) -> np.ndarray:
    """Bytes of OCP e5m2(x), RNE, for |x| <= 57344 (or NaN)."""
    return _cast(x, "e5m2")


def decode(bytes_: np.ndarray, fmt: str) -> np.ndarray:
    """fp32 value of each FP8 byte (finite codes only; NaN codes decode to NaN)."""
    bias, mbits, fmax = _FORMATS[fmt]
    b = np.asarray(bytes_, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    c = b & 0x7F
    e = c >> mbits
    m = c & ((1 << mbits) - 1)
    v = np.where(e == 0, m * 2.0 ** (1 - bias - mbits),
                 (1 + m / (1 << mbits)) * 2.0 ** (e - bias))
    v = np.where(v > fmax, np.nan, v)
    return (s * v).astype(np.float32)


# ---------------------------------------------------------------- scale rule
_LN2 = Decimal(2).ln()


def _half_spacing_toward(K: int) -> Decimal:
    """Half the fp32 spacing on the side of the integer K that log2(r) approaches
    from below (r < 2^K means log2(r) < K)."""
    if K == 0:
        return Decimal(0)  # values just below 0 are representable to ~1e-45
    aK = abs(K)
    e = aK.bit_length() - 1  # 2^e <= |K| < 2^(e+1)
    if K > 0:
        # next fp32 below K: spacing 2^(e-23), halved if K is a power of two
        spacing = Decimal(2) ** (e - 23)
        if aK == 1 << e:
            spacing /= 2
    else:
        # log2(r) = K - delta has |.| = |K| + delta: spacing above |K|
        spacing = Decimal(2) ** (e - 23)
    return spacing / 2


def band_nmax(K: int) -> int:
    """Largest n >= 0 such that the correctly rounded fp32 log2 of
    r = 2^K * (1 - n * 2^-24) (n fp32 ulps below 2^K) still rounds to K."""
    hs = _half_spacing_toward(K)
    n = 0
    while True:
        r = Decimal(1) - Decimal(n + 1) / Decimal(2 ** 24)
        delta = -(r.ln() / _LN2)
        if delta < hs:
            n += 1
        else:
            return n


@lru_cache(maxsize=None)
def _band_table(kmin: int, kmax: int) -> tuple:
    return tuple((K, band_nmax(K)) for K in range(kmin, kmax + 1))


def band_table(kmin: int = -125, kmax: int = 128) -> dict[int, int]:
    return dict(_band_table(kmin, kmax))


def floor_log2_cr(r: np.ndarray) -> np.ndarray:
    """floor(fl32(log2(r))) for positive normal fp32 r, with log2 correctly
    rounded to fp32, using the exact band table (no transcendental calls)."""
    r = np.asarray(r, dtype=np.float32)
    bits = r.view(np.uint32).astype(np.int64)
    if np.any((bits >> 23) == 0) or np.any(bits >> 31):
        raise ValueError("positive normal input expected")
    e = (bits >> 23) - 127
    m = bits & ((1 << 23) - 1)
    n = (1 << 23) - m
    lut = np.array([n for _, n in _band_table(-125, 128)], dtype=np.int64)
    K = e + 1
    if np.any((K < -125) | (K > 128)):
        raise ValueError("exponent outside the band table")
    nmax = lut[K + 125]
    return e + ((m != 0) & (n <= nmax)).astype(np.int64)


def pow2_scale(amax: np.ndarray, fmax: float, headroom: int, recip_first: bool = False) -> np.ndarray:
    """exp2(floor(log2(r)) - headroom) in fp32, exactly, for amax >= 0 (inf
    included).

    r = fmax / max(amax, 1e-30) for the scale roll (spark-gpt ``train.py:943``,
    a tensor/tensor divide, headroom 1); with ``recip_first`` r is
    (1 / max(amax, 1e-30)) * fmax, which is how torch evaluates the weight rule
    ``448.0 / tensor`` (``train.py:951``, headroom 0).  Each step is one
    IEEE-rounded fp32 operation.  An infinite amax gives r = 0, log2 = -inf and
    a scale of 0, as the reference's expression does."""
    a = np.maximum(np.asarray(amax, dtype=np.float32), np.float32(1e-30))
    with np.errstate(over="ignore", divide="ignore"):
        if recip_first:
            r = ((np.float32(1.0) / a).astype(np.float32) * np.float32(fmax)).astype(np.float32)
        else:
            r = (np.float32(fmax) / a).astype(np.float32)
    zero = r == 0
    k = floor_log2_cr(np.where(zero, np.float32(1.0), r)) - headroom
    out = np.ldexp(np.float32(1.0), k.astype(np.int32)).astype(np.float32)
    return np.where(zero, np.float32(0.0), out).astype(np.float32)
