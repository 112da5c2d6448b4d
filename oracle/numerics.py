"""bf16 and fp8-e4m3fn codecs on numpy arrays - test infrastructure (see oracle/__init__.py).

bf16 values travel as uint16 bit patterns, fp8 values as uint8 codes, so the oracle never relies on
a library's float type for these formats.

bf16: the upper 16 bits of an IEEE binary32. Encoding rounds to nearest, ties to even; NaN maps to
the canonical quiet NaN 0x7fc0 (the pattern torch produces).

fp8 e4m3fn (OCP FP8 E4M3, torch.float8_e4m3fn; the reference's FP8 at devstral2.py:33-34):
sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities, NaN = S.1111.111, largest finite
448. The encoder here is a nearest-value search over the decoded code table (a different method
from the bit manipulation the kernels use), with ties to the even code.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = 448.0


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    is_nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    # Finite values and infinities: add half an ulp of the kept part (minus one when the kept
    # lsb is 0) and truncate. No finite input overflows uint32 here.
    safe = np.where(is_nan, np.uint32(0), u)
    rounded = (safe + np.uint32(0x7FFF) + ((safe >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return np.where(is_nan, np.uint32(0x7FC0), rounded).astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 value, returned as fp32."""
    return bf16_to_f32(f32_to_bf16(x))


def _fp8_decode_table() -> np.ndarray:
    codes = np.arange(256, dtype=np.int64)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 0x7
    mag = np.where(exp == 0, man * 2.0 ** -9, (1.0 + man / 8.0) * 2.0 ** (exp - 7.0))
    values = sign * mag
    values[(exp == 15) & (man == 7)] = np.nan
    return values.astype(np.float32)


FP8_VALUES = _fp8_decode_table()            # code -> value (float32, NaN for 0x7f / 0xff)
_POS_VALUES = FP8_VALUES[:0x7F].astype(np.float64)   # codes 0x00..0x7e, ascending magnitudes


def fp8_to_f32(codes: np.ndarray) -> np.ndarray:
    return FP8_VALUES[np.asarray(codes, dtype=np.uint8)]


def f32_to_fp8_saturate(x: np.ndarray) -> np.ndarray:
    """clamp(x, -448, 448) then round to the nearest e4m3fn value, ties to the even code.

    NaN maps to 0x7f with the input's sign bit (0xff for negative NaN), as torch's clamp-then-cast
    does (devstral2.py:95).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    sign = ((x.view(np.uint32) >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    is_nan = np.isnan(x)
    mag = np.minimum(np.abs(np.where(is_nan, 0.0, x)).astype(np.float64), FP8_MAX)
    hi = np.searchsorted(_POS_VALUES, mag, side="left")            # first value >= mag
    hi = np.minimum(hi, len(_POS_VALUES) - 1)
    lo = np.maximum(hi - 1, 0)
    d_lo = mag - _POS_VALUES[lo]
    d_hi = _POS_VALUES[hi] - mag
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    exact = _POS_VALUES[hi] == mag
    code = np.where(exact | take_hi, hi, lo).astype(np.uint8)
    code = np.where(is_nan, np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)
