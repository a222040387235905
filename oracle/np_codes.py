"""Independent numpy restatement of the byte formats the Sage path uses
(TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing shipped).

The torch oracle (``sage_oracle.py``) relies on torch's own casts for
fp32 -> bf16 and fp32 -> float8_e4m3fn.  This module re-derives both from the
format definitions, in float64 arithmetic that is exact for every fp32 input,
so the tests can check the torch casts (and therefore the oracle's codes)
against the definitions rather than against themselves:

* bf16: the top 16 bits of fp32 after round-to-nearest-even on the low 16.
* OCP FP8 E4M3FN (the format the reference casts to with ``tl.float8e4nv``,
  sage_kernels.py:153, :1093, :1139, :1147): 1 sign bit, 4 exponent bits with
  bias 7, 3 mantissa bits, no infinities, NaN = S.1111.111, largest finite
  448 = 2^8 * 1.75, smallest normal 2^-6, subnormals k * 2^-9.
* int8 quantization: ``trunc(x * (127 / max(amax, 1e-12)))`` with the product
  and quotient rounded to fp32 (sage_kernels.py:1420-1422, :1447-1449).
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest, ties to even), returned as fp32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return (r.astype(np.uint32) << 16).view(np.float32)


def e4m3_decode_table() -> np.ndarray:
    """Value of each of the 256 E4M3FN codes (NaN for S.1111.111)."""
    vals = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = s * m * 2.0 ** -9
        else:
            vals[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


def _round_half_even(y: np.ndarray) -> np.ndarray:
    f = np.floor(y)
    d = y - f
    up = (d > 0.5) | ((d == 0.5) & (np.fmod(f, 2.0) != 0.0))
    return f + up


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> E4M3FN code (uint8), round to nearest even.

    Defined for |x| <= 464 (values that round to at most 448), which covers
    every product the quantizers form (|x * 448 / amax| <= 448 * (1 + 2^-23)).
    """
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    if np.any(np.abs(x) >= 464.0) or np.any(np.isnan(x)):
        raise ValueError("e4m3_encode: input outside the finite rounding range")
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    code = np.zeros(a.shape, dtype=np.int64)
    sub = a < 2.0 ** -6
    # subnormal range: multiples of 2^-9 (8 rounds up into the first normal)
    code[sub] = _round_half_even(a[sub] * 2.0 ** 9).astype(np.int64)
    nrm = ~sub
    if np.any(nrm):
        an = a[nrm]
        e = np.floor(np.log2(an)).astype(np.int64)
        # guard against log2 rounding at exact powers of two
        e = np.where(2.0 ** e > an, e - 1, e)
        e = np.where(2.0 ** (e + 1) <= an, e + 1, e)
        q = _round_half_even((an / 2.0 ** e - 1.0) * 8.0).astype(np.int64)
        carry = q == 8
        e = np.where(carry, e + 1, e)
        q = np.where(carry, 0, q)
        code[nrm] = ((e + 7) << 3) | q
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def quant_int8_rows(x: np.ndarray, amax: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """int8 codes and fp32 scales of rows of ``x`` (fp32) given their amax (fp32)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.asarray(amax, dtype=np.float32)
    inv = np.float32(127.0) / np.maximum(amax, np.float32(1e-12))
    y = (x * inv[..., None]).astype(np.float32)
    codes = np.trunc(y).astype(np.int8)
    return codes, (amax / np.float32(127.0)).astype(np.float32)


def quant_fp8_rows(x: np.ndarray, amax: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """E4M3FN codes (uint8) and fp32 scales of rows of ``x`` given their amax."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.asarray(amax, dtype=np.float32)
    inv = np.float32(E4M3_MAX) / np.maximum(amax, np.float32(1e-12))
    y = (x * inv[..., None]).astype(np.float32)
    return e4m3_encode(y), (amax / np.float32(E4M3_MAX)).astype(np.float32)


def qk_int32_bruteforce(qc: np.ndarray, kc: np.ndarray) -> np.ndarray:
    """Integer dot products ``qc @ kc^T`` in int64 (exact), returned as int32."""
    return (qc.astype(np.int64) @ kc.astype(np.int64).swapaxes(-1, -2)).astype(np.int32)
