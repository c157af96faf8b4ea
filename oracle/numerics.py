"""Rounding emulation used by the oracle (test infrastructure only).

The reference's fused Triton kernels cast q, K/V, the representative values and
the softmax weights to bfloat16 right before each ``tl.dot`` (CBT/page_attention.py
:86-90, :199-202, :230, :249-252) and accumulate in float32.  The oracle mirrors
those cast points with ``bf16_round``.  The fp8 KV variant has no counterpart in
the reference; its codec is the OCP e4m3fn format (1 sign, 4 exponent bits with
bias 7, 3 mantissa bits, no infinities, max finite 448).
"""

import numpy as np


def bf16_round(x):
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def bf16_bits(x):
    """bfloat16 bit patterns (uint16) of ``bf16_round(x)``."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).astype(np.uint32).view(np.float32)


def _e4m3_table():
    vals = np.zeros(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            vals[b] = np.nan
        elif e == 0:
            vals[b] = s * (m / 8.0) * 2.0 ** (-6)
        else:
            vals[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3_VALUES = _e4m3_table()
E4M3_MAX = 448.0


def e4m3_decode(codes):
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x):
    """Encode float values as e4m3fn codes: round to nearest, ties to even, saturate."""
    x = np.asarray(x, dtype=np.float32)
    finite = E4M3_VALUES[:0x7F]          # codes 0..126 are the non-negative finite values
    mag = np.minimum(np.abs(x), E4M3_MAX)
    idx = np.searchsorted(finite, mag, side="left")
    idx = np.clip(idx, 0, len(finite) - 1)
    lo = np.clip(idx - 1, 0, len(finite) - 1)
    d_hi = np.abs(finite[idx] - mag)
    d_lo = np.abs(mag - finite[lo])
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0) & (lo != idx))
    code = np.where(pick_lo, lo, idx).astype(np.uint8)
    code = code | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    return code.astype(np.uint8)
