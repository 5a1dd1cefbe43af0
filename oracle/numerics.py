"""Codecs and scalar functions shared by the oracle models."""

from __future__ import annotations

import numpy as np


def e4m3_decode_table() -> np.ndarray:
    """float64 value of every OCP E4M3FN byte (NaN for 0x7F / 0xFF)."""
    t = np.empty(256, dtype=np.float64)
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0**-9
        else:
            v = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        t[b] = -v if s else v
    return t


E4M3_TABLE = e4m3_decode_table()


def e4m3_decode(b: np.ndarray) -> np.ndarray:
    return E4M3_TABLE[np.asarray(b, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray, saturate: bool = False) -> np.ndarray:
    """fp32 -> E4M3FN bytes, round to nearest even; overflow -> NaN (0x7F)
    unless `saturate` (then +-448).  OCP 8-bit FP spec, section 5."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    sign = ((b >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    a = b & np.uint32(0x7FFFFFFF)
    r = a + np.uint32(0x7FFFF) + ((a >> np.uint32(20)) & np.uint32(1))
    normal = (((r >> np.uint32(23)) - np.uint32(120)) << np.uint32(3)) | ((r >> np.uint32(20)) & np.uint32(7))
    small = np.where(a < np.uint32(0x3C800000), a, np.uint32(0))
    sub = np.rint(small.view(np.float32) * np.float32(512.0)).astype(np.uint32)
    out = np.where(a >= np.uint32(0x3C800000), normal, sub)
    over = np.uint32(0x7E) if saturate else np.uint32(0x7F)
    out = np.where(a > np.uint32(0x43E80000), over, out)
    out = np.where(a > np.uint32(0x7F800000), np.uint32(0x7F), out)
    return (out.astype(np.uint8) | sign).astype(np.uint8)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, IEEE round to nearest even."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def sigmoid(x: np.ndarray) -> np.ndarray:
    """s = 1 / (1 + e) with e = exp(-x) rounded once to fp32 (evaluated in
    float64), then an fp32 add and an IEEE fp32 divide.  The GPU router
    evaluates the same sequence, so the two agree bit for bit."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-x.astype(np.float64)).astype(np.float32)
    d = (np.float32(1.0) + e).astype(np.float32)
    return (np.float32(1.0) / d).astype(np.float32)
