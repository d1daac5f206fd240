"""E4M3FN codec and per-(token, kv head) KV quantisation -- CPU definition.

``decode_e4m3fn`` / ``encode_e4m3fn`` restate the reference's software codec
(benchmarks/v0/probe_quant_support.py:24-56): nearest representable magnitude
after saturating at 448, ties to the even code, sign bit kept for -0 and for
values that round to zero, non-finite input rejected.  ``encode_array`` is the
same rule vectorised with numpy; ``quantize_kv`` restates the scale contract
of docs/project_manual.md:527-537:

    amax = max|x| over head_dim
    scale = 1 if amax == 0 else max(amax / 448, scale_floor)
    code = encode(clamp(x / scale, -448, 448))

with every operation in IEEE fp32 (numpy float32 division is correctly
rounded).  scale_floor is not fixed by the reference; this build freezes it to
2**-64.
"""
from __future__ import annotations

import bisect
import math

import numpy as np

FP8_MAX = 448.0
SCALE_FLOOR = 2.0 ** -64


def decode_e4m3fn(code: int) -> float:
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return math.nan
    if exp == 0:
        return sign * man * 2.0 ** -9
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


MAGNITUDES = [decode_e4m3fn(c) for c in range(127)]  # codes 0..126, increasing


def encode_e4m3fn(value: float) -> int:
    if not math.isfinite(value):
        raise ValueError("non-finite input has no E4M3FN code")
    sign = 0x80 if math.copysign(1.0, value) < 0 else 0
    mag = min(abs(value), FP8_MAX)
    i = bisect.bisect_left(MAGNITUDES, mag)
    lo, hi = max(0, min(126, i - 1)), max(0, min(126, i))
    d_lo, d_hi = abs(MAGNITUDES[lo] - mag), abs(MAGNITUDES[hi] - mag)
    if d_lo < d_hi:
        best = lo
    elif d_hi < d_lo:
        best = hi
    else:
        best = lo if lo % 2 == 0 else hi  # tie: even code
    return sign | best


_MAG = np.array(MAGNITUDES, dtype=np.float64)
DECODE_TABLE = np.array([decode_e4m3fn(c) for c in range(256)], dtype=np.float32)


def encode_array(x: np.ndarray) -> np.ndarray:
    """Vectorised ``encode_e4m3fn`` over a float32 array -> uint8 codes."""
    x = np.asarray(x, dtype=np.float32)
    if not np.isfinite(x).all():
        raise ValueError("non-finite input has no E4M3FN code")
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    mag = np.minimum(np.abs(x).astype(np.float64), FP8_MAX)
    i = np.searchsorted(_MAG, mag, side="left")
    lo = np.clip(i - 1, 0, 126)
    hi = np.clip(i, 0, 126)
    d_lo = np.abs(_MAG[lo] - mag)
    d_hi = np.abs(_MAG[hi] - mag)
    tie_pick = np.where(lo % 2 == 0, lo, hi)
    best = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, tie_pick))
    return (best.astype(np.uint8) | sign).astype(np.uint8)


def decode_array(codes: np.ndarray) -> np.ndarray:
    return DECODE_TABLE[np.asarray(codes, dtype=np.uint8)]


def quantize_kv(x: np.ndarray, scale_floor: float = SCALE_FLOOR):
    """Quantise ``x`` [..., head_dim] (bf16 values as float32) per leading index.

    Returns (codes uint8 [..., head_dim], scale float32 [...]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(amax == 0, np.float32(1.0),
                         np.maximum(amax / np.float32(FP8_MAX), np.float32(scale_floor))).astype(np.float32)
        y = np.clip(x / scale[..., None], np.float32(-FP8_MAX), np.float32(FP8_MAX)).astype(np.float32)
    return encode_array(y), scale


def dequantize_kv(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """x_hat = decode(code) * scale in fp32 (docs/project_manual.md:535)."""
    return decode_array(codes) * np.asarray(scale, dtype=np.float32)[..., None]
