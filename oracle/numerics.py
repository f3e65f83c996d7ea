"""Bit-level fp16/bf16/fp8 conversions and the parity metrics -- test infrastructure only.

Caches and activations travel as raw 16-bit words (``uint16``) or fp8 codes
(``uint8``) so the oracle never depends on a library's bf16 or fp8 support.
Pinned in ``tests/test_oracle.py``: the conversions against torch's own
``float32 <-> bfloat16/float16/float8_e4m3fn`` casts (every bf16 and fp16 bit
pattern, every fp8 code), the metrics against hand-computed cases.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bits_to_f32",
    "e4m3_to_f32",
    "f32_to_bits",
    "f32_to_e4m3",
    "half_ulp",
    "parity_report",
]


def bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Widen raw fp16 (``"fp16"``) or bf16 (``"bf16"``) words to float32, exactly."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)
    if dtype == "fp16":
        return bits.view(np.float16).astype(np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def f32_to_bits(values: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 to fp16/bf16 words, to nearest even; NaN stays a quiet NaN."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "fp16":
        with np.errstate(over="ignore"):
            return values.astype(np.float16).view(np.uint16)
    if dtype != "bf16":
        raise ValueError(f"unknown dtype {dtype!r}")
    u = values.view(np.uint32)
    rounded = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), rounded)
    return rounded.astype(np.uint16)


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """Decode OCP fp8 e4m3 codes (the ``float8_e4m3fn`` format) to float32, exactly.

    A code is sign (bit 7), exponent e (bits 6-3, bias 7) and mantissa m (bits
    2-0): (-1)^s (1 + m/8) 2^(e-7) for e >= 1, (-1)^s m 2^-9 for e = 0, and NaN
    for e = 15, m = 7 (there is no infinity).
    """
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e, m = (c >> 3) & 0xF, c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return (sign * mag).astype(np.float32)


def f32_to_e4m3(values: np.ndarray) -> np.ndarray:
    """Encode float32 to OCP fp8 e4m3 codes, to nearest even.

    Magnitudes that round above the largest finite value (448) and NaN give the
    NaN code (0x7F, with the sign bit of the input); there is no saturation.
    Subnormal results are m 2^-9, m in 0..7; the sign of zero is kept.
    """
    x = np.ascontiguousarray(values, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint32)
    a = np.abs(x.astype(np.float64))
    # normal results: round the float32 mantissa to 3 bits (ties to even), rebias 127 -> 7
    mag = u & np.uint32(0x7FFFFFFF)
    rounded = (mag + np.uint32(0x7FFFF) + ((mag >> np.uint32(20)) & np.uint32(1))) >> np.uint32(20)
    normal = rounded.astype(np.int64) - (120 << 3)
    # subnormal results: the nearest multiple of 2^-9 (np.rint rounds ties to even)
    with np.errstate(invalid="ignore"):
        sub = np.where(a < 2.0 ** -6, np.rint(a * 512.0), 0.0).astype(np.int64)
    code = np.where(a < 2.0 ** -6, sub, normal)
    code = np.where(np.isnan(a) | (code > 0x7E), 0x7F, code)
    return (code.astype(np.uint32) | sign).astype(np.uint8)


def f32_to_e4m3_scaled(values: np.ndarray, scale: float) -> np.ndarray:
    """Encode ``values / scale`` as a scaled fp8 e4m3 cache stores it: the inverse scale
    rounded once to float32, the product ``float32(x) * inverse`` rounded once to float32, then
    :func:`f32_to_e4m3`. Scale 1 is :func:`f32_to_e4m3` itself. Follows the codec this build adds
    beside the reference's only ``"raw"`` one (``python/ayaka/ops/kvcache.py:35-36``)."""
    inverse = np.float32(1.0) / np.float32(scale)
    return f32_to_e4m3(np.ascontiguousarray(values, dtype=np.float32) * inverse)


def half_ulp(values: np.ndarray, dtype: str) -> np.ndarray:
    """Half a unit in the last place of ``dtype`` at each |value| (what one rounding can cost)."""
    mantissa = {"bf16": 7, "fp16": 10}[dtype]
    min_exp = {"bf16": -126, "fp16": -14}[dtype]
    mag = np.abs(np.asarray(values, dtype=np.float64))
    with np.errstate(divide="ignore"):
        exp = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
    exp = np.maximum(np.where(mag > 0, exp, min_exp), min_exp)
    return 0.5 * np.exp2(exp - mantissa)


def parity_report(out: np.ndarray, expected: np.ndarray, dtype: str) -> dict[str, float]:
    """Errors of a rounded output against an fp32/fp64 oracle.

    * ``max_abs``: max |out - expected|.
    * ``max_abs_excess``: max over elements of |out - expected| minus half an
      ulp of the output dtype at the expected value -- the error left after the
      one rounding every implementation must make.
    * ``rel_l2``: ||out - round(expected)|| / ||expected||, the relative L2 error
      against the oracle rounded once to the output dtype, the form in which
      the reference returns it.
    * ``rel_l2_raw``: ||out - expected|| / ||expected||.
    """
    out = np.asarray(out, dtype=np.float64)
    exp = np.asarray(expected, dtype=np.float64)
    diff = np.abs(out - exp)
    rounded = bits_to_f32(f32_to_bits(exp.astype(np.float32), dtype), dtype).astype(np.float64)
    norm = float(np.linalg.norm(exp)) or 1.0
    return {
        "max_abs": float(diff.max(initial=0.0)),
        "max_abs_excess": float((diff - half_ulp(exp, dtype)).max(initial=0.0)),
        "rel_l2": float(np.linalg.norm(out - rounded)) / norm,
        "rel_l2_raw": float(np.linalg.norm(out - exp)) / norm,
    }
