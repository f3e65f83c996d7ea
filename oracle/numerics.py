"""Bit-level fp16/bf16 conversions and the parity metrics -- test infrastructure only.

Caches and activations travel as raw 16-bit words (``uint16``) so the oracle
never depends on a library's bf16 support. Pinned in ``tests/test_oracle.py``:
the conversions against torch's own ``float32 <-> bfloat16/float16`` casts on
every bf16 bit pattern (exhaustive), the metrics against hand-computed cases.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bits_to_f32",
    "f32_to_bits",
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
