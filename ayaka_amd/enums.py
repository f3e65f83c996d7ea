"""Enumerations the contract uses: step modes, cache layouts and compute dtypes.

Values equal the reference's (``python/ayaka/core/types.py:53-90``,
``python/ayaka/utils/dtypes.py``) and the code compares them by value, so the
engine's own enum members are accepted wherever these are.
"""

from __future__ import annotations

import enum

__all__ = ["DType", "ForwardMode", "KVLayoutKind"]


class KVLayoutKind(str, enum.Enum):
    """Physical layout of one cache block."""

    NHD = "nhd"  # [block_size, num_kv_heads, head_dim]
    HND = "hnd"  # [num_kv_heads, block_size, head_dim]
    NLD = "NLD"  # latent planes; no backend here serves it

    def __str__(self) -> str:
        return self.value


class ForwardMode(str, enum.Enum):
    """How a forward pass consumes its query rows."""

    PREFILL = "prefill"
    DECODE = "decode"
    MIXED = "mixed"
    IDLE = "idle"
    VERIFY = "verify"

    def __str__(self) -> str:
        return self.value


class DType(enum.Enum):
    """Compute dtypes, by label; ``torch_name`` is the torch attribute."""

    FP32 = ("fp32", "float32")
    FP16 = ("fp16", "float16")
    BF16 = ("bf16", "bfloat16")

    @property
    def label(self) -> str:
        return self.value[0]

    @property
    def torch_name(self) -> str:
        return self.value[1]


COMPUTE_DTYPES = frozenset({DType.FP32, DType.FP16, DType.BF16})

try:  # pragma: no cover - only where the engine is installed
    # Inside the engine its enums are the ones in every record; ours compare equal by value.
    from ayaka.core.types import ForwardMode, KVLayoutKind  # type: ignore[import-not-found] # noqa: F811
except ImportError:
    pass
