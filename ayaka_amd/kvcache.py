"""The paged KV-cache layout and the contract a backend implements to write it.

Restates the reference's layout definition (``python/ayaka/ops/kvcache.py:1-38``):

* ``k`` and ``v`` are separate contiguous tensors of one dtype, shaped
  ``[num_blocks, block_size, kv_heads, head_dim]`` (NHD) or
  ``[num_blocks, kv_heads, block_size, head_dim]`` (HND).
* Position ``pos`` of a request lives in ``slot = table[pos // block_size] *
  block_size + pos % block_size``. A request of ``length`` tokens uses the first
  ``ceil(length / block_size)`` entries of its table.
* Block 0 is the padding block: never assigned to a request; padding rows are
  stored into slot 0 and its contents are never read as context.
* ``codec`` names how values are stored. The reference defines ``"raw"`` only
  (values in the compute dtype). This package adds ``"fp8_e4m3"``: the
  tensors are ``torch.float8_e4m3fn``, one byte per element, holding what
  torch's cast to that type gives (round to nearest even; a magnitude that
  rounds above 448 becomes NaN); readers decode it exactly to the compute dtype.
  A layer may carry a key and a value scale (:func:`fp8_e4m3_codec`): the codes
  are then those of ``x / scale`` and readers multiply by the scale.

Importing this module does not import torch.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, NamedTuple, Protocol

from ayaka_amd.enums import KVLayoutKind

if TYPE_CHECKING:
    from torch import Tensor

    from ayaka_amd.attention import AttentionMetadata

__all__ = ["FP8_E4M3_CODEC", "RAW_CODEC", "KVBuffers", "KVCacheOps", "ScaledFp8Codec", "codec_scales", "fp8_e4m3_codec"]

RAW_CODEC = "raw"
#: Keys and values as OCP fp8 e4m3 codes (``torch.float8_e4m3fn``), no scale.
FP8_E4M3_CODEC = "fp8_e4m3"


class ScaledFp8Codec(str):
    """The ``"fp8_e4m3"`` codec of one layer with a key scale and a value scale.

    It is the string ``"fp8_e4m3"`` (equal to :data:`FP8_E4M3_CODEC`, so code that compares
    codecs keeps working) carrying ``k_scale`` and ``v_scale``: the cache holds the codes of
    ``k * (1 / k_scale)`` and ``v * (1 / v_scale)`` (the inverse rounded once to float32, the
    product once to float32, then encoded), and readers decode ``code * scale``. A layer whose
    keys reach 4,000 stores them finite with ``k_scale = 4000 / 448``. Scales of 1 are the
    unscaled codec, bit for bit. Make one with :func:`fp8_e4m3_codec`.
    """

    k_scale: float
    v_scale: float

    def __new__(cls, k_scale: float = 1.0, v_scale: float = 1.0) -> "ScaledFp8Codec":
        import math
        import struct

        scales = []
        for name, value in (("k_scale", k_scale), ("v_scale", v_scale)):
            value = struct.unpack("f", struct.pack("f", float(value)))[0]  # as the library reads it
            if not (math.isfinite(value) and value > 0.0):
                raise ValueError(f"{name} must be a positive finite float32, got {value!r}")
            scales.append(value)
        codec = super().__new__(cls, FP8_E4M3_CODEC)
        codec.k_scale, codec.v_scale = scales
        return codec

    def __repr__(self) -> str:
        return f"fp8_e4m3_codec(k_scale={self.k_scale!r}, v_scale={self.v_scale!r})"

    def __reduce__(self):
        return (ScaledFp8Codec, (self.k_scale, self.v_scale))


def fp8_e4m3_codec(k_scale: float = 1.0, v_scale: float = 1.0) -> ScaledFp8Codec:
    """The ``"fp8_e4m3"`` codec with a layer's key and value scales (see :class:`ScaledFp8Codec`)."""
    return ScaledFp8Codec(k_scale, v_scale)


def codec_scales(codec: str) -> tuple[float, float]:
    """``(k_scale, v_scale)`` of a codec: its own for a :class:`ScaledFp8Codec`, else (1, 1)."""
    return (getattr(codec, "k_scale", 1.0), getattr(codec, "v_scale", 1.0))


class _KVBuffers(NamedTuple):
    """The key and value tensors of one layer (reference ``ops/kvcache.py:58-91``)."""

    k: Tensor
    v: Tensor
    layout: KVLayoutKind
    codec: str

    @property
    def num_blocks(self) -> int:
        return int(self.k.shape[0])

    @property
    def block_size(self) -> int:
        return int(self.k.shape[1 if self.layout == KVLayoutKind.NHD else 2])

    @property
    def num_kv_heads(self) -> int:
        return int(self.k.shape[2 if self.layout == KVLayoutKind.NHD else 1])

    @property
    def head_dim(self) -> int:
        return int(self.k.shape[3])


try:  # pragma: no cover - only where the engine is installed
    from ayaka.ops.kvcache import KVBuffers  # type: ignore[import-not-found]
except ImportError:
    KVBuffers = _KVBuffers  # type: ignore[misc]


class KVCacheOps(Protocol):
    """Writing, reading and clearing the paged cache (reference ``ops/kvcache.py:94-144``)."""

    def layout(self) -> KVLayoutKind: ...

    def store(self, k: Tensor, v: Tensor, buffers: KVBuffers, meta: AttentionMetadata) -> None: ...

    def gather(
        self, buffers: KVBuffers, block_ids: Tensor, out_k: Tensor, out_v: Tensor
    ) -> None: ...

    def copy_blocks(self, buffers: KVBuffers, src: Tensor, dst: Tensor) -> None: ...

    def zero_blocks(self, buffers: KVBuffers, block_ids: Tensor) -> None: ...
