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

Importing this module does not import torch.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, NamedTuple, Protocol

from ayaka_amd.enums import KVLayoutKind

if TYPE_CHECKING:
    from torch import Tensor

    from ayaka_amd.attention import AttentionMetadata

__all__ = ["FP8_E4M3_CODEC", "RAW_CODEC", "KVBuffers", "KVCacheOps"]

RAW_CODEC = "raw"
#: Keys and values as OCP fp8 e4m3 codes (``torch.float8_e4m3fn``), no scale.
FP8_E4M3_CODEC = "fp8_e4m3"


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
