"""The attention contract: one step's metadata and the ops that plan and attend.

Restates the reference's row conventions (``python/ayaka/ops/attention.py:1-45``):
a step is a batch of requests, each contributing ``rows_per_request[b]``
consecutive query rows, which are the *last* rows of its sequence.
``kv_lengths[b]`` counts the tokens with keys and values after this step's rows
are stored; row ``j`` of request ``b`` is at position
``kv_lengths[b] - rows_per_request[b] + j`` and attends to positions 0 through
its own. A request with ``kv_lengths[b] == 0`` is padding: its rows go to slot
0 and their outputs are zero. Graph metadata is a fixed-address DECODE record
rewritten in place before each replay.

Importing this module does not import torch.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Protocol

if TYPE_CHECKING:
    from torch import Tensor, device

    from ayaka_amd.enums import ForwardMode
    from ayaka_amd.kvcache import KVBuffers

__all__ = ["AttentionMetadata", "AttentionOps"]


@dataclass(frozen=True, slots=True, eq=False)
class _AttentionMetadata:
    """Everything one step's attention and cache writes need (reference ``:62-95``).

    ``rows_per_request`` [B] int32, ``request_of_row`` [N] int32, ``positions``
    [N] int32 (0 for padding rows), ``slot_mapping`` [N] int64 (0 for padding
    rows), ``kv_lengths`` [B] int32, ``block_table`` the backend's form of the
    table (here the ``[B, max_blocks]`` int32 tensor) and ``plan`` the backend's
    own record, which ``attend`` checks to refuse metadata of another backend.
    """

    mode: ForwardMode
    block_size: int
    rows_per_request: Tensor
    request_of_row: Tensor
    positions: Tensor
    slot_mapping: Tensor
    kv_lengths: Tensor
    block_table: object
    plan: object | None


try:  # pragma: no cover - only where the engine is installed
    # Inside the engine, hand out its own record so nothing downstream sees a foreign type.
    from ayaka.ops.attention import AttentionMetadata  # type: ignore[import-not-found]
except ImportError:
    AttentionMetadata = _AttentionMetadata  # type: ignore[misc]


class AttentionOps(Protocol):
    """Planning a step and attending over the paged cache (reference ``:98-180``)."""

    def plan(
        self,
        mode: ForwardMode,
        rows_per_request: Tensor,
        kv_lengths: Tensor,
        block_rows: Tensor,
        block_size: int,
    ) -> AttentionMetadata: ...

    def attend(
        self, q: Tensor, buffers: KVBuffers, meta: AttentionMetadata, out: Tensor, *, scale: float
    ) -> None: ...

    def graph_metadata(
        self, num_requests: int, max_blocks: int, block_size: int, device: device
    ) -> AttentionMetadata: ...

    def update_graph_metadata(
        self, meta: AttentionMetadata, kv_lengths: Tensor, block_rows: Tensor
    ) -> None: ...
