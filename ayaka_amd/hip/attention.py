"""Attention over the paged cache with the MI355X kernels; implements the ``AttentionOps`` contract.

``plan`` runs on the host once per step. It checks the step and derives
positions, slots and lengths by the reference's rules
(``python/ayaka/ops/backends/torch/attention.py:64-164``) and records the host
facts ``attend`` needs to pick a launch without reading the device.

``attend`` launches one of two kernels through ``libayaka_hip.so``:

* v1 (``ayk_paged_attention_v1``): one launch, no scratch: a workgroup per row
  and 8 / n of its key/value heads, n = 1-8 waves per head each streaming every
  n-th chunk of the row's context, merged in LDS;
* v2 (``ayk_paged_attention_v2``): one workgroup per (row, key/value head,
  partition) that holds tokens, longest first, then a log-sum-exp merge.

:func:`choose_split` picks between them, v1's wave count and v2's partition size,
from the step's row lengths by a modelled schedule. Decode rows (one per request) use these kernels;
steps of several rows per request (prefill chunks, verify windows) use the multi-row
kernel (``ayk_paged_prefill``), where row ``j`` attends to positions
``0 .. position_j`` (the reference's causal rule, ``attention.py:209-234``).

``graph_metadata`` / ``update_graph_metadata`` follow the reference's
fixed-address record (``attention.py:274-374``): device tensors allocated once,
host staging pinned, asynchronous copies on the current stream. Each update also
stages the step's v2 partition size and work list on the device, so ``attend`` on
graph metadata reads nothing on the host that changes between replays: its
captured launch covers the bucket's capacity and the kernels read the step's split.
"""

from __future__ import annotations

import ctypes
import functools
import heapq
import math
from dataclasses import dataclass, field

import numpy as np
import torch

from ayaka_amd.enums import ForwardMode, KVLayoutKind
from ayaka_amd.attention import AttentionMetadata
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import _fastpath, _lib
from ayaka_amd.hip._checks import (
    compute_dtype,
    HEAD_DIMS,
    capturing,
    require_buffers,
    require_device,
    require_index_tensor,
    require_like,
    stream_handle,
)
from ayaka_amd.kvcache import FP8_E4M3_CODEC, KVBuffers, codec_scales

__all__ = [
    "PARTITION_SIZE",
    "HipAttentionPlan",
    "HipGraphPlan",
    "attend",
    "attend_with",
    "choose_partitions",
    "choose_split",
    "graph_metadata",
    "plan",
    "update_graph_metadata",
]

#: Default positions per v2 partition (callers that force a v2 launch without a size).
PARTITION_SIZE = 512
#: Graph replays: the smallest partition, the most partitions per row of the table width,
#: and the work items of a bucket of fewer rows (the captured grid, by key/value head
#: group, and the partial slots of its scratch).
GRAPH_MIN_PARTITION = 64
GRAPH_MAX_PARTITIONS = 256
GRAPH_MAX_ITEMS = 2048
#: Partition sizes an eagerly planned step chooses from (multiples of 64).
PARTITION_CANDIDATES = (64, 128, 192, 256, 320, 384, 448, 512, 576, 640, 704, 768, 896, 1024, 1280, 1536,
                        2048, 3072, 4096, 8192, 16384)
#: More sizes for fp8 caches. C5 over fp8 caches measured 219.9 us at 2560 against 229.8 at
#: 1280, the model's choice without it; over bf16 caches the model moves C5 to 2560 as well,
#: measured 404.7 against 399.0 at its 3072, so the size is offered to fp8 caches alone.
FP8_PARTITION_CANDIDATES = tuple(sorted(PARTITION_CANDIDATES + (2560,)))
#: Fixed cost of one workgroup, in positions of streaming (start-up, merge, partial write),
#: by bytes per cache element. Fitted to measured partition-size sweeps (256 ... 4096
#: positions) of the C3, C4 and C5 shapes: 320 for 16-bit caches (the modelled finish
#: time then tracks C5's ragged curve with correlation 0.87, against 0.11 at 80) and 160
#: for fp8 caches (0.99); with them the model picks the fastest measured size of all
#: three shapes for both.
WORKGROUP_COSTS = {2: 320, 1: 160, 4: 320}
WORKGROUP_COST = WORKGROUP_COSTS[2]
#: The same for a v1 workgroup, whose waves split each context among themselves and merge
#: in LDS (no partials, no second launch): fitted so that the model prefers v1 where it
#: measured faster than the best v2 launch (C3's 64 rows of 4096: 160.5 vs 162.8 us, with
#: fp8 caches 90.7 vs 92.8; C1's four short rows: 12.1 vs 15.9 us, with fp8 caches 11.3 vs
#: 15.7) and v2 where it is not (C2, C4, C5, both codecs).
V1_WORKGROUP_COSTS = {2: 240, 1: 80, 4: 240}
#: Waves a v1 workgroup may split each (row, key/value head)'s context among.
V1_WAVE_SPLITS = (1, 2, 4, 8)
#: XCDs of one MI355X; workgroups are dealt to them round-robin.
XCDS = 8
#: Heads per wave from which the library runs q.k on the matrix cores (mirrors the C library).
MFMA_MIN_HEADS = 3
#: (row, query head) pairs one workgroup of the multi-row kernel serves, by head width
#: (the C library's ``ayk_paged_prefill_tile_pairs``; a test checks they agree).
PREFILL_PAIRS = {64: 128, 128: 128, 256: 64}
#: Head widths whose multi-row kernel also runs the double tile: twice the pairs in an 8-wave
#: workgroup, one per compute unit, which stages each chunk once for all of them.
PREFILL_DOUBLE_TILE_DIMS = (128, 256)


def prefill_waves_per_group(head_dim: int, pairs: int) -> int:
    """How a tile of ``pairs`` runs: 1, 2 or 4 waves per group of 16 pairs in a 4-wave workgroup
    (the full tile, a half, a quarter), or 0 for the double tile (an 8-wave workgroup)."""
    full = PREFILL_PAIRS[head_dim]
    return 0 if pairs == 2 * full and head_dim in PREFILL_DOUBLE_TILE_DIMS else full // pairs
#: Rows per request (on average) from which a multi-row step runs the multi-row kernel.
PREFILL_MIN_ROWS = 2
#: Compute units of one MI355X; the split heuristic aims to keep all of them busy.
COMPUTE_UNITS = 256

_LAYOUT_CODES = {KVLayoutKind.NHD: 0, KVLayoutKind.HND: 1}
_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 3}
_KV_FP8_E4M3 = 2


def _kv_code(buffers: KVBuffers, dtype: torch.dtype) -> int:
    """The C ABI's cache element type: the compute dtype, or fp8 e4m3 codes."""
    return _KV_FP8_E4M3 if buffers.codec == FP8_E4M3_CODEC else _DTYPE_CODES[dtype]
_QK_FLAGS = {None: 0, "dpp": 1, "mfma": 2}
#: v2 flag: launch the partition kernel only (benchmarks time the dominant kernel with it).
PARTIALS_ONLY = 4
_MERGE_FLAGS = {None: 0, "reduce-kernel": 8, "in-kernel": 16}
#: AYK_FLAG_WAVES_*: waves sharing each (row, key/value head)'s context (v1) or partition (v2)
_WAVE_FLAGS = {None: 0, 1: 32, 2: 64, 4: 128, 8: 256}


@dataclass(frozen=True, slots=True)
class HipAttentionPlan:
    """Host facts of an eagerly planned step.

    ``rows`` / ``kv_lengths`` are the per-request lists ``plan`` read;
    ``max_length`` is the longest context any row attends to.
    """

    rows: tuple[int, ...]
    kv_lengths: tuple[int, ...]
    max_length: int
    total_length: int
    row_lengths: tuple[int, ...] = ()
    # v2 work lists built by the step's first attend, keyed by partition size, for the later layers
    work: dict[int, torch.Tensor] = field(default_factory=dict, compare=False, repr=False)
    # per-step choices shared by every layer: decode splits, multi-row partition sizes and launches,
    # window splits, and the multi-row row groups they are scored on
    splits: dict[tuple, object] = field(default_factory=dict, compare=False, repr=False)
    # library calls recorded by attend / store, replayed for the same objects (_fastpath)
    launches: dict = field(default_factory=dict, compare=False, repr=False)

    def split_for(self, num_kv_heads: int, group: int, kv_bytes: int = 2) -> Split:
        """The step's launch for this head shape and cache element size, chosen once and
        reused by every layer."""
        key = (num_kv_heads, group, kv_bytes)
        found = self.splits.get(key)
        if found is None:
            found = choose_split(len(self.row_lengths), num_kv_heads, group, self.max_length,
                                 row_lengths=self.row_lengths, kv_bytes=kv_bytes)
            self.splits[key] = found
        return found

    def prefill_group_arrays(self, group: int, pairs: int) -> tuple[np.ndarray, ...]:
        """(context length, first row, row count, request) of each group of rows the multi-row
        kernel serves together, as four int64 arrays, heaviest first (ties: the first row);
        built once per step and tile size.

        Each group holds consecutive rows of one request, at most ``pairs`` (row, query head)
        pairs; its context length is that of its last row (0 for a padding request).
        """
        key = ("groups", group, pairs)
        found = self.splits.get(key)
        if found is None:
            per_tile = max(1, pairs // group)
            rows = np.asarray(self.rows, dtype=np.int64)
            lengths = np.asarray(self.kv_lengths, dtype=np.int64)
            row_lengths = np.asarray(self.row_lengths, dtype=np.int64)
            first = np.cumsum(rows) - rows
            tiles = -(-rows // per_tile)
            request = np.repeat(np.arange(rows.size, dtype=np.int64), tiles)
            start = (np.arange(request.size, dtype=np.int64) - np.repeat(np.cumsum(tiles) - tiles, tiles)) * per_tile
            count = np.minimum(per_tile, rows[request] - start)
            row = first[request] + start
            last = np.where(lengths[request] > 0, row_lengths[row + count - 1], 0) if request.size else row
            order = np.lexsort((row, -last))
            found = (last[order], row[order], count[order], request[order])
            self.splits[key] = found
        return found

    def prefill_groups(self, group: int, pairs: int) -> list[tuple[int, int, int, int]]:
        """:meth:`prefill_group_arrays` as (context length, first row, row count, request) tuples."""
        return list(zip(*(a.tolist() for a in self.prefill_group_arrays(group, pairs))))

    def prefill_split(self, num_kv_heads: int, group: int, pairs: int, head_dim: int, kv_bytes: int = 2) -> int:
        """The partition size of the step's multi-row launch with tiles of ``pairs`` (0: none),
        chosen once for every layer."""
        key = ("prefill", num_kv_heads, group, pairs, head_dim, kv_bytes)
        found = self.splits.get(key)
        if found is None:
            lengths = self.prefill_group_arrays(group, pairs)[0]
            found = choose_prefill_partition(lengths, self.row_lengths, num_kv_heads, num_kv_heads * group,
                                             head_dim, prefill_waves_per_group(head_dim, pairs),
                                             self.context_bytes(num_kv_heads, head_dim, kv_bytes))
            self.splits[key] = found
        return found

    def context_bytes(self, num_kv_heads: int, head_dim: int, kv_bytes: int = 2) -> int:
        """K and V bytes of the contexts the step's multi-row requests read (once each)."""
        positions = sum(length for count, length in zip(self.rows, self.kv_lengths) if count)
        return positions * num_kv_heads * head_dim * 2 * kv_bytes

    def prefill_launch(self, num_kv_heads: int, group: int, head_dim: int, kv_bytes: int = 2) -> tuple[int, int]:
        """(tile pairs, partition size) of the step's multi-row launch: of the double tile (head
        widths 128 and 256), the full tile, a half and a quarter (each at its best partition
        size), the one with the smallest :func:`prefill_model_us`; chosen once for every layer."""
        key = ("prefill-launch", num_kv_heads, group, head_dim, kv_bytes)
        found = self.splits.get(key)
        if found is None:
            full = PREFILL_PAIRS[head_dim]
            context = self.context_bytes(num_kv_heads, head_dim, kv_bytes)
            best = None
            for waves in ((0, 1, 2, 4) if head_dim in PREFILL_DOUBLE_TILE_DIMS else (1, 2, 4)):
                pairs = 2 * full if waves == 0 else full // waves
                if pairs < group:
                    break
                size = self.prefill_split(num_kv_heads, group, pairs, head_dim, kv_bytes)
                lengths = self.prefill_group_arrays(group, pairs)[0]
                t = prefill_model_us(lengths, self.row_lengths, num_kv_heads, num_kv_heads * group, head_dim, size,
                                     waves, context)
                # a smaller tile (they come in decreasing size) must win by a margin: at a tie
                # the model under-prices the quarter tile's short steps (a 1024-row prompt:
                # modelled equal, measured 38.6 against 31.4 us on the half tile)
                if best is None or t < best[0] * (1 - PREFILL_SMALLER_TILE_MARGIN):
                    best = (t, pairs, size)
            found = (best[1], best[2])
            self.splits[key] = found
        return found

    def window_pairs(self, group: int) -> int:
        """(row, query head) pairs of a window tile (:func:`attend_with`'s ``window``):
        as many rows of a request as fit the decode kernel's 16 matrix-core columns, 0 when
        a request's rows do not fit one tile (or a group is wider than 16)."""
        if group > 16:
            return 0
        rows = 16 // group
        return rows * group if all(count <= rows for count in self.rows) else 0

    def window_split(self, num_kv_heads: int, group: int, kv_bytes: int = 2) -> int:
        """Partition size (0: none) of the step's window launch: the decode kernel's split
        model (:func:`choose_split`) over the tiles' contexts, one workgroup per tile,
        partition and 8 key/value heads, or, unsplit, each tile's context shared by up to 8
        waves per head as v1 shares a row's (the library sizes that split to the grid);
        chosen once for every layer."""
        key = ("window", num_kv_heads, group, kv_bytes)
        found = self.splits.get(key)
        if found is None:
            lengths = self.prefill_group_arrays(group, self.window_pairs(group))[0].tolist()
            found = window_partition_size([n for n in lengths if n > 0], num_kv_heads, kv_bytes)
            self.splits[key] = found
        return found

    def prefill_tiles(self, group: int, pairs: int, partition_size: int, device: torch.device,
                      capture: bool = False) -> torch.Tensor:
        """(first row, row count, request, partition) quadruples for the multi-row kernel.

        Without partitions (``partition_size`` 0) one tile per group of rows, heaviest
        first; with them, one per partition the group's last row sees, longest first.
        Built once per step and launch shape; building copies it to the device, which a
        graph capture cannot record (``capture``: raise instead).
        """
        key = (-group, pairs, partition_size)
        found = self.work.get(key)
        if found is None and capture:
            raise BackendError(
                "attention.attend: the multi-row tile list of this step is built on its first "
                "call; run the step once eagerly before capturing it",
                context={"op": "attention.attend"},
            )
        if found is None:
            length, row, count, request = self.prefill_group_arrays(group, pairs)
            if partition_size:
                parts = np.maximum(1, -(-length // partition_size))
                index = np.repeat(np.arange(length.size), parts)
                part = np.arange(index.size, dtype=np.int64) - np.repeat(np.cumsum(parts) - parts, parts)
                piece = np.minimum(partition_size, length[index] - part * partition_size)
                row, count, request = row[index], count[index], request[index]
                order = np.lexsort((part, request, count, row, -piece))  # longest piece first
                row, count, request, part = row[order], count[order], request[order], part[order]
            else:
                part = np.zeros_like(row)
            flat = np.stack((row, count, request, part), axis=1).reshape(-1).astype(np.int32)
            found = torch.from_numpy(flat).to(device)
            self.work[key] = found
        return found

    def work_items(self, partition_size: int, device: torch.device) -> torch.Tensor:
        """:func:`work_list` of the step's rows, on ``device``, built once per partition size."""
        found = self.work.get(partition_size)
        if found is None:
            found = torch.from_numpy(work_list(self.row_lengths, partition_size)).to(device)
            self.work[partition_size] = found
        return found


def work_list(row_lengths: "tuple[int, ...] | list[int] | np.ndarray", partition_size: int) -> np.ndarray:
    """The v2 work list: the (row, partition) pairs that hold tokens, flattened to int32
    ``[row0, part0, row1, part1, ...]``, longest partition first (ties by row, then
    partition), plus partition 0 of each row without context, last (it writes the row's zeros).

    Every full partition comes before any partial one, so the last workgroups to
    start are the short ones and consecutive workgroups land on different XCDs. Built by the
    library's host code (``ayk_work_list``).
    """
    lengths = np.ascontiguousarray(row_lengths, dtype=np.int64).reshape(-1)
    count = int(np.maximum(1, -(-lengths // max(partition_size, 1))).sum())
    out = np.empty(2 * count, dtype=np.int32)
    if _lib.lib().ayk_work_list(lengths.ctypes.data, lengths.size, partition_size, out.ctypes.data) != count:
        raise BackendError(f"attention.work_list: bad lengths or partition size {partition_size}",
                           context={"op": "attention.work_list"})
    return out


@dataclass(frozen=True, slots=True, eq=False)
class HipGraphPlan:
    """Pinned host staging of a graph bucket, its fixed table width, and the v2 launch
    staged on the device for every step.

    A captured v2 launch has a fixed grid of ``capacity`` work items over at most
    ``partitions`` partitions of at least ``min_size`` positions. Each update
    stages the step's own partition size (a multiple of 64, at least
    ``min_size``, whose work list fits the capacity) into ``staged`` (device) as
    ``[partition size, item count, first partial slot of each row, row0, part0,
    ...]``; workgroups past the item count return at once, and the rows' partials
    are packed into ``capacity`` slots. ``head_shape`` holds the ``(num_kv_heads,
    group, kv_bytes)`` of the first attend, which scores the staged split;
    ``staged_shape`` the shape the last staged split was scored for (an update before
    the first attend scores a guess, and that attend re-stages the split).
    """

    positions: torch.Tensor
    slot_mapping: torch.Tensor
    kv_lengths: torch.Tensor
    block_table: torch.Tensor
    max_blocks: int
    staged_host: torch.Tensor
    staged: torch.Tensor
    min_size: int
    partitions: int
    capacity: int
    host_all: torch.Tensor  # the pinned buffer every host record above is a view of
    device_all: torch.Tensor  # its device twin, holding the fixed records and `staged`
    staged_offset: int  # where `staged` starts in both, in bytes (it comes last)
    head_shape: list = field(default_factory=list)
    staged_shape: list = field(default_factory=list)
    launches: dict = field(default_factory=dict)

    @property
    def staged_partition_size(self) -> int:
        """The partition size the last update staged (the host copy)."""
        return int(self.staged_host[0])

    @property
    def work_offset(self) -> int:
        """Where the work list starts in ``staged``, in int32 words."""
        return 2 + self.positions.shape[0]


def plan(
    mode: ForwardMode,
    rows_per_request: torch.Tensor,
    kv_lengths: torch.Tensor,
    block_rows: torch.Tensor,
    block_size: int,
) -> AttentionMetadata:
    """Check one step and build its metadata (reference ``torch/attention.py:64-110``)."""
    op = "attention.plan"
    require_index_tensor(op, "rows_per_request", rows_per_request, ndim=1)
    require_index_tensor(op, "kv_lengths", kv_lengths, ndim=1)
    require_index_tensor(op, "block_rows", block_rows, ndim=2)
    batch = rows_per_request.shape[0]
    if kv_lengths.shape[0] != batch or block_rows.shape[0] != batch:
        raise BackendError(
            f"{op}: rows_per_request, kv_lengths and block_rows must all describe the same "
            f"requests, got {batch}, {kv_lengths.shape[0]} and {block_rows.shape[0]}",
            context={"op": op},
        )
    if block_size < 1:
        raise BackendError(f"{op}: block_size must be positive, got {block_size}", context={"op": op})
    rows_np = rows_per_request.to(device="cpu", dtype=torch.int64).numpy()
    lengths_np = kv_lengths.to(device="cpu", dtype=torch.int64).numpy()
    # the checks over all requests at once; the first failing request names the refusal
    bad = np.flatnonzero((rows_np < 0) | (lengths_np < 0) | ((lengths_np > 0) & (rows_np > lengths_np))
                         | ((rows_np != 1) if mode == ForwardMode.DECODE else False))
    if bad.size:
        index = int(bad[0])
        count, length = int(rows_np[index]), int(lengths_np[index])
        if count < 0 or length < 0:
            raise BackendError(
                f"{op}: request {index} has {count} rows and {length} tokens; neither can be "
                "negative",
                context={"op": op, "request": index},
            )
        if length and count > length:
            raise BackendError(
                f"{op}: request {index} has {count} query rows but only {length} tokens with "
                "keys after this step; kv_lengths counts this step's rows",
                context={"op": op, "request": index},
            )
        raise BackendError(
            f"{op}: a DECODE step has one row per request, request {index} has {count}",
            context={"op": op, "request": index},
        )
    rows, lengths = tuple(rows_np.tolist()), tuple(lengths_np.tolist())
    total = int(rows_np.sum())
    if mode == ForwardMode.IDLE and total:
        raise BackendError(f"{op}: an IDLE step has no rows, got {total}", context={"op": op})

    # The table: long enough for every request, and no padding block inside a used range.
    table_host = block_rows.to(device="cpu", dtype=torch.int64)
    max_blocks = table_host.shape[1]
    needed = -(-lengths_np // block_size)
    longest = int(needed.max(initial=0))
    if longest > max_blocks or (total > 0 and max_blocks == 0):
        raise BackendError(
            f"{op}: block_rows has {max_blocks} column(s) but the longest request needs "
            f"{longest} blocks of {block_size}",
            context={"op": op, "argument": "block_rows"},
        )
    table_np = table_host.numpy()
    if batch and max_blocks:
        used = np.arange(max_blocks)[None, :] < needed[:, None]
        if bool((used & (table_np == 0)).any()):
            raise BackendError(
                f"{op}: block_rows has the padding block 0 inside a request's blocks",
                context={"op": op, "argument": "block_rows"},
            )

    # Row j of a request of `count` rows and `length` tokens sits at position
    # length - count + j, in slot table[request][position // bs] * bs + position % bs; a
    # request without tokens (padding) gets position 0, slot 0 and no context.
    request_of_row = np.repeat(np.arange(batch, dtype=np.int64), rows_np)
    first = np.cumsum(rows_np) - rows_np
    j = np.arange(total, dtype=np.int64) - np.repeat(first, rows_np)
    row_length = lengths_np[request_of_row]
    live = row_length > 0
    positions_np = np.where(live, row_length - rows_np[request_of_row] + j, 0)
    blocks = table_np[request_of_row, positions_np // block_size] if total else np.zeros(0, dtype=np.int64)
    slots_np = np.where(live, blocks * block_size + positions_np % block_size, 0)
    row_lengths = tuple(np.where(live, positions_np + 1, 0).tolist())

    device = rows_per_request.device
    return AttentionMetadata(
        mode=mode,
        block_size=block_size,
        rows_per_request=torch.from_numpy(rows_np.astype(np.int32)).to(device),
        request_of_row=torch.from_numpy(request_of_row.astype(np.int32)).to(device),
        positions=torch.from_numpy(positions_np.astype(np.int32)).to(device),
        slot_mapping=torch.from_numpy(slots_np).to(device),
        kv_lengths=torch.from_numpy(lengths_np.astype(np.int32)).to(device),
        block_table=block_rows.to(device=device, dtype=torch.int32).contiguous(),
        plan=HipAttentionPlan(rows, lengths, max(lengths, default=0), sum(row_lengths), row_lengths),
    )


def _wants_prefill_kernel(step: object) -> bool:
    """Multi-row steps with >= :data:`PREFILL_MIN_ROWS` rows per request (on average) use the
    multi-row kernel, which reads each request's context once for all its rows (split into
    partitions when the tiles are too few to fill the GPU); steps of single rows use the
    decode kernels."""
    if not isinstance(step, HipAttentionPlan):
        return False
    requests = sum(1 for count in step.rows if count)
    return requests > 0 and sum(step.rows) >= PREFILL_MIN_ROWS * requests


def head_chunks(group: int) -> int:
    """Chunks the query heads of one key/value head are split into (at most 8 heads each)."""
    for chunks in range(1, group + 1):
        if group % chunks == 0 and group // chunks <= 8:
            return chunks
    return group


def uses_matrix_cores(group: int) -> bool:
    """Whether the library picks the MFMA q.k kernel for this group size (3+ heads per wave)."""
    return group // head_chunks(group) >= MFMA_MIN_HEADS


#: Most partitions per row the in-kernel merge serves (``kInKernelMaxPartitions`` in ``api.hip``).
IN_KERNEL_MAX_PARTITIONS = 4


def merge_site_for(workgroups: int, partitions: int) -> str:
    """Where the library merges the v2 partitions of a grid of ``workgroups`` whose rows hold up
    to ``partitions`` partitions: ``"in-kernel"`` for a quarter round of the compute units at
    most and a few partitions per row, ``"reduce-kernel"`` otherwise (the rule of
    ``merge_in_kernel`` in ``api.hip``)."""
    small = workgroups <= COMPUTE_UNITS // 4 and partitions <= IN_KERNEL_MAX_PARTITIONS
    return "in-kernel" if small else "reduce-kernel"


def merge_site(num_kv_heads: int, group: int, step: "HipAttentionPlan", partition_size: int) -> str:
    """Where the library merges the v2 partitions of an eagerly planned step (its work list)."""
    groups = -(-num_kv_heads * head_chunks(group) // 8)
    items = sum(max(1, -(-n // partition_size)) for n in step.row_lengths)
    return merge_site_for(items * groups, -(-step.max_length // partition_size))


def graph_merge_site(items: int, num_kv_heads: int, group: int, partitions: int) -> str:
    """Where the library merges the v2 partitions of a launch over a grid of ``items`` work
    items (a graph replay's capacity, or the rows x partitions of a forced dense grid) whose
    rows hold up to ``partitions`` partitions."""
    return merge_site_for(items * -(-num_kv_heads * head_chunks(group) // 8), partitions)


@dataclass(frozen=True, slots=True)
class Split:
    """A launch: ``partitions == 0`` is v1, otherwise v2 over partitions of ``partition_size``.
    ``waves`` (v1): waves sharing each (row, key/value head)'s context, 0 for the C
    library's own rule."""

    partition_size: int
    partitions: int
    waves: int = 0


def schedule_makespans(row_lengths: "list[int] | np.ndarray", sizes: "list[int] | tuple[int, ...]",
                       groups: int = 1, cost: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Modelled finish times, in positions, of v2 over partitions of each of ``sizes``, and
    the work items per key/value head group at each size.

    Workgroups start in work-list order (longest partition first); the GPU hands
    workgroup i to XCD i mod 8 and each XCD to whichever of its 32 CUs frees up
    first, one 8-wave workgroup per CU at a time. A workgroup costs its
    positions plus ``cost`` (default :data:`WORKGROUP_COST`: start-up, the final
    merge, writing the partial). Computed by the library's host code
    (``ayk_split_model``), one call for every size.
    """
    cost = WORKGROUP_COST if cost is None else cost
    lengths = np.ascontiguousarray(row_lengths, dtype=np.int64).reshape(-1)
    sizes = np.ascontiguousarray(sizes, dtype=np.int32).reshape(-1)
    makespans = np.empty(sizes.size, dtype=np.int64)
    items = np.empty(sizes.size, dtype=np.int64)
    rc = _lib.lib().ayk_split_model(lengths.ctypes.data, lengths.size, sizes.ctypes.data, sizes.size, groups, cost,
                                    COMPUTE_UNITS, XCDS, makespans.ctypes.data, items.ctypes.data)
    if rc != 0:
        raise BackendError(f"attention.schedule_makespans: bad sizes {sizes.tolist()}, groups {groups} or cost {cost}",
                           context={"op": "attention.schedule_makespans"})
    return makespans, items


def schedule_makespan(row_lengths: list[int], size: int, groups: int = 1, cost: int | None = None) -> int:
    """:func:`schedule_makespans` at one partition size."""
    return int(schedule_makespans(row_lengths, (size,), groups, cost)[0][0])


_split_cache: dict[tuple, int] = {}
#: Work lists longer than this many rounds of the GPU are not considered (start-up cost dominates).
MAX_ROUNDS = 8


def v1_makespan(row_lengths: list[int], waves: int, virtual_heads: int, cost: int) -> int:
    """Modelled finish time, in positions, of v1 with each context split among ``waves`` waves:
    a workgroup per row and ``8 / waves`` virtual heads, each wave streaming a ``1 / waves``
    share of its row in 16-position chunks, scheduled as :func:`schedule_makespan` schedules
    v2's workgroups."""
    shares = -(-np.asarray(row_lengths, dtype=np.int64) // (16 * waves)) * 16
    groups = -(-virtual_heads * waves // 8)
    return schedule_makespan(shares, int(shares.max(initial=0)) + 1, groups, cost)


def window_waves(n_items: int, num_kv_heads: int) -> int:
    """Waves per key/value head of a window launch of ``n_items`` work items (tiles, or tile
    partitions), as the C library sizes it: the most (up to 8) that keep items x heads x
    waves within one round of 8-wave workgroups."""
    waves = 1
    while waves < 8 and n_items * num_kv_heads * waves * 2 <= COMPUTE_UNITS * 8:
        waves *= 2
    return waves


def window_partition_size(lengths: list[int], num_kv_heads: int, kv_bytes: int = 2) -> int:
    """Partition size (0: none) of a window launch over tiles of these contexts: each
    candidate's work items (a tile, or a partition of one) shared by the waves the library
    gives them (:func:`window_waves`), scored as v1's wave split is (:func:`v1_makespan`),
    with v1's workgroup cost unsplit and v2's (partials, merge) split; of sizes that model
    the same, the largest (fewest partials; measured: 8 tiles over 8K, 256 -> 1024 took
    63.7 -> 51.1 us)."""
    if not lengths:
        return 0
    longest = max(lengths)
    best = (v1_makespan(lengths, window_waves(len(lengths), num_kv_heads), num_kv_heads,
                        V1_WORKGROUP_COSTS[kv_bytes]), 0)
    for size in PARTITION_CANDIDATES:
        if size >= longest:
            break
        parts = [min(size, n - start) for n in lengths for start in range(0, n, size)]
        t = v1_makespan(parts, window_waves(len(parts), num_kv_heads), num_kv_heads, WORKGROUP_COSTS[kv_bytes])
        if t <= best[0] and (best[1] or t < best[0]):  # ties: the larger size, fewer partials to merge
            best = (t, size)
    return best[1]


def fits_schedule(lengths: list[int], size: int, groups: int = 1) -> bool:
    """Whether partitions of ``size`` keep the work list within :data:`MAX_ROUNDS` rounds."""
    items = sum(-(-n // size) for n in lengths) * groups
    return items <= MAX_ROUNDS * COMPUTE_UNITS


def _best_size(lengths: list[int], max_length: int, groups: int, kv_bytes: int = 2, min_size: int = 0,
               max_items: int = 0) -> int:
    """The candidate partition size (of ``min_size`` or more, and with ``max_items`` work
    items at most when that is positive) with the smallest :func:`schedule_makespan`; sizes
    whose work list exceeds :data:`MAX_ROUNDS` rounds are left out unless none is left, and
    no size past the first that covers ``max_length`` is scored."""
    offered = FP8_PARTITION_CANDIDATES if kv_bytes == 1 else PARTITION_CANDIDATES
    candidates = [size for size in offered if size >= min_size] or [min_size]
    for i, size in enumerate(candidates):
        if size >= max_length:
            candidates = candidates[:i + 1]
            break
    lengths = np.ascontiguousarray(lengths, dtype=np.int64)
    sizes = np.ascontiguousarray(candidates, dtype=np.int32)
    best = ctypes.c_int32(-1)
    rc = _lib.lib().ayk_best_split(lengths.ctypes.data, lengths.size, sizes.ctypes.data, sizes.size, groups,
                                   WORKGROUP_COSTS[kv_bytes], COMPUTE_UNITS, XCDS, max_items,
                                   MAX_ROUNDS * COMPUTE_UNITS, ctypes.byref(best))
    if rc != 0:
        raise BackendError(f"attention.choose_split: bad sizes {candidates} or groups {groups}",
                           context={"op": "attention.choose_split"})
    if best.value < 0:  # no size keeps the work list within max_items: one partition per row
        return -(-max_length // 64) * 64
    return candidates[best.value]


def choose_split(
    n_rows: int,
    num_kv_heads: int,
    group: int,
    max_length: int,
    total_length: int | None = None,
    row_lengths: "tuple[int, ...] | np.ndarray | None" = None,
    kv_bytes: int = 2,
    min_size: int = 0,
    max_items: int = 0,
    v1: bool = True,
) -> Split:
    """Pick v1 or v2 and the partition size from the step's shape.

    Every candidate partition size is scored with :func:`schedule_makespan` and
    the fastest wins; a single partition per row is v1. An eagerly planned step
    is scored on its rows' lengths; graph metadata, where only the table width
    is fixed, on ``n_rows`` rows of ``max_length``. The choice is cached under a
    coarse signature of the lengths (row count, longest row to a power of two,
    total to 4 significant bits), which successive decode steps -- every length
    one longer than the step before -- keep hitting. ``kv_bytes`` is the cache's bytes
    per element (2, or 1 for fp8), which sets the modelled workgroup cost; ``min_size``
    leaves out smaller partition sizes, and ``max_items`` sizes whose work list over the
    rows with context is longer (a graph replay's grid and scratch are sized for both).
    An eagerly planned step also scores v1 with each context split among 1-8 waves
    (:func:`v1_makespan`) and takes it, with its wave count, when it models faster than the
    best v2 launch (``v1`` False leaves that out: the best v2 launch).
    """
    del total_length
    if max_length <= 0:
        return Split(0, 0)
    virtual_heads = num_kv_heads * head_chunks(group)
    groups = -(-virtual_heads // 8)
    if row_lengths is not None:
        lengths = np.asarray(row_lengths, dtype=np.int64)
        lengths = lengths[lengths > 0]
    else:
        lengths = np.full(n_rows, max_length, dtype=np.int64)
    total = int(lengths.sum())
    # The total to 4 significant bits, the longest row to a power of two, the row count.
    top = max(total.bit_length() - 4, 0)
    key = (virtual_heads, kv_bytes, min_size, max_items, v1, lengths.size, max_length.bit_length(), total >> top,
           top)
    found = _split_cache.get(key)
    if found is None:
        if len(_split_cache) > 4096:
            _split_cache.clear()
        size = _best_size(lengths, max_length, groups, kv_bytes, min_size, max_items)
        waves = 0
        # v1 with a wave split, scored by the same schedule: eager plans only (a graph replay's
        # launch is the staged v2 split, sized by min_size and max_items)
        if v1 and not min_size and not max_items and lengths.size:
            v2 = schedule_makespan(lengths, size, groups, WORKGROUP_COSTS[kv_bytes]) if size < max_length else None
            best = None
            for ws in (V1_WAVE_SPLITS if kv_bytes != 4 else (1,)):  # fp32: one wave per head
                t = v1_makespan(lengths, ws, virtual_heads, V1_WORKGROUP_COSTS[kv_bytes])
                if best is None or t < best[0]:
                    best = (t, ws)
            if v2 is None or best[0] < v2:
                size, waves = 0, best[1]  # v1 (the key covers other lengths: no size is kept)
        found = (size, waves)
        _split_cache[key] = found
    size, waves = found
    if not size or max_length <= size:
        return Split(0, 0, waves)
    return Split(size, -(-max_length // size))


def choose_partitions(n_rows: int, num_kv_heads: int, group: int, max_length: int, kv_bytes: int = 2) -> int:
    """Partitions for a step known only by its longest context, as graph metadata is (0 = v1)."""
    return choose_split(n_rows, num_kv_heads, group, max_length, kv_bytes=kv_bytes).partitions


#: Multi-row workgroups one compute unit runs at a time (the kernel's launch bounds).
PREFILL_WORKGROUPS_PER_CU = 2
#: Positions one multi-row workgroup folds per step, the time of a step by head width and waves
#: per pair group (0: the double tile, an 8-wave workgroup, one per compute unit; 1, 2, 4: the
#: full tile, a half and a quarter), and each workgroup's fixed time by tile (its prologue,
#: and the fold of a group's waves at the end); with the streaming rate, the partials' rate and
#: the reduce launch below, fitted to a sweep of 52 step shapes (head widths 64, 128 and 256,
#: 3 to 8 key/value heads, GQA 3, 4 and 8, 1 to 4096 rows per request over 512 to 8192
#: positions, decode rows beside a chunk) x every tile x 5 partition sizes on MI355X: the
#: library's choice averaged 1.2% and at worst 14% above the fastest measured launch (over fp8
#: caches, 8 shapes: 1.0% and 5.8%), against 4.2% and 28% with the constants fitted before to
#: head width 128 alone.
PREFILL_CHUNK = 64
PREFILL_CHUNK_US = {
    (64, 1): 0.99, (64, 2): 0.81, (64, 4): 0.60,
    (128, 0): 2.05, (128, 1): 2.38, (128, 2): 1.68, (128, 4): 1.40,
    (256, 0): 2.84, (256, 1): 2.93, (256, 2): 2.56, (256, 4): 3.81,
}
PREFILL_WORKGROUP_US = {0: 4.56, 1: 3.98, 2: 2.09, 4: 2.70}
#: How much faster a smaller tile must model to be chosen over a larger one.
PREFILL_SMALLER_TILE_MARGIN = 0.03
#: Rate (bytes per us) at which a launch streams K and V it reads once (about 7 TB/s).
PREFILL_STREAM_BYTES_PER_US = 7.0e6
#: Rate (bytes per us) at which partials are written and read back, and the reduce launch.
PREFILL_PARTIALS_BYTES_PER_US = 5.4e6
PREFILL_REDUCE_US = 9.9
#: Whether steps whose requests' rows all fit one window tile run on the decode kernel's window
#: launch (``ayk_paged_attention_windows``) rather than the multi-row kernel.
WINDOWS = True
#: Partition sizes a multi-row launch chooses from.
PREFILL_PARTITION_CANDIDATES = (128, 256, 512, 1024, 2048, 4096)


def _dispatch_makespan(steps: "list[float] | np.ndarray", slots: int) -> float:
    """Finish time of workgroups of these durations started longest first, each in the first of
    ``slots`` identical slots to free up (the library's host code, ``ayk_dispatch_makespan``)."""
    steps = np.ascontiguousarray(steps, dtype=np.float64).reshape(-1)
    out = ctypes.c_double()
    rc = _lib.lib().ayk_dispatch_makespan(steps.ctypes.data, steps.size, slots, ctypes.byref(out))
    if rc != 0:
        raise BackendError(f"attention._dispatch_makespan: {steps.size} durations over {slots} slots",
                           context={"op": "attention._dispatch_makespan"})
    return out.value


def prefill_model_us(group_lengths: list[int], row_lengths: tuple[int, ...] | list[int], num_kv_heads: int,
                     num_heads: int, head_dim: int, partition_size: int, waves_per_group: int = 1,
                     context_bytes: int = 0) -> float:
    """Modelled time (us) of a multi-row launch.

    Its workgroups (one per tile, partition and key/value head) start longest first, each
    in the first of the GPU's workgroup slots to free up (:func:`_dispatch_makespan`), taking
    :data:`PREFILL_CHUNK_US` per 64-position chunk plus :data:`PREFILL_WORKGROUP_US`, but the
    launch takes no less than streaming the requests' K and V once (``context_bytes``).
    With partitions, writing and reading back the partials of rows that span several and
    the reduce launch are added.
    """
    slots = COMPUTE_UNITS * (PREFILL_WORKGROUPS_PER_CU if waves_per_group else 1)
    chunk_us = PREFILL_CHUNK_US[(head_dim, waves_per_group)]
    fixed_us = PREFILL_WORKGROUP_US[waves_per_group]
    lengths = np.asarray(group_lengths, dtype=np.int64)
    if partition_size:
        # each length's full partitions, its remainder, and one empty piece for a length of 0
        full, rest = np.divmod(lengths, partition_size)
        chunks = np.concatenate((np.full(int(full.sum()), -(-partition_size // PREFILL_CHUNK), dtype=np.int64),
                                 -(-rest[rest > 0] // PREFILL_CHUNK), np.zeros(int((lengths == 0).sum()), np.int64)))
    else:
        chunks = -(-lengths // PREFILL_CHUNK)
    steps = np.repeat(chunks * chunk_us + fixed_us, num_kv_heads)
    t = _dispatch_makespan(steps, slots)
    t = max(t, context_bytes / PREFILL_STREAM_BYTES_PER_US)
    if partition_size:
        rows = np.asarray(row_lengths, dtype=np.int64)
        parts = int((-(-rows[rows > partition_size] // partition_size)).sum())
        t += 2 * parts * num_heads * (head_dim + 2) * 4 / PREFILL_PARTIALS_BYTES_PER_US + PREFILL_REDUCE_US
    return t


def choose_prefill_partition(group_lengths: list[int], row_lengths: tuple[int, ...] | list[int],
                             num_kv_heads: int, num_heads: int, head_dim: int, waves_per_group: int = 1,
                             context_bytes: int = 0) -> int:
    """Partition size of a multi-row launch (0: none) for groups of rows with these context
    lengths: the candidate with the smallest :func:`prefill_model_us`, considered only when
    the unsplit grid fills at most two rounds of the GPU (beyond that the partials' traffic
    outweighs any balance gained)."""
    slots = COMPUTE_UNITS * (PREFILL_WORKGROUPS_PER_CU if waves_per_group else 1)
    group_lengths = np.asarray(group_lengths, dtype=np.int64)
    if not group_lengths.size or group_lengths.size * num_kv_heads >= 2 * slots:
        return 0
    longest = int(group_lengths.max())
    model = functools.partial(prefill_model_us, group_lengths, row_lengths, num_kv_heads, num_heads, head_dim,
                              waves_per_group=waves_per_group, context_bytes=context_bytes)
    best = (model(0), 0)
    for size in PREFILL_PARTITION_CANDIDATES:
        if size >= longest:
            break
        if int((-(-group_lengths // size)).sum()) * num_kv_heads > 8 * slots:
            continue  # more than 8 rounds of partitions: their partials outweigh any balance
        t = model(size)
        if t < best[0]:
            best = (t, size)
    return best[1]


_workspaces: dict[torch.device, torch.Tensor] = {}
# Buffers a larger one replaced: a captured graph may still point at them, so they are never freed.
_retired: list[torch.Tensor] = []


#: The stream (raw handle) whose calls last used each device's shared scratch and counters.
_scratch_streams: dict[torch.device, int] = {}


def _order_scratch(device: torch.device, stream: int, capture: bool) -> None:
    """Order this call's use of the device's shared v2 scratch and arrival counters after
    every use already queued on another stream: an event recorded now on that stream, which
    this one waits for (one per change of stream; nothing when the stream stays the same).
    A capture is ordered after its stream's earlier work by the capture itself; replays of a
    captured graph must not overlap calls on another stream (they share the buffers)."""
    last = _scratch_streams.get(device)
    if capture:
        return
    if last is not None and last != stream:
        event = torch.cuda.Event()
        event.record(torch.cuda.ExternalStream(last, device=device))
        torch.cuda.ExternalStream(stream, device=device).wait_event(event)
    _scratch_streams[device] = stream


def _workspace(op: str, device: torch.device, nbytes: int, capture: bool, stream: int) -> torch.Tensor:
    _order_scratch(device, stream, capture)
    found = _workspaces.get(device)
    if found is not None and found.numel() >= nbytes:
        return found
    if capture:
        raise BackendError(
            f"{op}: the v2 scratch for this step ({nbytes} bytes) is larger than the one "
            "allocated so far; run the step once eagerly before capturing it",
            context={"op": op},
        )
    size = max(nbytes, 2 * found.numel() if found is not None else 0, 1 << 20)
    with torch.inference_mode(False):
        fresh = torch.empty(size, dtype=torch.uint8, device=device)
    if found is not None:
        _retired.append(found)
    _workspaces[device] = fresh
    return fresh


_counters: dict[torch.device, torch.Tensor] = {}


def _arrivals(op: str, device: torch.device, words: int, capture: bool) -> torch.Tensor:
    """The v2 arrival counters of ``device``: zero-filled once, and every v2 call
    leaves them zero again, so they are shared by all calls on the device's stream."""
    found = _counters.get(device)
    if found is not None and found.numel() >= words:
        return found
    if capture:
        raise BackendError(
            f"{op}: the v2 arrival counters for this step ({words} words) outnumber the ones "
            "allocated so far; run the step once eagerly before capturing it",
            context={"op": op},
        )
    size = max(words, 2 * found.numel() if found is not None else 0, 1 << 14)
    with torch.inference_mode(False):
        fresh = torch.zeros(size, dtype=torch.int32, device=device)
    if found is not None:
        _retired.append(found)
    _counters[device] = fresh
    return fresh


def _call(op: str, fn, args: tuple, stream: int, device: torch.device, scratch: bool,
          record: "_fastpath.Recorder | None") -> None:
    """Make one library call (``stream`` last), and hand it to ``record`` for replays."""
    if record is not None:
        record(op, fn, args, device, scratch)
    _lib.check(op, fn(*args, stream))


def attend(
    q: torch.Tensor,
    buffers: KVBuffers,
    meta: AttentionMetadata,
    out: torch.Tensor,
    *,
    scale: float,
) -> None:
    """Write every query row's attention output into ``out`` (reference ``attention.py:167-234``).

    The first call with a combination of q, out, buffers and step metadata is checked in full;
    its library call is recorded in the step's plan, and later calls with the same buffers and
    metadata and with q and out at the same addresses, shapes, strides and dtype (the engine's
    per-layer tensors, every layer of a step) replay it on the current stream.
    """
    cache = getattr(meta.plan, "launches", None)
    if cache is None:
        attend_with(q, buffers, meta, out, scale=scale, partitions=None)
        return
    key = ("attend", id(buffers), id(meta), scale, _fastpath.signature((q, out, buffers.k, buffers.v)))
    found = _fastpath.lookup(cache, key)
    if found is not None:
        stream = stream_handle(found.device)
        if found.scratch:
            _order_scratch(found.device, stream, capturing(q))
        _fastpath.run(found, stream)
        return
    record = _fastpath.Recorder()
    attend_with(q, buffers, meta, out, scale=scale, partitions=None, _record=record)
    _fastpath.remember(cache, key, (buffers, meta), record)


def attend_with(
    q: torch.Tensor,
    buffers: KVBuffers,
    meta: AttentionMetadata,
    out: torch.Tensor,
    *,
    scale: float,
    partitions: int | None,
    qk: str | None = None,
    partition_size: int | None = None,
    partials_only: bool = False,
    prefill: bool | None = None,
    merge: str | None = None,
    tile_pairs: int | None = None,
    window: bool | None = None,
    waves: int | None = None,
    _record: "_fastpath.Recorder | None" = None,
) -> None:
    """:func:`attend` with the launch chosen by the caller.

    ``partitions`` 0 runs v1, a positive count runs v2 over that many partitions
    of ``partition_size`` (default :data:`PARTITION_SIZE`; together they must
    cover the step's longest context), ``None`` lets :func:`choose_split` decide. ``qk`` forces the q.k implementation,
    ``"dpp"`` (VALU dot2 + DPP butterflies) or ``"mfma"`` (matrix cores); ``None``
    lets the library pick. ``partials_only`` (v2) runs the partition kernel alone
    and leaves the rows of several partitions unwritten; ``merge`` (v2) forces
    where the partitions are merged, ``"in-kernel"`` (the partition kernel's
    last workgroup of a row) or ``"reduce-kernel"`` (a second launch); ``None``
    lets the library pick. For the multi-row kernel (``prefill``: ``True`` forces it,
    ``False`` the decode kernels, ``None`` lets the row count decide) ``partitions`` 0
    covers each tile's context in one workgroup, ``partition_size`` splits it into
    partitions of that size (a multiple of 64) merged by the reduce kernel, and ``None``
    for both lets :func:`choose_prefill_partition` decide; ``tile_pairs`` forces the tile
    capacity (:data:`PREFILL_PAIRS`, a half or a quarter of it, or twice it at head widths 128 and
    256, an 8-wave workgroup; ``None``:
    :meth:`HipAttentionPlan.prefill_launch`). ``waves`` (1, 2, 4 or 8) forces how many
    waves share each (row, key/value head)'s context (v1) or partition (v2) (``None``: the
    split model's choice, else the library's).
    Benchmarks and tests use them to time and check every kernel on one step.
    """
    op = "attention.attend"
    require_buffers(op, buffers)
    step = meta.plan
    table = meta.block_table
    if not isinstance(step, (HipAttentionPlan, HipGraphPlan)) or not isinstance(table, torch.Tensor):
        raise BackendError(
            f"{op}: this step was planned by another backend; plan it with the same ops",
            context={"op": op, "argument": "meta"},
        )
    if meta.block_size != buffers.block_size:
        raise BackendError(
            f"{op}: the step was planned for blocks of {meta.block_size} positions "
            f"but the cache has blocks of {buffers.block_size}",
            context={"op": op, "argument": "meta"},
        )
    heads = q.shape[1] if q.ndim == 3 else 0
    n_rows = meta.request_of_row.shape[0]
    require_like(op, "q", q, (n_rows, heads, buffers.head_dim), compute_dtype(op, "q", q, buffers))
    require_like(op, "out", out, q.shape, q.dtype)
    kv_heads = buffers.num_kv_heads
    if heads == 0 or heads % kv_heads:
        raise BackendError(
            f"{op}: q has {heads} heads, which is not a positive multiple of the cache's "
            f"{kv_heads} key/value heads",
            context={"op": op, "argument": "q"},
        )
    if buffers.head_dim not in HEAD_DIMS:
        raise BackendError(
            f"{op}: the hip kernels are built for head widths {sorted(HEAD_DIMS)}, "
            f"not {buffers.head_dim}",
            context={"op": op, "argument": "buffers"},
        )
    block_size = buffers.block_size
    device = buffers.k.device
    for name, tensor in (
        ("q", q),
        ("out", out),
        ("meta.kv_lengths", meta.kv_lengths),
        ("meta.block_table", table),
        ("meta.request_of_row", meta.request_of_row),
        ("meta.positions", meta.positions),
    ):
        require_device(op, name, tensor, device)
    decode = meta.mode == ForwardMode.DECODE
    if isinstance(step, HipGraphPlan):
        if not decode:
            raise BackendError(f"{op}: graph metadata must be a DECODE step", context={"op": op})
        max_length, row_lengths = step.max_blocks * block_size, None
    else:
        max_length, row_lengths = step.max_length, step.row_lengths
    if n_rows == 0:
        return
    if table.dtype != torch.int32 or not table.is_contiguous() or table.ndim != 2:
        raise BackendError(f"{op}: meta.block_table must be a contiguous int32 [B, max_blocks] tensor")

    lib = _lib.lib()
    stream = stream_handle(device)
    if q.dtype == torch.float32:
        # fp32 models run on the decode kernel for fp32, each row of a multi-row step on its own
        if prefill or window or (qk is not None) or (waves not in (None, 1)) or merge == "in-kernel":
            raise BackendError(f"{op}: fp32 runs one launch shape: the per-row decode kernel, one wave per "
                               "head, partitions merged by the reduce kernel", context={"op": op})
        prefill = False
    if prefill is None:
        prefill = not decode and _wants_prefill_kernel(step)
    if prefill and isinstance(step, HipAttentionPlan):
        group = heads // kv_heads
        if window is None:
            window = tile_pairs is None and WINDOWS and step.window_pairs(group) > 0
        if window:
            _attend_windows(op, q, buffers, meta, out, step, scale, partitions, partition_size, stream, _record)
            return
    if prefill:
        if not isinstance(step, HipAttentionPlan):
            raise BackendError(f"{op}: the multi-row kernel needs a planned step", context={"op": op})
        pairs = tile_pairs or step.prefill_launch(kv_heads, heads // kv_heads, buffers.head_dim,
                                                  buffers.k.element_size())[0]
        if heads // kv_heads > pairs:
            raise BackendError(
                f"{op}: {heads // kv_heads} query heads per key/value head exceed the multi-row "
                f"kernel's tile of {pairs}",
                context={"op": op, "argument": "q"},
            )
        group = heads // kv_heads
        kv_bytes = buffers.k.element_size()
        if partitions == 0:
            size = 0
        elif partition_size is not None:
            size = partition_size
        else:
            size = step.prefill_split(kv_heads, group, pairs, buffers.head_dim, kv_bytes)
        tiles = step.prefill_tiles(group, pairs, size, device, capturing(q))
        scratch, nbytes = None, 0
        if size:
            max_partitions = -(-table.shape[1] * block_size // size)
            nbytes = lib.ayk_paged_attention_v2_workspace_bytes(n_rows, heads, buffers.head_dim, max_partitions)
        if q.dtype == torch.bfloat16 and _kv_code(buffers, q.dtype) == _DTYPE_CODES[torch.bfloat16]:
            # one int32 per workgroup after the partials: the fp16 values pass hands a workgroup
            # whose values fp16 cannot hold to the bf16 pass through it
            nbytes = -(-nbytes // 16) * 16 + 4 * (tiles.numel() // 4) * kv_heads
        if nbytes:
            scratch = _workspace(op, device, nbytes, capturing(q), stream)
        _call(op, lib.ayk_paged_prefill, (
            out.data_ptr(), q.data_ptr(), buffers.k.data_ptr(), buffers.v.data_ptr(), table.data_ptr(),
            table.stride(0), meta.kv_lengths.data_ptr(), meta.request_of_row.data_ptr(),
            meta.positions.data_ptr(), tiles.data_ptr(), tiles.numel() // 4, pairs, n_rows, heads, kv_heads,
            buffers.head_dim, buffers.num_blocks, block_size, table.shape[1],
            _LAYOUT_CODES[KVLayoutKind(buffers.layout)], _DTYPE_CODES[q.dtype], _kv_code(buffers, q.dtype),
            float(scale), *codec_scales(buffers.codec), size, scratch.data_ptr() if scratch is not None else 0,
            scratch.numel() if scratch is not None else 0,
        ), stream, device, scratch is not None, _record)
        return
    # Decode rows need no per-row indirection: row n is request n and sees its whole context.
    row_request = 0 if decode else meta.request_of_row.data_ptr()
    row_position = 0 if decode else meta.positions.data_ptr()
    group = heads // kv_heads
    common = (
        out.data_ptr(),
        q.data_ptr(),
        buffers.k.data_ptr(),
        buffers.v.data_ptr(),
        table.data_ptr(),
        table.stride(0),
        meta.kv_lengths.data_ptr(),
        row_request,
        row_position,
        n_rows,
        heads,
        kv_heads,
        buffers.head_dim,
        buffers.num_blocks,
        block_size,
        table.shape[1],
        _LAYOUT_CODES[KVLayoutKind(buffers.layout)],
        _DTYPE_CODES[q.dtype],
        _kv_code(buffers, q.dtype),
        float(scale),
        *codec_scales(buffers.codec),
    )
    staged = None
    if partitions is None:
        kv_bytes = buffers.k.element_size()
        if isinstance(step, HipAttentionPlan):
            split = step.split_for(kv_heads, group, kv_bytes)
        else:
            if not step.head_shape:
                step.head_shape.extend((kv_heads, group, kv_bytes))
                if step.staged_shape and step.staged_shape != step.head_shape and not capturing(q):
                    # the last update scored a guessed head shape: re-stage its step's split
                    used = _stage_split(step, step.kv_lengths.numpy(), block_size)
                    step.staged[:used].copy_(step.staged_host[:used], non_blocking=True)
            # v2 over the staged split (rows of one partition write their output directly),
            # or v1 when the table holds one partition at most
            split = Split(0, 0)
            if step.partitions > 1:
                staged = step.staged
                split = Split(step.min_size, step.partitions)
        partitions, partition_size = split.partitions, split.partition_size
        # a forced DPP q.k streams each head's context in one wave
        waves = waves or (split.waves if qk != "dpp" else None) or None
    partition_size = partition_size or PARTITION_SIZE
    if partitions and partitions * partition_size < max_length:
        raise BackendError(
            f"{op}: {partitions} partitions of {partition_size} do not cover {max_length} positions",
            context={"op": op},
        )
    flags = _QK_FLAGS[qk] | (PARTIALS_ONLY if partials_only else 0) | _MERGE_FLAGS[merge]
    if partitions == 0:
        _call(op, lib.ayk_paged_attention_v1, (*common, flags | _WAVE_FLAGS[waves]), stream, device, False,
              _record)
        return
    if staged is not None:  # the rows' partials packed into one slot per work item
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(step.capacity, heads, buffers.head_dim, 1)
    else:
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(n_rows, heads, buffers.head_dim, partitions)
    scratch = _workspace(op, device, nbytes, capturing(q), stream)
    arrivals = _arrivals(op, device, n_rows * heads, capturing(q))
    # A planned step runs only the partitions that hold tokens, longest first. Graph
    # metadata's launch reads the same list and its partition size from the staged
    # buffer, over a grid of the bucket's capacity; forced launches on graph metadata
    # keep the dense grid.
    work, n_work = 0, 0
    if staged is not None:
        work, n_work = staged.data_ptr() + 4 * step.work_offset, step.capacity
    elif isinstance(step, HipAttentionPlan) and not capturing(q):
        items = step.work_items(partition_size, device)
        work, n_work = items.data_ptr(), items.numel() // 2
    _call(op, lib.ayk_paged_attention_v2, (
        *common, partition_size, partitions, work, n_work, staged.data_ptr() if staged is not None else 0,
        scratch.data_ptr(), scratch.numel(), arrivals.data_ptr(), flags | _WAVE_FLAGS[waves],
    ), stream, device, True, _record)


def _attend_windows(op: str, q: torch.Tensor, buffers: KVBuffers, meta: AttentionMetadata, out: torch.Tensor,
                    step: HipAttentionPlan, scale: float, partitions: int | None, partition_size: int | None,
                    stream: int, record: "_fastpath.Recorder | None" = None) -> None:
    """A step of few rows per request on the decode kernel (``ayk_paged_attention_windows``):
    one tile per request, its (row, query head) pairs the kernel's 16 matrix-core columns."""
    heads, kv_heads = q.shape[1], buffers.num_kv_heads
    group = heads // kv_heads
    pairs = step.window_pairs(group)
    if not pairs:
        raise BackendError(
            f"{op}: a window tile holds 16 (row, query head) pairs; this step has a request of more "
            f"rows than {16 // group if group <= 16 else 0} at {group} query heads per key/value head",
            context={"op": op, "argument": "meta"},
        )
    kv_bytes = buffers.k.element_size()
    if partitions == 0:
        size = 0
    elif partition_size is not None:
        size = partition_size
    else:
        size = step.window_split(kv_heads, group, kv_bytes)
    device = buffers.k.device
    tiles = step.prefill_tiles(group, pairs, size, device, capturing(q))
    table = meta.block_table
    n_rows = meta.request_of_row.shape[0]
    lib = _lib.lib()
    scratch, nbytes = None, 0
    if size:
        max_partitions = -(-table.shape[1] * buffers.block_size // size)
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(n_rows, heads, buffers.head_dim, max_partitions)
        scratch = _workspace(op, device, nbytes, capturing(q), stream)
    _call(op, lib.ayk_paged_attention_windows, (
        out.data_ptr(), q.data_ptr(), buffers.k.data_ptr(), buffers.v.data_ptr(), table.data_ptr(),
        table.stride(0), meta.kv_lengths.data_ptr(), meta.request_of_row.data_ptr(), meta.positions.data_ptr(),
        tiles.data_ptr(), tiles.numel() // 4, n_rows, heads, kv_heads, buffers.head_dim, buffers.num_blocks,
        buffers.block_size, table.shape[1], _LAYOUT_CODES[KVLayoutKind(buffers.layout)], _DTYPE_CODES[q.dtype],
        _kv_code(buffers, q.dtype), float(scale), *codec_scales(buffers.codec), size,
        scratch.data_ptr() if scratch is not None else 0,
        scratch.numel() if scratch is not None else 0,
    ), stream, device, scratch is not None, record)


def graph_metadata(
    num_requests: int, max_blocks: int, block_size: int, device: torch.device
) -> AttentionMetadata:
    """Allocate the fixed metadata of a decode bucket (reference ``attention.py:274-305``)."""
    if num_requests < 1 or max_blocks < 1 or block_size < 1:
        raise BackendError(
            "attention.graph_metadata: num_requests, max_blocks and block_size must be "
            f"positive, got {num_requests}, {max_blocks} and {block_size}",
            context={"op": "attention.graph_metadata"},
        )
    target = torch.device(device)
    # Replays run v2 over partitions of at least min_size (64 positions, or the share of the
    # table width that keeps a row within GRAPH_MAX_PARTITIONS of them) and a grid of
    # `capacity` work items: GRAPH_MAX_ITEMS, or one per row for a larger bucket.
    max_length = max_blocks * block_size
    min_size = max(GRAPH_MIN_PARTITION, -(-max_length // (64 * GRAPH_MAX_PARTITIONS)) * 64)
    capacity = max(num_requests, GRAPH_MAX_ITEMS)
    work = 2 + num_requests
    # The records a replay reads at fixed addresses (a decode step: one row per request, row n
    # is request n), then the staged split, laid out in one device buffer with a pinned host
    # twin that update_graph_metadata fills, so each update is one asynchronous copy (of
    # everything up to the end of the step's work list).
    records = {
        "block_table": ((num_requests, max_blocks), torch.int32),
        "positions": ((num_requests,), torch.int32),
        "slot_mapping": ((num_requests,), torch.int64),
        "kv_lengths": ((num_requests,), torch.int32),
        "staged": ((work + 2 * capacity,), torch.int32),
    }
    offsets, total = {}, 0
    for name, (shape, dtype) in records.items():
        offsets[name] = total
        nbytes = math.prod(shape) * torch.tensor([], dtype=dtype).element_size()
        total += -(-nbytes // 256) * 256
    host_all = torch.zeros(total, dtype=torch.uint8, pin_memory=target.type == "cuda")
    device_all = torch.zeros(total, dtype=torch.uint8, device=target)

    def view(buffer: torch.Tensor, name: str) -> torch.Tensor:
        shape, dtype = records[name]
        nbytes = math.prod(shape) * torch.tensor([], dtype=dtype).element_size()
        return buffer[offsets[name]:offsets[name] + nbytes].view(dtype).view(shape)

    fixed = {name: view(device_all, name) for name in records if name != "staged"}
    twins = {name: view(host_all, name) for name in records if name != "staged"}
    # Until the first update every row is one item.
    staged_host = view(host_all, "staged")
    staged_host[0], staged_host[1] = min_size, num_requests
    staged_host[work:work + 2 * num_requests:2] = torch.arange(num_requests, dtype=torch.int32)
    staged = view(device_all, "staged")
    staged.copy_(staged_host)
    staging = HipGraphPlan(
        **twins,
        max_blocks=max_blocks,
        staged_host=staged_host,
        staged=staged,
        min_size=min_size,
        partitions=-(-max_length // min_size),
        capacity=capacity,
        host_all=host_all,
        device_all=device_all,
        staged_offset=offsets["staged"],
    )
    return AttentionMetadata(
        mode=ForwardMode.DECODE,
        block_size=block_size,
        rows_per_request=torch.ones(num_requests, dtype=torch.int32, device=target),
        request_of_row=torch.arange(num_requests, dtype=torch.int32, device=target),
        plan=staging,
        **fixed,
    )


def _require_host_ints(op: str, name: str, tensor: torch.Tensor, shape: tuple[int, ...]) -> np.ndarray:
    """``tensor`` as a numpy view, if it is an int32 CPU tensor of ``shape`` (the message is the
    reference's, ``torch/attention.py:341-352``)."""
    if tuple(tensor.shape) != shape or tensor.dtype != torch.int32 or tensor.device.type != "cpu":
        raise BackendError(
            f"{op}: {name} must be an int32 CPU tensor of shape {list(shape)}, got "
            f"{tensor.dtype} {list(tensor.shape)} on {tensor.device}",
            context={"op": op, "argument": name},
        )
    return tensor.numpy()


def update_graph_metadata(
    meta: AttentionMetadata, kv_lengths: torch.Tensor, block_rows: torch.Tensor
) -> None:
    """Write the next decode step into ``meta`` without waiting on the device.

    The contract of the reference's update (``attention.py:308-374``): int32 CPU inputs,
    every length within the table, each request's newest token at position
    ``length - 1`` and its slot read from the table (a padding request, length 0,
    gets position and slot 0). Everything is computed on the host into the pinned
    staging, together with the step's v2 split, and copied to the fixed device
    records with asynchronous copies on the current stream.
    """
    op = "attention.update_graph_metadata"
    staging = meta.plan
    table = meta.block_table
    if not isinstance(staging, HipGraphPlan) or not isinstance(table, torch.Tensor):
        raise BackendError(
            f"{op}: meta was not made by this backend's graph_metadata",
            context={"op": op, "argument": "meta"},
        )
    requests, width = staging.block_table.shape
    lens = _require_host_ints(op, "kv_lengths", kv_lengths, (requests,)).astype(np.int64)
    rows = _require_host_ints(op, "block_rows", block_rows, (requests, width))
    block_size = meta.block_size
    limit = width * block_size
    if lens.size and (int(lens.min()) < 0 or int(lens.max()) > limit):
        raise BackendError(
            f"{op}: every length must be in [0, {limit}] for a table of {width} blocks of {block_size}",
            context={"op": op, "argument": "kv_lengths"},
        )
    newest = np.maximum(lens - 1, 0)
    block = rows[np.arange(requests), newest // block_size].astype(np.int64)
    staging.positions.numpy()[:] = newest
    staging.slot_mapping.numpy()[:] = np.where(lens > 0, block * block_size + newest % block_size, 0)
    staging.kv_lengths.numpy()[:] = lens
    staging.block_table.numpy()[:] = rows
    used = _stage_split(staging, lens, block_size)
    end = staging.staged_offset + 4 * used
    staging.device_all[:end].copy_(staging.host_all[:end], non_blocking=True)


def _stage_split(staging: HipGraphPlan, lengths: np.ndarray, block_size: int) -> int:
    """Fill ``staging.staged_host`` with this step's partition size, the rows' first partial
    slots and the work list (the eager plan's choice among sizes of ``staging.min_size`` up
    whose list fits the capacity); returns the int32 words used."""
    kv_heads, group, kv_bytes = staging.head_shape or (8, 1, 2)
    staging.staged_shape[:] = [kv_heads, group, kv_bytes]
    lengths = lengths.astype(np.int64)
    longest = int(lengths.max()) if lengths.size else 0
    empty = int((lengths == 0).sum())
    split = choose_split(lengths.size, kv_heads, group, max(longest, 1), row_lengths=lengths,
                         kv_bytes=kv_bytes, min_size=staging.min_size, max_items=staging.capacity - empty)
    # one partition per row when the model prefers v1
    size = split.partition_size or max(staging.min_size, -(-longest // 64) * 64)
    items = work_list(lengths, size)
    if items.size > 2 * staging.capacity:  # cannot happen for sizes the model returns; stay safe
        size = max(staging.min_size, -(-longest // 64) * 64)
        items = work_list(lengths, size)
    counts = -(-lengths // size)
    assert items.size <= 2 * staging.capacity and int(counts.max(initial=0)) <= staging.partitions
    host = staging.staged_host.numpy()
    work = staging.work_offset
    host[0], host[1] = size, items.size // 2
    host[2:work] = np.cumsum(counts) - counts  # each row's first partial slot
    host[work:work + items.size] = items
    return work + items.size


