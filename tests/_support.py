"""Builders shared by the tests: small paged scenarios with NaN-poisoned caches.

Modelled on the reference's test builder (``tests/ops/test_attention_contract.py:72-141``):
each request gets random keys/values at its positions, its blocks are drawn
from a seeded permutation of the pool (never block 0), and every slot nobody
wrote holds NaN, so reading block 0, an unused block or the unwritten tail of a
block shows up as NaN. Values are drawn in float32 and rounded to the cache
dtype, and kept both as raw 16-bit words (for the device) and widened back to
float32 (for the oracle), so both sides see identical inputs.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import paged
from oracle.numerics import bits_to_f32, f32_to_bits

NAN_BITS = {"bf16": 0x7FC0, "fp16": 0x7E00}


@dataclass
class Scenario:
    dtype: str
    layout: str
    block_size: int
    heads: int
    kv_heads: int
    head_dim: int
    rows: list[int]
    lengths: list[int]
    mode: str
    table: np.ndarray  # [B, max_blocks] int64
    q_bits: np.ndarray  # [N, H, D] uint16
    k_bits: np.ndarray  # cache words in the scenario's layout
    v_bits: np.ndarray
    plan: dict[str, np.ndarray]
    scale: float

    @property
    def q(self) -> np.ndarray:
        return bits_to_f32(self.q_bits, self.dtype)

    @property
    def k(self) -> np.ndarray:
        return bits_to_f32(self.k_bits, self.dtype)

    @property
    def v(self) -> np.ndarray:
        return bits_to_f32(self.v_bits, self.dtype)

    def expected(self, precision: type = np.float64, k: np.ndarray | None = None,
                 v: np.ndarray | None = None) -> np.ndarray:
        """The oracle's output; ``k``/``v`` replace the cache values (e.g. decoded fp8 codes)."""
        decode = self.mode == "decode"
        return paged.attention(
            self.q,
            self.k if k is None else k,
            self.v if v is None else v,
            self.table,
            np.asarray(self.lengths),
            scale=self.scale,
            layout=self.layout,
            request_of_row=None if decode else self.plan["request_of_row"],
            positions=None if decode else self.plan["positions"],
            precision=precision,
        )


def build_scenario(
    steps: list[tuple[int, int]],
    *,
    dtype: str = "bf16",
    layout: str = "nhd",
    heads: int = 4,
    kv_heads: int = 2,
    head_dim: int = 64,
    block_size: int = 4,
    mode: str = "mixed",
    seed: int = 0,
    spare_blocks: int = 3,
    scale: float | None = None,
) -> Scenario:
    """A paged cache holding each request's context; ``steps`` is ``[(rows, length), ...]``."""
    rng = np.random.default_rng(seed)
    needed = [-(-length // block_size) for _, length in steps]
    num_blocks = 1 + sum(needed) + spare_blocks
    nhd_shape = (num_blocks, block_size, kv_heads, head_dim)
    k_nhd = np.full(nhd_shape, NAN_BITS[dtype], dtype=np.uint16)
    v_nhd = np.full(nhd_shape, NAN_BITS[dtype], dtype=np.uint16)
    free = list(rng.permutation(np.arange(1, num_blocks)))
    table = np.zeros((len(steps), max(needed, default=0) or 1), dtype=np.int64)
    for b, ((_, length), n) in enumerate(zip(steps, needed)):
        blocks = [int(free.pop()) for _ in range(n)]
        table[b, :n] = blocks
        ctx_k = f32_to_bits(rng.standard_normal((length, kv_heads, head_dim)).astype(np.float32), dtype)
        ctx_v = f32_to_bits(rng.standard_normal((length, kv_heads, head_dim)).astype(np.float32), dtype)
        for pos in range(length):
            k_nhd[blocks[pos // block_size], pos % block_size] = ctx_k[pos]
            v_nhd[blocks[pos // block_size], pos % block_size] = ctx_v[pos]
    rows = [r for r, _ in steps]
    lengths = [n for _, n in steps]
    q_bits = f32_to_bits(
        rng.standard_normal((sum(rows), heads, head_dim)).astype(np.float32), dtype
    )
    if layout == "hnd":
        k_bits = np.ascontiguousarray(k_nhd.transpose(0, 2, 1, 3))
        v_bits = np.ascontiguousarray(v_nhd.transpose(0, 2, 1, 3))
    else:
        k_bits, v_bits = k_nhd, v_nhd
    return Scenario(
        dtype=dtype,
        layout=layout,
        block_size=block_size,
        heads=heads,
        kv_heads=kv_heads,
        head_dim=head_dim,
        rows=rows,
        lengths=lengths,
        mode=mode,
        table=table,
        q_bits=q_bits,
        k_bits=k_bits,
        v_bits=v_bits,
        plan=paged.plan(mode, rows, lengths, table, block_size),
        scale=head_dim**-0.5 if scale is None else scale,
    )


def brute_force(s: Scenario) -> np.ndarray:
    """Pure-Python float64 attention, one row, head and position at a time (tiny inputs only)."""
    q, k, v = s.q.astype(np.float64), paged.nhd(s.k, s.layout), paged.nhd(s.v, s.layout)
    group = s.heads // s.kv_heads
    out = np.zeros(q.shape)
    row = 0
    for b, (count, length) in enumerate(zip(s.rows, s.lengths)):
        for j in range(count):
            if length:
                visible = length - count + j + 1
                for h in range(s.heads):
                    kvh = h // group
                    scores = []
                    for pos in range(visible):
                        blk, off = s.table[b, pos // s.block_size], pos % s.block_size
                        dot = 0.0
                        for d in range(s.head_dim):
                            dot += q[row, h, d] * float(k[blk, off, kvh, d])
                        scores.append(dot * s.scale)
                    top = max(scores)
                    weights = [np.exp(x - top) for x in scores]
                    total = sum(weights)
                    for pos in range(visible):
                        blk, off = s.table[b, pos // s.block_size], pos % s.block_size
                        for d in range(s.head_dim):
                            out[row, h, d] += weights[pos] / total * float(v[blk, off, kvh, d])
            row += 1
    return out


def oracle_rows(step, rows: list[int], precision: type = np.float64, chunk: int = 16) -> np.ndarray:
    """The oracle's output for decode rows ``rows`` of a ``workloads`` step.

    Rows are taken ``chunk`` at a time in order of length, each chunk with its table cut to
    the blocks its longest row reads: the oracle gathers a padded table per row, and on a
    ragged batch the full width would multiply its work (same semantics: what lies past a
    row's length is masked either way).
    """
    from ayaka_amd import workloads
    from oracle import paged

    sample = workloads.sample_rows(step, rows)
    bs = step.config.block_size
    order = np.argsort(sample["lengths"], kind="stable")
    out = np.zeros((len(rows), *sample["q"].shape[1:]), dtype=precision)
    for start in range(0, len(rows), chunk):
        pick = order[start:start + chunk]
        width = max(1, -(-int(sample["lengths"][pick].max()) // bs))
        out[pick] = paged.attention(sample["q"][pick], sample["k"], sample["v"], sample["table"][pick, :width],
                                    sample["lengths"][pick], scale=step.config.scale, precision=precision,
                                    chunk=chunk)
    return out


# --- the host launch model, stated in plain Python -------------------------------------------
# The library computes these in C++ (ayk_split_model, ayk_work_list); the tests check that its
# answers are these, on random and edge-case inputs.


def python_schedule_makespan(row_lengths, size: int, groups: int = 1, cost: int = 320,
                             compute_units: int = 256, xcds: int = 8) -> int:
    """Finish time of v2 over partitions of ``size``: work items longest first, each repeated
    ``groups`` times, dealt to XCD i mod ``xcds``; each XCD hands its next item to whichever
    of its units frees first; an item costs its positions plus ``cost``."""
    import heapq

    items: list[int] = []
    for length in row_lengths:
        if length <= 0:
            continue
        full, rest = divmod(int(length), size)
        items.extend([size] * full)
        if rest:
            items.append(rest)
    items.sort(reverse=True)
    items = [item for item in items for _ in range(groups)]
    loads = [[0] * (compute_units // xcds) for _ in range(xcds)]
    for index, item in enumerate(items):
        heap = loads[index % xcds]
        heapq.heapreplace(heap, heap[0] + item + cost)
    return max(max(heap) for heap in loads)


def python_work_list(row_lengths, partition_size: int) -> np.ndarray:
    """(row, partition) pairs holding tokens, longest partition first (ties by row, then
    partition), then partition 0 of each row without context; flattened int32."""
    entries = []
    for row, length in enumerate(row_lengths):
        length = int(length)
        if length <= 0:
            entries.append((0, row, 0))
            continue
        for part in range(-(-length // partition_size)):
            entries.append((-min(partition_size, length - part * partition_size), row, part))
    entries.sort()
    return np.array([x for _, row, part in entries for x in (row, part)], dtype=np.int32)
