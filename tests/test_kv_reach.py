"""Every K/V address the attention kernels form stays inside the cache (CPU, no GPU).

The library's host address walk (``ayk_debug_kv_reach_begin`` / ``_end``) runs an entry
point's checks and launch preparation as usual and then, instead of launching, enumerates every
K/V load of the prepared launch with the kernels' own loops and address arithmetic
(``csrc/kv_address.h``). These tests drive every attention entry point -- v1 and v2 on both q.k
kernels, v2 over a work list, a dense grid and a staged split, the window launch and the
multi-row kernel with each tile size, with and without partitions -- over small pools of every
head width, both codecs, both layouts and block sizes from 1 to 100, and assert:

* every load reads bytes inside the cache: ``0 <= lo`` and ``hi <= num_blocks * block bytes``;
* the reach is the one the step's tables imply, exactly: the lowest byte is the start of the
  lowest block a context uses, and a context that fills the pool's last block reaches its end
  (so a load computed in the wrong units -- elements for bytes -- or from a stale table index
  shows, not only a fault);
* every block-table entry read lies inside the table.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from ayaka_amd.hip import _lib
from ayaka_amd.hip import attention as hip_attention

FAKE = 1 << 40  # a stand-in device address for pointers the walk never dereferences
FLAG_DPP, FLAG_MFMA, FLAG_SEPARATE_REDUCE, FLAG_SINGLE_LAUNCH = 1, 2, 8, 16
FLAG_WAVES = {1: 32, 2: 64, 4: 128, 8: 256}


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


class Step:
    """A paged pool and the requests of one step: contexts of ``lengths``, each request's
    blocks drawn from the pool (block 0 never), the last request ending on a full block that
    is the pool's last one."""

    def __init__(self, rng: np.random.Generator, lengths: list[int], block_size: int, kv_heads: int,
                 head_dim: int, kv8: bool, layout: int, spare: int = 3, fp32: bool = False) -> None:
        self.fp32 = fp32
        self.lengths = np.asarray(lengths, dtype=np.int32)
        self.block_size, self.kv_heads, self.head_dim, self.kv8, self.layout = (block_size, kv_heads, head_dim,
                                                                                 kv8, layout)
        need = [-(-n // block_size) for n in lengths]
        self.num_blocks = 1 + sum(need) + spare
        free = list(rng.permutation(np.arange(1, self.num_blocks - 1)))
        width = max(max(need), 1) + int(rng.integers(0, 3))  # tables wider than any context
        self.table = np.zeros((len(lengths), width), dtype=np.int32)
        for r, n in enumerate(need):
            ids = [int(free.pop()) for _ in range(n)]
            if r == len(lengths) - 1 and n:
                ids[-1] = self.num_blocks - 1  # the pool's last block holds this request's end
            self.table[r, :n] = ids
        self.width = width
        elem = 1 if kv8 else 4 if fp32 else 2
        self.elem = elem
        self.block_bytes = block_size * kv_heads * head_dim * elem
        self.pool_bytes = self.num_blocks * self.block_bytes

    def expected_reach(self) -> tuple[int, int]:
        """(lowest byte, one past the highest byte) the step's contexts occupy."""
        lo, hi = None, 0
        elem = self.elem
        for r, n in enumerate(self.lengths):
            for b in range(-(-int(n) // self.block_size)):
                block = int(self.table[r, b])
                start = block * self.block_bytes
                lo = start if lo is None else min(lo, start)
                used = min(self.block_size, int(n) - b * self.block_size)  # positions read in the block
                if self.layout == 0:  # NHD: [token][head][dim]
                    end = start + used * self.kv_heads * self.head_dim * elem
                else:  # HND: [head][token][dim], the last head's rows end last
                    end = start + ((self.kv_heads - 1) * self.block_size + used) * self.head_dim * elem
                hi = max(hi, end)
        return (lo or 0), hi


def _walk(step: Step, call) -> np.ndarray:
    lib = _lib.lib()
    assert lib.ayk_debug_kv_reach_begin(step.table.size) == 0
    try:
        rc = call(lib)
    finally:
        reach = np.zeros(5, dtype=np.int64)
        assert lib.ayk_debug_kv_reach_end(reach.ctypes.data) == 0
    assert rc == 0, lib.ayk_last_error()
    return reach


def _check(step: Step, reach: np.ndarray, label: str) -> None:
    lo, hi, loads, table_lo, table_hi = (int(x) for x in reach)
    assert loads > 0, label
    assert 0 <= lo and hi <= step.pool_bytes, f"{label}: reach [{lo}, {hi}) outside [0, {step.pool_bytes})"
    assert (lo, hi) == step.expected_reach(), f"{label}: reach [{lo}, {hi}) vs {step.expected_reach()}"
    assert 0 <= table_lo and table_hi <= step.table.size, f"{label}: table entries [{table_lo}, {table_hi})"


def _common(step: Step, heads: int, rows: int, request_of_row, positions) -> tuple:
    dtype = 3 if step.fp32 else 1
    kv_dtype = 2 if step.kv8 else dtype
    return (FAKE, FAKE, FAKE, FAKE, _ptr(step.table), step.width, _ptr(step.lengths), _ptr(request_of_row),
            _ptr(positions), rows, heads, step.kv_heads, step.head_dim, step.num_blocks, step.block_size,
            step.width, step.layout, dtype, kv_dtype, ctypes.c_float(0.125), 1.0, 1.0)


def walk_v1(step: Step, heads: int, flags: int) -> np.ndarray:
    args = _common(step, heads, len(step.lengths), None, None)
    return _walk(step, lambda lib: lib.ayk_paged_attention_v1(*args, flags, None))


def walk_v2(step: Step, heads: int, size: int, grid: str, flags: int) -> np.ndarray:
    rows = len(step.lengths)
    # a staged launch is sized for its smallest partition (64), as graph metadata sizes it
    parts = -(-step.width * step.block_size // (64 if grid == "staged" else size))
    keep = []
    work, n_work, staged = None, 0, None
    if grid == "work list":
        work = hip_attention.work_list(step.lengths, size)
        n_work = work.size // 2
    elif grid == "staged":  # as a graph replay: size, item count, partial offsets, then the list
        items = hip_attention.work_list(step.lengths, size)
        counts = [max(1, -(-int(n) // size)) for n in step.lengths]
        staged = np.array([size, items.size // 2, *np.cumsum([0] + counts[:-1]), *items], dtype=np.int32)
        work, n_work = staged[2 + rows:], items.size // 2
    keep.append((work, staged))
    nbytes = _lib.lib().ayk_paged_attention_v2_workspace_bytes(max(rows, n_work), heads, step.head_dim, parts)
    args = _common(step, heads, rows, None, None)
    return _walk(step, lambda lib: lib.ayk_paged_attention_v2(
        *args, 64 if staged is not None else size, parts, _ptr(work), n_work, _ptr(staged), FAKE, nbytes,
        FAKE if flags & FLAG_SINGLE_LAUNCH else None, flags, None))


def _rows(step: Step, rows_per_request: list[int]) -> tuple[np.ndarray, np.ndarray]:
    req, pos = [], []
    for r, (count, n) in enumerate(zip(rows_per_request, step.lengths)):
        for j in range(count):
            req.append(r)
            pos.append(max(int(n) - count + j, 0))
    return np.asarray(req, dtype=np.int32), np.asarray(pos, dtype=np.int32)


def _tiles(rows_per_request: list[int], rows_per_tile: int, partitions: int) -> np.ndarray:
    tiles, first = [], 0
    for r, count in enumerate(rows_per_request):
        for start in range(0, count, rows_per_tile):
            for part in range(partitions):
                tiles.append((first + start, min(rows_per_tile, count - start), r, part))
        first += count
    return np.asarray(tiles, dtype=np.int32).reshape(-1)


def walk_prefill(step: Step, heads: int, rows_per_request: list[int], tile_pairs: int, size: int) -> np.ndarray:
    group = heads // step.kv_heads
    req, pos = _rows(step, rows_per_request)
    parts = -(-step.width * step.block_size // size) if size else 1
    tiles = _tiles(rows_per_request, max(1, tile_pairs // group), parts)
    nbytes = _lib.lib().ayk_paged_attention_v2_workspace_bytes(len(req), heads, step.head_dim, parts)
    args = _common(step, heads, len(req), req, pos)
    return _walk(step, lambda lib: lib.ayk_paged_prefill(
        *args[:9], _ptr(tiles), tiles.size // 4, tile_pairs, *args[9:], size, FAKE, nbytes, None))


def walk_windows(step: Step, heads: int, rows_per_request: list[int], size: int) -> np.ndarray:
    req, pos = _rows(step, rows_per_request)
    parts = -(-step.width * step.block_size // size) if size else 1
    tiles = _tiles(rows_per_request, max(rows_per_request), parts)
    nbytes = _lib.lib().ayk_paged_attention_v2_workspace_bytes(len(req), heads, step.head_dim, parts)
    args = _common(step, heads, len(req), req, pos)
    return _walk(step, lambda lib: lib.ayk_paged_attention_windows(
        *args[:9], _ptr(tiles), tiles.size // 4, *args[9:], size, FAKE, nbytes, None))


BLOCK_SIZES = [1, 3, 5, 16, 24, 64, 100]


def _lengths(rng: np.random.Generator, block_size: int, n: int) -> list[int]:
    edges = [1, block_size - 1, block_size, block_size + 1, 2 * block_size + 1, 0]
    out = [int(rng.choice([e for e in edges if e > 0] + [int(rng.integers(1, 700))])) for _ in range(n - 1)]
    return out + [int(rng.integers(1, 4)) * block_size]  # the last request fills its last block


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("kv8", [False, True], ids=["16-bit", "fp8"])
def test_decode_loads_stay_in_the_cache(head_dim: int, kv8: bool) -> None:
    rng = np.random.default_rng(head_dim + kv8)
    for case in range(24):
        bs = BLOCK_SIZES[case % len(BLOCK_SIZES)]
        kv_heads, group = [(2, 4), (3, 1), (1, 8), (4, 2)][case % 4]
        step = Step(rng, _lengths(rng, bs, int(rng.integers(1, 6))), bs, kv_heads, head_dim, kv8, case % 2)
        heads = kv_heads * group
        qk = [FLAG_MFMA] if kv8 else [FLAG_MFMA, FLAG_DPP]
        for flag in qk:
            waves = [1] if flag == FLAG_DPP else [1, 2, 4, 8]
            for w in waves:
                label = f"v1 case {case} bs {bs} heads {heads}/{kv_heads} qk {flag} waves {w}"
                _check(step, walk_v1(step, heads, flag | FLAG_WAVES[w]), label)
            _check(step, walk_v1(step, heads, flag), f"v1 case {case} library waves")
            for size in (64, 128, 320):
                for grid in ("work list", "dense", "staged"):
                    for merge in (FLAG_SEPARATE_REDUCE, FLAG_SINGLE_LAUNCH):
                        label = f"v2 case {case} bs {bs} size {size} {grid} qk {flag} merge {merge}"
                        _check(step, walk_v2(step, heads, size, grid, flag | merge), label)


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("kv8", [False, True], ids=["16-bit", "fp8"])
def test_multi_row_and_window_loads_stay_in_the_cache(head_dim: int, kv8: bool) -> None:
    rng = np.random.default_rng(100 + head_dim + kv8)
    full = _lib.lib().ayk_paged_prefill_tile_pairs(head_dim)
    for case in range(16):
        bs = BLOCK_SIZES[case % len(BLOCK_SIZES)]
        kv_heads, group = [(2, 4), (1, 8), (2, 1), (4, 2)][case % 4]
        step = Step(rng, _lengths(rng, bs, int(rng.integers(1, 5))), bs, kv_heads, head_dim, kv8, case % 2)
        heads = kv_heads * group
        rows = [int(rng.integers(1, min(n, 40) + 1)) if n else 1 for n in step.lengths]
        for tile_pairs in ((2 * full,) if head_dim != 64 else ()) + (full, full // 2, full // 4):
            if group > tile_pairs:
                continue
            for size in (0, 64, 192):
                label = f"multi-row case {case} bs {bs} tile {tile_pairs} size {size}"
                _check(step, walk_prefill(step, heads, rows, tile_pairs, size), label)
        if group <= 16:
            window_rows = [min(r, 16 // group) or 1 for r in rows]
            for size in (0, 64, 256):
                label = f"windows case {case} bs {bs} size {size}"
                _check(step, walk_windows(step, heads, window_rows, size), label)


def test_the_walk_reports_out_of_range_tables() -> None:
    # the walk itself bites: a table entry outside the pool reads block 0 (as the kernels map
    # it), which moves the reach down to byte 0 instead of the lowest used block
    rng = np.random.default_rng(7)
    step = Step(rng, [40, 33], 16, 2, 128, False, 0)
    step.table[0, 1] = step.num_blocks + 5
    reach = walk_v1(step, 8, FLAG_MFMA | FLAG_WAVES[1])
    assert reach[0] == 0 and reach[1] <= step.pool_bytes
    # a walk left on by a failed call is turned off by the next end, and nothing launches
    lib = _lib.lib()
    assert lib.ayk_debug_kv_reach_begin(-1) == 1


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_fp32_decode_loads_stay_in_the_cache(head_dim: int) -> None:
    # the fp32 kernel: 16-byte loads of 4 floats, D / 4 lanes per position, v1 and v2 over every
    # grid kind; multi-row steps of an fp32 model run row by row on it (rows carry positions)
    rng = np.random.default_rng(300 + head_dim)
    for case in range(20):
        bs = BLOCK_SIZES[case % len(BLOCK_SIZES)]
        kv_heads, group = [(2, 4), (3, 1), (1, 8), (4, 2)][case % 4]
        step = Step(rng, _lengths(rng, bs, int(rng.integers(1, 6))), bs, kv_heads, head_dim, False, case % 2,
                    fp32=True)
        heads = kv_heads * group
        _check(step, walk_v1(step, heads, FLAG_WAVES[1]), f"fp32 v1 case {case} bs {bs}")
        for size in (64, 128, 320):
            for grid in ("work list", "dense", "staged"):
                _check(step, walk_v2(step, heads, size, grid, FLAG_SEPARATE_REDUCE),
                       f"fp32 v2 case {case} bs {bs} size {size} {grid}")
