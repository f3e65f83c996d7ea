"""Host logic of the hip backend, on the CPU: plan, graph metadata, checks and the registry.

``plan`` and ``update_graph_metadata`` run on the host, so they are checked here
against the known answers of the reference's tests
(``tests/ops/test_attention_contract.py:393-467``,
``tests/ops/test_attention_graph.py:56-143``) and against the oracle's plan.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from ayaka_amd import backend as registry
from ayaka_amd import workloads
from ayaka_amd.enums import DType, ForwardMode, KVLayoutKind
from ayaka_amd.errors import BackendError, CapabilityError, ConfigError
from ayaka_amd.hip import attention as hip_attention
from ayaka_amd.hip import kvcache as hip_kvcache
from ayaka_amd.kvcache import FP8_E4M3_CODEC, RAW_CODEC, KVBuffers
from oracle import paged

KNOWN = json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())


def _ints(*values: int) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.int32)


@pytest.mark.parametrize("case", KNOWN["plan"], ids=lambda c: c["mode"])
def test_plan_known_answers(case: dict) -> None:
    meta = hip_attention.plan(
        ForwardMode(case["mode"]), _ints(*case["rows"]), _ints(*case["lengths"]),
        torch.tensor(case["table"]), case["block_size"],
    )
    assert meta.request_of_row.tolist() == case["request_of_row"]
    assert meta.positions.tolist() == case["positions"]
    assert meta.slot_mapping.tolist() == case["slot_mapping"]
    assert meta.slot_mapping.dtype == torch.int64 and meta.rows_per_request.dtype == torch.int32
    assert meta.kv_lengths.tolist() == case["lengths"] and meta.block_size == case["block_size"]


@pytest.mark.parametrize("case", KNOWN["plan_refusals"], ids=lambda c: c["message"])
def test_plan_refusals(case: dict) -> None:
    with pytest.raises(BackendError, match=case["message"]):
        hip_attention.plan(ForwardMode(case["mode"]), torch.tensor(case["rows"]),
                           torch.tensor(case["lengths"]), torch.tensor(case["table"]), 4)


def test_plan_matches_the_oracle_on_random_steps() -> None:
    rng = np.random.default_rng(0)
    for _ in range(40):
        batch, bs = int(rng.integers(1, 7)), int(rng.choice([1, 4, 16, 32]))
        lengths = [int(x) for x in rng.integers(0, 100, size=batch)]
        rows = [int(rng.integers(1, n + 1)) if n else int(rng.integers(0, 3)) for n in lengths]
        width = max(max(-(-n // bs) for n in lengths), 1)
        table = rng.integers(1, 999, size=(batch, width))
        meta = hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), torch.from_numpy(table), bs)
        want = paged.plan("mixed", rows, lengths, table, bs)
        for key in ("request_of_row", "positions", "slot_mapping"):
            assert getattr(meta, key).tolist() == want[key].tolist()
        assert meta.plan.max_length == max(lengths)
        # the host record the split model reads: plain ints, each row's visible context
        assert meta.plan.rows == tuple(rows) and meta.plan.kv_lengths == tuple(lengths)
        assert meta.plan.row_lengths == tuple(p + 1 if lengths[r] else 0
                                              for r, p in zip(want["request_of_row"].tolist(),
                                                              want["positions"].tolist()))
        assert all(type(x) is int for x in meta.plan.row_lengths + meta.plan.rows + meta.plan.kv_lengths)
    for _ in range(10):  # decode steps: one row per request, padding requests among them
        batch, bs = int(rng.integers(1, 40)), int(rng.choice([1, 16, 32]))
        lengths = [int(x) for x in rng.integers(0, 300, size=batch)]
        width = max(max(-(-n // bs) for n in lengths), 1)
        table = rng.integers(1, 999, size=(batch, width + 2))
        meta = hip_attention.plan(ForwardMode.DECODE, _ints(*[1] * batch), _ints(*lengths), torch.from_numpy(table), bs)
        want = paged.plan("decode", [1] * batch, lengths, table, bs)
        for key in ("request_of_row", "positions", "slot_mapping"):
            assert getattr(meta, key).tolist() == want[key].tolist()


def test_plan_rejects_mismatched_batches_and_bad_types() -> None:
    with pytest.raises(BackendError, match=r"same requests, got 2, 1 and 2"):
        hip_attention.plan(ForwardMode.MIXED, _ints(1, 1), _ints(2), torch.tensor([[1], [2]]), 4)
    with pytest.raises(BackendError, match="rows_per_request must be an int32 or int64"):
        hip_attention.plan(ForwardMode.MIXED, torch.ones(1), _ints(2), torch.tensor([[1]]), 4)
    with pytest.raises(BackendError, match="block_size must be positive"):
        hip_attention.plan(ForwardMode.MIXED, _ints(1), _ints(1), torch.tensor([[1]]), 0)


def test_metadata_is_a_frozen_snapshot() -> None:
    meta = hip_attention.plan(ForwardMode.DECODE, _ints(1), _ints(3), torch.tensor([[1]]), 4)
    with pytest.raises(AttributeError):
        meta.mode = ForwardMode.PREFILL  # type: ignore[misc]


def test_graph_metadata_starts_as_padding_and_updates_in_place() -> None:
    meta = hip_attention.graph_metadata(3, 4, 4, torch.device("cpu"))
    assert meta.mode == ForwardMode.DECODE and meta.kv_lengths.tolist() == [0, 0, 0]
    addresses = [t.data_ptr() for t in (meta.positions, meta.slot_mapping, meta.kv_lengths, meta.block_table)]
    table = torch.tensor([[3, 1, 0, 0], [0, 0, 0, 0], [2, 4, 5, 0]], dtype=torch.int32)
    hip_attention.update_graph_metadata(meta, _ints(5, 0, 10), table)
    planned = hip_attention.plan(ForwardMode.DECODE, _ints(1, 1, 1), _ints(5, 0, 10), table, 4)
    for key in ("positions", "slot_mapping", "kv_lengths"):
        assert getattr(meta, key).tolist() == getattr(planned, key).tolist()
    assert meta.block_table.tolist() == table.tolist()
    assert addresses == [t.data_ptr() for t in (meta.positions, meta.slot_mapping, meta.kv_lengths, meta.block_table)]


def test_work_list_order_and_the_staged_graph_split() -> None:
    # longest partition first, ties by row then partition; a row without context keeps partition 0
    items = hip_attention.work_list([300, 0, 512, 40], 256).reshape(-1, 2).tolist()
    assert items == [[0, 0], [2, 0], [2, 1], [0, 1], [3, 0], [1, 0]]
    assert hip_attention.work_list([], 64).size == 0
    # brute force over small cases: every partition with tokens once, sizes never rising
    rng = np.random.default_rng(3)
    for _ in range(50):
        lengths = rng.integers(0, 700, size=int(rng.integers(1, 9)))
        size = int(rng.choice([64, 128, 256]))
        pairs = hip_attention.work_list(lengths, size).reshape(-1, 2)
        want = {(r, p) for r, n in enumerate(lengths) for p in range(max(1, -(-int(n) // size)))}
        assert {tuple(x) for x in pairs.tolist()} == want and len(pairs) == len(want)
        sizes = [min(size, int(lengths[r]) - p * size) for r, p in pairs.tolist()]
        assert sizes == sorted(sizes, reverse=True)
    # a bucket of 8 requests x 1024 blocks of 16: partitions of 64 positions at least (256 per
    # row), a grid of 2048 work items whose partials the scratch packs
    meta = hip_attention.graph_metadata(8, 1024, 16, torch.device("cpu"))
    plan = meta.plan
    assert (plan.min_size, plan.partitions, plan.capacity, plan.work_offset) == (64, 256, 2048, 10)
    assert plan.staged_host[:10].tolist() == [64, 8] + [0] * 8
    assert plan.staged_host[10:26:2].tolist() == list(range(8)) and plan.staged_host[11:26:2].tolist() == [0] * 8
    table = torch.arange(8 * 1024, dtype=torch.int32).reshape(8, 1024)

    def check(lengths: list[int]) -> int:
        hip_attention.update_graph_metadata(meta, _ints(*lengths), table)
        size, count = plan.staged_partition_size, int(plan.staged_host[1])
        assert size % 64 == 0 and size >= plan.min_size and -(-max(lengths) // size) <= plan.partitions
        assert count <= plan.capacity
        counts = [-(-n // size) for n in lengths]
        assert plan.staged_host[2:10].tolist() == [sum(counts[:r]) for r in range(8)]  # first partial slots
        assert plan.staged_host[10:10 + 2 * count].tolist() == hip_attention.work_list(lengths, size).tolist()
        return size

    check([16384, 9000, 0, 1, 4096, 2048, 100, 16000])
    # a few long rows split as finely as an eager plan splits them
    size = check([16384, 16384, 0, 0, 0, 0, 0, 0])
    eager = hip_attention.choose_split(8, 8, 1, 16384, row_lengths=(16384, 16384, 0, 0, 0, 0, 0, 0))
    assert size == eager.partition_size
    # all rows empty: one item per row, the minimum size
    hip_attention.update_graph_metadata(meta, _ints(*[0] * 8), table)
    assert plan.staged_host[:2].tolist() == [64, 8]
    # a large bucket: one item per row at least; sizes whose list would overflow it are left out
    big = hip_attention.graph_metadata(4096, 64, 16, torch.device("cpu"))
    assert (big.plan.min_size, big.plan.partitions, big.plan.capacity) == (64, 16, 4096)
    hip_attention.update_graph_metadata(big, torch.full((4096,), 1024, dtype=torch.int32),
                                        torch.zeros((4096, 64), dtype=torch.int32))
    assert int(big.plan.staged_host[1]) <= 4096 and big.plan.staged_partition_size == 1024


def test_graph_metadata_update_refusals() -> None:
    meta = hip_attention.graph_metadata(2, 2, 4, torch.device("cpu"))
    with pytest.raises(BackendError, match=r"must be in \[0, 8\]"):
        hip_attention.update_graph_metadata(meta, _ints(9, 0), torch.zeros((2, 2), dtype=torch.int32))
    with pytest.raises(BackendError, match="int32 CPU tensor of shape"):
        hip_attention.update_graph_metadata(meta, torch.tensor([1, 0]), torch.zeros((2, 2), dtype=torch.int32))
    planned = hip_attention.plan(ForwardMode.DECODE, _ints(1), _ints(3), torch.tensor([[1]]), 4)
    with pytest.raises(BackendError, match="not made by this backend's graph_metadata"):
        hip_attention.update_graph_metadata(planned, _ints(1), torch.zeros((1, 1), dtype=torch.int32))
    with pytest.raises(BackendError, match="must be positive"):
        hip_attention.graph_metadata(0, 2, 4, torch.device("cpu"))


def test_the_split_covers_every_context_and_follows_the_modelled_schedule() -> None:
    choose = hip_attention.choose_split
    # one long row must be split across the GPU; a 64-position row is never split
    assert choose(1, 8, 4, 32768, row_lengths=(32768,)).partitions > 16
    assert choose(4, 8, 4, 64, row_lengths=(64, 1, 3, 64)).partitions == 0
    rng = np.random.default_rng(1)
    for _ in range(20):
        lengths = tuple(int(x) for x in rng.integers(1, 20000, size=int(rng.integers(1, 300))))
        hip_attention._split_cache.clear()
        split = choose(len(lengths), 8, 4, max(lengths), row_lengths=lengths)
        if split.partitions:
            assert split.partition_size % 64 == 0
            assert split.partitions * split.partition_size >= max(lengths)
            # no worse, under the model, than any size whose work list fits the round limit
            cost = hip_attention.schedule_makespan(list(lengths), split.partition_size)
            for size in (256, 512, 1024, 2048):
                if size < max(lengths) and hip_attention.fits_schedule(list(lengths), size):
                    assert cost <= hip_attention.schedule_makespan(list(lengths), size)
    # graph metadata (lengths unknown) is scored as every row at the table width
    assert choose(64, 8, 4, 4096) == choose(64, 8, 4, 4096, row_lengths=(4096,) * 64)
    assert hip_attention.head_chunks(4) == 1 and hip_attention.head_chunks(12) == 2
    assert hip_attention.head_chunks(16) == 2 and hip_attention.head_chunks(11) == 11


def test_v1_with_a_wave_split_is_chosen_where_it_models_faster() -> None:
    choose = hip_attention.choose_split
    hip_attention._split_cache.clear()
    # C3: 64 rows of 4096 at 8 key/value heads: v1, each context split among 4 waves (256
    # workgroups of 2 heads), which models (and measured) faster than any v2 launch
    assert choose(64, 8, 4, 4096, row_lengths=(4096,) * 64) == hip_attention.Split(0, 0, 4)
    assert choose(64, 8, 4, 4096, row_lengths=(4096,) * 64, kv_bytes=1) == hip_attention.Split(0, 0, 4)
    # without v1, the best v2 launch: one round of 1024-position partitions
    assert choose(64, 8, 4, 4096, row_lengths=(4096,) * 64, v1=False) == hip_attention.Split(1024, 4)
    # a few long rows (C4) and a ragged batch stay on v2
    assert choose(8, 8, 4, 32768, row_lengths=(8192, 16384, 24576, 32768, 32768, 32768, 12288, 2048)).partitions
    lengths = workloads.config(5).lengths  # log-uniform in [16, 16384]
    assert choose(256, 8, 8, max(lengths), row_lengths=lengths).partitions
    # a cached v1 choice serves every step of the same signature (a longer one included)
    assert choose(4, 3, 3, 121, row_lengths=(121, 100, 90, 64)) == choose(4, 3, 3, 127, row_lengths=(127, 100, 90, 64))
    assert choose(4, 3, 3, 127, row_lengths=(127, 100, 90, 64)).partitions == 0
    # graph replays (a minimum partition size) never take the v1 candidate
    assert choose(64, 8, 4, 4096, row_lengths=(4096,) * 64, min_size=64).partitions
    # the model: a wave's share of its row, in 16-position chunks, plus the fixed cost
    assert hip_attention.v1_makespan([4096] * 64, 4, 8, 240) == 1024 + 240
    assert hip_attention.v1_makespan([4096] * 64, 8, 8, 240) == 2 * (512 + 240)


def test_the_modelled_schedule() -> None:
    # 256 equal workgroups fill the 256 CUs once; one more starts a second round
    assert hip_attention.schedule_makespan([1024] * 256, 1024) == 1024 + hip_attention.WORKGROUP_COST
    assert hip_attention.schedule_makespan([1024] * 257, 1024) == 2 * (1024 + hip_attention.WORKGROUP_COST)


def test_the_native_launch_model_is_the_python_statement() -> None:
    # ayk_split_model and ayk_work_list (C++, host) against the plain-Python statement of the
    # same schedule and order, on random ragged steps, edge lengths and every group count
    from tests._support import python_schedule_makespan, python_work_list

    rng = np.random.default_rng(17)
    cases = [[0], [1], [64], [65], [4096] * 64, [1024] * 257, [0, 0, 3], list(range(0, 3000, 7))]
    for _ in range(120):
        n = int(rng.integers(1, 400))
        cases.append([int(x) for x in np.exp(rng.uniform(0, np.log(40000), n)).astype(int) * (rng.random(n) > 0.1)])
    for lengths in cases:
        sizes = [int(x) for x in rng.choice(hip_attention.PARTITION_CANDIDATES, size=4)] + [max(lengths) + 1]
        groups, cost = int(rng.integers(1, 4)), int(rng.choice([0, 80, 160, 240, 320]))
        makespans, items = hip_attention.schedule_makespans(lengths, sizes, groups, cost)
        for size, got, count in zip(sizes, makespans, items):
            assert got == python_schedule_makespan(lengths, size, groups, cost), (lengths, size, groups, cost)
            assert count == sum(-(-n // size) for n in lengths if n > 0)
        size = int(rng.choice([64, 128, 320, 512, 4096]))
        assert hip_attention.work_list(lengths, size).tolist() == python_work_list(lengths, size).tolist()
    with pytest.raises(BackendError):
        hip_attention.schedule_makespans([10], [0])


@pytest.mark.parametrize("index,kv_bytes,expected", [
    (1, 2, (0, 8)), (1, 1, (0, 8)), (2, 2, (320, 0)), (2, 1, (320, 0)), (3, 2, (0, 4)), (3, 1, (0, 4)),
    (4, 2, (704, 0)), (4, 1, (704, 0)), (5, 2, (3072, 0)), (5, 1, (2560, 0))])
def test_the_launches_chosen_for_the_benchmark_steps(index: int, kv_bytes: int, expected: tuple) -> None:
    # the library's launch for each benchmark configuration: (partition size, v1 waves per head),
    # (0, n) being v1 with each context split among n waves (measured choices: C3 v1 at 4 waves,
    # C1 v1 at 8, C2 v2 at 320, C4 v2 at 704, C5 v2 at 3072, or 2560 over fp8 caches)
    cfg = workloads.config(index)
    hip_attention._split_cache.clear()
    split = hip_attention.choose_split(cfg.batch, cfg.kv_heads, cfg.heads // cfg.kv_heads, max(cfg.lengths),
                                       row_lengths=tuple(cfg.lengths), kv_bytes=kv_bytes)
    assert (split.partition_size, split.waves) == expected


def test_multi_row_tiles_list_every_partition_a_group_sees_once() -> None:
    rows, lengths = [37, 5, 1, 8, 0], [37, 900, 2, 130, 0]
    table = torch.ones(len(rows), 64, dtype=torch.int32)
    step = hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), table, 16).plan
    groups = step.prefill_groups(4, 128)  # 32 rows per group at 4 query heads per key/value head
    assert sorted((row, n) for _, row, n, _ in groups) == [(0, 32), (32, 5), (37, 5), (42, 1), (43, 8)]
    assert [g[0] for g in groups] == sorted((g[0] for g in groups), reverse=True)
    for size in (0, 64, 192, 512):
        tiles = step.prefill_tiles(4, 128, size, torch.device("cpu")).view(-1, 4).tolist()
        for length, row, n, request in groups:
            parts = sorted(t[3] for t in tiles if t[0] == row)
            assert all(t[1:3] == [n, request] for t in tiles if t[0] == row)
            assert parts == (list(range(max(1, -(-length // size)))) if size else [0]), (size, row)
        # longest first: the positions each tile covers never grow down the list
        length_of = {row: length for length, row, _, _ in groups}
        work = [min(size, length_of[row] - part * size) if size else length_of[row] for row, _, _, part in tiles]
        assert work == sorted(work, reverse=True)


def test_multi_row_groups_and_tiles_match_a_loop_restatement() -> None:
    # the array builders against the definition written as loops: groups of at most
    # pairs // group consecutive rows of one request, each with its last row's context (0 for
    # a padding request), heaviest first then by first row; tiles of one group per partition
    # its context reaches (one for an empty context), longest piece first
    rng = np.random.default_rng(41)
    for _ in range(60):
        count = int(rng.integers(1, 30))
        rows = [int(x) for x in rng.integers(0, 70, count)]
        lengths = [r + int(rng.integers(0, 3000)) if r else int(rng.integers(0, 2)) * 40 for r in rows]
        if not any(rows):
            rows[0], lengths[0] = 1, max(lengths[0], 1)
        table = torch.ones(count, max(lengths) // 16 + 2, dtype=torch.int32)
        step = hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), table, 16).plan
        group, pairs = int(rng.choice([1, 4, 8])), int(rng.choice([16, 32, 64, 128]))
        per_tile, want, first = max(1, pairs // group), [], 0
        for request, (n_rows, length) in enumerate(zip(rows, lengths)):
            for start in range(0, n_rows, per_tile):
                n = min(per_tile, n_rows - start)
                want.append((step.row_lengths[first + start + n - 1] if length else 0, first + start, n, request))
            first += n_rows
        want.sort(key=lambda g: (-g[0], g[1]))
        assert step.prefill_groups(group, pairs) == want
        for size in (0, 64, 448, 1024):
            tiles = []
            for length, row, n, request in want:
                for part in range(max(1, -(-length // size)) if size else 1):
                    tiles.append((-min(size, length - part * size) if size else -length, row, n, request, part))
            flat = [v for _, row, n, request, part in sorted(tiles) for v in (row, n, request, part)]
            assert step.prefill_tiles(group, pairs, size, torch.device("cpu")).tolist() == flat


def test_multi_row_partition_choice() -> None:
    choose = hip_attention.choose_prefill_partition
    # 16 verify windows of 8 rows over 1K fill 128 of 512 workgroup slots: split
    rows = [1017 + i for i in range(8)] * 16
    assert choose([1024] * 16, rows, 8, 32, 128) > 0
    # 4 requests x 512 rows over 4K fill the GPU already (64 tiles x 8 heads): no split
    lengths = [3584 + 32 * (i + 1) for i in range(16)] * 4
    assert choose(lengths, list(range(3585, 4097)) * 4, 8, 32, 128) == 0
    # a short context is never split
    assert choose([100, 60], [100] * 32 + [60] * 32, 8, 32, 128) == 0
    # the chosen size is the modelled optimum among the candidates
    model = hip_attention.prefill_model_us
    size = choose([1024] * 16, rows, 8, 32, 128)
    for other in (0, *hip_attention.PREFILL_PARTITION_CANDIDATES):
        if other < 1024:
            assert model([1024] * 16, rows, 8, 32, 128, size) <= model([1024] * 16, rows, 8, 32, 128, other)


def test_dispatch_makespan() -> None:
    makespan = hip_attention._dispatch_makespan
    assert makespan([5, 3, 9], 4) == 9                      # every item starts at once
    assert makespan([7] * 9, 4) == 21                       # equal items: three rounds
    assert makespan([10, 10, 2, 2, 2, 2, 2], 2) == 16        # the short ones share the slots
    # against every order-respecting assignment on tiny cases: greedy longest-first dispatch
    rng = np.random.default_rng(3)
    for _ in range(200):
        steps = [int(x) for x in rng.integers(1, 20, size=int(rng.integers(1, 9)))]
        slots = int(rng.integers(1, 4))
        loads = [0] * slots
        for s in sorted(steps, reverse=True):
            loads[loads.index(min(loads))] += s
        assert makespan(steps, slots) == max(loads)


def test_multi_row_launch_choice() -> None:
    def launch(rows: list[int], lengths: list[int]) -> tuple[int, int]:
        table = torch.ones(len(rows), max(lengths) // 16 + 1, dtype=torch.int32)
        step = hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), table, 16).plan
        return step.prefill_launch(8, 4, 128)
    # long chunks that fill the GPU: double tiles (8-wave workgroups), no partitions
    assert launch([512] * 4, [4096] * 4) == (256, 0)
    # one 2048-row prompt and 128-row chunks: a double tile per compute unit would leave the
    # causal triangle's short tiles unbalanced; half tiles measured within 1% and 8% of the best
    assert launch([2048], [2048]) == (64, 0) and launch([128] * 8, [2048] * 8) == (64, 0)
    # a 1024-row prompt: half tiles (31.4 us), not quarter tiles (38.6), which model about equal
    assert launch([1024], [1024]) == (64, 0)
    # short verify windows: small tiles; few of them: partitions as well
    assert launch([2] * 64, [2048] * 64)[0] < 128
    pairs, size = launch([8] * 16, [1024] * 16)
    assert pairs < 128 and size > 0
    # decode rows beside one chunk: small tiles, split (they would stream alone otherwise)
    pairs, size = launch([1] * 64 + [64], [4096] * 65)
    assert pairs < 128 and size > 0


def test_multi_row_launch_choice_by_head_width() -> None:
    def launch(rows: list[int], lengths: list[int], heads: int, head_dim: int, kv_heads: int = 8) -> tuple[int, int]:
        table = torch.ones(len(rows), max(lengths) // 16 + 1, dtype=torch.int32)
        step = hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), table, 16).plan
        return step.prefill_launch(kv_heads, heads // kv_heads, head_dim)
    # the measured fastest launches of a sweep on MI355X (us, chosen against the runner-up)
    # head_dim 64: a 2048-row prompt on unsplit half tiles (34.6), not full tiles in partitions
    # of 1024 (41.0)
    assert launch([2048], [2048], 32, 64) == (64, 0)
    # head_dim 256: 128-row chunks on double tiles in partitions of 1024 (66.6, against
    # 85.8 on unsplit quarter tiles), and long chunks on unsplit double tiles
    assert launch([128] * 8, [2048] * 8, 16, 256) == (128, 1024)
    assert launch([512] * 4, [4096] * 4, 16, 256) == (128, 0)
    # GQA 8: long chunks on unsplit double tiles
    assert launch([512] * 4, [4096] * 4, 64, 128) == (256, 0)
    # TinyLlama (32/4/64): 256 rows over 2048 on half tiles in partitions of 512 (21.3, against
    # 24.7 on unsplit quarter tiles)
    assert launch([256], [2048], 32, 64, kv_heads=4) == (64, 512)


def test_window_tiles_and_split() -> None:
    def step(rows: list[int], lengths: list[int]):
        table = torch.ones(len(rows), max(lengths) // 16 + 1, dtype=torch.int32)
        return hip_attention.plan(ForwardMode.MIXED, _ints(*rows), _ints(*lengths), table, 16).plan
    # 16 columns: 4 rows at 4 query heads per key/value head, 2 at 8, 1 at 16, none past 16
    assert step([2, 1, 4], [900, 17, 40]).window_pairs(4) == 16
    assert step([2, 1, 5], [900, 17, 40]).window_pairs(4) == 0
    assert step([2, 2], [900, 17]).window_pairs(8) == 16 and step([3], [40]).window_pairs(8) == 0
    assert step([1, 1], [9, 9]).window_pairs(16) == 16 and step([1], [9]).window_pairs(32) == 0
    assert step([3, 3], [100, 100]).window_pairs(3) == 15  # 5 rows x 3 heads
    # the decode split model over the tiles: many long tiles stay whole-ish, few are split
    few = step([4] * 8, [4096] * 8).window_split(8, 4)
    assert few % 64 == 0 and 0 < few < 4096
    assert step([4], [64]).window_split(8, 4) == 0
    # the waves the library gives each head: the most (up to 8) within one round of 8-wave
    # workgroups on 256 CUs (items x heads x waves <= 1024)
    assert [hip_attention.window_waves(n, 8) for n in (16, 32, 64, 128, 256)] == [8, 8, 4, 2, 1]
    assert hip_attention.window_waves(4, 1) == 8 and hip_attention.window_waves(2048, 8) == 1
    # measured on MI355X: many 4K tiles run unsplit at 8 waves per head (32 x 4-row windows
    # 89.3 us, the best split 86.5), few long ones split into large partitions (8 x 8K:
    # 2048, 52.0 us; 1024 measured fastest at 50.5, 256 63.0)
    assert hip_attention.window_partition_size([4096] * 32, 8) == 0
    assert hip_attention.window_partition_size([2048] * 64, 8) == 0
    assert hip_attention.window_partition_size([8192] * 8, 8) in (1024, 2048)
    assert hip_attention.window_partition_size([32768] * 2, 8) in (1024, 2048, 4096)
    assert hip_attention.window_partition_size([], 8) == 0


def _cpu_buffers(**changes: object) -> KVBuffers:
    k = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16)
    buffers = KVBuffers(k, k.clone(), KVLayoutKind.NHD, RAW_CODEC)
    return buffers._replace(**changes)


def test_ops_refuse_caches_they_cannot_serve() -> None:
    meta = hip_attention.plan(ForwardMode.DECODE, _ints(1), _ints(3), torch.tensor([[1]]), 16)
    q = torch.zeros(1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(BackendError, match="serves the NHD and HND layouts"):
        hip_attention.attend(q, _cpu_buffers(layout=KVLayoutKind.NLD), meta, q.clone(), scale=1.0)
    with pytest.raises(BackendError, match="stores the 'raw' and 'fp8_e4m3' codecs, not 'fp8'"):
        hip_kvcache.store(q[:, :2], q[:, :2], _cpu_buffers(codec="fp8"), meta)
    fp64 = torch.zeros(4, 16, 2, 64, dtype=torch.float64)
    with pytest.raises(BackendError, match="computes in float16, bfloat16, float32"):
        hip_attention.attend(q, KVBuffers(fp64, fp64, KVLayoutKind.NHD, RAW_CODEC), meta, q.clone(), scale=1.0)
    fp32 = torch.zeros(4, 16, 2, 64)  # accepted as a cache (it fails on the device, as every CPU tensor does)
    with pytest.raises(BackendError, match="runs on a HIP device"):
        hip_attention.attend(q, KVBuffers(fp32, fp32, KVLayoutKind.NHD, RAW_CODEC), meta, q.clone(), scale=1.0)
    with pytest.raises(BackendError, match="stores the 'fp8_e4m3' codec as float8_e4m3fn"):
        hip_attention.attend(q, _cpu_buffers(codec=FP8_E4M3_CODEC), meta, q.clone(), scale=1.0)
    with pytest.raises(BackendError, match="runs on a HIP device"):
        hip_attention.attend(q, _cpu_buffers(), meta, q.clone(), scale=1.0)
    bad_v = torch.zeros(4, 16, 2, 65, dtype=torch.bfloat16)
    with pytest.raises(BackendError, match=r"buffers.v must be bfloat16 \[4, 16, 2, 64\]"):
        hip_kvcache.store(q[:, :2], q[:, :2], _cpu_buffers(v=bad_v), meta)


def test_registry_selection_and_refusals(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(registry, "_registry", dict(registry._registry))
    calls: list[str] = []

    def fake_loader() -> dict[str, object]:
        calls.append("fake")
        return {"attention": "fake-attention", "kvcache": "fake-kvcache"}

    registry.register_backend(
        registry.BackendCaps(
            name="fake", families=frozenset({"attention", "kvcache"}), platforms=frozenset({"linux"}),
            devices=frozenset({"cpu"}), dtypes=frozenset({DType.BF16}), multi_row_attention=True,
        ),
        fake_loader,
    )
    chosen = registry.load_backend(["hip", "fake"], device="cpu", dtype=DType.BF16)
    assert chosen.providers == {"kvcache": "fake", "attention": "fake"} and calls == ["fake"]
    with pytest.raises(ConfigError, match="hip has no cpu support"):
        registry.load_backend(["hip"], device="cpu", dtype=DType.BF16)
    with pytest.raises(ConfigError, match="cannot run inside a CUDA graph"):
        registry.load_backend(["fake"], device="cpu", dtype=DType.BF16, cuda_graph=True)
    with pytest.raises(ConfigError, match="BACKEND_UNKNOWN"):
        registry.load_backend(["nope"], device="cpu", dtype=DType.BF16)
    with pytest.raises(ValueError, match="already registered"):
        registry.register_backend(registry.available_backends()[0], fake_loader)


def test_hip_backend_is_unavailable_without_a_device(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(CapabilityError, match="no HIP device"):
        from ayaka_amd.hip import load

        load()
    with pytest.raises(ConfigError, match="hip is unavailable"):
        registry.load_backend(["hip"], device="cuda", dtype=DType.BF16)


def test_recorded_launches_replay_only_for_the_same_storage() -> None:
    # the repeated-call record: keyed by the long-lived objects' ids and by every tensor's data
    # pointer, shape, strides and dtype; it holds no activation tensor
    import gc
    import weakref

    from ayaka_amd.hip import _fastpath

    calls = []
    cache: dict = {}
    owner = object()  # stands in for the buffers and metadata a record keeps
    q, out = torch.zeros(4, 8), torch.zeros(4, 8)

    def key_of(*tensors):
        return ("attend", id(owner), _fastpath.signature(tensors))

    assert _fastpath.lookup(cache, key_of(q, out)) is None
    record = _fastpath.Recorder()
    record("op", lambda *args: calls.append(args) or 0, (1, 2), torch.device("cpu"), False)
    _fastpath.remember(cache, key_of(q, out), (owner,), record)
    found = _fastpath.lookup(cache, key_of(q, out))
    assert found is not None and found.keep == (owner,)
    _fastpath.run(found, 7)
    assert calls == [(1, 2, 7)]
    # the record does not keep q or out alive
    dead = weakref.ref(q)
    del q, found
    gc.collect()
    assert dead() is None
    q = torch.zeros(4, 8)
    # new storage, a new shape, new strides or a new dtype behind the same object miss
    base = key_of(q, out)
    _fastpath.remember(cache, base, (owner,), record)
    q.set_(torch.zeros(4, 8).untyped_storage())
    assert _fastpath.lookup(cache, key_of(q, out)) is None
    same = torch.zeros(8, 4)
    _fastpath.remember(cache, key_of(same, out), (owner,), record)
    assert _fastpath.lookup(cache, key_of(same.t(), out)) is None  # same address, other strides
    assert _fastpath.lookup(cache, key_of(same.view(torch.int32), out)) is None
    assert _fastpath.lookup(cache, key_of(same.view(32), out)) is None
    assert _fastpath.lookup(cache, key_of(same, out)) is not None
    # an empty recorder (a call that launched nothing) records nothing; the cache is bounded
    _fastpath.remember(cache, ("none",), (), _fastpath.Recorder())
    assert ("none",) not in cache
    for i in range(_fastpath.MAX_RECORDS + 1):
        _fastpath.remember(cache, ("k", i), (), record)
    assert len(cache) <= _fastpath.MAX_RECORDS


def test_recorded_library_arguments_keep_their_values() -> None:
    # a recorded library call converts its arguments once to the export's declared types;
    # the values (pointers, sizes, numpy scalars, the float scale) must come through unchanged
    import ctypes

    import numpy as np

    from ayaka_amd.hip import _fastpath, _lib

    types = _lib.EXPORTS["ayk_paged_attention_v1"][1][:-1]
    args = tuple(range(1000, 1000 + len(types)))
    args = args[:5] + (np.int64(64),) + (None,) + args[7:19] + (np.float32(0.125),) + args[20:]
    converted = _fastpath.convert(types, args)
    assert [type(c) for c in converted] == types
    assert converted[6].value is None and converted[5].value == 64 and converted[19].value == 0.125
    assert [c.value for i, c in enumerate(converted) if i not in (5, 6, 19)] == \
        [a for i, a in enumerate(args) if i not in (5, 6, 19)]
    with pytest.raises(ValueError):
        _fastpath.convert(types, args[:-1])
    assert isinstance(_fastpath.convert([ctypes.c_int32], (ctypes.c_int32(3),))[0], ctypes.c_int32)


def test_plan_accepts_int64_inputs() -> None:
    # tests/ops/test_attention_contract.py:414-423: int64 step tensors plan as int32 do
    as32 = hip_attention.plan(ForwardMode.MIXED, _ints(2, 1), _ints(5, 3), torch.tensor([[3, 4], [7, 0]]), 4)
    as64 = hip_attention.plan(ForwardMode.MIXED, torch.tensor([2, 1]), torch.tensor([5, 3]),
                              torch.tensor([[3, 4], [7, 0]], dtype=torch.int64), 4)
    for key in ("rows_per_request", "request_of_row", "positions", "slot_mapping", "kv_lengths", "block_table"):
        a, b = getattr(as32, key), getattr(as64, key)
        assert a.dtype == b.dtype and a.tolist() == b.tolist(), key
    assert as64.positions.tolist() == [3, 4, 2] and as64.slot_mapping.tolist() == [15, 16, 30]


def test_the_pruned_best_split_is_the_exhaustive_one() -> None:
    # ayk_best_split schedules only candidates whose lower bound can still win; its choice must
    # be the first smallest exact finish time among the eligible candidates, as an exhaustive
    # scoring of every candidate (the plain-Python schedule) picks it
    from tests._support import python_schedule_makespan

    rng = np.random.default_rng(23)
    for trial in range(150):
        n = int(rng.integers(1, 300))
        lengths = [int(x) for x in np.exp(rng.uniform(0, np.log(40000), n)).astype(int)]
        if trial % 3 == 0:
            lengths = [int(rng.choice([512, 1024, 4096]))] * n  # equal rows: ties between sizes
        groups = int(rng.integers(1, 3))
        kv_bytes = int(rng.choice([1, 2]))
        max_items = int(rng.choice([0, 0, 64, 2048]))
        cost = hip_attention.WORKGROUP_COSTS[kv_bytes]
        sizes = list(hip_attention.FP8_PARTITION_CANDIDATES if kv_bytes == 1 else hip_attention.PARTITION_CANDIDATES)
        got = hip_attention._best_size(lengths, max(lengths), groups, kv_bytes, 0, max_items)
        cands = sizes
        for i, size in enumerate(sizes):
            if size >= max(lengths):
                cands = sizes[:i + 1]
                break
        counts = [sum(-(-x // size) for x in lengths) for size in cands]
        eligible = [i for i, c in enumerate(counts) if not max_items or c <= max_items]
        if not eligible:
            assert got == -(-max(lengths) // 64) * 64
            continue
        scored = [i for k, i in enumerate(eligible)
                  if k == len(eligible) - 1 or counts[i] * groups <= hip_attention.MAX_ROUNDS * 256]
        times = {i: python_schedule_makespan(lengths, cands[i], groups, cost) for i in scored}
        want = min(scored, key=lambda i: (times[i], i))
        assert got == cands[want], (trial, got, cands[want])
