"""Parity of the HIP path with the oracle, on a HIP device (MI355X).

Every call goes through the C ABI of ``libayaka_hip.so`` (via the ``hip``
backend's ops, and once directly with ctypes). Bars:

* KV write and block ops: bit-exact.
* Attention: against the float64 oracle, ``max_abs_excess`` (error beyond half
  an output ulp) <= 2e-3 and ``rel_l2`` (against the oracle rounded once to the
  output dtype) <= 1e-3 (or a raw relative L2 within 1e-4 of the once-rounded
  oracle's own, for outputs whose excess is only rounding flips); plus the reference tests' own bound
  ``|out - exact| <= 4 eps max|y|`` (``tests/ops/test_parity.py:196-201``).
  The oracle's own rounded fp32 result is held to the same metrics and reported.
"""

from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from ayaka_amd import workloads
from ayaka_amd.enums import ForwardMode, KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import _lib
from ayaka_amd.hip import attention as hip_attention
from ayaka_amd.hip import kvcache as hip_kvcache
from ayaka_amd.kvcache import FP8_E4M3_CODEC, RAW_CODEC, KVBuffers
from oracle import paged
from oracle.numerics import bits_to_f32, e4m3_to_f32, f32_to_bits, f32_to_e4m3, parity_report
from tests._support import Scenario, build_scenario, oracle_rows

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TORCH_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}
EPS = {"bf16": 2.0**-7, "fp16": 2.0**-10}
DEV = torch.device("cuda:0")


def to_device(bits: np.ndarray, dtype: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(TORCH_DTYPES[dtype]).to(DEV)


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_parity(out: torch.Tensor, expected: np.ndarray, dtype: str, label: str = "") -> dict:
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{label}: non-finite output"
    rep = parity_report(got, expected, dtype)
    ref = parity_report(bits_to_f32(f32_to_bits(expected.astype(np.float32), dtype), dtype), expected, dtype)
    bound = 4 * EPS[dtype] * float(np.abs(expected).max(initial=0.0))
    worst = float(np.abs(got - expected).max(initial=0.0))
    assert rep["max_abs_excess"] <= 2e-3, f"{label}: {rep} (reference rounding: {ref})"
    # rel_l2 counts every rounding flip at a full ulp. On an output of a few hundred elements, a
    # handful of values within a hair of a rounding midpoint can flip and carry it past 1e-3
    # while the output is as close to the exact result as the oracle rounded once (sweep case
    # 29207: raw 1.74052e-3 against 1.74048e-3). Such an output passes when its raw distance from
    # the exact result is within 1e-4 of the once-rounded oracle's; a real excess (one bf16
    # weight per P.V product: raw ~2.3e-3 against ~1.6e-3) still fails.
    assert rep["rel_l2"] <= 1e-3 or rep["rel_l2_raw"] <= ref["rel_l2_raw"] + 1e-4, \
        f"{label}: {rep} (reference rounding: {ref})"
    assert worst <= max(bound, 1e-6), f"{label}: {worst} > 4 eps max|y| = {bound}"
    return rep


def scenario_buffers(s: Scenario) -> KVBuffers:
    layout = KVLayoutKind.NHD if s.layout == "nhd" else KVLayoutKind.HND
    return KVBuffers(to_device(s.k_bits, s.dtype), to_device(s.v_bits, s.dtype), layout, RAW_CODEC)


def plan_scenario(s: Scenario):
    mode = ForwardMode(s.mode)
    return hip_attention.plan(
        mode,
        torch.tensor(s.rows, dtype=torch.int32, device=DEV),
        torch.tensor(s.lengths, dtype=torch.int32, device=DEV),
        torch.from_numpy(s.table).to(DEV),
        s.block_size,
    )


QK = ["dpp", "mfma"]


def run_attention(s: Scenario, partitions: int | None = None, qk: str | None = None,
                  prefill: bool | None = None, **launch) -> torch.Tensor:
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    q = to_device(s.q_bits, s.dtype)
    out = torch.full_like(q, 7.0)
    if partitions is not None and prefill is None:
        prefill = False  # a forced v1/v2 launch means the decode kernels
    hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, partitions=partitions, qk=qk, prefill=prefill,
                              **launch)
    torch.cuda.synchronize()
    return out


# --- KV write --------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("head_dim", [64, 128, 8, 12])
def test_store_is_bit_exact(dtype: str, layout: str, head_dim: int) -> None:
    s = build_scenario([(3, 9), (1, 2), (2, 0), (5, 40)], dtype=dtype, layout=layout, head_dim=head_dim,
                       block_size=4, seed=21)
    rng = np.random.default_rng(5)
    n = sum(s.rows)
    k_new = f32_to_bits(rng.standard_normal((n, s.kv_heads, head_dim)).astype(np.float32), dtype)
    v_new = f32_to_bits(rng.standard_normal((n, s.kv_heads, head_dim)).astype(np.float32), dtype)
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    assert meta.slot_mapping.cpu().tolist() == s.plan["slot_mapping"].tolist()
    hip_kvcache.store(to_device(k_new, dtype), to_device(v_new, dtype), buffers, meta)
    torch.cuda.synchronize()
    want_k, want_v = s.k_bits.copy(), s.v_bits.copy()
    paged.store(want_k, want_v, k_new, v_new, s.plan["slot_mapping"], layout)
    got_k, got_v = to_bits(buffers.k), to_bits(buffers.v)
    # block 0 receives the padding rows in an unspecified order; every other block is exact
    assert np.array_equal(got_k[1:], want_k[1:])
    assert np.array_equal(got_v[1:], want_v[1:])


def test_store_of_an_empty_step_is_a_no_op() -> None:
    s = build_scenario([(1, 3)], mode="decode", seed=2)
    buffers = scenario_buffers(s)
    meta = hip_attention.plan(
        ForwardMode.IDLE,
        torch.zeros(0, dtype=torch.int32, device=DEV),
        torch.zeros(0, dtype=torch.int32, device=DEV),
        torch.zeros((0, 1), dtype=torch.int32, device=DEV),
        s.block_size,
    )
    empty = torch.empty((0, s.kv_heads, s.head_dim), dtype=torch.bfloat16, device=DEV)
    hip_kvcache.store(empty, empty, buffers, meta)
    out = torch.empty((0, s.heads, s.head_dim), dtype=torch.bfloat16, device=DEV)
    hip_attention.attend(out, buffers, meta, out.clone(), scale=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(buffers.k), s.k_bits)


# --- attention: the reference's contract cases ---------------------------------------------

CASES = [
    ("one-block", [(1, 16), (1, 16)], "decode"),
    ("block-multiples", [(1, 32), (1, 48)], "decode"),
    ("ends-inside-blocks", [(1, 1), (1, 15), (1, 17), (1, 31), (1, 33)], "decode"),
    ("padding-requests", [(1, 6), (1, 0), (1, 70), (1, 0)], "decode"),
    ("parity-lengths", [(1, 1), (1, 16), (1, 17), (1, 70)], "decode"),
    ("prefill-chunks", [(16, 16), (5, 5), (3, 11), (4, 12), (1 + 3, 9)], "mixed"),
    ("mixed-batch", [(7, 7), (1, 9), (4, 16), (2, 2), (1, 1), (3, 6), (2, 0)], "mixed"),
]


@pytest.mark.parametrize("qk", QK)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("name,steps,mode", CASES, ids=[c[0] for c in CASES])
def test_attention_contract_cases(dtype: str, layout: str, name: str, steps: list, mode: str, qk: str) -> None:
    s = build_scenario(steps, dtype=dtype, layout=layout, heads=8, kv_heads=2, head_dim=64,
                       block_size=16, mode=mode, seed=31)
    expected = s.expected(np.float64)
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    for partitions, prefill in ((0, False), (1, False), (None, True)):
        out = run_attention(s, partitions, qk, prefill)
        assert_parity(out, expected, dtype, f"{name}/{partitions}/{prefill}")
        if padding_rows:
            assert torch.count_nonzero(out[padding_rows]) == 0


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 2), (6, 1), (8, 4), (8, 1), (12, 4), (9, 3), (64, 8), (16, 1)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("qk", QK)
def test_grouped_query_heads(heads: int, kv_heads: int, head_dim: int, qk: str) -> None:
    s = build_scenario([(1, 37), (1, 200), (3, 10)], heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                       block_size=16, seed=41)
    for partitions in (0, 1):
        out = run_attention(s, partitions, qk)
        assert_parity(out, s.expected(np.float64), "bf16", f"{heads}/{kv_heads}/{head_dim}/{partitions}")


PREFILL_CASES = [
    ("long-prompt", [(300, 300)]),
    ("chunk-after-context", [(77, 1500), (5, 40)]),
    ("verify-windows", [(5, 900), (3, 17), (1, 2), (4, 0)]),
    ("many-requests", [(int(n), int(n) + 11) for n in np.random.default_rng(2).integers(1, 60, size=12)]),
]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 2, 64), (32, 8, 128), (12, 4, 128), (4, 4, 256),
                                                     (64, 8, 128), (16, 1, 64)])
@pytest.mark.parametrize("name,steps", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_multi_row_kernel(dtype: str, heads: int, kv_heads: int, head_dim: int, name: str, steps: list) -> None:
    s = build_scenario(steps, dtype=dtype, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16,
                       mode="mixed", seed=67, spare_blocks=2)
    out = run_attention(s, None, None, True, window=False)
    assert_parity(out, s.expected(np.float64), dtype, f"prefill/{name}")
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    if padding_rows:
        assert torch.count_nonzero(out[padding_rows]) == 0


@pytest.mark.parametrize("size", [0, 64, 512, None])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 2, 64), (32, 8, 128), (12, 4, 128), (4, 4, 256),
                                                     (64, 8, 128), (16, 1, 64)])
def test_window_kernel(size: int | None, dtype: str, heads: int, kv_heads: int, head_dim: int) -> None:
    # steps of few rows per request on the decode kernel's window launch: a tile's (row, head)
    # pairs are the 16 matrix-core columns, each row masked at its own position; rows of one
    # to 16 / group per request, a padding request, contexts across partitions and blocks
    rows = 16 // (heads // kv_heads)
    steps = [(min(rows, 2), 900), (1, 17), (rows, rows), (1, 0), (min(rows, 3), 300), (rows, 1041)]
    s = build_scenario(steps, dtype=dtype, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16,
                       mode="mixed", seed=69, spare_blocks=2)
    launch = dict(partitions=0) if size == 0 else dict(partition_size=size) if size else {}
    assert plan_scenario(s).plan.window_pairs(heads // kv_heads) > 0
    out = run_attention(s, prefill=True, window=True, **launch)
    assert_parity(out, s.expected(np.float64), dtype, f"windows/{size}")
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    assert torch.count_nonzero(out[padding_rows]) == 0


@pytest.mark.parametrize("waves", [0, 1, 2, 4])
@pytest.mark.parametrize("size", [0, 64, 192, 512])
@pytest.mark.parametrize("heads,kv_heads,head_dim,dtype", [(8, 2, 64, "fp16"), (32, 8, 128, "bf16"),
                                                           (4, 4, 256, "bf16")])
@pytest.mark.parametrize("name,steps", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_multi_row_partitions(size: int, waves: int, heads: int, kv_heads: int, head_dim: int, dtype: str,
                              name: str, steps: list) -> None:
    # size 0: each tile's whole context in one workgroup; otherwise partitions of `size`
    # positions merged by the reduce kernel, each row over the partitions it sees. waves:
    # tiles of the full pair capacity, or of a half or a quarter whose 2 or 4 waves per
    # pair group split every chunk and merge their states at the end; waves 0: the double tile
    # (twice the pairs in an 8-wave workgroup, head widths 128 and 256)
    if waves == 0 and head_dim not in hip_attention.PREFILL_DOUBLE_TILE_DIMS:
        pytest.skip("no double tile at this head width")
    s = build_scenario(steps, dtype=dtype, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16,
                       mode="mixed", seed=68, spare_blocks=2)
    launch = dict(partitions=0) if size == 0 else dict(partition_size=size)
    full = hip_attention.PREFILL_PAIRS[head_dim]
    pairs = 2 * full if waves == 0 else full // waves
    out = run_attention(s, prefill=True, tile_pairs=pairs, **launch)
    assert_parity(out, s.expected(np.float64), dtype, f"prefill/{name}/{size}/{pairs}")
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    if padding_rows:
        assert torch.count_nonzero(out[padding_rows]) == 0


@pytest.mark.parametrize("size", [0, 256])
@pytest.mark.parametrize("tile", ["double", "full", "half"])
@pytest.mark.parametrize("kind", ["a-huge-value", "all-small", "one-request-small", "normal"])
def test_multi_row_values_fp16_cannot_hold(kind: str, tile: str, size: int) -> None:
    # bf16 caches: the kernel runs P.V in fp16 where a chunk's values allow it and hands the
    # workgroups that met any other chunk to a bf16 pass (full and double tiles; split tiles run
    # the bf16 pass alone). A value of 65536 or more, or a context whose values all lie below
    # 2^-10, sends its tiles there; the rest stay on the fp16 pass
    s = build_scenario([(40, 600), (3, 300), (20, 200)], dtype="bf16", heads=8, kv_heads=2, head_dim=128,
                       block_size=16, mode="mixed", seed=70)
    v = s.v.copy()
    if kind == "a-huge-value":
        pos = 100  # request 0, a position every one of its rows sees
        v[s.table[0][pos // 16], pos % 16, 1, 5] = 99840.0
    elif kind == "all-small":
        v *= 1e-4
    elif kind == "one-request-small":
        for b in s.table[1][: -(-300 // 16)]:
            v[b] *= 1e-4
    s.v_bits = f32_to_bits(v, "bf16")
    full = hip_attention.PREFILL_PAIRS[128]
    pairs = {"double": 2 * full, "full": full, "half": full // 2}[tile]
    launch = dict(partitions=0) if size == 0 else dict(partition_size=size)
    out = run_attention(s, prefill=True, window=False, tile_pairs=pairs, **launch)
    assert_parity(out, s.expected(np.float64), "bf16", f"{kind}/{tile}/{size}")
    if tile == "half":
        return  # split tiles run one bf16 pass: no hand-off slots are written
    # the hand-off slots (one int32 per workgroup, after the partials in the shared workspace)
    meta = plan_scenario(s)
    n_slots = meta.plan.prefill_tiles(4, pairs, size, DEV, False).numel() // 4 * 2
    offset = 0
    if size:
        parts = -(-meta.block_table.shape[1] * 16 // size)
        offset = -(-_lib.lib().ayk_paged_attention_v2_workspace_bytes(sum(s.rows), 8, 128, parts) // 16) * 16
    slots = hip_attention._workspaces[DEV][offset:offset + 4 * n_slots].view(torch.int32).cpu()
    handed = int(slots.sum())
    if kind == "normal":
        assert handed == 0, "every workgroup stays on the fp16 pass"
    elif kind == "all-small":
        assert handed == n_slots
    else:
        assert 0 < handed < n_slots, (handed, n_slots)


@pytest.mark.parametrize("block_size", [1, 2])
def test_multi_row_partitions_across_table_segments(block_size: int) -> None:
    # partitions of 512 positions of one- and two-position blocks each span several staged
    # table segments (at most 511 entries at a time)
    s = build_scenario([(40, 1300), (9, 1400), (3, 5)], block_size=block_size, head_dim=128, heads=8,
                       kv_heads=2, mode="mixed", seed=45)
    expected = s.expected(np.float64)
    for size in (0, 512, 1024):
        launch = dict(partitions=0) if size == 0 else dict(partition_size=size)
        assert_parity(run_attention(s, prefill=True, **launch), expected, "bf16", f"bs{block_size}/{size}")


@pytest.mark.parametrize("requests,rows,context,heads,dim,dtype",
                         [(4, 512, 4096, 32, 128, "bf16"), (1, 2048, 2048, 32, 128, "bf16"),
                          (4, 512, 4096, 32, 64, "fp16")],
                         ids=["4x512-over-4K", "2048-row-prompt", "4x512-over-4K-fp16-d64"])
def test_multi_row_full_size_against_the_oracle(requests: int, rows: int, context: int, heads: int, dim: int,
                                                 dtype: str) -> None:
    # the benchmark's prefill chunks at full size (Llama-3-8B and -3.2-1B head shapes, block
    # 16, a permuted pool), the library's launch against the float64 oracle, every row
    print(f"full-size multi-row: {requests} x {rows} over {context}, D {dim}, {dtype}", flush=True)
    kv_heads, bs = 8, 16
    torch_dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[dtype]
    blocks = requests * (context // bs) + 1
    gen = torch.Generator(device=DEV).manual_seed(rows + dim)
    k = torch.randn((blocks, bs, kv_heads, dim), generator=gen, device=DEV).to(torch_dtype)
    v = torch.randn((blocks, bs, kv_heads, dim), generator=gen, device=DEV).to(torch_dtype)
    ids = torch.randperm(blocks - 1, generator=gen, device=DEV) + 1
    table = ids.view(requests, context // bs).to(torch.int32)
    meta = hip_attention.plan(ForwardMode.MIXED, torch.full((requests,), rows, dtype=torch.int32, device=DEV),
                              torch.full((requests,), context, dtype=torch.int32, device=DEV), table, bs)
    q = torch.randn((requests * rows, heads, dim), generator=gen, device=DEV).to(torch_dtype)
    out = torch.full_like(q, 7.0)
    hip_attention.attend(q, KVBuffers(k, v, KVLayoutKind.NHD, RAW_CODEC), meta, out, scale=dim**-0.5)
    torch.cuda.synchronize()
    expected = paged.attention_of_requests(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                           v.float().cpu().numpy(), table.cpu().numpy(),
                                           np.full(requests, context), scale=dim**-0.5,
                                           request_of_row=meta.request_of_row.cpu().numpy(),
                                           positions=meta.positions.cpu().numpy())
    assert_parity(out, expected, dtype, f"{requests} x {rows} over {context}")


@pytest.mark.parametrize("launch", [dict(partitions=0), dict(partitions=None, partition_size=128),
                                    dict(partitions=None, partition_size=128, tile_pairs=256, window=False)],
                         ids=["whole", "partitions", "double-tile"])
@pytest.mark.parametrize("steps", [[(40, 600), (3, 3), (7, 300)], [(4, 600), (3, 3), (1, 300), (2, 0)]],
                         ids=["multi-row-kernel", "window-launch"])
def test_multi_row_step_in_a_captured_graph(launch: dict, steps: list) -> None:
    # an eagerly planned multi-row step captures once it has run eagerly (its tile list and
    # workspace exist); every replay, with eager work between, matches the eager call. With at
    # most 16 / G rows per request the step takes the decode kernel's window launch.
    s = build_scenario(steps, heads=8, kv_heads=2, head_dim=128, block_size=16, mode="mixed", seed=46)
    buffers, meta = scenario_buffers(s), plan_scenario(s)
    assert (meta.plan.window_pairs(4) > 0) == (max(rows for rows, _ in steps) <= 4)
    q = to_device(s.q_bits, s.dtype)
    eager, out = torch.full_like(q, 7.0), torch.full_like(q, 7.0)
    hip_attention.attend_with(q, buffers, meta, eager, scale=s.scale, prefill=True, **launch)
    torch.cuda.synchronize()
    assert_parity(eager, s.expected(np.float64), "bf16", "eager")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, prefill=True, **launch)
    for _ in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    # a step never run eagerly has no tile list yet: capture refuses it before any launch, so
    # the capture ends empty (torch warns about that, and the warning is expected here)
    fresh = plan_scenario(s)
    with pytest.warns(UserWarning, match="Graph is empty"):
        with pytest.raises(BackendError, match="run the step once eagerly before capturing it"):
            with torch.cuda.graph(torch.cuda.CUDAGraph()):
                hip_attention.attend_with(q, buffers, fresh, out, scale=s.scale, prefill=True, **launch)
    torch.cuda.synchronize()


@pytest.mark.parametrize("block_size", [1, 3, 4, 5, 8, 12, 16, 24, 32, 48, 64, 100])
@pytest.mark.parametrize("qk", QK)
def test_block_sizes(block_size: int, qk: str) -> None:
    # any block size (the reference's CacheConfig accepts every positive one): powers of two
    # and others, odd ones included, whose positions the kernels divide by a magic number
    s = build_scenario([(1, 1), (1, 63), (1, 130), (2, 70), (1, 301)], block_size=block_size, head_dim=128,
                       heads=8, kv_heads=2, seed=43)
    expected = s.expected(np.float64)
    for prefill, window in ((False, None), (True, False), (True, True)):
        out = run_attention(s, None, qk, prefill, window=window)
        assert_parity(out, expected, "bf16", f"bs{block_size}/{prefill}/{window}")
    # v1 (one and several waves per head), v2 partitions that start inside a block, and the
    # multi-row kernel's partitions and smaller tiles
    launches = [dict(partitions=0, prefill=False), dict(partitions=3, partition_size=128, prefill=False),
                dict(partitions=None, partition_size=64, prefill=True, window=False),
                dict(partitions=None, partition_size=192, prefill=True, tile_pairs=32)]
    if qk == "mfma":
        launches.append(dict(partitions=0, prefill=False, waves=8))
    for launch in launches:
        out = run_attention(s, qk=qk if not launch.get("prefill") else None, **launch)
        assert_parity(out, expected, "bf16", f"bs{block_size}/{launch}")


EXTREME_CASES = [
    # a 128K-position context (v2 up to 2048 partitions of 64, v1 at 8 waves per head)
    ("long-context", dict(steps=[(1, 131072), (1, 5)], heads=8, kv_heads=1, head_dim=128, block_size=16)),
    # 4096 short decode rows (grids of tens of thousands of workgroups, work lists of 4096 items)
    ("many-rows", dict(steps=[(1, int(n)) for n in np.random.default_rng(7).integers(1, 40, size=4096)], heads=8,
                       kv_heads=2, head_dim=64, block_size=16)),
    # the largest block size the library takes, with a context spanning two blocks
    ("block-65536", dict(steps=[(1, 70000), (1, 3), (3, 65537)], heads=4, kv_heads=1, head_dim=64,
                         block_size=65536, mode="mixed")),
]


@pytest.mark.parametrize("name,shape", EXTREME_CASES, ids=[c[0] for c in EXTREME_CASES])
def test_extreme_shapes(name: str, shape: dict) -> None:
    shape = dict(shape)
    steps = shape.pop("steps")
    s = build_scenario(steps, seed=47, spare_blocks=1, **{"mode": "decode", **shape})
    expected = s.expected(np.float64)
    longest = max(n for _, n in steps)
    launches = [dict(partitions=None), dict(partitions=0, prefill=False, waves=8),
                dict(partitions=-(-longest // 64), partition_size=64, prefill=False)]
    if s.mode == "mixed":
        launches += [dict(partitions=None, prefill=True, window=False),
                     dict(partitions=None, partition_size=4096, prefill=True, window=False)]
    for launch in launches:
        out = run_attention(s, **launch)
        assert_parity(out, expected, s.dtype, f"{name}/{launch}")


@pytest.mark.parametrize("block_size", [1, 2, 3])
def test_table_segments(block_size: int) -> None:
    # a workgroup stages at most 511 table entries at a time: with blocks of 1-2 positions these
    # contexts span several staged segments, and the rows end at positions in different ones
    s = build_scenario([(40, 1300), (1, 1100), (9, 1400)], block_size=block_size, head_dim=128, heads=8,
                       kv_heads=2, mode="mixed", seed=44)
    expected = s.expected(np.float64)
    for prefill in (False, True):
        assert_parity(run_attention(s, None, None, prefill), expected, "bf16", f"bs{block_size}/{prefill}")
    # windows of 2-4 rows over contexts that span several segments
    w = build_scenario([(2, 1300), (1, 1100), (4, 1400)], block_size=block_size, head_dim=128, heads=8,
                       kv_heads=2, mode="mixed", seed=45)
    for launch in (dict(partitions=0), dict(partition_size=512)):
        assert_parity(run_attention(w, prefill=True, window=True, **launch), w.expected(np.float64), "bf16",
                      f"bs{block_size}/windows/{launch}")


@pytest.mark.parametrize("heads,qk", [(1, "dpp"), (4, "mfma")])
def test_first_table_segment_wider_than_its_prefetch(heads: int, qk: str) -> None:
    # One key/value head makes one-wave (64-thread) workgroups, whose read-ahead of the first
    # table segment covers 128 entries; with blocks of one position that segment holds 511, so
    # the rest are read when it is staged. v1 over whole contexts, v2 over partitions of 1024.
    s = build_scenario([(1, 1300), (1, 700), (1, 129), (1, 0), (1, 1024)], block_size=1, head_dim=128, heads=heads,
                       kv_heads=1, mode="decode", seed=46)
    expected = s.expected(np.float64)
    for launch in (dict(partitions=0, waves=1), dict(partitions=2, partition_size=1024)):
        assert_parity(run_attention(s, qk=qk, **launch), expected, "bf16", f"{qk}/{launch}")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("qk", QK)
def test_split_partitions_agree_with_the_oracle_and_v1(dtype: str, head_dim: int, qk: str) -> None:
    # contexts across several 512-position partitions, one ending inside a block and a partition
    s = build_scenario([(1, 1500), (1, 513), (1, 512), (1, 2048), (1, 7), (1, 0)], dtype=dtype,
                       head_dim=head_dim, heads=8, kv_heads=2, block_size=16, mode="decode", seed=47)
    expected = s.expected(np.float64)
    v1 = run_attention(s, 0, qk)
    v2 = run_attention(s, 4, qk)
    assert_parity(v1, expected, dtype, "v1")
    assert_parity(v2, expected, dtype, "v2")
    auto = run_attention(s, None, qk)
    assert_parity(auto, expected, dtype, "auto")


@pytest.mark.parametrize("waves", [1, 2, 4, 8])
@pytest.mark.parametrize("heads,kv_heads,head_dim,dtype", [(8, 2, 64, "fp16"), (32, 8, 128, "bf16"),
                                                           (4, 4, 256, "bf16"), (16, 1, 128, "fp16"),
                                                           (40, 10, 128, "bf16"), (9, 3, 64, "bf16")])
def test_v1_context_split_among_waves(waves: int, heads: int, kv_heads: int, head_dim: int, dtype: str) -> None:
    # v1 with each (row, key/value head)'s context shared by 1-8 waves (every n-th chunk each,
    # states merged in LDS in wave order): contexts shorter than one chunk per wave, ending
    # inside blocks and chunks, a padding row, and a head count that leaves a workgroup's
    # last head slots idle (10 heads at 8 / waves per workgroup)
    s = build_scenario([(1, 1), (1, 17), (1, 0), (1, 2047), (1, 300), (1, 64), (1, 95)], dtype=dtype,
                       heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16, mode="decode", seed=93)
    expected = s.expected(np.float64)
    out = run_attention(s, 0, "mfma", waves=waves)
    assert_parity(out, expected, dtype, f"v1/{waves} waves")
    assert torch.count_nonzero(out[2]) == 0
    again = run_attention(s, 0, "mfma", waves=waves)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    # v2: each partition shared by the waves the same way, either merge site
    for merge in ("reduce-kernel", "in-kernel"):
        out = run_attention(s, 8, "mfma", waves=waves, partition_size=256, merge=merge)
        assert_parity(out, expected, dtype, f"v2/{waves} waves/{merge}")
        assert torch.count_nonzero(out[2]) == 0
    assert counters_are_clear()


@pytest.mark.parametrize("block_size", [1, 2])
def test_v1_context_split_across_table_segments(block_size: int) -> None:
    # one- and two-position blocks: each wave's chunks cross the staged table segments
    s = build_scenario([(1, 1300), (1, 1100), (1, 3)], block_size=block_size, head_dim=128, heads=8,
                       kv_heads=2, mode="decode", seed=94)
    expected = s.expected(np.float64)
    for waves in (2, 8):
        assert_parity(run_attention(s, 0, "mfma", waves=waves), expected, "bf16", f"bs{block_size}/{waves}")


# --- fp8 e4m3 codec ---------------------------------------------------------------------------


def fp8_buffers(s: Scenario) -> tuple[KVBuffers, np.ndarray, np.ndarray]:
    """The scenario's caches encoded to fp8 codes by the oracle (NaN slots stay NaN codes)."""
    kc, vc = f32_to_e4m3(s.k), f32_to_e4m3(s.v)
    layout = KVLayoutKind.NHD if s.layout == "nhd" else KVLayoutKind.HND
    k = torch.from_numpy(kc).view(torch.float8_e4m3fn).to(DEV)
    v = torch.from_numpy(vc).view(torch.float8_e4m3fn).to(DEV)
    return KVBuffers(k, v, layout, FP8_E4M3_CODEC), kc, vc


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("head_dim", [64, 128, 12, 8])
def test_fp8_store_is_bit_exact(dtype: str, layout: str, head_dim: int) -> None:
    s = build_scenario([(3, 9), (1, 2), (2, 30)], dtype=dtype, layout=layout, head_dim=head_dim, block_size=4,
                       kv_heads=2, seed=83)
    buffers, kc, vc = fp8_buffers(s)
    rng = np.random.default_rng(84)
    n = len(s.plan["slot_mapping"])
    vals = rng.standard_normal((2, n, s.kv_heads, head_dim)) * np.exp2(rng.uniform(-13, 9, (2, n, s.kv_heads, 1)))
    special = [448.0, 464.0, 470.0, 500.0, -0.0, 1e-3, 2.0 ** -10, 3 * 2.0 ** -10, np.nan, np.inf, -600.0]
    vals.reshape(-1)[: len(special)] = special
    bits = f32_to_bits(vals.astype(np.float32), dtype)
    rows = bits_to_f32(bits, dtype)
    meta = plan_scenario(s)
    hip_kvcache.store(to_device(bits[0], dtype), to_device(bits[1], dtype), buffers, meta)
    torch.cuda.synchronize()
    paged.store(kc, vc, f32_to_e4m3(rows[0]), f32_to_e4m3(rows[1]), s.plan["slot_mapping"], layout)
    assert np.array_equal(buffers.k.view(torch.uint8).cpu().numpy(), kc)
    assert np.array_equal(buffers.v.view(torch.uint8).cpu().numpy(), vc)
    with pytest.raises(BackendError, match="over a 'fp8_e4m3' cache the hip backend computes in float16"):
        hip_kvcache.store(to_device(bits[0], dtype).float(), to_device(bits[1], dtype).float(), buffers, meta)


FP8_CASES = [
    ("decode", [(1, 16), (1, 0), (1, 1300), (1, 33), (1, 517)], "decode"),
    ("mixed", [(7, 7), (1, 9), (40, 600), (2, 0), (3, 1100)], "mixed"),
    ("windows", [(2, 700), (1, 0), (2, 1300), (1, 9)], "mixed"),
]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 2, 128), (32, 8, 64), (64, 8, 128), (4, 4, 256), (32, 8, 256)])
@pytest.mark.parametrize("name,steps,mode", FP8_CASES, ids=[c[0] for c in FP8_CASES])
def test_fp8_attention_matches_the_oracle_on_decoded_values(dtype: str, layout: str, heads: int, kv_heads: int,
                                                            head_dim: int, name: str, steps: list, mode: str) -> None:
    s = build_scenario(steps, dtype=dtype, layout=layout, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                       block_size=16, mode=mode, seed=89)
    buffers, kc, vc = fp8_buffers(s)
    expected = s.expected(np.float64, k=e4m3_to_f32(kc), v=e4m3_to_f32(vc))
    meta = plan_scenario(s)
    q = to_device(s.q_bits, dtype)
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    launches = [("v1", dict(partitions=0, prefill=False)),
                ("v1/1 wave", dict(partitions=0, prefill=False, waves=1)),
                ("v1/8 waves", dict(partitions=0, prefill=False, waves=8)),
                ("v2/in-kernel", dict(partitions=6, partition_size=256, merge="in-kernel", prefill=False)),
                ("v2/reduce-kernel", dict(partitions=6, partition_size=256, merge="reduce-kernel", prefill=False)),
                ("auto", dict(partitions=None))]
    if mode == "mixed":
        launches.append(("multi-row", dict(partitions=None, prefill=True, window=False)))
        if meta.plan.window_pairs(heads // kv_heads):
            launches.append(("windows", dict(partitions=None, prefill=True, window=True)))
            launches.append(("windows/256", dict(partitions=None, partition_size=256, prefill=True, window=True)))
        full = hip_attention.PREFILL_PAIRS[head_dim]
        for waves in (2, 4):
            if full // waves >= heads // kv_heads:
                launches.append((f"multi-row/{waves} waves per group",
                                 dict(partitions=None, partition_size=256, prefill=True, tile_pairs=full // waves)))
    for label, launch in launches:
        out = torch.full_like(q, 7.0)
        hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, **launch)
        torch.cuda.synchronize()
        assert_parity(out, expected, dtype, f"fp8 {name} {label}")
        if padding_rows:
            assert torch.count_nonzero(out[padding_rows]) == 0
    assert counters_are_clear()


SCALED_STEPS = [(1, 16), (1, 0), (1, 1300), (7, 600), (2, 33), (3, 1100)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 2, 128), (32, 8, 64)])
def test_scaled_fp8_cache_holds_large_keys(dtype: str, layout: str, heads: int, kv_heads: int,
                                           head_dim: int) -> None:
    # a layer whose keys reach 4,000 (and values 0.015): stored with k_scale = 4000 / 448 and
    # v_scale = 0.02 / 448 they stay finite; the KV write is bit-exact against the oracle's
    # scaled encoder, and every launch's output matches the float64 oracle on code * scale
    from ayaka_amd.kvcache import fp8_e4m3_codec
    from oracle.numerics import f32_to_e4m3_scaled

    s = build_scenario(SCALED_STEPS, dtype=dtype, layout=layout, heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, block_size=16, mode="mixed", seed=91)
    k_scale, v_scale = 4000.0 / 448.0, 0.02 / 448.0
    codec = fp8_e4m3_codec(k_scale, v_scale)
    k_scale, v_scale = codec.k_scale, codec.v_scale
    rng = np.random.default_rng(92)
    big_k = np.clip(rng.standard_normal(s.k.shape) * 1500.0, -4000, 4000)
    small_v = s.v * 0.003
    kc = f32_to_e4m3_scaled(bits_to_f32(f32_to_bits(big_k.astype(np.float32), dtype), dtype), k_scale)
    vc = f32_to_e4m3_scaled(bits_to_f32(f32_to_bits(small_v.astype(np.float32), dtype), dtype), v_scale)
    kind = KVLayoutKind.NHD if layout == "nhd" else KVLayoutKind.HND
    buffers = KVBuffers(torch.from_numpy(kc).view(torch.float8_e4m3fn).to(DEV),
                        torch.from_numpy(vc).view(torch.float8_e4m3fn).to(DEV), kind, codec)
    meta = plan_scenario(s)
    # the step's own rows written through the library: large keys, small values
    n = len(s.plan["slot_mapping"])
    rows_k = np.clip(rng.standard_normal((n, kv_heads, head_dim)) * 1500.0, -4000, 4000).astype(np.float32)
    rows_k.reshape(-1)[:4] = [4000.0, -4000.0, 3999.0, 0.5]
    rows_v = (rng.standard_normal((n, kv_heads, head_dim)) * 0.003).astype(np.float32)
    bits_k, bits_v = f32_to_bits(rows_k, dtype), f32_to_bits(rows_v, dtype)
    hip_kvcache.store(to_device(bits_k, dtype), to_device(bits_v, dtype), buffers, meta)
    torch.cuda.synchronize()
    paged.store(kc, vc, f32_to_e4m3_scaled(bits_to_f32(bits_k, dtype), k_scale),
                f32_to_e4m3_scaled(bits_to_f32(bits_v, dtype), v_scale), s.plan["slot_mapping"], layout)
    assert np.array_equal(buffers.k.view(torch.uint8).cpu().numpy(), kc)
    assert np.array_equal(buffers.v.view(torch.uint8).cpu().numpy(), vc)
    context = np.zeros(kc.shape, dtype=bool)  # every cache element some context reads
    context_nhd = paged.nhd(context, layout)
    for r, n in enumerate(s.lengths):
        for t in range(n):
            context_nhd[s.table[r, t // 16], t % 16] = True
    assert np.isfinite(e4m3_to_f32(kc)[context]).all() and np.isfinite(e4m3_to_f32(vc)[context]).all()
    real = s.plan["slot_mapping"] != 0
    stored = e4m3_to_f32(paged.nhd(kc, layout).reshape(-1, kv_heads, head_dim)[s.plan["slot_mapping"][real]])
    assert np.isfinite(stored).all() and np.abs(stored * k_scale).max() > 3000  # large keys kept finite
    q = to_device(f32_to_bits((s.q * 0.01).astype(np.float32), dtype), dtype)  # scores of a sane range
    expected = paged.attention(bits_to_f32(f32_to_bits((s.q * 0.01).astype(np.float32), dtype), dtype),
                               e4m3_to_f32(kc).astype(np.float64) * k_scale,
                               e4m3_to_f32(vc).astype(np.float64) * v_scale, s.table, np.asarray(s.lengths),
                               scale=s.scale, layout=layout, request_of_row=s.plan["request_of_row"],
                               positions=s.plan["positions"], precision=np.float64)
    full = hip_attention.PREFILL_PAIRS[head_dim]
    launches = [("multi-row", dict(partitions=None, prefill=True, window=False)),
                ("multi-row/256/quarter", dict(partitions=None, partition_size=256, prefill=True, tile_pairs=full // 4)),
                ("per-row v1", dict(partitions=0, prefill=False)),
                ("per-row v2/in-kernel", dict(partitions=6, partition_size=256, merge="in-kernel", prefill=False)),
                ("per-row v2/reduce-kernel", dict(partitions=6, partition_size=256, merge="reduce-kernel",
                                                  prefill=False)),
                ("auto", dict(partitions=None))]
    for label, launch in launches:
        out = torch.full_like(q, 7.0)
        hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, **launch)
        torch.cuda.synchronize()
        assert_parity(out, expected, dtype, f"scaled fp8 {label}")
    # decode rows of the same caches: v1, v2 and the window launch
    decode = build_scenario([(1, n) for n in s.lengths], dtype=dtype, layout=layout, heads=heads, kv_heads=kv_heads,
                            head_dim=head_dim, block_size=16, mode="decode", seed=93)
    decode.table = s.table
    dmeta = plan_scenario(decode)
    dq = to_device(f32_to_bits((decode.q * 0.01).astype(np.float32), dtype), dtype)
    dexpected = paged.attention(bits_to_f32(f32_to_bits((decode.q * 0.01).astype(np.float32), dtype), dtype),
                                e4m3_to_f32(kc).astype(np.float64) * k_scale,
                                e4m3_to_f32(vc).astype(np.float64) * v_scale, s.table, np.asarray(s.lengths),
                                scale=s.scale, layout=layout, precision=np.float64)
    for label, launch in [("v1", dict(partitions=0)), ("v1/8 waves", dict(partitions=0, waves=8)),
                          ("v2", dict(partitions=11, partition_size=128)), ("auto", dict(partitions=None))]:
        out = torch.full_like(dq, 7.0)
        hip_attention.attend_with(dq, buffers, dmeta, out, scale=s.scale, **launch)
        torch.cuda.synchronize()
        assert_parity(out, dexpected, dtype, f"scaled fp8 decode {label}")


def test_unit_scales_are_the_unscaled_codec_bit_for_bit() -> None:
    # fp8_e4m3_codec(1, 1) stores and reads exactly as the plain codec
    from ayaka_amd.kvcache import fp8_e4m3_codec

    s = build_scenario([(1, 700), (1, 33), (40, 300)], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="mixed", seed=94)
    plain, _, _ = fp8_buffers(s)
    unit = KVBuffers(plain.k.clone(), plain.v.clone(), plain.layout, fp8_e4m3_codec(1.0, 1.0))
    meta = plan_scenario(s)
    rng = np.random.default_rng(95)
    n = len(s.plan["slot_mapping"])
    rows = to_device(f32_to_bits((rng.standard_normal((2, n, 2, 128)) * 50).astype(np.float32), "bf16"), "bf16")
    for buffers in (plain, unit):
        hip_kvcache.store(rows[0], rows[1], buffers, meta)
    q = to_device(s.q_bits, "bf16")
    outs = []
    for buffers in (plain, unit):
        out = torch.full_like(q, 7.0)
        hip_attention.attend(q, buffers, meta, out, scale=s.scale)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(plain.k.view(torch.uint8), unit.k.view(torch.uint8))
    assert torch.equal(plain.v.view(torch.uint8), unit.v.view(torch.uint8))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def counters_are_clear() -> bool:
    return all(int(c.abs().max()) == 0 for c in hip_attention._counters.values())


@pytest.mark.parametrize("shape", ["8 slots, 3 batches", "4 slots, 2 batches", "1 slot"])
def test_reduce_kernel_slot_shapes(shape: str) -> None:
    # the reduce kernel's three shapes, chosen by partitions per row and the grid: 8 slots per
    # (row, head) pair for few pairs of many partitions (here 133 partitions of 64: three
    # batches of 8 per slot), 4 slots for many pairs of many partitions (41: two batches),
    # one slot for many pairs of at most 16 (most rows here hold one partition)
    rng = np.random.default_rng(71)
    if shape == "8 slots, 3 batches":
        lengths = [8500, 4100, 0, 64, 65]
    elif shape == "4 slots, 2 batches":
        lengths = [2600, 0, 1] + rng.integers(1, 2600, 61).tolist()
    else:
        lengths = [1000, 0] + rng.integers(1, 64, 200).tolist() + rng.integers(64, 1000, 54).tolist()
    s = build_scenario([(1, n) for n in lengths], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="decode", seed=72)
    parts = -(-max(lengths) // 64)
    out = run_attention(s, parts, "mfma", partition_size=64, merge="reduce-kernel")
    assert_parity(out, s.expected(np.float64), "bf16", shape)
    assert torch.count_nonzero(out[lengths.index(0)]) == 0


@pytest.mark.parametrize("qk", QK)
@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (40, 10), (96, 12), (12, 12)])
def test_single_launch_merge_agrees_with_the_reduce_kernel(qk: str, heads: int, kv_heads: int) -> None:
    # 10 and 12 key/value heads leave idle waves in the second workgroup of a row; rows of
    # 0, 1 and many partitions, one ending inside a partition
    s = build_scenario([(1, 2500), (1, 0), (1, 64), (1, 1024), (1, 1500), (1, 7)], heads=heads,
                       kv_heads=kv_heads, head_dim=128, block_size=16, mode="decode", seed=67)
    expected = s.expected(np.float64)
    fused = run_attention(s, 10, qk, merge="in-kernel")
    assert counters_are_clear()
    separate = run_attention(s, 10, qk, partition_size=256, merge="reduce-kernel")
    fused256 = run_attention(s, 10, qk, partition_size=256, merge="in-kernel")
    assert counters_are_clear()
    for name, out in (("fused", fused), ("separate", separate), ("fused256", fused256)):
        assert_parity(out, expected, "bf16", name)
    # a smaller step in between leaves the counters ready for the next one
    small = build_scenario([(1, 700), (1, 300)], heads=heads, kv_heads=kv_heads, head_dim=128, block_size=16,
                           mode="decode", seed=68)
    assert_parity(run_attention(small, 3, qk, partition_size=256, merge="in-kernel"), small.expected(np.float64),
                  "bf16", "small")
    again = run_attention(s, 10, qk, merge="in-kernel")
    assert counters_are_clear()
    assert torch.equal(fused.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("qk", QK)
def test_one_partition_reproduces_v1_bit_for_bit(qk: str) -> None:
    s = build_scenario([(1, 300), (1, 17), (1, 512)], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="decode", seed=53)
    v1 = run_attention(s, 0, qk, waves=1)
    v2 = run_attention(s, 1, qk)
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))


def test_outlier_keys_keep_the_max_tracking_exact() -> None:
    # keys scaled by 20 at a few positions, late in the context, after the running max settled
    s = build_scenario([(1, 3000), (1, 700), (1, 40)], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="decode", seed=59)
    k = paged.nhd(s.k, "nhd").copy()
    rng = np.random.default_rng(3)
    for b, length in enumerate(s.lengths):
        for pos in rng.choice(length, size=max(1, length // 300), replace=False):
            blk, off = s.table[b, pos // 16], pos % 16
            k[blk, off] *= 20.0
    s.k_bits = f32_to_bits(k, "bf16")
    expected = s.expected(np.float64)
    for qk in QK:
        for partitions in (0, 6):
            assert_parity(run_attention(s, partitions, qk), expected, "bf16", f"outliers/{qk}/{partitions}")


def test_one_visible_key_returns_its_value_exactly() -> None:
    s = build_scenario([(1, 1), (1, 1)], heads=4, kv_heads=2, head_dim=64, block_size=16, mode="decode", seed=3)
    out = run_attention(s)
    v = paged.nhd(s.v_bits, s.layout)
    for b in range(2):
        want = np.repeat(v[s.table[b, 0], 0], 2, axis=0)
        assert np.array_equal(to_bits(out[b]), want)


def test_scale_zero_averages_the_visible_values() -> None:
    s = build_scenario([(2, 600)], heads=4, kv_heads=2, head_dim=64, block_size=16, seed=5, scale=0.0)
    assert_parity(run_attention(s), s.expected(np.float64), "bf16", "scale0")


def test_the_cache_is_only_read() -> None:
    s = build_scenario([(3, 90), (1, 700)], heads=4, kv_heads=2, head_dim=64, block_size=16, seed=6)
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    q = to_device(s.q_bits, s.dtype)
    out = torch.empty_like(q)
    hip_attention.attend(q, buffers, meta, out, scale=s.scale)
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(buffers.k), s.k_bits) and np.array_equal(to_bits(buffers.v), s.v_bits)


def test_golden_fixture() -> None:
    data = np.load(GOLDEN / "smollm2_small.npz")
    buffers = KVBuffers(to_device(data["k_cache_before"], "fp16"), to_device(data["v_cache_before"], "fp16"),
                        KVLayoutKind.NHD, RAW_CODEC)
    table = torch.from_numpy(data["table"]).to(DEV)
    lengths = torch.from_numpy(data["lengths"]).to(DEV)
    write = hip_attention.plan(ForwardMode.MIXED, torch.from_numpy(data["rows_per_request"]).to(DEV), lengths,
                               table, 16)
    assert write.slot_mapping.cpu().numpy().tolist() == data["slot_mapping"].tolist()
    hip_kvcache.store(to_device(data["k_new"], "fp16"), to_device(data["v_new"], "fp16"), buffers, write)
    decode = hip_attention.plan(ForwardMode.DECODE, torch.ones(4, dtype=torch.int32, device=DEV), lengths, table, 16)
    q = to_device(data["q"], "fp16")
    out = torch.empty_like(q)
    hip_attention.attend(q, buffers, decode, out, scale=float(data["scale"]))
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(buffers.k), data["k_cache"])
    assert np.array_equal(to_bits(buffers.v), data["v_cache"])
    assert_parity(out, data["expected"], "fp16", "golden")


# --- benchmark configurations at full size --------------------------------------------------

def _report(out: torch.Tensor, e32: np.ndarray, e64: np.ndarray, dtype: str) -> dict:
    """The north star's raw figures against the float32 oracle (max-abs, relative L2), and the
    net-of-rounding ones against the float64 oracle that the tests bound."""
    got = out.float().cpu().numpy().astype(np.float64)
    norm = float(np.linalg.norm(e32)) or 1.0
    net = parity_report(got, e64, dtype)
    return {"max_abs": float(np.abs(got - e32).max()), "rel_l2": float(np.linalg.norm(got - e32)) / norm,
            "max_abs_excess_fp64": net["max_abs_excess"], "rel_l2_rounded_fp64": net["rel_l2"]}


@pytest.mark.parametrize("index", [1, 2, 3, 4, 5])
def test_benchmark_configuration(index: int) -> None:
    # every row of every configuration against the oracle; the raw figures (ours, and the
    # reference's own rounding of the float32 result) are written to $AYAKA_PARITY_DIR
    cfg = workloads.config(index)
    print(f"config {index} {cfg.name}", flush=True)
    step = workloads.build(cfg, DEV)
    layout = KVLayoutKind.NHD
    buffers = KVBuffers(step.k_cache, step.v_cache, layout, RAW_CODEC)
    write = hip_attention.plan(ForwardMode.MIXED, step.rows_per_request, step.lengths, step.table, cfg.block_size)
    hip_kvcache.store(step.k_new, step.v_new, buffers, write)
    # the write is bit-exact: read the slots back
    slots = write.slot_mapping
    got_k = step.k_cache.view(-1, cfg.kv_heads, cfg.head_dim)[slots]
    got_v = step.v_cache.view(-1, cfg.kv_heads, cfg.head_dim)[slots]
    assert torch.equal(got_k.view(torch.int16), step.k_new.view(torch.int16))
    assert torch.equal(got_v.view(torch.int16), step.v_new.view(torch.int16))

    decode = hip_attention.plan(ForwardMode.DECODE, torch.ones(cfg.batch, dtype=torch.int32, device=DEV),
                                step.lengths, step.table, cfg.block_size)
    outs = {}
    v2_parts = -(-max(cfg.lengths) // hip_attention.PARTITION_SIZE)
    for name, parts, qk, merge in (("v1-dpp", 0, "dpp", None), ("v1-mfma", 0, "mfma", None),
                                   ("v2-dpp", v2_parts, "dpp", None), ("v2-mfma", v2_parts, "mfma", None),
                                   ("v2-reduce-kernel", v2_parts, None, "reduce-kernel"),
                                   ("v2-in-kernel", v2_parts, None, "in-kernel"), ("auto", None, None, None)):
        out = torch.empty_like(step.q)
        hip_attention.attend_with(step.q, buffers, decode, out, scale=cfg.scale, partitions=parts, qk=qk,
                                  merge=merge)
        outs[name] = out
    torch.cuda.synchronize()
    rows = list(range(cfg.batch))
    expected = oracle_rows(step, rows, np.float64)
    e32 = oracle_rows(step, rows, np.float32).astype(np.float64)
    for name, out in outs.items():
        assert_parity(out, expected, cfg.dtype_label, f"config {index} {name}")
    assert counters_are_clear()
    rounded = bits_to_f32(f32_to_bits(e32.astype(np.float32), cfg.dtype_label), cfg.dtype_label)
    split = decode.plan.split_for(cfg.kv_heads, cfg.heads // cfg.kv_heads)
    record = {
        "config": f"C{index} {cfg.name}", "dtype": cfg.dtype_label, "rows": cfg.batch,
        "auto_launch": f"v1, {split.waves} waves" if not split.partitions else
                       f"v2, {split.partitions} x {split.partition_size}",
        "reference_rounding": _report(torch.from_numpy(rounded), e32, expected, cfg.dtype_label),
        **{name: _report(outs[name], e32, expected, cfg.dtype_label) for name in ("auto", "v1-mfma", "v2-mfma")},
    }
    target = os.environ.get("AYAKA_PARITY_DIR")
    if target:
        Path(target).mkdir(parents=True, exist_ok=True)
        (Path(target) / f"parity_c{index}.json").write_text(json.dumps(record, indent=1))


def test_full_size_verify_windows() -> None:
    # the benchmark's verify-window step (32 requests x 4 rows over 4K, Llama-3-8B shape) on the
    # window launch, every row against the oracle
    requests, rows, context, bs = 32, 4, 4096, 16
    gen = torch.Generator(device=DEV).manual_seed(4)
    blocks = requests * context // bs + 1
    k = torch.randn((blocks, bs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn((blocks, bs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    k[0], v[0] = float("nan"), float("nan")
    ids = torch.randperm(blocks - 1, generator=gen, device=DEV) + 1
    table = ids.view(requests, context // bs).to(torch.int32)
    meta = hip_attention.plan(ForwardMode.MIXED, torch.full((requests,), rows, dtype=torch.int32, device=DEV),
                              torch.full((requests,), context, dtype=torch.int32, device=DEV), table, bs)
    assert meta.plan.window_pairs(4) > 0
    q = torch.randn((requests * rows, 32, 128), generator=gen, device=DEV).to(torch.bfloat16)
    buffers = KVBuffers(k, v, KVLayoutKind.NHD, RAW_CODEC)
    for launch in (dict(partitions=None), dict(partitions=0)):
        out = torch.full_like(q, 7.0)
        hip_attention.attend_with(q, buffers, meta, out, scale=128 ** -0.5, prefill=True, window=True, **launch)
        torch.cuda.synchronize()
        expected = paged.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                   table.cpu().numpy(), np.full(requests, context),
                                   request_of_row=meta.request_of_row.cpu().numpy(),
                                   positions=meta.positions.cpu().numpy(), scale=128 ** -0.5, precision=np.float64)
        assert_parity(out, expected, "bf16", f"windows {launch}")


# --- graph metadata and capture ---------------------------------------------------------------


@pytest.mark.parametrize("heads,kv_heads,max_blocks,bucket,fp8,layout",
                         [(8, 2, 80, 4, False, "nhd"), (8, 2, 80, 4, False, "hnd"), (32, 8, 512, 16, False, "nhd"),
                          (32, 8, 512, 16, True, "nhd"), (16, 8, 512, 16, False, "nhd")])
def test_graph_metadata_replays_match_eager_steps(heads: int, kv_heads: int, max_blocks: int, bucket: int,
                                                  fp8: bool, layout: str) -> None:
    # (16, 8): two query heads per key/value head, which the DPP q.k kernel serves
    rng = np.random.default_rng(61)
    dim, bs = 128, 16
    num_blocks = 1 + bucket * max_blocks
    cache_dtype = torch.float8_e4m3fn if fp8 else torch.bfloat16
    shape = (num_blocks, bs, kv_heads, dim) if layout == "nhd" else (num_blocks, kv_heads, bs, dim)
    k_cache = (torch.randn(shape, device=DEV)).to(cache_dtype)
    v_cache = (torch.randn(shape, device=DEV)).to(cache_dtype)
    kind = KVLayoutKind.NHD if layout == "nhd" else KVLayoutKind.HND
    buffers = KVBuffers(k_cache, v_cache, kind, FP8_E4M3_CODEC if fp8 else RAW_CODEC)
    perm = rng.permutation(np.arange(1, num_blocks)).reshape(bucket, max_blocks).astype(np.int32)
    meta = hip_attention.graph_metadata(bucket, max_blocks, bs, DEV)
    q = torch.zeros((bucket, heads, dim), dtype=torch.bfloat16, device=DEV)
    k_new = torch.zeros((bucket, kv_heads, dim), dtype=torch.bfloat16, device=DEV)
    v_new = torch.zeros_like(k_new)
    out = torch.zeros_like(q)

    def step() -> None:
        hip_kvcache.store(k_new, v_new, buffers, meta)
        hip_attention.attend(q, buffers, meta, out, scale=dim**-0.5)

    # one eager step sizes the scratch, then capture
    lengths0 = torch.ones(bucket, dtype=torch.int32)
    hip_attention.update_graph_metadata(meta, lengths0, torch.from_numpy(perm))
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    if bucket == 4:
        trials = [[5, 0, 1000, 17], [1280, 640, 0, 0], [33, 1, 2, 900]]
    else:  # ragged batches: the staged partition size and work list change from step to step
        cap = max_blocks * bs
        trials = [[int(x) for x in rng.integers(0, cap + 1, size=bucket)] for _ in range(2)]
        trials += [[cap] + [0] * (bucket - 1), [1] * bucket, [cap] * bucket]
    for trial, lens in enumerate(trials):
        lengths = torch.tensor(lens, dtype=torch.int32)
        table = torch.from_numpy(perm.copy())
        q.copy_(torch.randn(q.shape, device=DEV).to(torch.bfloat16))
        k_new.copy_(torch.randn(k_new.shape, device=DEV).to(torch.bfloat16))
        v_new.copy_(torch.randn(v_new.shape, device=DEV).to(torch.bfloat16))
        hip_attention.update_graph_metadata(meta, lengths, table)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        # The same step planned eagerly. With the replay's launch shape (the split a
        # graph bucket gets from its table width) it is the same arithmetic, bit for bit; with
        # the eager plan's own split it agrees within the contract's tolerance
        # (the reference compares graph and planned steps with a tolerance too,
        # tests/ops/test_attention_graph.py:56-73).
        eager_meta = hip_attention.plan(ForwardMode.DECODE, torch.ones(bucket, dtype=torch.int32, device=DEV),
                                        lengths.to(DEV), table.to(DEV), bs)
        assert eager_meta.slot_mapping.tolist() == meta.slot_mapping.tolist()
        assert eager_meta.positions.tolist() == meta.positions.tolist()
        # a v2 replay runs the partition size the update staged, over a grid of the bucket's
        # capacity and the bucket's partition count (which sets the reduce kernel's fold
        # width), so the library may merge the partitions at another site than the eager
        # work list's; the same site and partition count fold in the same order
        staged_size = meta.plan.staged_partition_size
        assert staged_size % 64 == 0 and staged_size >= meta.plan.min_size
        site = hip_attention.graph_merge_site(meta.plan.capacity, kv_heads, heads // kv_heads,
                                              meta.plan.partitions)
        same_shape = torch.empty_like(out)
        if meta.plan.partitions > 1:
            hip_attention.attend_with(q, buffers, eager_meta, same_shape, scale=dim**-0.5,
                                      partitions=meta.plan.partitions, partition_size=staged_size,
                                      merge=site)
        else:
            hip_attention.attend_with(q, buffers, eager_meta, same_shape, scale=dim**-0.5, partitions=0)
        eager_out = torch.empty_like(out)
        hip_attention.attend(q, buffers, eager_meta, eager_out, scale=dim**-0.5)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), same_shape.view(torch.int16)), f"replay {trial}"
        diff = (replayed.float() - eager_out.float()).abs().max().item()
        assert diff <= 4 * EPS["bf16"] * eager_out.float().abs().max().item(), f"replay {trial}: {diff}"
        assert torch.count_nonzero(replayed[[i for i, n in enumerate(lens) if n == 0]]) == 0
        if trial in (0, len(trials) - 1):  # the replay itself against the float64 oracle
            expected = paged.attention(q.float().cpu().numpy(), k_cache.float().cpu().numpy(),
                                       v_cache.float().cpu().numpy(), table.numpy(), np.array(lens),
                                       scale=dim**-0.5, layout=layout, precision=np.float64)
            assert_parity(replayed, expected, "bf16", f"replay {trial} against the oracle")


# --- block ops ------------------------------------------------------------------------------


@pytest.mark.parametrize("mode,steps", [("decode", [(1, 900), (1, 0), (1, 5000)]),
                                        ("mixed", [(40, 600), (3, 3), (7, 300)]),
                                        ("mixed", [(4, 600), (3, 3), (1, 300)])], ids=["decode", "multi-row", "windows"])
def test_repeated_calls_replay_the_recorded_launch(mode: str, steps: list) -> None:
    # attend and store record their library call in the step's plan; later calls with the same
    # objects replay it: new contents of the same tensors are read, other objects are checked anew
    s = build_scenario(steps, heads=8, kv_heads=2, head_dim=128, block_size=16, mode=mode, seed=99)
    buffers, meta = scenario_buffers(s), plan_scenario(s)
    q = to_device(s.q_bits, "bf16")
    out = torch.full_like(q, 7.0)
    for _ in range(3):
        hip_attention.attend(q, buffers, meta, out, scale=s.scale)
    torch.cuda.synchronize()
    assert len(meta.plan.launches) == 1
    assert_parity(out, s.expected(np.float64), "bf16", "replayed")
    first = out.clone()
    q.mul_(-1.0)  # same tensor, new contents: the replay reads them
    hip_attention.attend(q, buffers, meta, out, scale=s.scale)
    fresh = torch.full_like(out, 7.0)
    hip_attention.attend_with(q, buffers, meta, fresh, scale=s.scale, partitions=None)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), fresh.view(torch.int16))
    assert not torch.equal(out, first)
    other = torch.full_like(out, 7.0)  # another out: a second record
    hip_attention.attend(q, buffers, meta, other, scale=s.scale)
    assert len(meta.plan.launches) == 2
    # a bad argument on a new object is still refused before any launch
    with pytest.raises(BackendError):
        hip_attention.attend(q, buffers, meta, torch.empty_like(out[:1]), scale=s.scale)
    # store: the same rows twice, then new contents of the same k/v objects
    rng = np.random.default_rng(3)
    k_new = torch.from_numpy(rng.standard_normal((len(s.plan["slot_mapping"]), 2, 128)).astype(np.float32))
    k_new = k_new.to(DEV).to(torch.bfloat16)
    v_new = -k_new
    for _ in range(2):
        hip_kvcache.store(k_new, v_new, buffers, meta)
    k_new.mul_(2.0)
    hip_kvcache.store(k_new, v_new, buffers, meta)
    torch.cuda.synchronize()
    slots = meta.slot_mapping
    real = slots != 0
    got = buffers.k.view(-1, 2, 128)[slots[real]]
    assert torch.equal(got.view(torch.int16), k_new[real].view(torch.int16))


def test_fresh_layer_tensors_are_not_kept_alive() -> None:
    # the reference layer (layers/attention/dense.py:113-124) makes new q/k/v and output tensors
    # for every layer: the recorded launches must not hold them, so the device memory after a
    # step of many layers is what it was before, and the caching allocator's reuse of their
    # addresses keeps the record count small
    import gc

    s = build_scenario([(1, 700), (1, 33), (1, 1500)], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="decode", seed=96)
    buffers, meta = scenario_buffers(s), plan_scenario(s)
    q0 = to_device(s.q_bits, "bf16")
    rows = q0.shape[0]
    warm = torch.empty_like(q0)  # grows the library's device-wide scratch before measuring
    hip_attention.attend_with(q0, buffers, meta, warm, scale=s.scale, partitions=None)
    del warm
    gc.collect()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    for _ in range(64):
        q = q0 * 1.0  # a fresh activation per layer
        out = torch.empty_like(q)
        k = torch.randn(rows, 2, 128, device=DEV, dtype=torch.bfloat16)
        hip_kvcache.store(k, -k, buffers, meta)
        hip_attention.attend(q, buffers, meta, out, scale=s.scale)
        del q, out, k
    torch.cuda.synchronize()
    gc.collect()
    assert torch.cuda.memory_allocated() == before
    assert len(meta.plan.launches) <= 8


def test_calls_on_two_streams_share_the_scratch_in_order() -> None:
    # two v2 steps queued back to back on two streams with no synchronisation between them: the
    # second stream waits for the first one's use of the shared scratch and counters, so both
    # results are those of the steps run alone
    s1 = build_scenario([(1, 3000), (1, 2500), (1, 4000)] * 6, heads=32, kv_heads=8, head_dim=128, block_size=16,
                        mode="decode", seed=97)
    s2 = build_scenario([(1, 1700), (1, 90), (1, 4000)] * 6, heads=32, kv_heads=8, head_dim=128, block_size=16,
                        mode="decode", seed=98)
    alone = [run_attention(s, 40, partition_size=128, merge="reduce-kernel") for s in (s1, s2)]
    for merge in ("reduce-kernel", "in-kernel"):
        setups = [(scenario_buffers(s), plan_scenario(s), to_device(s.q_bits, "bf16")) for s in (s1, s2)]
        outs = [torch.full_like(q, 7.0) for _, _, q in setups]
        torch.cuda.synchronize()
        for (buffers, meta, q), out, stream in zip(setups, outs, (torch.cuda.Stream(), torch.cuda.Stream())):
            with torch.cuda.stream(stream):
                for _ in range(3):
                    hip_attention.attend_with(q, buffers, meta, out, scale=s1.scale, partitions=40,
                                              partition_size=128, merge=merge, prefill=False)
        torch.cuda.synchronize()
        for got, want in zip(outs, alone):
            if merge == "reduce-kernel":
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), merge
        assert_parity(outs[0], s1.expected(np.float64), "bf16", f"stream 1 {merge}")
        assert_parity(outs[1], s2.expected(np.float64), "bf16", f"stream 2 {merge}")
    assert counters_are_clear()


def test_graph_metadata_restages_the_split_for_the_real_head_shape() -> None:
    # an update before the first attend scores the split for a guessed head shape; the first
    # eager attend knows the real one (GQA 8 over fp8 caches here) and stages that split
    bucket, max_blocks, bs = 8, 256, 16
    meta = hip_attention.graph_metadata(bucket, max_blocks, bs, DEV)
    lengths = torch.tensor([4096, 4096, 100, 0, 2000, 4096, 1, 3000], dtype=torch.int32)
    table = torch.arange(1, 1 + bucket * max_blocks, dtype=torch.int32).view(bucket, max_blocks)
    hip_attention.update_graph_metadata(meta, lengths, table)
    assert meta.plan.staged_shape == [8, 1, 2]
    k = torch.randn((1 + bucket * max_blocks, bs, 8, 128), device=DEV).to(torch.float8_e4m3fn)
    buffers = KVBuffers(k, k.clone(), KVLayoutKind.NHD, FP8_E4M3_CODEC)
    q = torch.randn((bucket, 64, 128), device=DEV).to(torch.bfloat16)
    out = torch.empty_like(q)
    hip_attention.attend(q, buffers, meta, out, scale=128 ** -0.5)
    torch.cuda.synchronize()
    assert meta.plan.head_shape == meta.plan.staged_shape == [8, 8, 1]
    expected = hip_attention.choose_split(bucket, 8, 8, max_blocks * bs, row_lengths=tuple(lengths.tolist()),
                                          kv_bytes=1, min_size=meta.plan.min_size,
                                          max_items=meta.plan.capacity - 1)
    staged = meta.plan.staged.cpu()
    assert int(staged[0]) == (expected.partition_size or int(staged[0]))
    assert torch.equal(staged[:2], meta.plan.staged_host[:2])


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
def test_block_ops_are_bit_exact(layout: str, ids_dtype: torch.dtype) -> None:
    s = build_scenario([(1, 40), (1, 9)], layout=layout, head_dim=128, block_size=16, spare_blocks=6, seed=7)
    buffers = scenario_buffers(s)
    k0, v0 = s.k_bits.copy(), s.v_bits.copy()
    ids = torch.tensor([5, 1, 5, 3], dtype=ids_dtype, device=DEV)
    out_k = torch.empty((4, *buffers.k.shape[1:]), dtype=buffers.k.dtype, device=DEV)
    out_v = torch.empty_like(out_k)
    hip_kvcache.gather(buffers, ids, out_k, out_v)
    hip_kvcache.copy_blocks(buffers, torch.tensor([1, 2], dtype=ids_dtype, device=DEV),
                            torch.tensor([6, 7], dtype=ids_dtype, device=DEV))
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(out_k), k0[[5, 1, 5, 3]]) and np.array_equal(to_bits(out_v), v0[[5, 1, 5, 3]])
    want_k, want_v = k0.copy(), v0.copy()
    paged.copy_blocks(want_k, want_v, np.array([1, 2]), np.array([6, 7]))
    assert np.array_equal(to_bits(buffers.k), want_k) and np.array_equal(to_bits(buffers.v), want_v)
    hip_kvcache.zero_blocks(buffers, torch.tensor([2, 4], dtype=ids_dtype, device=DEV))
    torch.cuda.synchronize()
    paged.zero_blocks(want_k, want_v, np.array([2, 4]))
    assert np.array_equal(to_bits(buffers.k), want_k) and np.array_equal(to_bits(buffers.v), want_v)


# --- the C ABI called directly ----------------------------------------------------------------


def test_c_abi_direct_call() -> None:
    s = build_scenario([(1, 100), (1, 1), (1, 0)], heads=8, kv_heads=2, head_dim=128, block_size=16,
                       mode="decode", seed=71)
    k, v, q = to_device(s.k_bits, "bf16"), to_device(s.v_bits, "bf16"), to_device(s.q_bits, "bf16")
    table = torch.from_numpy(s.table.astype(np.int32)).to(DEV)
    lengths = torch.tensor(s.lengths, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ayk_paged_attention_v1(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                                    table.shape[1], lengths.data_ptr(), None, None, 3, 8, 2, 128,
                                    k.shape[0], 16, table.shape[1], 0, 1, 1, ctypes.c_float(s.scale), 1.0, 1.0, 0, stream)
    assert rc == 0, lib.ayk_last_error()
    torch.cuda.synchronize()
    assert_parity(out, s.expected(np.float64), "bf16", "abi")
    rc = lib.ayk_paged_attention_v1(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                                    table.shape[1], lengths.data_ptr(), None, None, 3, 8, 2, 96,
                                    k.shape[0], 16, table.shape[1], 0, 1, 1, ctypes.c_float(1.0), 1.0, 1.0, 0, stream)
    assert rc == 2 and b"head_dim 96" in lib.ayk_last_error()


@pytest.mark.parametrize("heads", [8, 4], ids=["mfma", "dpp"])
@pytest.mark.parametrize("merge_flag", [8, 16], ids=["reduce-kernel", "in-kernel"])
def test_c_abi_v2_follows_the_staged_split(merge_flag: int, heads: int) -> None:
    # ayk_paged_attention_v2 with staged parameters (as a graph replay calls it): the grid covers
    # a capacity of work items; the partition size, the rows' first partial slots and the item
    # list are read from device memory, and the partials are packed. The result equals, bit for
    # bit, the same call given that size and list directly (partials at (row, head, partition)).
    s = build_scenario([(1, 700), (1, 1), (1, 0), (1, 300)], heads=heads, kv_heads=2, head_dim=128,
                       block_size=16, mode="decode", seed=73)
    k, v, q = to_device(s.k_bits, "bf16"), to_device(s.v_bits, "bf16"), to_device(s.q_bits, "bf16")
    table = torch.from_numpy(s.table.astype(np.int32)).to(DEV)
    lengths = torch.tensor(s.lengths, dtype=torch.int32, device=DEV)
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    n_rows, width = len(s.lengths), table.shape[1]
    min_size = 64
    max_partitions = -(-width * 16 // min_size)
    capacity = n_rows * max_partitions
    nbytes = lib.ayk_paged_attention_v2_workspace_bytes(n_rows, heads, 128, max_partitions)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    arrivals = torch.zeros(1024, dtype=torch.int32, device=DEV)
    common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), width, lengths.data_ptr(), None, None,
              n_rows, heads, 2, 128, k.shape[0], 16, width, 0, 1, 1, ctypes.c_float(s.scale), 1.0, 1.0)
    staged = torch.zeros(2 + n_rows + 2 * capacity, dtype=torch.int32, device=DEV)
    work = 2 + n_rows
    for size in (256, 128, 704):
        items = hip_attention.work_list(s.lengths, size)
        counts = [-(-n // size) for n in s.lengths]
        first = [sum(counts[:r]) for r in range(n_rows)]
        staged[:work + items.size] = torch.tensor([size, items.size // 2, *first, *items.tolist()],
                                                  dtype=torch.int32)
        direct = torch.from_numpy(items).to(DEV)
        outs = []
        for staged_call in (True, False):
            out = torch.full_like(q, float("nan"))
            if staged_call:
                rc = lib.ayk_paged_attention_v2(out.data_ptr(), *common, min_size, max_partitions,
                                                staged.data_ptr() + 4 * work, capacity, staged.data_ptr(),
                                                scratch.data_ptr(),
                                                nbytes, arrivals.data_ptr(), merge_flag, stream)
            else:
                rc = lib.ayk_paged_attention_v2(out.data_ptr(), *common, size, max_partitions, direct.data_ptr(),
                                                items.size // 2, None, scratch.data_ptr(), nbytes,
                                                arrivals.data_ptr(), merge_flag, stream)
            assert rc == 0, lib.ayk_last_error()
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), f"size {size}"
        assert_parity(outs[0], s.expected(np.float64), "bf16", f"staged {size}")
    assert int(arrivals.abs().sum()) == 0  # the in-kernel merge leaves its counters at zero


def test_attend_refuses_what_the_reference_contract_refuses() -> None:
    # the reference contract's refusals (tests/ops/test_attention_contract.py:252-391)
    import dataclasses

    s = build_scenario([(1, 10), (1, 7)], heads=4, kv_heads=2, head_dim=64, block_size=16, mode="decode")
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    q = to_device(s.q_bits, s.dtype)
    foreign = dataclasses.replace(meta, plan=object())
    with pytest.raises(BackendError, match="planned by another backend"):
        hip_attention.attend(q, buffers, foreign, torch.empty_like(q), scale=1.0)
    small = dataclasses.replace(meta, block_size=8)
    with pytest.raises(BackendError, match="planned for blocks of 8 positions but the cache has blocks of 16"):
        hip_attention.attend(q, buffers, small, torch.empty_like(q), scale=1.0)
    with pytest.raises(BackendError, match=r"q must be bfloat16 \[2, 4, 64\]"):
        hip_attention.attend(q[:1], buffers, meta, torch.empty_like(q[:1]), scale=1.0)
    with pytest.raises(BackendError, match=r"out must be bfloat16 \[2, 4, 64\]"):
        hip_attention.attend(q, buffers, meta, torch.empty_like(q, dtype=torch.float32), scale=1.0)  # never cast into
    q3 = q[:, :3].contiguous()
    with pytest.raises(BackendError, match="not a positive multiple of the cache's 2 key/value heads"):
        hip_attention.attend(q3, buffers, meta, torch.empty_like(q3), scale=1.0)


def test_kvcache_refuses_what_the_reference_contract_refuses() -> None:
    # the reference contract's refusals (tests/ops/test_kvcache_contract.py:200-296), raised
    # before a launch; nothing in the cache changes
    s = build_scenario([(2, 9), (1, 4)], heads=4, kv_heads=2, head_dim=64, block_size=16, seed=5)
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    before = (buffers.k.clone(), buffers.v.clone())
    rows = sum(s.rows)
    k = torch.zeros((rows, 2, 64), dtype=torch.bfloat16, device=buffers.k.device)
    with pytest.raises(BackendError, match=r"k must be bfloat16 \[3, 2, 64\]"):
        hip_kvcache.store(k[:2], k[:2], buffers, meta)  # one row short of the slot mapping
    with pytest.raises(BackendError, match=r"v must be bfloat16 \[3, 2, 64\]"):
        hip_kvcache.store(k, k.half(), buffers, meta)
    with pytest.raises(BackendError, match="planned for blocks of 8 positions but the cache has blocks of 16"):
        import dataclasses
        hip_kvcache.store(k, k, buffers, dataclasses.replace(meta, block_size=8))
    ids = torch.tensor([1, 2], dtype=torch.int32, device=buffers.k.device)
    with pytest.raises(BackendError, match="src has 2 blocks but dst has 1"):
        hip_kvcache.copy_blocks(buffers, ids, ids[:1])
    with pytest.raises(BackendError, match="int32 or int64 tensor"):
        hip_kvcache.zero_blocks(buffers, ids.float())
    out = torch.empty((1, *buffers.k.shape[1:]), dtype=buffers.k.dtype, device=buffers.k.device)
    with pytest.raises(BackendError, match="out_k must be bfloat16"):
        hip_kvcache.gather(buffers, ids, out, out)  # one block of output for two ids
    torch.cuda.synchronize()
    for now, then in zip((buffers.k, buffers.v), before):  # the caches hold NaN padding: compare bits
        assert torch.equal(now.view(torch.int16), then.view(torch.int16))


def test_unsupported_shapes_are_refused_before_launch() -> None:
    s = build_scenario([(1, 10)], head_dim=64, block_size=16, mode="decode")
    buffers = scenario_buffers(s)
    meta = plan_scenario(s)
    q = to_device(s.q_bits, s.dtype)
    with pytest.raises(BackendError, match="not a positive multiple"):
        hip_attention.attend(q[:, :3], buffers, meta, torch.empty_like(q[:, :3]), scale=1.0)
    odd = build_scenario([(1, 10)], head_dim=96, block_size=16, mode="decode")
    with pytest.raises(BackendError, match="head widths"):
        q96 = to_device(odd.q_bits, odd.dtype)
        hip_attention.attend(q96, scenario_buffers(odd), plan_scenario(odd), torch.empty_like(q96), scale=1.0)
