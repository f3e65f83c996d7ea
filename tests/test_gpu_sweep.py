"""Seeded sweep over the attention launch space, against the float64 oracle, on a HIP device.

The parity suite covers each launch dimension on its own; this sweep crosses them. Each case
draws (from ``numpy.random.default_rng(5000 + case)``) a head shape (G 1-8, head_dim 64 / 128 /
256), a cache dtype, layout and codec (16-bit values or fp8 e4m3 codes), a block size from 1 to 64
(powers of two and not), and a step: single-row decode or multi-row (prefill chunks and verify
windows beside decode rows), with edge lengths (0, 1, block_size - 1, block_size + 1) among
random ones. Every case runs the library's own launch and forced ones: v1 at a random wave split,
v2 at a random partition size and merge site (decode), the multi-row kernel at a random tile size
and partition size, and the window launch where the step allows it (multi-row). Each output is
held to the parity suite's bar (``max_abs_excess`` <= 2e-3, ``rel_l2`` <= 1e-3 against the
oracle, and the reference tests' 4 eps max|y|), padding rows must be zero, and a forced launch
the library refuses must be refused before any kernel runs (a ``BackendError``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ayaka_amd.enums import KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import attention as hip_attention
from ayaka_amd.kvcache import FP8_E4M3_CODEC, RAW_CODEC, KVBuffers
from oracle.numerics import e4m3_to_f32, f32_to_e4m3
from tests._support import build_scenario
from tests.test_gpu_parity import DEV, assert_parity, plan_scenario, to_device

pytestmark = pytest.mark.gpu

SHAPES = [(4, 4, 64), (8, 2, 64), (9, 3, 64), (32, 8, 64), (8, 1, 128), (12, 4, 128), (32, 8, 128), (64, 8, 128),
          (6, 6, 128), (4, 4, 256), (16, 8, 256), (8, 2, 256)]
BLOCK_SIZES = [1, 2, 3, 5, 7, 8, 12, 16, 24, 32, 48, 64]
PARTITION_SIZES = [64, 128, 192, 256, 320, 512, 704, 1024]
CASES = 160


def draw(case: int) -> dict:
    rng = np.random.default_rng(5000 + case)
    heads, kv_heads, head_dim = SHAPES[rng.integers(len(SHAPES))]
    bs = int(BLOCK_SIZES[rng.integers(len(BLOCK_SIZES))])
    mode = "decode" if rng.random() < 0.5 else "mixed"
    edge = [0, 1, max(1, bs - 1), bs + 1, 2 * bs + 1]
    steps = []
    for _ in range(int(rng.integers(1, 6))):
        length = int(edge[rng.integers(len(edge))]) if rng.random() < 0.35 else int(rng.integers(1, 1400))
        if mode == "decode":
            rows = 1
        else:
            kind = rng.random()
            rows = (1 if kind < 0.3 else int(rng.integers(2, 6)) if kind < 0.7 else int(rng.integers(6, 70)))
            rows = min(rows, max(length, 1))
        steps.append((rows, length))
    return dict(heads=int(heads), kv_heads=int(kv_heads), head_dim=int(head_dim), block_size=bs, mode=mode,
                steps=steps, dtype=["bf16", "fp16"][rng.integers(2)], layout=["nhd", "hnd"][rng.integers(2)],
                codec=["raw", "raw", "fp8"][rng.integers(3)], seed=int(rng.integers(1 << 30)), rng=rng)


def launches(d: dict, meta) -> list[tuple[str, dict]]:
    rng = d["rng"]
    group = d["heads"] // d["kv_heads"]
    longest = max(n for _, n in d["steps"])
    out = [("auto", dict(partitions=None))]
    if d["mode"] == "decode":
        waves = int([1, 2, 4, 8][rng.integers(4)])
        out.append((f"v1/{waves} waves", dict(partitions=0, prefill=False, waves=waves)))
        size = int(PARTITION_SIZES[rng.integers(len(PARTITION_SIZES))])
        merge = ["in-kernel", "reduce-kernel"][rng.integers(2)]
        out.append((f"v2/{size}/{merge}", dict(partitions=max(1, -(-longest // size)), partition_size=size,
                                                merge=merge, prefill=False)))
        if d["codec"] == "raw" and rng.random() < 0.5:
            out.append(("v1/dpp", dict(partitions=0, prefill=False, qk="dpp")))
    else:
        full = hip_attention.PREFILL_PAIRS[d["head_dim"]]
        tiles = [full // w for w in (1, 2, 4) if full // w >= group]
        pairs = int(tiles[rng.integers(len(tiles))])
        size = int([0, 64, 256, 512][rng.integers(4)])
        launch = dict(partitions=0) if size == 0 else dict(partitions=None, partition_size=size)
        out.append((f"multi-row/{pairs} pairs/{size}", dict(prefill=True, window=False, tile_pairs=pairs, **launch)))
        if meta.plan.window_pairs(group):
            wsize = int([0, 64, 256][rng.integers(3)])
            wlaunch = dict(partitions=0) if wsize == 0 else dict(partitions=None, partition_size=wsize)
            out.append((f"windows/{wsize}", dict(prefill=True, window=True, **wlaunch)))
    return out


@pytest.mark.parametrize("case", range(CASES))
def test_sweep(case: int) -> None:
    d = draw(case)
    s = build_scenario(d["steps"], dtype=d["dtype"], layout=d["layout"], heads=d["heads"], kv_heads=d["kv_heads"],
                       head_dim=d["head_dim"], block_size=d["block_size"], mode=d["mode"], seed=d["seed"])
    layout = KVLayoutKind.NHD if s.layout == "nhd" else KVLayoutKind.HND
    if d["codec"] == "fp8":
        kc, vc = f32_to_e4m3(s.k), f32_to_e4m3(s.v)
        buffers = KVBuffers(torch.from_numpy(kc).view(torch.float8_e4m3fn).to(DEV),
                            torch.from_numpy(vc).view(torch.float8_e4m3fn).to(DEV), layout, FP8_E4M3_CODEC)
        expected = s.expected(np.float64, k=e4m3_to_f32(kc), v=e4m3_to_f32(vc))
    else:
        buffers = KVBuffers(to_device(s.k_bits, s.dtype), to_device(s.v_bits, s.dtype), layout, RAW_CODEC)
        expected = s.expected(np.float64)
    meta = plan_scenario(s)
    q = to_device(s.q_bits, s.dtype)
    padding_rows = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    desc = {k: v for k, v in d.items() if k != "rng"}
    for label, launch in launches(d, meta):
        print(f"case {case} {label}: {desc}", flush=True)
        out = torch.full_like(q, 7.0)
        try:
            hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, **launch)
        except BackendError as err:
            # only a forced launch may be refused, and only before anything ran
            assert label != "auto", f"case {case}: the library's own launch refused: {err}"
            assert bool((out == 7.0).all()), f"case {case} {label}: refused after writing"
            print(f"case {case} {label}: refused ({err})", flush=True)
            continue
        torch.cuda.synchronize()
        assert_parity(out, expected, s.dtype, f"case {case} {label} {desc}")
        if padding_rows:
            assert torch.count_nonzero(out[padding_rows]) == 0, f"case {case} {label}: padding rows"
