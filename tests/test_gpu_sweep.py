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
oracle or a raw error within 1e-4 of the once-rounded oracle's, and the reference tests' 4 eps
max|y|), padding rows must be zero, and a forced launch
the library refuses must be refused before any kernel runs (a ``BackendError``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ayaka_amd.enums import KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import attention as hip_attention
from ayaka_amd.hip import kvcache as hip_kvcache
from ayaka_amd.kvcache import FP8_E4M3_CODEC, RAW_CODEC, KVBuffers
from oracle import paged
from oracle.numerics import bits_to_f32, e4m3_to_f32, f32_to_bits, f32_to_e4m3
from tests._support import build_scenario
from tests.test_gpu_parity import DEV, assert_parity, plan_scenario, to_bits, to_device

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
        if d["head_dim"] in hip_attention.PREFILL_DOUBLE_TILE_DIMS:  # the 8-wave double tile, same split
            out.append((f"multi-row/{2 * full} pairs/{size}",
                        dict(prefill=True, window=False, tile_pairs=2 * full, **launch)))
        if meta.plan.window_pairs(group):
            wsize = int([0, 64, 256][rng.integers(3)])
            wlaunch = dict(partitions=0) if wsize == 0 else dict(partitions=None, partition_size=wsize)
            out.append((f"windows/{wsize}", dict(prefill=True, window=True, **wlaunch)))
    return out


@pytest.mark.parametrize("case", [*range(CASES), 29207])  # 29207: one row of 512 outputs, rounding flips
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


# --- the bit-exact ops: KV write (both codecs) and block ops ------------------------------------

OPS_CASES = 48


@pytest.mark.parametrize("case", range(OPS_CASES))
def test_sweep_bit_exact_ops(case: int) -> None:
    """A seeded shape (``default_rng(7000 + case)``: head_dim 8-256, 1-8 key/value heads, block size
    1-64, NHD/HND, fp16/bf16, 16-bit or fp8 caches, steps of prefill and decode rows with padding
    requests), then the step's KV write and, on 16-bit caches, gather / copy_blocks / zero_blocks
    with int32 or int64 ids: every cache byte against the oracle's, except block 0 (padding rows'
    slot, written in an unspecified order)."""
    rng = np.random.default_rng(7000 + case)
    head_dim = int([8, 12, 16, 64, 128, 256][rng.integers(6)])
    kv_heads = int(rng.integers(1, 9))
    bs = int(BLOCK_SIZES[rng.integers(len(BLOCK_SIZES))])
    dtype = ["bf16", "fp16"][rng.integers(2)]
    layout = ["nhd", "hnd"][rng.integers(2)]
    fp8 = rng.random() < 0.4
    steps = []
    for _ in range(int(rng.integers(1, 6))):
        length = 0 if rng.random() < 0.15 else int(rng.integers(1, 300))
        steps.append((max(1, min(int(rng.integers(1, 40)), length)) if length else int(rng.integers(1, 3)), length))
    s = build_scenario(steps, dtype=dtype, layout=layout, heads=kv_heads, kv_heads=kv_heads, head_dim=head_dim,
                       block_size=bs, mode="mixed", seed=int(rng.integers(1 << 30)), spare_blocks=8)
    desc = dict(head_dim=head_dim, kv_heads=kv_heads, block_size=bs, dtype=dtype, layout=layout, fp8=fp8,
                steps=steps)
    print(f"case {case}: {desc}", flush=True)
    n = len(s.plan["slot_mapping"])
    rows = rng.standard_normal((2, n, kv_heads, head_dim)) * np.exp2(rng.uniform(-10, 8, (2, n, kv_heads, 1)))
    bits = f32_to_bits(rows.astype(np.float32), dtype)
    meta = plan_scenario(s)
    kind = KVLayoutKind.NHD if layout == "nhd" else KVLayoutKind.HND
    if fp8:
        kc, vc = f32_to_e4m3(s.k), f32_to_e4m3(s.v)
        buffers = KVBuffers(torch.from_numpy(kc).view(torch.float8_e4m3fn).to(DEV),
                            torch.from_numpy(vc).view(torch.float8_e4m3fn).to(DEV), kind, FP8_E4M3_CODEC)
        hip_kvcache.store(to_device(bits[0], dtype), to_device(bits[1], dtype), buffers, meta)
        torch.cuda.synchronize()
        decoded = bits_to_f32(bits, dtype)
        paged.store(kc, vc, f32_to_e4m3(decoded[0]), f32_to_e4m3(decoded[1]), s.plan["slot_mapping"], layout)
        got_k, got_v = buffers.k.view(torch.uint8).cpu().numpy(), buffers.v.view(torch.uint8).cpu().numpy()
        assert np.array_equal(got_k[1:], kc[1:]) and np.array_equal(got_v[1:], vc[1:]), f"case {case}: {desc}"
        return
    buffers = KVBuffers(to_device(s.k_bits, dtype), to_device(s.v_bits, dtype), kind, RAW_CODEC)
    hip_kvcache.store(to_device(bits[0], dtype), to_device(bits[1], dtype), buffers, meta)
    torch.cuda.synchronize()
    want_k, want_v = s.k_bits.copy(), s.v_bits.copy()
    paged.store(want_k, want_v, bits[0], bits[1], s.plan["slot_mapping"], layout)
    got_k, got_v = to_bits(buffers.k), to_bits(buffers.v)
    assert np.array_equal(got_k[1:], want_k[1:]) and np.array_equal(got_v[1:], want_v[1:]), f"case {case}: {desc}"
    # block ops on the written caches (block 0 included now: made deterministic first)
    buffers.k[0].zero_()
    buffers.v[0].zero_()
    torch.cuda.synchronize()
    cur_k, cur_v = to_bits(buffers.k), to_bits(buffers.v)
    blocks = buffers.k.shape[0]
    ids_dtype = [torch.int32, torch.int64][rng.integers(2)]
    picks = rng.integers(0, blocks, size=int(rng.integers(1, 2 * blocks)))
    out_k = torch.empty((len(picks), *buffers.k.shape[1:]), dtype=buffers.k.dtype, device=DEV)
    out_v = torch.empty_like(out_k)
    hip_kvcache.gather(buffers, torch.tensor(picks, dtype=ids_dtype, device=DEV), out_k, out_v)
    perm = rng.permutation(blocks)
    pairs = int(rng.integers(1, blocks // 2 + 1))
    src, dst = perm[:pairs], perm[pairs:2 * pairs]  # disjoint, so the result does not depend on order
    hip_kvcache.copy_blocks(buffers, torch.tensor(src, dtype=ids_dtype, device=DEV),
                            torch.tensor(dst, dtype=ids_dtype, device=DEV))
    zero = rng.choice(blocks, size=int(rng.integers(1, blocks + 1)), replace=False)
    hip_kvcache.zero_blocks(buffers, torch.tensor(zero, dtype=ids_dtype, device=DEV))
    torch.cuda.synchronize()
    want_gk, want_gv = paged.gather(cur_k, cur_v, picks)
    assert np.array_equal(to_bits(out_k), want_gk) and np.array_equal(to_bits(out_v), want_gv), f"case {case}"
    paged.copy_blocks(cur_k, cur_v, src, dst)
    paged.zero_blocks(cur_k, cur_v, zero)
    assert np.array_equal(to_bits(buffers.k), cur_k) and np.array_equal(to_bits(buffers.v), cur_v), f"case {case}"
