"""fp32 models on the hip backend: the fp32 decode kernel against the float64 oracle.

The reference's torch backend serves fp32 (``python/ayaka/ops/backends/torch/_checks.py:30-38``);
its contract tests hold fp32 outputs to ``4 * eps * max|y| + 1e-6`` against float64
(``tests/ops/test_attention_contract.py:168-171``), the bound used here. Decode steps run v1
and v2 (either grid, partitions merged by the fp32 reduce kernel); multi-row steps run row by
row on the same kernel; graph replays read their staged split.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ayaka_amd.enums import ForwardMode, KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import attention as hip_attention
from ayaka_amd.hip import kvcache as hip_kvcache
from ayaka_amd.kvcache import RAW_CODEC, KVBuffers
from oracle import paged
from tests._support import build_scenario

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
EPS32 = 2.0**-23


def f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def assert_close(out: torch.Tensor, expected: np.ndarray, label: str) -> None:
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all(), f"{label}: non-finite output"
    bound = 4 * EPS32 * float(np.abs(expected).max(initial=0.0)) + 1e-6
    worst = float(np.abs(got - expected).max(initial=0.0))
    assert worst <= bound, f"{label}: {worst} > {bound}"


def scenario(steps, heads: int, kv_heads: int, head_dim: int, layout: str, mode: str, seed: int):
    s = build_scenario(steps, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16, layout=layout,
                       mode=mode, seed=seed)
    kind = KVLayoutKind.NHD if layout == "nhd" else KVLayoutKind.HND
    buffers = KVBuffers(f32(s.k), f32(s.v), kind, RAW_CODEC)  # NaN in every slot no context holds
    meta = hip_attention.plan(ForwardMode(mode), torch.tensor(s.rows, dtype=torch.int32, device=DEV),
                              torch.tensor(s.lengths, dtype=torch.int32, device=DEV),
                              torch.from_numpy(s.table.astype(np.int32)).to(DEV), 16)
    return s, buffers, meta, f32(s.q)


STEPS = [
    ("decode", [(1, 16), (1, 0), (1, 1300), (1, 33), (1, 517), (1, 1), (1, 15), (1, 17)], "decode"),
    ("mixed", [(7, 7), (1, 9), (40, 600), (2, 0), (3, 1100)], "mixed"),
]


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 2, 128), (32, 8, 64), (4, 4, 256), (64, 8, 128),
                                                     (16, 1, 64), (12, 4, 256)])
@pytest.mark.parametrize("name,steps,mode", STEPS, ids=[s[0] for s in STEPS])
def test_fp32_attention_matches_the_oracle(layout: str, heads: int, kv_heads: int, head_dim: int, name: str,
                                           steps: list, mode: str) -> None:
    s, buffers, meta, q = scenario(steps, heads, kv_heads, head_dim, layout, mode, seed=101)
    expected = s.expected(np.float64)
    padding = [i for i, r in enumerate(s.plan["request_of_row"]) if s.lengths[r] == 0]
    launches = [("auto", dict(partitions=None)), ("v1", dict(partitions=0)),
                ("v2/128", dict(partitions=11, partition_size=128)),
                ("v2/64 partials only then merged", dict(partitions=21, partition_size=64)),
                ("v2/512", dict(partitions=3, partition_size=512, merge="reduce-kernel"))]
    for label, launch in launches:
        out = torch.full_like(q, 7.0)
        hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, **launch)
        torch.cuda.synchronize()
        assert_close(out, expected, f"fp32 {name} {label}")
        if padding:
            assert torch.count_nonzero(out[padding]) == 0
    out = torch.full_like(q, 7.0)
    hip_attention.attend(q, buffers, meta, out, scale=s.scale)  # the library's launch, recorded and replayed
    hip_attention.attend(q, buffers, meta, out, scale=s.scale)
    torch.cuda.synchronize()
    assert_close(out, expected, f"fp32 {name} attend")


def test_fp32_refuses_the_other_launch_shapes() -> None:
    s, buffers, meta, q = scenario(STEPS[1][1], 8, 2, 128, "nhd", "mixed", seed=102)
    out = torch.empty_like(q)
    for launch in (dict(partitions=None, prefill=True), dict(partitions=0, qk="mfma"),
                   dict(partitions=0, waves=4), dict(partitions=3, partition_size=512, merge="in-kernel")):
        with pytest.raises(BackendError, match="fp32 runs one launch shape"):
            hip_attention.attend_with(q, buffers, meta, out, scale=s.scale, **launch)


def test_fp32_store_and_block_ops_are_bit_exact() -> None:
    s, buffers, meta, _ = scenario(STEPS[1][1], 8, 2, 128, "nhd", "mixed", seed=103)
    rng = np.random.default_rng(104)
    n = len(s.plan["slot_mapping"])
    k_new = rng.standard_normal((n, 2, 128)).astype(np.float32)
    v_new = rng.standard_normal((n, 2, 128)).astype(np.float32)
    kc, vc = s.k.copy(), s.v.copy()
    hip_kvcache.store(f32(k_new), f32(v_new), buffers, meta)
    torch.cuda.synchronize()
    paged.store(kc, vc, k_new, v_new, s.plan["slot_mapping"], "nhd")
    # block 0 receives the padding rows in an unspecified order; every other block is exact
    assert np.array_equal(buffers.k.cpu().numpy()[1:].view(np.uint32), kc[1:].view(np.uint32))
    assert np.array_equal(buffers.v.cpu().numpy()[1:].view(np.uint32), vc[1:].view(np.uint32))
    ids = torch.tensor([3, 1, 2], dtype=torch.int64, device=DEV)
    out_k, out_v = torch.empty((3, *buffers.k.shape[1:]), device=DEV), torch.empty((3, *buffers.k.shape[1:]), device=DEV)
    hip_kvcache.gather(buffers, ids, out_k, out_v)
    torch.cuda.synchronize()
    assert np.array_equal(out_k.cpu().numpy().view(np.uint32), kc[[3, 1, 2]].view(np.uint32))
    assert np.array_equal(out_v.cpu().numpy().view(np.uint32), vc[[3, 1, 2]].view(np.uint32))


def test_fp32_graph_replays_match_eager_and_the_oracle() -> None:
    # a decode bucket of fp32 layers captured once, replayed over steps whose staged split
    # changes: each replay bit for bit the same step run eagerly on the graph metadata, and
    # within the contract's bound of the float64 oracle
    rng = np.random.default_rng(105)
    bucket, max_blocks, bs, heads, kv_heads, dim = 6, 64, 16, 16, 4, 128
    num_blocks = 1 + bucket * max_blocks
    k_cache = torch.randn((num_blocks, bs, kv_heads, dim), device=DEV)
    v_cache = torch.randn((num_blocks, bs, kv_heads, dim), device=DEV)
    buffers = KVBuffers(k_cache, v_cache, KVLayoutKind.NHD, RAW_CODEC)
    perm = rng.permutation(np.arange(1, num_blocks)).reshape(bucket, max_blocks).astype(np.int32)
    meta = hip_attention.graph_metadata(bucket, max_blocks, bs, DEV)
    q = torch.zeros((bucket, heads, dim), device=DEV)
    out = torch.zeros_like(q)
    hip_attention.update_graph_metadata(meta, torch.ones(bucket, dtype=torch.int32), torch.from_numpy(perm))
    hip_attention.attend(q, buffers, meta, out, scale=dim**-0.5)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_attention.attend(q, buffers, meta, out, scale=dim**-0.5)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        hip_attention.attend(q, buffers, meta, out, scale=dim**-0.5)
    torch.cuda.synchronize()
    cap = max_blocks * bs
    for lens in ([5, 0, 1000, 17, 1, 33], [cap, 0, 0, 0, 0, 1], [int(x) for x in rng.integers(0, cap + 1, bucket)]):
        q.copy_(torch.randn(q.shape, device=DEV))
        hip_attention.update_graph_metadata(meta, torch.tensor(lens, dtype=torch.int32), torch.from_numpy(perm))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = torch.empty_like(out)
        hip_attention.attend(q, buffers, meta, eager, scale=dim**-0.5)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int32), eager.view(torch.int32)), lens
        expected = paged.attention(q.cpu().numpy(), k_cache.cpu().numpy(), v_cache.cpu().numpy(), perm,
                                   np.array(lens), scale=dim**-0.5, precision=np.float64)
        assert_close(replayed, expected, f"fp32 replay {lens}")
