"""Decode-attention benchmark on one MI355X: µs per call, KV bytes/s and the HBM roofline fraction.

The workload is the headline configuration: Llama-3-8B-shape decode attention
(32 query heads, 8 key/value heads, head_dim 128, bf16, block 16), batch 64 at
4096 context, random block permutation over a 40000-block pool, synthetic
N(0,1) data. A step is one ``attend`` call over the batch, with every input
already resident in HBM. ``value`` is algorithmic bytes per call / time per call.

Also reported, in the same JSON line: v1 and v2 timed separately, the
roofline record of the dominant kernel, and the reference CPU algorithm
(the oracle's restatement of ``_attend_decode``) timed on a bounded sample of
the same workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0

# HBM bytes per launch of the dominant kernel, measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE on `bench.py --config C --only` and scaled by what the same counters read
# for a 1 GiB device copy (FETCH x2.0, WRITE x1.0). Reported only when this run's launch is
# the one profiled: (config, kernel, partition size) -> (read bytes, write bytes, summary).
PROFILED_TRAFFIC = {
    (3, "paged_attention_mfma_kernel (v1, 4 waves per head)", 0):
        (1_080_177_728, 524_288, "profiles/paged_attention_mfma_kernel_c3_llama3_8b_decode.md"),
    (3, "paged_attention_mfma_kernel (v1, 4 waves per head, fp8 cache)", 0):
        (544_024_803, 524_288, "profiles/paged_attention_mfma_kernel_c3_llama3_8b_decode_fp8_cache.md"),
    (4, "paged_attention_mfma_kernel (v2, merge reduce-kernel)", 704):
        (668_605_302, 4_054_928, "profiles/paged_attention_mfma_kernel_c4_long_context.md"),
    (5, "paged_attention_mfma_kernel (v2, merge reduce-kernel)", 3072):
        (2_598_158_371, 10_319_456, "profiles/paged_attention_mfma_kernel_c5_ragged_gqa8.md"),
    (2, "paged_attention_mfma_kernel (v2, merge reduce-kernel)", 320):
        (148_332_170, 2_128_368, "profiles/paged_attention_mfma_kernel_c2_llama32_1b_decode.md"),
    (1, "paged_attention_mfma_kernel (v1, 8 waves per head)", 0):
        (1_634_780, 4_608, "profiles/paged_attention_mfma_kernel_c1_smollm2_decode.md"),
    (5, "paged_attention_mfma_kernel (v2, merge reduce-kernel, fp8 cache)", 2560):
        (1_307_048_278, 11_526_016, "profiles/paged_attention_mfma_kernel_c5_ragged_gqa8_fp8_cache.md"),
}


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, help="benchmark configuration 1-5 (3 = headline)")
    ap.add_argument("--only", action="store_true",
                    help="time only the headline launch, on one pool (for profiler runs)")
    ap.add_argument("--layout", choices=["nhd", "hnd"], default=None,
                    help="cache layout (default: the one the hip backend asks the pool for)")
    ap.add_argument("--codec", choices=["raw", "fp8_e4m3"], default="raw",
                    help="KV-cache codec: 16-bit values, or fp8 e4m3 codes decoded in the kernel")
    ap.add_argument("--fp32", action="store_true",
                    help="only time C1-C5 as fp32 models (fp32 q, out and caches, the fp32 decode kernel), "
                         "one JSON record each")
    ap.add_argument("--model-dtype", choices=["config", "fp32"], default="config",
                    help="with --record: the configuration's own dtype, or fp32 throughout")
    ap.add_argument("--qk", choices=["dpp", "mfma"], default=None,
                    help="force the q.k implementation (default: the library's choice)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=64, help="rows of the CPU baseline sample")
    ap.add_argument("--record", action="store_true",
                    help="print only the record of --config (with --codec): µs per call, GB/s, kernel")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-configuration records (C1-C5, both codecs) of the default run")
    ap.add_argument("--graph-step", action="store_true",
                    help="time a 32-layer decode step (KV write + attention per layer) eagerly and as a "
                         "captured graph replay (and eagerly on a planned step), at the C1-C5 shapes")
    ap.add_argument("--multi-row", action="store_true",
                    help="only time the multi-row (prefill / verify) kernel on its workloads, one JSON line each")
    ap.add_argument("--block-ops", action="store_true",
                    help="only time the block ops (gather / copy_blocks / zero_blocks) at the C3 pool shape")
    ap.add_argument("--reference-shapes", action="store_true",
                    help="only time the reference's own op-benchmark matrix (TinyLlama 32/4/64 and SmolLM2 "
                         "9/3/64, fp16: five decode and two prefill steps), one JSON line per step")
    ap.add_argument("--host-trace", action="store_true",
                    help="only time the host side of decode steps (update_graph_metadata, and plan plus the "
                         "split choice of an eager step) over a continuous-batching trace at the C5 shape")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (scales profiler byte counters)")
    return ap.parse_args()


def time_calls(fn, steps: int, warmup: int, repeats: int = 5) -> dict:
    """Time ``steps`` back-to-back calls between two HIP events on the current stream.

    An event recorded between every pair of calls would add a cache-flushing
    barrier to each call, so only the region is bracketed. The region is
    repeated ``repeats`` times; the median region gives µs per call.
    """
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    regions, walls = [], []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        regions.append(start.elapsed_time(end) * 1000.0 / steps)  # µs per call
    return {"median_us": statistics.median(regions), "min_us": min(regions),
            "wall_ms_per_step": statistics.median(walls) * 1000.0 / steps}


def settle(fn, steps: int, limit_s: float = 2.0, min_s: float = 0.3) -> int:
    """Run ``fn`` in regions of ``steps`` calls for at least ``min_s`` and then until two
    consecutive regions agree within 1% (or ``limit_s`` passes); returns the calls made. After
    an idle spell the first calls of a compute-heavier kernel run slower on MI355X for a few
    tens of milliseconds of sustained work (fp8 C3 v1: ~104-108 µs, then 89-90; the bf16
    kernels, bound by memory throughout, hardly move), so the per-configuration records,
    which are not the driver's headline step, are timed once that has passed."""
    import torch

    calls, last, t0 = 0, None, time.perf_counter()
    while time.perf_counter() - t0 < limit_s:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        calls += steps
        us = start.elapsed_time(end)
        if time.perf_counter() - t0 >= min_s and last is not None and abs(us - last) <= 0.01 * last:
            break
        last = us
    return calls


def cpu_baseline(step, cfg, rows: int, kv_bytes: int = 2, chunk: int | None = None, runs: int = 5) -> dict:
    """The reference's CPU decode (``_attend_decode``, restated in torch by
    ``oracle.torch_decode``) timed on this host over ``rows`` rows of the step: the padded
    tables gathered from a bf16/fp16 cache, float32 matmuls and softmax, as the reference's
    torch backend runs it, on as many threads as this process may use. ``chunk`` runs the
    requests in groups of that many (same padded width, same arithmetic per request: C5's
    whole padded gather would need ~34 GB); ``runs`` timed runs follow one warm-up."""
    import torch

    from ayaka_amd import workloads
    from oracle.torch_decode import attend_decode

    nproc = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(nproc, int(omp)) if omp.isdigit() and int(omp) > 0 else nproc
    torch.set_num_threads(threads)
    rows = min(rows, cfg.batch)
    sample = workloads.sample_rows(step, list(range(rows)))
    # the cache in its own dtype (fp8 caches: their decoded values, which the reference has no codec for)
    keys = torch.from_numpy(sample["k"]).to(cfg.dtype)
    values = torch.from_numpy(sample["v"]).to(cfg.dtype)
    q = torch.from_numpy(sample["q"]).to(cfg.dtype)
    table, lengths = torch.from_numpy(sample["table"]), torch.from_numpy(sample["lengths"])
    step_rows = chunk or rows
    times = []
    for _ in range(runs + 1):  # 1 warm-up + `runs` timed
        t0 = time.perf_counter()
        for r0 in range(0, rows, step_rows):
            attend_decode(q[r0:r0 + step_rows], keys, values, table[r0:r0 + step_rows], lengths[r0:r0 + step_rows],
                          scale=cfg.scale)
        times.append(time.perf_counter() - t0)
    seconds = statistics.median(times[1:]) * cfg.batch / rows  # scaled to the whole batch
    scaled = "all of them" if rows == cfg.batch else f"scaled by {cfg.batch}/{rows} to one call"
    if chunk:
        scaled += f", in groups of {chunk} requests"
    return {
        "value": workloads.algorithmic_bytes(cfg, kv_bytes) / seconds / 1e9,
        "unit": "GB/s",
        "us_per_call": seconds * 1e6,
        "cores": threads,
        "nproc": nproc,
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} of {cfg.batch} rows of the same step ({scaled}): the reference's _attend_decode "
                  f"restated in torch "
                  f"(oracle/torch_decode.py) on the CPU, bf16 cache gathered per padded table, float32 "
                  f"matmuls and softmax; median of {runs} runs after 1 warm-up, torch.set_num_threads({threads})",
    }


# Multi-row workloads, all Llama-3-8B-shaped (D 128, bf16, block 16) unless noted:
# (requests, rows per request, context per request, query heads, key/value heads).
MULTI_ROW_WORKLOADS = [
    (4, 512, 4096, 32, 8),    # chunked prefill: 512-row chunks at the end of 4K contexts
    (1, 2048, 2048, 32, 8),   # one whole 2K prompt
    (8, 128, 2048, 32, 8),    # small chunks
    (16, 8, 1024, 32, 8),     # verify windows of 8 draft tokens
    (4, 512, 4096, 64, 8),    # GQA 8
    (32, 4, 4096, 32, 8),     # verify windows of 4 draft tokens over 4K
    (64, 2, 2048, 32, 8),     # verify windows of 2 draft tokens over 2K
    (4, 512, 4096, 32, 8, 128, "fp16"),  # the first workload with an fp16 model (one P.V MFMA per step)
    (4, 512, 4096, 32, 8, 64, "fp16"),   # Llama-3.2-1B shape (D 64, fp16)
    (4, 512, 4096, 32, 8, 128, "bf16", "fp8_e4m3"),  # the first workload over fp8 caches
    (32, 4, 4096, 32, 8, 128, "bf16", "fp8_e4m3"),   # verify windows over fp8 caches
    (4, 512, 4096, 16, 8, 256, "bf16"),  # Gemma-2-9B shape (head_dim 256)
    (64, 2, 2048, 64, 8),     # verify windows of 2 draft tokens at GQA 8 (16 columns: 2 rows x 8 heads)
]
MFMA_BF16_PEAK_TFLOPS = 2500.0


def multi_row(args) -> int:
    """Time a multi-row step as the library launches it (the multi-row kernel, or the decode kernel's
    window launch when every request's rows fit one 16-column tile) and, beside it, the same
    step through the per-row decode kernels and through the multi-row kernel."""
    import torch

    from ayaka_amd.enums import ForwardMode, KVLayoutKind
    from ayaka_amd.hip import _lib
    from ayaka_amd.hip import attention as hip_attention
    from ayaka_amd.kvcache import FP8_E4M3_CODEC, KVBuffers

    _lib.lib()
    dev = torch.device("cuda:0")
    for requests, rows, context, heads, kv_heads, *shape in MULTI_ROW_WORKLOADS:
        dim, dtype_name, codec = (*shape, "raw")[:3] if shape else (128, "bf16", "raw")
        dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[dtype_name]
        bs = 16
        blocks = requests * (context // bs) + 1
        gen = torch.Generator(device=dev).manual_seed(rows)
        k = torch.randn((blocks, bs, kv_heads, dim), generator=gen, device=dev).to(dtype)
        v = torch.randn((blocks, bs, kv_heads, dim), generator=gen, device=dev).to(dtype)
        ids = torch.randperm(blocks - 1, generator=gen, device=dev)[: blocks - 1] + 1
        table = ids.view(requests, context // bs).to(torch.int32)
        meta = hip_attention.plan(ForwardMode.MIXED, torch.full((requests,), rows, dtype=torch.int32, device=dev),
                                  torch.full((requests,), context, dtype=torch.int32, device=dev), table, bs)
        q = torch.randn((requests * rows, heads, dim), generator=gen, device=dev).to(dtype)
        out, per_row = torch.empty_like(q), torch.empty_like(q)
        if codec == FP8_E4M3_CODEC:
            k, v = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
        buffers = KVBuffers(k, v, KVLayoutKind.NHD, codec)
        scale = dim ** -0.5
        # timed once the part's clocks have settled under sustained calls (see settle), as the
        # per-configuration decode records are: the first ~100 ms of these compute-bound calls run
        # about 10% slower
        launch = lambda: hip_attention.attend_with(q, buffers, meta, out, scale=scale, partitions=None,  # noqa: E731
                                                    prefill=True)
        settle(launch, args.steps)
        kernel = time_calls(launch, args.steps, args.warmup)
        kv_code = 1 if codec == FP8_E4M3_CODEC else 2
        window = hip_attention.WINDOWS and meta.plan.window_pairs(heads // kv_heads) > 0
        if window:
            pairs, size = meta.plan.window_pairs(heads // kv_heads), meta.plan.window_split(kv_heads, heads // kv_heads,
                                                                                           kv_code)
        else:
            pairs, size = meta.plan.prefill_launch(kv_heads, heads // kv_heads, dim, kv_code)
        unsplit = kernel if not size else time_calls(
            lambda: hip_attention.attend_with(q, buffers, meta, per_row, scale=scale, partitions=0, prefill=True),
            args.steps, args.warmup)
        multi_row_kernel = kernel if not window else time_calls(
            lambda: hip_attention.attend_with(q, buffers, meta, per_row, scale=scale, partitions=None, prefill=True,
                                              window=False), args.steps, args.warmup)
        old = time_calls(lambda: hip_attention.attend_with(q, buffers, meta, per_row, scale=scale, partitions=None,
                                                           prefill=False), 3, 1, repeats=1)
        torch.cuda.synchronize()
        # positions each row sees (causal within the chunk), and the flops of q.k and p.v on them
        visible = requests * sum(context - rows + j + 1 for j in range(rows))
        flops = 4 * heads * dim * visible
        kv_bytes = requests * context * kv_heads * dim * 2 * (1 if codec == FP8_E4M3_CODEC else 2)
        us = kernel["median_us"]
        print(json.dumps({
            "workload": f"{requests} requests x {rows} rows over {context} positions, Hq {heads}, Hkv {kv_heads}, "
                        f"D {dim}, {dtype_name}, block {bs}" + (", fp8 e4m3 cache" if codec == FP8_E4M3_CODEC else ""),
            "us_per_call": round(us, 2),
            "launch": "windows" if window else "multi-row",
            "tile_pairs": pairs,
            "partition_size": size,
            "unsplit_us": round(unsplit["median_us"], 2),
            "multi_row_kernel_us": round(multi_row_kernel["median_us"], 2),
            "tflops": round(flops / us / 1e6, 1),
            "mfma_fraction": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
            "kv_gbs": round(kv_bytes / us / 1e3, 1),
            "per_row_decode_kernels_us": round(old["median_us"], 1),
            "speedup": round(old["median_us"] / us, 2),
            "max_abs_diff_vs_per_row": float((out.float() - per_row.float()).abs().max()),
        }), flush=True)
    return 0


GRAPH_STEP_LAYERS = 32


def graph_step(args) -> int:
    """A decode step of GRAPH_STEP_LAYERS layers, each a KV write and an attention call over one
    shared pool (every layer has the same shape, so one pool times them all), on graph metadata:
    run eagerly (the Python ops per call) and as one captured graph replayed per step; and, as
    the reference point of a GPU-bound step, eagerly on a planned step (its own work list)."""
    import torch

    from ayaka_amd import workloads
    from ayaka_amd.hip import _lib
    from ayaka_amd.hip import attention as hip_attention
    from ayaka_amd.hip import kvcache as hip_kvcache
    from ayaka_amd.enums import ForwardMode, KVLayoutKind
    from ayaka_amd.kvcache import RAW_CODEC, KVBuffers

    _lib.lib()
    dev = torch.device("cuda:0")
    for index in (1, 2, 3, 4, 5):
        cfg = workloads.config(index)
        step = workloads.build(cfg, dev, poison=False)
        buffers = KVBuffers(step.k_cache, step.v_cache, KVLayoutKind.NHD, RAW_CODEC)
        meta = hip_attention.graph_metadata(cfg.batch, step.table.shape[1], cfg.block_size, dev)
        hip_attention.update_graph_metadata(meta, step.lengths.cpu(), step.table.cpu())
        rows = step.k_new.shape[0]
        k_new, v_new = step.k_new[:cfg.batch].contiguous(), step.v_new[:cfg.batch].contiguous()
        if rows < cfg.batch:
            raise RuntimeError("graph step: fewer new rows than sequences")
        out = torch.empty_like(step.q)

        planned = hip_attention.plan(ForwardMode.DECODE, torch.ones(cfg.batch, dtype=torch.int32, device=dev),
                                     step.lengths, step.table, cfg.block_size)

        def one_step(meta=meta) -> None:
            for _ in range(GRAPH_STEP_LAYERS):
                hip_kvcache.store(k_new, v_new, buffers, meta)
                hip_attention.attend(step.q, buffers, meta, out, scale=cfg.scale)

        eager = time_calls(one_step, max(3, args.steps // 20), 2, repeats=3)
        eager_planned = time_calls(lambda: one_step(planned), max(3, args.steps // 20), 2, repeats=3)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            one_step()
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            one_step()
        replay = time_calls(graph.replay, max(3, args.steps // 20), 2, repeats=3)
        print(json.dumps({
            "workload": f"C{index} {cfg.name}: {GRAPH_STEP_LAYERS} layers of KV write + decode attention "
                        f"(graph metadata, batch {cfg.batch})",
            "planned_us_per_step": round(eager_planned["median_us"], 1),
            "eager_us_per_step": round(eager["median_us"], 1),
            "graph_us_per_step": round(replay["median_us"], 1),
            "planned_us_per_layer": round(eager_planned["median_us"] / GRAPH_STEP_LAYERS, 2),
            "eager_us_per_layer": round(eager["median_us"] / GRAPH_STEP_LAYERS, 2),
            "graph_us_per_layer": round(replay["median_us"] / GRAPH_STEP_LAYERS, 2),
        }), flush=True)
    return 0


def block_ops(args) -> int:
    """Time gather / copy_blocks / zero_blocks on the C3 pool (40000 blocks of 16 positions x 8
    key/value heads x 128 bf16, 32 KiB per block and cache) over 4096 distinct random blocks:
    one JSON line each, with the bytes the op must move (read + write, both caches) per second."""
    import torch

    from ayaka_amd import workloads
    from ayaka_amd.enums import KVLayoutKind
    from ayaka_amd.hip import _lib
    from ayaka_amd.hip import kvcache as hip_kvcache
    from ayaka_amd.kvcache import KVBuffers

    _lib.lib()
    dev = torch.device("cuda:0")
    cfg = workloads.config(3)
    shape = (cfg.num_blocks, cfg.block_size, cfg.kv_heads, cfg.head_dim)
    gen = torch.Generator(device=dev).manual_seed(7)
    buffers = KVBuffers(torch.randn(shape, generator=gen, device=dev).to(cfg.dtype),
                        torch.randn(shape, generator=gen, device=dev).to(cfg.dtype), KVLayoutKind.NHD, "raw")
    n = 4096
    ids = torch.randperm(cfg.num_blocks - 1, generator=gen, device=dev)[: 2 * n] + 1
    src, dst = ids[:n].contiguous(), ids[n:].contiguous()
    out_k = torch.empty((n, *shape[1:]), dtype=cfg.dtype, device=dev)
    out_v = torch.empty_like(out_k)
    block = cfg.block_size * cfg.kv_heads * cfg.head_dim * 2  # bytes per block and cache
    ops = {
        "gather": (lambda: hip_kvcache.gather(buffers, src, out_k, out_v), 2 * 2 * n * block),
        "copy_blocks": (lambda: hip_kvcache.copy_blocks(buffers, src, dst), 2 * 2 * n * block),
        "zero_blocks": (lambda: hip_kvcache.zero_blocks(buffers, dst), 2 * n * block),
    }
    for name, (fn, nbytes) in ops.items():
        us = time_calls(fn, args.steps, args.warmup, repeats=3)["median_us"]
        print(json.dumps({"op": name, "blocks": n, "block_bytes_per_cache": block, "bytes_moved": nbytes,
                          "us_per_call": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                          "hbm_fraction": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
    return 0


#: The reference's op benchmark (benchmarks/ops/attention.py:33-36): (query heads, key/value
#: heads, head width) of TinyLlama-1.1B and SmolLM2-135M; decode (batch, context) and prefill
#: (rows, context) steps of one request; block 16.
REFERENCE_SHAPES = {"tinyllama": (32, 4, 64), "smollm2-135m": (9, 3, 64)}
REFERENCE_DECODE = [(1, 512), (1, 2048), (1, 8192), (4, 2048), (8, 2048)]
REFERENCE_PREFILL = [(512, 512), (256, 2048)]


def reference_shapes(args) -> int:
    """The reference's op-benchmark matrix on this backend, fp16 as its default. Each step's
    requests hold contiguous blocks, as the reference lays them out; the step is planned over
    many disjoint copies of its blocks in one pool of about 1 GiB, and consecutive calls take
    consecutive copies, so every call reads its K/V from HBM rather than from the last call's
    cache lines (these steps hold 0.3-8 MB of K/V, well inside the 256 MB Infinity Cache). The
    time is the mean over back-to-back calls between two HIP events (median of 5 regions);
    ``us_one_pool_event`` is the reference's own method (one call per event pair, the median,
    always the same copy) for comparison. GB/s counts K/V read, q read and output written."""
    import numpy as np
    import torch

    from ayaka_amd.enums import ForwardMode, KVLayoutKind
    from ayaka_amd.hip import _lib
    from ayaka_amd.hip import attention as hip_attention
    from ayaka_amd.kvcache import RAW_CODEC, KVBuffers

    _lib.lib()
    dev, bs, dtype = torch.device("cuda:0"), 16, torch.float16
    for shape, (heads, kv_heads, dim) in REFERENCE_SHAPES.items():
        group = heads // kv_heads
        steps = [("decode", [1] * b, [n] * b) for b, n in REFERENCE_DECODE]
        steps += [("prefill", [rows], [n]) for rows, n in REFERENCE_PREFILL]
        for kind, rows, lengths in steps:
            need = [-(-n // bs) for n in lengths]
            per_copy = sum(need)
            block_bytes = bs * kv_heads * dim * 2
            copies = max(1, min(4096, (1 << 30) // (2 * block_bytes * per_copy)))
            gen = torch.Generator(device=dev).manual_seed(sum(lengths) + len(rows))
            k = torch.randn((copies * per_copy + 1, bs, kv_heads, dim), generator=gen, device=dev).to(dtype)
            v = torch.randn(k.shape, generator=gen, device=dev).to(dtype)
            buffers = KVBuffers(k, v, KVLayoutKind.NHD, RAW_CODEC)
            width = max(need)
            mode = ForwardMode.DECODE if kind == "decode" else ForwardMode.PREFILL
            rows_t = torch.tensor(rows, dtype=torch.int32, device=dev)
            lengths_t = torch.tensor(lengths, dtype=torch.int32, device=dev)
            metas = []
            for c in range(copies):
                table = np.zeros((len(lengths), width), dtype=np.int32)
                first = 1 + c * per_copy
                for r, n in enumerate(need):
                    table[r, :n] = np.arange(first, first + n)
                    first += n
                metas.append(hip_attention.plan(mode, rows_t, lengths_t, torch.from_numpy(table).to(dev), bs))
            q = torch.randn((sum(rows), heads, dim), generator=gen, device=dev).to(dtype)
            out = torch.empty_like(q)
            scale = dim ** -0.5
            turn = [0]

            def call() -> None:
                meta = metas[turn[0]]
                turn[0] = (turn[0] + 1) % copies
                hip_attention.attend(q, buffers, meta, out, scale=scale)

            for meta in metas:  # plan each copy's launch (work list, tiles) before timing
                hip_attention.attend(q, buffers, meta, out, scale=scale)
            timed = time_calls(call, max(args.steps, copies), args.warmup)

            def one() -> None:
                hip_attention.attend(q, buffers, metas[0], out, scale=scale)

            for _ in range(args.warmup):
                one()
            torch.cuda.synchronize()
            single = []
            for _ in range(50):
                start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                one()
                stop.record()
                stop.synchronize()
                single.append(start.elapsed_time(stop) * 1000.0)
            plan = metas[0].plan
            if kind == "decode":
                split = plan.split_for(kv_heads, group, 2)
                if split.partitions:
                    merge = hip_attention.merge_site(kv_heads, group, plan, split.partition_size)
                    launch = f"v2, {split.partitions} x {split.partition_size}, merge {merge}"
                else:
                    launch = f"v1, {split.waves or 'library'} waves per head"
            elif hip_attention.WINDOWS and plan.window_pairs(group) > 0:
                launch = f"windows, partition {plan.window_split(kv_heads, group, 2)}"
            else:
                pairs, size = plan.prefill_launch(kv_heads, group, dim, 2)
                launch = f"multi-row, tiles of {pairs} pairs, partition {size}"
            nbytes = sum(lengths) * kv_heads * dim * 2 * 2 + 2 * q.numel() * 2
            us = timed["median_us"]
            record = {"shape": shape, "heads": [heads, kv_heads, dim], "kind": kind, "dtype": "fp16",
                      "batch": len(rows), "rows": sum(rows), "context": lengths[0], "us_per_call": round(us, 2),
                      "gbs": round(nbytes / us / 1e3, 1), "launch": launch, "copies": copies,
                      "us_one_pool_event": round(statistics.median(single), 2)}
            if kind == "prefill":
                visible = sum(n - rows[0] + j + 1 for j in range(rows[0]) for n in lengths)
                record["tflops"] = round(4 * heads * dim * visible / us / 1e6, 1)
            else:
                # as the engine's decode runs: replays of one captured graph of up to 128 calls,
                # each over its own copy of the blocks
                calls = min(copies, 128)
                graph = torch.cuda.CUDAGraph()
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    hip_attention.attend(q, buffers, metas[0], out, scale=scale)
                torch.cuda.current_stream().wait_stream(side)
                torch.cuda.synchronize()
                with torch.cuda.graph(graph):
                    for c in range(calls):
                        hip_attention.attend(q, buffers, metas[c], out, scale=scale)
                record["us_graph"] = round(time_calls(graph.replay, 10, 3)["median_us"] / calls, 2)
                del graph
            print(json.dumps(record), flush=True)
            del metas, k, v, buffers
            torch.cuda.empty_cache()
    return 0


HOST_TRACE_STEPS = 3000


def continuous_batching_trace(steps: int, bucket: int, capacity: int, seed: int = 5) -> list:
    """Per-step int32 lengths of a decode bucket under continuous batching, C5-like: prompts
    log-uniform in [16, 16384]; every step each running request grows by one; every 4 steps
    0-3 requests finish (their rows go vacant, length 0) and 0-3 new ones take vacant rows,
    keeping 200-256 running. The row count of running requests changes at most steps, which
    is what defeats a choice cached under the step's shape."""
    import numpy as np

    rng = np.random.default_rng(seed)

    def draw(n: int):
        return np.minimum(np.exp(rng.uniform(np.log(16), np.log(16384), n)).astype(np.int64), capacity - steps - 1)

    lengths, out = draw(bucket), []
    for step in range(steps):
        lengths = np.where(lengths > 0, lengths + 1, 0)
        if step % 4 == 0:
            busy, free = np.flatnonzero(lengths > 0), np.flatnonzero(lengths == 0)
            k = int(rng.integers(0, 4))
            if k and busy.size > 200:
                lengths[rng.choice(busy, k, replace=False)] = 0
            k = min(int(rng.integers(0, 4)), free.size)
            if k:
                lengths[rng.choice(free, k, replace=False)] = draw(k)
        out.append(lengths.astype(np.int32))
    return out


def host_trace(args) -> int:
    """Host time per decode step over :func:`continuous_batching_trace` (C5 head shape: 64
    query heads over 8 key/value heads, block 32, a bucket of 256 rows by 512 blocks): the
    graph path's ``update_graph_metadata`` (positions, slots, table and the staged v2 split,
    one asynchronous copy), and the eager path's ``plan`` plus the split choice its first
    ``attend`` makes. Percentiles in µs over the trace; the split model's cache misses are
    counted."""
    import numpy as np
    import torch

    from ayaka_amd.enums import ForwardMode
    from ayaka_amd.hip import _lib
    from ayaka_amd.hip import attention as hip_attention

    _lib.lib()
    dev = torch.device("cuda:0")
    bucket, width, bs = 256, 512, 32
    trace = continuous_batching_trace(HOST_TRACE_STEPS, bucket, width * bs)
    rng = np.random.default_rng(6)
    table = torch.from_numpy(rng.integers(1, 100_000, (bucket, width)).astype(np.int32))
    meta = hip_attention.graph_metadata(bucket, width, bs, dev)
    meta.plan.head_shape.extend((8, 8, 2))
    hip_attention.update_graph_metadata(meta, torch.from_numpy(trace[0]), table)  # first-use costs
    torch.cuda.synchronize()
    hip_attention._split_cache.clear()
    misses, graph_us = 0, []
    for lengths in trace:
        host = torch.from_numpy(lengths)
        before = len(hip_attention._split_cache)
        t0 = time.perf_counter()
        hip_attention.update_graph_metadata(meta, host, table)
        graph_us.append((time.perf_counter() - t0) * 1e6)
        misses += len(hip_attention._split_cache) != before
        torch.cuda.synchronize()  # the step's replay and token read would wait here
    torch.cuda.synchronize()
    device_table = table.to(dev)
    ones = torch.ones(bucket, dtype=torch.int32, device=dev)
    eager_us = []
    hip_attention.plan(ForwardMode.DECODE, ones, torch.from_numpy(trace[0]).to(dev), device_table, bs)
    hip_attention._split_cache.clear()
    for lengths in trace[:1000]:
        device_lengths = torch.from_numpy(lengths).to(dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step = hip_attention.plan(ForwardMode.DECODE, ones, device_lengths, device_table, bs)
        step.plan.split_for(8, 8, 2)
        eager_us.append((time.perf_counter() - t0) * 1e6)

    def pct(values: list) -> dict:
        return {f"p{q}": round(float(np.percentile(values, q)), 1) for q in (50, 90, 99)} | \
               {"max": round(max(values), 1), "max_at_step": int(np.argmax(values))}

    print(json.dumps({"workload": "continuous-batching decode trace: 256-row bucket x 512 blocks of 32, "
                                  "64/8 heads, lengths log-uniform in [16, 16384], requests joining and "
                                  "leaving every 4 steps",
                      "steps": len(trace), "split_model_misses": misses,
                      "update_graph_metadata_us": pct(graph_us),
                      "eager_plan_and_split_us": pct(eager_us),
                      "host_cpus": os.cpu_count()}), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this build runs the "
              "decode path on one MI355X (sequences and key/value heads shard across GPUs without a "
              "collective, so a multi-GPU figure would be N independent copies of this one)", file=sys.stderr)
        return 2
    import torch

    if args.multi_row:
        return multi_row(args)
    if args.graph_step:
        return graph_step(args)
    if args.block_ops:
        return block_ops(args)
    if args.host_trace:
        return host_trace(args)
    if args.reference_shapes:
        return reference_shapes(args)
    if args.fp32:
        for index in (1, 2, 3, 4, 5):
            args.model_dtype = "fp32"
            rec = child_record(index, "raw", args)
            print(json.dumps({"config": f"C{index}", "model_dtype": "fp32", **rec}), flush=True)
        return 0
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel()}))
        return 0

    from ayaka_amd.hip import _lib

    _lib.lib()
    if args.record:
        print(json.dumps(measure(args.config, args, args.codec, args.layout)), flush=True)
        return 0
    head = measure(args.config, args, args.codec, args.layout, headline=True)
    line = head.pop("line")
    if not args.only and not args.no_configs:
        # every benchmark configuration, both codecs, as the library launches it (the
        # headline's own record is the one above). Each runs in a child process of its
        # own: a fresh allocator gives every pool the same placement a first run gets
        # (in one process, after the rotated pools of C1/C2 came and went, the later
        # configurations measured 5-10% slower).
        for codec, key in (("raw", "configs"), ("fp8_e4m3", "configs_fp8")):
            line[key] = {}
            for index in (1, 2, 3, 4, 5):
                if index == args.config and codec == args.codec:
                    line[key][f"C{index}"] = head
                    continue
                line[key][f"C{index}"] = child_record(index, codec, args)
        # the same configurations as fp32 models (fp32 q, out and caches: the fp32 decode kernel)
        line["configs_fp32"] = {}
        dtype_arg, args.model_dtype = args.model_dtype, "fp32"
        for index in (1, 2, 3, 4, 5):
            line["configs_fp32"][f"C{index}"] = child_record(index, "raw", args)
        args.model_dtype = dtype_arg
    print(json.dumps(line), flush=True)
    return 0


def child_record(index: int, codec: str, args) -> dict:
    """One configuration's record, measured by ``bench.py --record`` in a child process."""
    import subprocess

    cmd = [sys.executable, str(Path(__file__).resolve()), "--record", "--config", str(index), "--codec", codec,
           "--steps", str(args.steps), "--warmup", str(args.warmup)]
    if args.layout:
        cmd += ["--layout", args.layout]
    if args.qk:
        cmd += ["--qk", args.qk]
    if args.no_cpu_baseline:
        cmd += ["--no-cpu-baseline"]
    if args.model_dtype != "config":
        cmd += ["--model-dtype", args.model_dtype]
    done = subprocess.run(cmd, capture_output=True, text=True, timeout=300, check=False)
    sys.stderr.write(done.stderr)
    if done.returncode != 0:
        return {"error": f"exit status {done.returncode}"}
    return json.loads(done.stdout.strip().splitlines()[-1])


# Caches whose K/V working set fits MI355X's 256 MB Infinity Cache are timed over rotating
# copies of the pool, at least this many bytes of K/V in all, so that consecutive calls read
# HBM rather than the last call's lines.
ROTATION_BYTES = 1 << 30


def kernel_label(mfma: bool, split, merge: str | None, kv_bytes: int) -> str:
    """The dominant kernel of a launch, as the bench line and the profiles name it."""
    if kv_bytes == 4:
        what = "v1" if not split.partitions else "v2, merge reduce-kernel"
        return f"paged_attention_f32_kernel ({what})"
    name = "paged_attention_mfma_kernel" if mfma else "paged_attention_kernel"
    what = f"v1, {split.waves} waves per head" if not split.partitions else f"v2, merge {merge}"
    return f"{name} ({what}{', fp8 cache' if kv_bytes == 1 else ''})"


def measure(index: int, args, codec: str, layout_name: str | None, headline: bool = False) -> dict:
    """Time configuration ``index`` as ``attend`` launches it: µs per call, GB/s, the HBM
    fraction and the dominant kernel alone. The headline configuration also times v1 and
    v2 (partition 512, the reference's) and the best v2 launch, the KV write, the
    roofline record and the CPU baseline, and returns the bench line under "line"."""
    import torch

    from ayaka_amd import workloads
    from ayaka_amd.enums import ForwardMode, KVLayoutKind
    from ayaka_amd.hip import attention as hip_attention
    from ayaka_amd.hip import kvcache as hip_kvcache
    from ayaka_amd.kvcache import KVBuffers

    dev = torch.device("cuda:0")
    cfg = workloads.config(index)
    if args.model_dtype == "fp32":
        if codec != "raw" or headline:
            raise SystemExit("fp32 models are measured per configuration (--record or --fp32), raw caches only")
        cfg = dataclasses.replace(cfg, dtype=torch.float32)
    group = cfg.heads // cfg.kv_heads
    layout = KVLayoutKind(layout_name) if layout_name else KVLayoutKind(hip_kvcache.layout())
    step = workloads.build(cfg, dev, poison=False, layout=str(layout.value), codec=codec)
    buffers = KVBuffers(step.k_cache, step.v_cache, layout, codec)
    kv_bytes = 1 if codec == "fp8_e4m3" else cfg.dtype.itemsize
    write = hip_attention.plan(ForwardMode.MIXED, step.rows_per_request, step.lengths, step.table, cfg.block_size)
    hip_kvcache.store(step.k_new, step.v_new, buffers, write)
    meta = hip_attention.plan(ForwardMode.DECODE, torch.ones(cfg.batch, dtype=torch.int32, device=dev),
                              step.lengths, step.table, cfg.block_size)
    out = torch.empty_like(step.q)
    nbytes = workloads.algorithmic_bytes(cfg, kv_bytes)
    kv_set = sum(cfg.lengths) * cfg.kv_heads * cfg.head_dim * 2 * kv_bytes
    copies = 1 if headline and args.only else max(1, -(-ROTATION_BYTES // kv_set)) if kv_set < (256 << 20) else 1
    pools = [buffers] + [KVBuffers(step.k_cache.clone(), step.v_cache.clone(), layout, codec)
                         for _ in range(copies - 1)]
    turn = [0]

    def pool():
        turn[0] += 1
        return pools[turn[0] % len(pools)]

    auto = meta.plan.split_for(cfg.kv_heads, group, kv_bytes)  # what attend will launch
    mfma = args.qk == "mfma" or (args.qk is None and (hip_attention.uses_matrix_cores(group) or kv_bytes == 1
                                                      or (auto.partitions == 0 and auto.waves > 1)))
    merge = None if not auto.partitions else "reduce-kernel" if kv_bytes == 4 else \
        hip_attention.merge_site(cfg.kv_heads, group, meta.plan, auto.partition_size)
    kernel = kernel_label(mfma, auto, merge, kv_bytes)

    def call():
        hip_attention.attend(step.q, pool(), meta, out, scale=cfg.scale)

    settled = 0 if headline else settle(call, args.steps)
    result = time_calls(call, args.steps, args.warmup, repeats=1 if headline else 3)
    if auto.partitions and merge == "reduce-kernel":
        kernel_us = time_calls(
            lambda: hip_attention.attend_with(step.q, pool(), meta, out, scale=cfg.scale, partitions=None,
                                              partials_only=True), args.steps, args.warmup)["median_us"]
    else:
        kernel_us = result["median_us"]
    us = result["median_us"]
    record = {
        "us_per_call": round(us, 2),
        "gbs": round(nbytes / us / 1e3, 1),
        "hbm_fraction": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
        "launch": f"v1, {auto.waves} waves per head" if not auto.partitions else
                  f"v2 x{auto.partitions} partitions of {auto.partition_size}, merge {merge}",
        "kernel": kernel,
        "kernel_us": round(kernel_us, 2),
        "kernel_gbs": round(nbytes / kernel_us / 1e3, 1),
        "kernel_hbm_fraction": round(nbytes / kernel_us / 1e3 / HBM_PEAK_GBS, 4),
        "algorithmic_bytes": nbytes,
        "pools": len(pools),
        "settling_calls": settled,
    }
    profiled = PROFILED_TRAFFIC.get((cfg.index, kernel, auto.partition_size))
    if profiled is not None:  # HBM bytes of the dominant kernel per launch (rocprofv3 counters)
        record["traffic_read_write"] = [profiled[0], profiled[1]]
        record["traffic_source"] = profiled[2]
    if len(pools) > 1:  # the same call over one pool: what the Infinity Cache serves
        record["cache_resident_us"] = round(time_calls(
            lambda: hip_attention.attend(step.q, buffers, meta, out, scale=cfg.scale), args.steps,
            args.warmup)["median_us"], 2)
    if not headline and index != 1:
        # v2 at the reference's partition size (512; C4: up to 64 partitions per row), as the
        # configurations name it, beside the library's own launch
        ref_split = dict(partitions=-(-max(cfg.lengths) // hip_attention.PARTITION_SIZE),
                         partition_size=hip_attention.PARTITION_SIZE)
        r = time_calls(lambda: hip_attention.attend_with(step.q, pool(), meta, out, scale=cfg.scale, qk=args.qk,
                                                         **ref_split), args.steps, args.warmup, repeats=3)
        record["v2_512"] = {"us_per_call": round(r["median_us"], 2), "gbs": round(nbytes / r["median_us"] / 1e3, 1),
                            "hbm_fraction": round(nbytes / r["median_us"] / 1e3 / HBM_PEAK_GBS, 4), **ref_split}
    if not headline and kv_bytes == 2 and not args.no_cpu_baseline:
        # the reference's CPU path on the same step (it has no fp8 codec): every request,
        # C5 in groups of 16 with 3 timed runs (its padded gather is 7x its context)
        big = index == 5
        base = cpu_baseline(step, cfg, cfg.batch, kv_bytes, chunk=16 if big else None, runs=3 if big else 5)
        record["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in base.items()
                                  if k in ("value", "unit", "us_per_call", "cores", "kind", "sample")}
    print(f"[bench] C{index} {cfg.name} {codec}: {us:.1f} us/call {nbytes / us / 1e3:.0f} GB/s "
          f"({record['launch']}; kernel {kernel_us:.1f} us, {len(pools)} pools)", file=sys.stderr, flush=True)
    if not headline:
        del pools, step, buffers
        torch.cuda.empty_cache()
        return record

    # The headline: the other launches of the same step, then the bench line.
    max_len = max(cfg.lengths)
    best_v2 = hip_attention.choose_split(cfg.batch, cfg.kv_heads, group, max_len, row_lengths=cfg.lengths,
                                         kv_bytes=kv_bytes, v1=False)
    launches = {
        "v1": dict(partitions=0),
        "v2": dict(partitions=-(-max_len // hip_attention.PARTITION_SIZE),
                   partition_size=hip_attention.PARTITION_SIZE),
        "v2-best": dict(partitions=best_v2.partitions, partition_size=best_v2.partition_size or None),
    }
    kernels = {"auto": {"us_per_call": record["us_per_call"], "gbs": record["gbs"], "launch": record["launch"]}}
    if not args.only:
        for name, launch in launches.items():
            r = time_calls(lambda launch=launch: hip_attention.attend_with(step.q, pool(), meta, out, scale=cfg.scale,
                                                                          qk=args.qk, **launch),
                           args.steps, args.warmup, repeats=3)
            kernels[name] = {"us_per_call": round(r["median_us"], 2), "gbs": round(nbytes / r["median_us"] / 1e3, 1),
                             **{k: v for k, v in launch.items() if v is not None}}
            print(f"[bench] {cfg.name} {name}: {r['median_us']:.1f} us/call", file=sys.stderr, flush=True)
    store_us = time_calls(lambda: hip_kvcache.store(step.k_new, step.v_new, buffers, write), 50, 5)["median_us"]
    line = {
        "metric": "decode-attention µs/call + achieved HBM GB/s (% of peak) at 1 MI355X",
        "value": record["gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(result["wall_ms_per_step"], 4),
        "us_per_call": record["us_per_call"],
        "hbm_fraction": record["hbm_fraction"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype_label,
        "data": "synthetic (seeded N(0,1) K/V/Q, random block permutation)",
        "config": {
            "workload": f"C{cfg.index} {cfg.name} decode attention: Hq {cfg.heads}, Hkv {cfg.kv_heads}, "
                        f"D {cfg.head_dim}, {cfg.dtype_label}, {layout.value.upper()} "
                        f"{'fp8 e4m3 ' if kv_bytes == 1 else ''}cache, "
                        f"block {cfg.block_size}, batch {cfg.batch}, "
                        f"context {min(cfg.lengths)}-{max(cfg.lengths)} (sum {sum(cfg.lengths)}), "
                        f"pool {cfg.num_blocks} blocks",
            "algorithmic_bytes_per_call": nbytes,
            "launch": record["launch"],
        },
        "kernels": kernels,
        "kv_write": {"us_per_call": round(store_us, 2), "rows": int(step.k_new.shape[0]),
                     "bytes": workloads.store_bytes(cfg, kv_bytes)},
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "kernel_us": record["kernel_us"],
            "achieved": record["kernel_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": record["kernel_hbm_fraction"],
            "traffic": None if profiled is None else profiled[0] + profiled[1],
            "traffic_read_write": None if profiled is None else [profiled[0], profiled[1]],
            "traffic_source": None if profiled is None else profiled[2],
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(step, cfg, args.cpu_rows, kv_bytes)
    record["line"] = line
    return record


if __name__ == "__main__":
    sys.exit(main())
