"""Write ``smollm2_small.npz``: a small SmolLM2-shape step, its KV write and its float64 output.

Shape of benchmark configuration 1 (9 query heads, 3 key/value heads, head_dim
64, fp16, block 16) at the reference parity test's lengths {1, 16, 17, 70}
(``tests/ops/test_parity.py:207-208``), 4 new tokens per sequence (1 for the
one-token sequence). Inputs are drawn from ``numpy.random.default_rng(1)`` and
rounded to fp16; the expected output is the oracle's float64 gather-then-softmax
on the cache after the write. The device tests replay the write and the
attention on these exact words.

Run from the repository root: ``python -m tests.golden.make_golden``.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import paged
from oracle.numerics import bits_to_f32, f32_to_bits

HERE = Path(__file__).resolve().parent


def main() -> None:
    rng = np.random.default_rng(1)
    heads, kv_heads, dim, bs = 9, 3, 64, 16
    lengths = [1, 16, 17, 70]
    new = [min(4, n) for n in lengths]
    needed = [-(-n // bs) for n in lengths]
    num_blocks = 1 + sum(needed) + 4
    order = rng.permutation(np.arange(1, num_blocks))
    table = np.zeros((len(lengths), max(needed)), dtype=np.int64)
    first = 0
    for b, n in enumerate(needed):
        table[b, :n] = order[first:first + n]
        first += n
    nan = np.uint16(0x7E00)
    k_cache = np.full((num_blocks, bs, kv_heads, dim), nan, dtype=np.uint16)
    v_cache = np.full_like(k_cache, nan)
    for b, n in enumerate(lengths):
        for pos in range(n - new[b]):
            blk, off = table[b, pos // bs], pos % bs
            k_cache[blk, off] = f32_to_bits((0.5 * rng.standard_normal((kv_heads, dim))).astype(np.float32), "fp16")
            v_cache[blk, off] = f32_to_bits((0.5 * rng.standard_normal((kv_heads, dim))).astype(np.float32), "fp16")
    step = paged.plan("mixed", new, lengths, table, bs)
    k_new = f32_to_bits((0.5 * rng.standard_normal((sum(new), kv_heads, dim))).astype(np.float32), "fp16")
    v_new = f32_to_bits((0.5 * rng.standard_normal((sum(new), kv_heads, dim))).astype(np.float32), "fp16")
    q = f32_to_bits((0.5 * rng.standard_normal((len(lengths), heads, dim))).astype(np.float32), "fp16")
    k_after, v_after = k_cache.copy(), v_cache.copy()
    paged.store(k_after, v_after, k_new, v_new, step["slot_mapping"], "nhd")
    scale = 1.0 / 8.0
    expected = paged.attention(
        bits_to_f32(q, "fp16"), bits_to_f32(k_after, "fp16"), bits_to_f32(v_after, "fp16"),
        table, np.asarray(lengths), scale=scale, precision=np.float64,
    )
    np.savez_compressed(
        HERE / "smollm2_small.npz",
        q=q, k_cache_before=k_cache, v_cache_before=v_cache, k_new=k_new, v_new=v_new,
        rows_per_request=np.asarray(new, dtype=np.int32), slot_mapping=step["slot_mapping"],
        k_cache=k_after, v_cache=v_after, table=table, lengths=np.asarray(lengths, dtype=np.int32),
        scale=np.float64(scale), expected=expected,
    )


if __name__ == "__main__":
    main()
