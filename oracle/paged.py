"""numpy restatement of the reference's paged-cache ops -- test infrastructure only.

Every function restates one reference function (cited in its docstring) and
names the checks in ``tests/test_oracle.py`` that pin it. Caches are NHD or HND
arrays of float32 (already widened from fp16/bf16 words by
:func:`oracle.numerics.bits_to_f32`) or of raw words for the bit-exact ops.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "PlanError",
    "attention",
    "copy_blocks",
    "gather",
    "nhd",
    "plan",
    "store",
    "zero_blocks",
]


class PlanError(ValueError):
    """A step the reference's ``plan`` refuses."""


def nhd(cache: np.ndarray, layout: str) -> np.ndarray:
    """View a cache as ``[block, offset, head, dim]`` (reference ``torch/kvcache.py:34-36``)."""
    return cache if layout == "nhd" else cache.transpose(0, 2, 1, 3)


def plan(
    mode: str, rows: list[int], lengths: list[int], table: np.ndarray, block_size: int
) -> dict[str, np.ndarray]:
    """Row numbering, positions and slots of one step.

    Restates ``python/ayaka/ops/backends/torch/attention.py:64-164`` (``plan``,
    ``_check_step``, ``_check_table``). Pinned by the reference tests' known
    answers (``tests/ops/test_attention_contract.py:393-467``) and against a
    brute-force walk over tokens.
    """
    table = np.asarray(table, dtype=np.int64).reshape(len(rows), -1)
    if len(lengths) != len(rows):
        raise PlanError("rows and lengths describe different requests")
    if block_size < 1:
        raise PlanError("block_size must be positive")
    for index, (count, length) in enumerate(zip(rows, lengths)):
        if count < 0 or length < 0:
            raise PlanError(f"request {index}: neither can be negative")
        if length and count > length:
            raise PlanError(f"request {index} has {count} query rows but only {length} tokens")
        if mode == "decode" and count != 1:
            raise PlanError("a DECODE step has one row per request")
    if mode == "idle" and sum(rows):
        raise PlanError("an IDLE step has no rows")
    needed = [-(-length // block_size) for length in lengths]
    max_blocks = table.shape[1]
    if max(needed, default=0) > max_blocks or (sum(rows) and max_blocks == 0):
        raise PlanError(f"the longest request needs {max(needed)} blocks of {block_size}")
    for b, n in enumerate(needed):
        if (table[b, :n] == 0).any():
            raise PlanError("padding block 0 inside a request's blocks")
    request_of_row, positions, slots = [], [], []
    for b, (count, length) in enumerate(zip(rows, lengths)):
        for j in range(count):
            request_of_row.append(b)
            pos = length - count + j if length else 0
            positions.append(pos)
            slots.append(int(table[b, pos // block_size]) * block_size + pos % block_size if length else 0)
    return {
        "request_of_row": np.asarray(request_of_row, dtype=np.int32),
        "positions": np.asarray(positions, dtype=np.int32),
        "slot_mapping": np.asarray(slots, dtype=np.int64),
    }


def store(
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    slot_mapping: np.ndarray,
    layout: str,
) -> None:
    """Write row i of k/v into slot ``slot_mapping[i]``, in place, bit for bit.

    Restates ``python/ayaka/ops/backends/torch/kvcache.py:65-80`` (an
    ``index_put`` through the NHD view). Pinned by the reference tests' known
    answer (``tests/ops/test_kvcache_contract.py:85-125``).
    """
    block_size = nhd(k_cache, layout).shape[1]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    blocks, offsets = slots // block_size, slots % block_size
    nhd(k_cache, layout)[blocks, offsets] = k
    nhd(v_cache, layout)[blocks, offsets] = v


def gather(k_cache: np.ndarray, v_cache: np.ndarray, block_ids: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Whole blocks in the order of ``block_ids`` (reference ``torch/kvcache.py:83-93``)."""
    ids = np.asarray(block_ids, dtype=np.int64)
    return k_cache[ids].copy(), v_cache[ids].copy()


def copy_blocks(k_cache: np.ndarray, v_cache: np.ndarray, src: np.ndarray, dst: np.ndarray) -> None:
    """Block ``dst[i]`` = block ``src[i]``, both caches (reference ``torch/kvcache.py:96-107``)."""
    src, dst = np.asarray(src, dtype=np.int64), np.asarray(dst, dtype=np.int64)
    k_cache[dst] = k_cache[src]
    v_cache[dst] = v_cache[src]


def zero_blocks(k_cache: np.ndarray, v_cache: np.ndarray, block_ids: np.ndarray) -> None:
    """Every element of the listed blocks set to zero (reference ``torch/kvcache.py:110-115``)."""
    ids = np.asarray(block_ids, dtype=np.int64)
    k_cache[ids] = 0
    v_cache[ids] = 0


def attention(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    table: np.ndarray,
    kv_lengths: np.ndarray,
    *,
    scale: float,
    layout: str = "nhd",
    request_of_row: np.ndarray | None = None,
    positions: np.ndarray | None = None,
    precision: type = np.float32,
    chunk: int = 16,
) -> np.ndarray:
    """Paged attention of every query row, gather-then-softmax.

    Restates the reference's decode path ``_attend_decode``
    (``python/ayaka/ops/backends/torch/attention.py:237-271``): gather each
    row's whole padded table, scores ``scale * q.k`` in ``precision``, mask
    positions at or past the row's length to -inf, softmax, zero the weights of
    a row with nothing visible and the values past the length (0 * NaN is NaN),
    then the weighted sum. Query head h reads key/value head h // G.

    With ``request_of_row`` and ``positions`` it is the reference's multi-row
    rule (``attention.py:209-234``, row-causal SDPA): row n reads request
    ``request_of_row[n]``'s table and sees positions ``0 .. positions[n]``; a row
    of a request with ``kv_lengths == 0`` is a padding row and gets zeros.
    Rows are processed ``chunk`` at a time so the padded gather stays small
    (same semantics).

    Pinned by a pure-Python float64 loop on small inputs, by torch's
    ``scaled_dot_product_attention`` (a library routine), and by the invariants
    of the reference's tests: one visible key returns its value, scale 0 returns
    the mean of the visible values, padding rows are zero, NaN in unread slots
    does not leak.
    """
    q = np.asarray(q)
    n_rows, heads, dim = q.shape
    keys, values = nhd(k_cache, layout), nhd(v_cache, layout)
    block_size, kv_heads = keys.shape[1], keys.shape[2]
    group = heads // kv_heads
    table = np.asarray(table, dtype=np.int64)
    lengths = np.asarray(kv_lengths, dtype=np.int64)
    if request_of_row is None:
        req = np.arange(n_rows)
        row_len = lengths[:n_rows]
    else:
        req = np.asarray(request_of_row, dtype=np.int64)
        pos = np.asarray(positions, dtype=np.int64)
        row_len = np.where(lengths[req] > 0, pos + 1, 0)
    out = np.zeros((n_rows, heads, dim), dtype=precision)
    width = table.shape[1] * block_size
    for start in range(0, n_rows, chunk):
        rows = slice(start, min(n_rows, start + chunk))
        blocks = table[req[rows]]  # [r, MB]
        ctx_k = keys[blocks].reshape(blocks.shape[0], width, kv_heads, dim).astype(precision)
        ctx_v = values[blocks].reshape(blocks.shape[0], width, kv_heads, dim).astype(precision)
        query = q[rows].astype(precision).reshape(-1, kv_heads, group, dim)
        # [r, Hkv, G, D] @ [r, Hkv, D, W] -> [r, Hkv, G, W]
        scores = np.matmul(query, ctx_k.transpose(0, 2, 3, 1)) * precision(scale)
        visible = np.arange(width)[None, :] < row_len[rows][:, None]  # [r, W]
        scores = np.where(visible[:, None, None, :], scores, -np.inf)
        peak = scores.max(axis=-1, keepdims=True)
        peak = np.where(np.isfinite(peak), peak, 0.0)
        with np.errstate(invalid="ignore", over="ignore"):
            weights = np.exp(scores - peak)
            weights = weights / weights.sum(axis=-1, keepdims=True)
        weights = np.where(visible.any(axis=-1)[:, None, None, None], weights, 0.0)
        ctx_v = np.where(visible[:, :, None, None], ctx_v, 0.0)
        # [r, Hkv, G, W] @ [r, Hkv, W, D] -> [r, Hkv, G, D]
        result = np.matmul(weights.astype(precision), ctx_v.transpose(0, 2, 1, 3))
        out[rows] = result.reshape(-1, heads, dim)
    return out


def attention_of_requests(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    table: np.ndarray,
    kv_lengths: np.ndarray,
    *,
    scale: float,
    request_of_row: np.ndarray,
    positions: np.ndarray,
    layout: str = "nhd",
    precision: type = np.float64,
    rows_per_pass: int = 64,
) -> np.ndarray:
    """:func:`attention`'s multi-row rule (reference ``attention.py:209-234``) with the rows of
    one request sharing one gather of its context, so that full-size prefill chunks (thousands of
    rows over thousands of positions) finish in seconds.

    Same semantics as :func:`attention` given ``request_of_row`` and ``positions``: row n sees
    positions ``0 .. positions[n]`` of its request, a request of length 0 gives zero rows, and
    the values at or past the request's length are zeroed before the weighted sum. Pinned
    against :func:`attention` on mixed steps with padding requests and NaN-poisoned slots.
    """
    q = np.asarray(q)
    n_rows, heads, dim = q.shape
    keys, values = nhd(k_cache, layout), nhd(v_cache, layout)
    block_size, kv_heads = keys.shape[1], keys.shape[2]
    group = heads // kv_heads
    table = np.asarray(table, dtype=np.int64)
    lengths = np.asarray(kv_lengths, dtype=np.int64)
    req = np.asarray(request_of_row, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    width = table.shape[1] * block_size
    out = np.zeros((n_rows, heads, dim), dtype=precision)
    for r in np.unique(req):
        rows = np.flatnonzero(req == r)
        if lengths[r] <= 0:
            continue
        # [W, Hkv, D] -> [Hkv, D, W] keys and [Hkv, W, D] values, values past the length zeroed
        ctx_k = keys[table[r]].reshape(width, kv_heads, dim).astype(precision).transpose(1, 2, 0)
        ctx_v = values[table[r]].reshape(width, kv_heads, dim).astype(precision)
        ctx_v = np.where((np.arange(width) < lengths[r])[:, None, None], ctx_v, 0.0).transpose(1, 0, 2)
        for start in range(0, rows.size, rows_per_pass):
            part = rows[start:start + rows_per_pass]
            # [n, Hq, D] -> [Hkv, G, n, D] @ [Hkv, 1, D, W] -> [Hkv, G, n, W]
            query = q[part].astype(precision).reshape(-1, kv_heads, group, dim).transpose(1, 2, 0, 3)
            scores = np.matmul(query, ctx_k[:, None]) * precision(scale)
            visible = np.arange(width)[None, :] <= pos[part][:, None]  # [n, W]
            scores = np.where(visible[None, None], scores, -np.inf)
            peak = scores.max(axis=-1, keepdims=True)
            with np.errstate(invalid="ignore", over="ignore"):
                weights = np.exp(scores - peak)
                weights = weights / weights.sum(axis=-1, keepdims=True)
            # [Hkv, G, n, W] @ [Hkv, 1, W, D] -> [Hkv, G, n, D] -> [n, Hq, D]
            result = np.matmul(weights, ctx_v[:, None])
            out[part] = result.transpose(2, 0, 1, 3).reshape(-1, heads, dim)
    return out
