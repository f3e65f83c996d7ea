"""The reference's CPU decode algorithm restated in torch -- test and benchmark infrastructure only.

``attend_decode`` follows ``_attend_decode``
(``python/ayaka/ops/backends/torch/attention.py:237-271``), the path the reference's
torch backend runs for a decode step on the CPU: gather every request's whole padded
table, widen K and V to float32, scores ``scale * q.k`` per key/value head group, mask
positions at or past the length to -inf, softmax, zero the weights of a request with
nothing visible and the values past the length (0 * NaN is NaN), weighted sum, one
rounding into ``out``'s dtype. ``bench.py`` times it on the host as the CPU baseline;
``tests/test_oracle.py`` pins it against the numpy oracle (``oracle.paged.attention``)
and against the float64 loop that pins that one.
"""

from __future__ import annotations

import torch

__all__ = ["attend_decode"]


def attend_decode(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, table: torch.Tensor,
                  lengths: torch.Tensor, *, scale: float) -> torch.Tensor:
    """Decode attention of ``q`` ``[B, Hq, D]`` over NHD caches ``[blocks, bs, Hkv, D]`` with
    int ``table`` ``[B, max_blocks]`` and ``lengths`` ``[B]``; returns ``[B, Hq, D]`` in q's dtype."""
    batch, heads, dim = q.shape
    kv_heads = keys.shape[2]
    ids = table.long()
    width = ids.shape[1] * keys.shape[1]
    # [B, max_blocks, bs, Hkv, D] -> [B, Hkv, W, D], float32
    ctx_k = keys[ids].reshape(batch, width, kv_heads, dim).permute(0, 2, 1, 3).float()
    ctx_v = values[ids].reshape(batch, width, kv_heads, dim).permute(0, 2, 1, 3).float()
    query = q.float().reshape(batch, kv_heads, heads // kv_heads, dim)
    seen = torch.arange(width)[None, :] < lengths.long()[:, None]  # [B, W]
    scores = torch.matmul(query, ctx_k.transpose(-1, -2)) * scale  # [B, Hkv, G, W]
    scores = scores.masked_fill(~seen[:, None, None, :], float("-inf"))
    weights = torch.softmax(scores, dim=-1)
    weights = torch.where(seen.any(dim=-1)[:, None, None, None], weights, torch.zeros((), dtype=weights.dtype))
    ctx_v = torch.where(seen[:, None, :, None], ctx_v, torch.zeros((), dtype=ctx_v.dtype))
    out = torch.matmul(weights, ctx_v)  # [B, Hkv, G, D]
    return out.reshape(batch, heads, dim).to(q.dtype)
