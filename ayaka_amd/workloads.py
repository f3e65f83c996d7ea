"""Seeded synthetic decode steps at the benchmark shapes.

Five configurations, numbered as in the benchmark definition:

1. SmolLM2-135M shape: 9/3/64 fp16, block 16, 4 sequences of {128, 300, 512, 1000},
   values 0.5 N(0,1), a pool of 256 blocks, 4 new tokens per sequence written by
   the KV write.
2. Llama-3.2-1B shape: 32/8/64 fp16, block 16, 32 sequences of U[512, 4096] with
   three of length 1, a pool of 16384 blocks.
3. Llama-3-8B shape: 32/8/128 bf16, block 16, 64 sequences of 4096, a pool of
   40000 blocks (the headline shape).
4. Long context: 32/8/128 bf16, block 16, 8 sequences of {8K, 16K, 24K, 32K, 32K,
   32K, 12K, 2K}, 0.1% of key positions scaled by 20.
5. Ragged continuous batching: 64/8/128 bf16, block 32, 256 sequences of
   log-uniform length in [16, 16384].

Every configuration ends its step with the KV write of each sequence's newest
``new_tokens`` positions (``store``) followed by decode attention over all
sequences. Those slots are free before the step (never written, NaN) and lie in
blocks drawn from a random permutation of the pool, so C5's "256 new tokens into
random free slots" is its 256 sequences' newest tokens, scattered over the pool. Blocks come from a seeded permutation of the pool (never block 0).
Every slot that is not part of a context holds NaN, so a kernel that reads past
a length, an unused table entry or block 0 shows it. Lengths are drawn on the
host from ``numpy.random.default_rng(1000 + index)``; tensors from a
``torch.Generator`` seeded with ``1000 + index`` on the target device.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

__all__ = ["Config", "Step", "algorithmic_bytes", "build", "config", "sample_rows"]


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    heads: int
    kv_heads: int
    head_dim: int
    dtype: torch.dtype
    block_size: int
    lengths: tuple[int, ...]
    num_blocks: int
    new_tokens: int = 1
    q_std: float = 1.0
    kv_std: float = 1.0
    outlier_fraction: float = 0.0
    outlier_scale: float = 20.0

    @property
    def batch(self) -> int:
        return len(self.lengths)

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def dtype_label(self) -> str:
        return {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[self.dtype]


def config(index: int) -> Config:
    """The benchmark configuration ``index`` (1-5)."""
    rng = np.random.default_rng(1000 + index)
    if index == 1:
        return Config(1, "smollm2-135m", 9, 3, 64, torch.float16, 16, (128, 300, 512, 1000), 256,
                      new_tokens=4, q_std=0.5, kv_std=0.5)
    if index == 2:
        lengths = rng.integers(512, 4097, size=32)
        lengths[[5, 17, 29]] = 1  # three one-token sequences
        return Config(2, "llama-3.2-1b", 32, 8, 64, torch.float16, 16, tuple(int(x) for x in lengths),
                      16384)
    if index == 3:
        return Config(3, "llama-3-8b", 32, 8, 128, torch.bfloat16, 16, (4096,) * 64, 40000)
    if index == 4:
        lengths = tuple(k * 1024 for k in (8, 16, 24, 32, 32, 32, 12, 2))
        used = sum(-(-n // 16) for n in lengths)
        return Config(4, "llama-3-8b-long", 32, 8, 128, torch.bfloat16, 16, lengths, used + 1 + 1024,
                      outlier_fraction=0.001)
    if index == 5:
        lengths = np.floor(np.exp(rng.uniform(math.log(16), math.log(16384), size=256))).astype(int)
        used = int(sum(-(-int(n) // 32) for n in lengths))
        return Config(5, "ragged-gqa8", 64, 8, 128, torch.bfloat16, 32, tuple(int(x) for x in lengths),
                      used + 1 + 4096)
    raise ValueError(f"no configuration {index}")


@dataclass
class Step:
    """One synthetic decode step: a filled pool, its table, the rows to store and the queries."""

    config: Config
    k_cache: torch.Tensor  # [num_blocks, block_size, kv_heads, head_dim] (NHD) or HND
    v_cache: torch.Tensor
    table: torch.Tensor  # [B, max_blocks] int32
    lengths: torch.Tensor  # [B] int32
    rows_per_request: torch.Tensor  # [B] int32, the rows of the KV write
    k_new: torch.Tensor  # [sum rows, kv_heads, head_dim]
    v_new: torch.Tensor
    q: torch.Tensor  # [B, heads, head_dim], the decode queries


def build(cfg: Config, device: torch.device | str = "cpu", *, poison: bool = True, layout: str = "nhd",
          codec: str = "raw") -> Step:
    """Fill a pool for ``cfg`` on ``device``. The newest ``new_tokens`` positions of every
    sequence are left unwritten (NaN): the step's KV write fills them. ``layout`` "hnd"
    returns the same values in HND caches (``[num_blocks, kv_heads, block_size, head_dim]``);
    ``codec`` "fp8_e4m3" returns them cast to ``torch.float8_e4m3fn``."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(1000 + cfg.index)
    host = np.random.default_rng(2000 + cfg.index)
    bs, hkv, dim = cfg.block_size, cfg.kv_heads, cfg.head_dim
    needed = [-(-n // bs) for n in cfg.lengths]
    max_blocks = max(needed)
    if sum(needed) > cfg.num_blocks - 1:
        raise ValueError(f"{cfg.name}: {sum(needed)} blocks do not fit a pool of {cfg.num_blocks}")
    order = host.permutation(np.arange(1, cfg.num_blocks))
    table = np.zeros((cfg.batch, max_blocks), dtype=np.int32)
    first = 0
    for b, n in enumerate(needed):
        table[b, :n] = order[first:first + n]
        first += n
    used = torch.from_numpy(order[:first].astype(np.int64)).to(device)

    fill = float("nan") if poison else 0.0
    shape = (cfg.num_blocks, bs, hkv, dim)
    k_cache = torch.full(shape, fill, dtype=cfg.dtype, device=device)
    v_cache = torch.full(shape, fill, dtype=cfg.dtype, device=device)
    # Positions written before this step: [0, L - new_tokens) of each sequence.
    valid = np.zeros((first, bs), dtype=bool)
    first = 0
    for n, length in zip(needed, cfg.lengths):
        written = max(0, length - cfg.new_tokens)
        flat = np.zeros(n * bs, dtype=bool)
        flat[:written] = True
        valid[first:first + n] = flat.reshape(n, bs)
        first += n
    mask = torch.from_numpy(valid).to(device)[:, :, None, None]
    for cache, std in ((k_cache, cfg.kv_std), (v_cache, cfg.kv_std)):
        chunk = 4096
        for start in range(0, used.numel(), chunk):
            ids = used[start:start + chunk]
            vals = torch.randn((ids.numel(), bs, hkv, dim), generator=gen, device=device) * std
            if cache is k_cache and cfg.outlier_fraction:
                hit = torch.rand((ids.numel(), bs, 1, 1), generator=gen, device=device)
                vals = torch.where(hit < cfg.outlier_fraction, vals * cfg.outlier_scale, vals)
            vals = vals.to(cfg.dtype)
            cache[ids] = torch.where(mask[start:start + chunk], vals, cache[ids])
    rows = [min(cfg.new_tokens, n) for n in cfg.lengths]
    k_new = (torch.randn((sum(rows), hkv, dim), generator=gen, device=device) * cfg.kv_std).to(cfg.dtype)
    v_new = (torch.randn((sum(rows), hkv, dim), generator=gen, device=device) * cfg.kv_std).to(cfg.dtype)
    q = (torch.randn((cfg.batch, cfg.heads, dim), generator=gen, device=device) * cfg.q_std).to(cfg.dtype)
    if layout == "hnd":
        k_cache = k_cache.permute(0, 2, 1, 3).contiguous()
        v_cache = v_cache.permute(0, 2, 1, 3).contiguous()
    if codec == "fp8_e4m3":
        k_cache, v_cache = k_cache.to(torch.float8_e4m3fn), v_cache.to(torch.float8_e4m3fn)
    elif codec != "raw":
        raise ValueError(f"unknown codec {codec!r}")
    return Step(
        config=cfg,
        k_cache=k_cache,
        v_cache=v_cache,
        table=torch.from_numpy(table).to(device),
        lengths=torch.tensor(cfg.lengths, dtype=torch.int32, device=device),
        rows_per_request=torch.tensor(rows, dtype=torch.int32, device=device),
        k_new=k_new,
        v_new=v_new,
        q=q,
    )


def algorithmic_bytes(cfg: Config, kv_bytes: int = 2) -> int:
    """Bytes one decode-attention call must move: K and V of every context position (``kv_bytes``
    per element: 2, 1 for fp8 caches, 4 for fp32 models), q read, out written, the used table entries and the
    lengths (v2 scratch not counted). q and out have the model's element size."""
    s = cfg.dtype.itemsize
    kv = sum(cfg.lengths) * cfg.kv_heads * cfg.head_dim * 2 * kv_bytes
    qo = 2 * cfg.batch * cfg.heads * cfg.head_dim * s
    table = 4 * sum(-(-n // cfg.block_size) for n in cfg.lengths)
    return kv + qo + table + 4 * cfg.batch


def store_bytes(cfg: Config, kv_bytes: int = 2) -> int:
    """Bytes of the step's KV write: read k and v rows (the model's element size), write them
    (``kv_bytes`` per element), read the slots."""
    rows = sum(min(cfg.new_tokens, n) for n in cfg.lengths)
    return 2 * rows * cfg.kv_heads * cfg.head_dim * (cfg.dtype.itemsize + kv_bytes) + 8 * rows


def sample_rows(step: Step, rows: list[int]) -> dict[str, np.ndarray]:
    """Copy what the decode rows ``rows`` read to the host, with their blocks renumbered 1..n.

    Returns float32 ``q`` [r, H, D], ``k``/``v`` [n + 1, bs, Hkv, D] (block 0 NaN),
    ``table`` [r, max_blocks] and ``lengths`` [r], so an oracle can recompute those
    rows without the whole pool.
    """
    table = step.table[rows].cpu().numpy().astype(np.int64)
    lengths = step.lengths[rows].cpu().numpy().astype(np.int64)
    bs = step.config.block_size
    used = np.arange(table.shape[1])[None, :] < -(-lengths[:, None] // bs)  # the table entries each row reads
    ids = np.unique(table[used])
    new_table = np.where(used, np.searchsorted(ids, table) + 1, 0)
    index = torch.from_numpy(ids).to(step.k_cache.device)
    k_nhd, v_nhd = step.k_cache[index], step.v_cache[index]
    if k_nhd.shape[1] != bs:  # HND caches: back to [block, offset, head, dim]
        k_nhd, v_nhd = k_nhd.permute(0, 2, 1, 3), v_nhd.permute(0, 2, 1, 3)
    nan_block = torch.full((1, *k_nhd.shape[1:]), float("nan"))
    k = torch.cat([nan_block, k_nhd.float().cpu()]).numpy()
    v = torch.cat([nan_block, v_nhd.float().cpu()]).numpy()
    return {
        "q": step.q[rows].float().cpu().numpy(),
        "k": k,
        "v": v,
        "table": new_table,
        "lengths": lengths,
    }
