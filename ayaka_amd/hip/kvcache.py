"""KV-cache ops with the MI355X kernels; implements the ``KVCacheOps`` contract.

``store`` is the KV write (``ayk_reshape_and_cache``): row ``i`` of ``k``/``v``
lands bit for bit in slot ``meta.slot_mapping[i]`` (reference
``python/ayaka/ops/backends/torch/kvcache.py:65-80``); into a ``"fp8_e4m3"``
cache it lands encoded (``ayk_reshape_and_cache_e4m3``). ``gather``,
``copy_blocks`` and ``zero_blocks`` move whole blocks (same file, ``:83-115``).
Both layouts are served; NHD is preferred, as the reference's ``layout()``
returns (``:30-31``).
"""

from __future__ import annotations

import torch

from ayaka_amd.attention import AttentionMetadata
from ayaka_amd.enums import KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.hip import _fastpath, _lib
from ayaka_amd.hip._checks import (
    compute_dtype,
    require_buffers,
    require_device,
    require_index_tensor,
    require_like,
    stream_handle,
)
from ayaka_amd.kvcache import FP8_E4M3_CODEC, KVBuffers, codec_scales

__all__ = ["copy_blocks", "gather", "layout", "store", "zero_blocks"]

_LAYOUT_CODES = {KVLayoutKind.NHD: 0, KVLayoutKind.HND: 1}
_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}


def layout() -> KVLayoutKind:
    return KVLayoutKind.NHD


def _stream(device: torch.device) -> int:
    return stream_handle(device)


def _block_bytes(buffers: KVBuffers) -> int:
    return buffers.k[0].numel() * buffers.k.element_size()


def _ids(op: str, name: str, ids: torch.Tensor, device: torch.device) -> None:
    require_index_tensor(op, name, ids, ndim=1)
    require_device(op, name, ids, device)
    if not ids.is_contiguous():
        raise BackendError(f"{op}: {name} must be contiguous", context={"op": op, "argument": name})


def store(k: torch.Tensor, v: torch.Tensor, buffers: KVBuffers, meta: AttentionMetadata) -> None:
    """Write each row's k and v into its slot (reference ``torch/kvcache.py:65-80``).

    As ``attend``: the first call with a combination of k, v, buffers and step metadata is
    checked in full and recorded in the step's plan; later calls with the same buffers and
    metadata, and k and v at the same addresses, shapes, strides and dtype, replay the library
    call on the current stream.
    """
    cache = getattr(meta.plan, "launches", None)
    if cache is None:
        _store(k, v, buffers, meta, None)
        return
    key = ("store", id(buffers), id(meta), _fastpath.signature((k, v, buffers.k, buffers.v)))
    found = _fastpath.lookup(cache, key)
    if found is not None:
        _fastpath.run(found, _stream(found.device))
        return
    record = _fastpath.Recorder()
    _store(k, v, buffers, meta, record)
    _fastpath.remember(cache, key, (buffers, meta), record)


def _store(k: torch.Tensor, v: torch.Tensor, buffers: KVBuffers, meta: AttentionMetadata,
           record: "_fastpath.Recorder | None") -> None:
    op = "kvcache.store"
    require_buffers(op, buffers)
    if meta.block_size != buffers.block_size:
        raise BackendError(
            f"{op}: the step was planned for blocks of {meta.block_size} positions "
            f"but the cache has blocks of {buffers.block_size}",
            context={"op": op, "argument": "meta"},
        )
    rows = meta.slot_mapping.shape[0]
    shape = (rows, buffers.num_kv_heads, buffers.head_dim)
    dtype = compute_dtype(op, "k", k, buffers)
    require_like(op, "k", k, shape, dtype)
    require_like(op, "v", v, shape, dtype)
    device = buffers.k.device
    for name, tensor in (("k", k), ("v", v), ("meta.slot_mapping", meta.slot_mapping)):
        require_device(op, name, tensor, device)
    slots = meta.slot_mapping
    if slots.dtype != torch.int64 or not slots.is_contiguous():
        raise BackendError(f"{op}: meta.slot_mapping must be a contiguous int64 tensor")
    if rows == 0:
        return
    if buffers.codec == FP8_E4M3_CODEC:
        fn = _lib.lib().ayk_reshape_and_cache_e4m3
        args = (k.data_ptr(), v.data_ptr(), buffers.k.data_ptr(), buffers.v.data_ptr(), slots.data_ptr(), rows,
                buffers.num_kv_heads, buffers.head_dim, buffers.num_blocks, buffers.block_size,
                _LAYOUT_CODES[KVLayoutKind(buffers.layout)], _DTYPE_CODES[dtype], *codec_scales(buffers.codec))
    else:
        fn = _lib.lib().ayk_reshape_and_cache
        args = (k.data_ptr(), v.data_ptr(), buffers.k.data_ptr(), buffers.v.data_ptr(), slots.data_ptr(), rows,
                buffers.num_kv_heads, buffers.head_dim, buffers.num_blocks, buffers.block_size,
                _LAYOUT_CODES[KVLayoutKind(buffers.layout)], buffers.k.element_size())
    if record is not None:
        record(op, fn, args, device, False)
    _lib.check(op, fn(*args, _stream(device)))


def gather(
    buffers: KVBuffers, block_ids: torch.Tensor, out_k: torch.Tensor, out_v: torch.Tensor
) -> None:
    op = "kvcache.gather"
    require_buffers(op, buffers)
    device = buffers.k.device
    _ids(op, "block_ids", block_ids, device)
    shape = (block_ids.shape[0], *buffers.k.shape[1:])
    require_like(op, "out_k", out_k, shape, buffers.k.dtype)
    require_like(op, "out_v", out_v, shape, buffers.k.dtype)
    require_device(op, "out_k", out_k, device)
    require_device(op, "out_v", out_v, device)
    if block_ids.shape[0] == 0:
        return
    _lib.check(
        op,
        _lib.lib().ayk_gather_blocks(
            buffers.k.data_ptr(),
            buffers.v.data_ptr(),
            out_k.data_ptr(),
            out_v.data_ptr(),
            block_ids.data_ptr(),
            int(block_ids.dtype == torch.int64),
            block_ids.shape[0],
            buffers.num_blocks,
            _block_bytes(buffers),
            _stream(device),
        ),
    )


def copy_blocks(buffers: KVBuffers, src: torch.Tensor, dst: torch.Tensor) -> None:
    op = "kvcache.copy_blocks"
    require_buffers(op, buffers)
    device = buffers.k.device
    _ids(op, "src", src, device)
    _ids(op, "dst", dst, device)
    if src.shape != dst.shape:
        raise BackendError(
            f"{op}: src has {src.shape[0]} blocks but dst has {dst.shape[0]}",
            context={"op": op, "argument": "dst"},
        )
    if src.shape[0] == 0:
        return
    if src.dtype != dst.dtype:
        src, dst = src.to(torch.int64), dst.to(torch.int64)
    _lib.check(
        op,
        _lib.lib().ayk_copy_blocks(
            buffers.k.data_ptr(),
            buffers.v.data_ptr(),
            src.data_ptr(),
            dst.data_ptr(),
            int(src.dtype == torch.int64),
            src.shape[0],
            buffers.num_blocks,
            _block_bytes(buffers),
            _stream(device),
        ),
    )


def zero_blocks(buffers: KVBuffers, block_ids: torch.Tensor) -> None:
    op = "kvcache.zero_blocks"
    require_buffers(op, buffers)
    device = buffers.k.device
    _ids(op, "block_ids", block_ids, device)
    if block_ids.shape[0] == 0:
        return
    _lib.check(
        op,
        _lib.lib().ayk_zero_blocks(
            buffers.k.data_ptr(),
            buffers.v.data_ptr(),
            block_ids.data_ptr(),
            int(block_ids.dtype == torch.int64),
            block_ids.shape[0],
            buffers.num_blocks,
            _block_bytes(buffers),
            _stream(device),
        ),
    )
