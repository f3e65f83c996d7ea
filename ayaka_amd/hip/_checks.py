"""Argument checks of the hip ops.

The messages follow the reference's (``python/ayaka/ops/backends/torch/_checks.py:21-59``,
``kvcache.py:39-62``) so that callers and tests read the same refusals. The
hip backend computes in fp16, bf16 and fp32 (fp32 on a decode kernel of its own, row by row),
on HIP devices, for head widths of 64, 128 and 256 and block sizes of 1 to 65536 positions; it
stores the ``"raw"`` codec (fp16/bf16/fp32 caches) and ``"fp8_e4m3"`` (``float8_e4m3fn`` caches,
read by fp16/bf16 models).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from ayaka_amd.enums import KVLayoutKind
from ayaka_amd.errors import BackendError
from ayaka_amd.kvcache import FP8_E4M3_CODEC, RAW_CODEC, KVBuffers

__all__ = [
    "HEAD_DIMS",
    "capturing",
    "compute_dtype",
    "dtype_name",
    "require_buffers",
    "require_device",
    "require_index_tensor",
    "require_like",
    "stream_handle",
]

HEAD_DIMS = frozenset({64, 128, 256})
_DTYPES = (torch.float16, torch.bfloat16)  # compute dtypes over a quantised codec
_RAW_DTYPES = (torch.float16, torch.bfloat16, torch.float32)  # the raw codec's, fp32 on its own kernel
_NAMES = {
    torch.float16: "float16",
    torch.bfloat16: "bfloat16",
    torch.float32: "float32",
    torch.float64: "float64",
    torch.int32: "int32",
    torch.int64: "int64",
    torch.float8_e4m3fn: "float8_e4m3fn",
}
# The cache element type of each codec this backend stores.
_CODEC_DTYPES = {RAW_CODEC: _RAW_DTYPES, FP8_E4M3_CODEC: (torch.float8_e4m3fn,)}


def dtype_name(dtype: torch.dtype) -> str:
    return _NAMES.get(dtype, str(dtype).removeprefix("torch."))


def capturing(tensor: torch.Tensor) -> bool:
    """Whether ``tensor``'s device is capturing a graph on the current stream."""
    return tensor.is_cuda and torch._C._cuda_isCurrentStreamCapturing()


# torch's raw handle of the current stream, without building a Stream object per call
# (about 3 us of host time each): the ops launch once per layer and per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The HIP stream behind torch's current stream on ``device``: the ops launch there."""
    if _raw_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(index)


def require_like(
    op: str, name: str, tensor: torch.Tensor, shape: Sequence[int], dtype: torch.dtype
) -> None:
    if tuple(tensor.shape) != tuple(shape) or tensor.dtype != dtype:
        raise BackendError(
            f"{op}: {name} must be {dtype_name(dtype)} {list(shape)}, "
            f"got {dtype_name(tensor.dtype)} {list(tensor.shape)}",
            context={"op": op, "argument": name},
        )
    if not tensor.is_contiguous():
        raise BackendError(f"{op}: {name} must be contiguous", context={"op": op, "argument": name})


def require_index_tensor(op: str, name: str, tensor: torch.Tensor, *, ndim: int) -> None:
    if tensor.dtype not in (torch.int32, torch.int64) or tensor.ndim != ndim:
        raise BackendError(
            f"{op}: {name} must be an int32 or int64 tensor with {ndim} dimension(s), "
            f"got {dtype_name(tensor.dtype)} {list(tensor.shape)}",
            context={"op": op, "argument": name},
        )


def require_device(op: str, name: str, tensor: torch.Tensor, device: torch.device) -> None:
    if tensor.device != device:
        raise BackendError(
            f"{op}: {name} is on {tensor.device}, the cache is on {device}",
            context={"op": op, "argument": name},
        )


def compute_dtype(op: str, name: str, tensor: torch.Tensor, buffers: KVBuffers) -> torch.dtype:
    """The compute dtype of a call: the cache's for ``"raw"``, ``tensor``'s (fp16 or bf16)
    for a quantised codec, whose cache does not say."""
    if buffers.codec == RAW_CODEC:
        return buffers.k.dtype
    if tensor.dtype not in _DTYPES:
        raise BackendError(
            f"{op}: {name} is {dtype_name(tensor.dtype)}; over a {buffers.codec!r} cache the hip "
            "backend computes in float16, bfloat16",
            context={"op": op, "argument": name},
        )
    return tensor.dtype


def require_buffers(op: str, buffers: KVBuffers) -> None:
    """Refuse a cache these kernels cannot read: layout, codec, shape, dtype, device, strides."""
    if buffers.layout not in (KVLayoutKind.NHD, KVLayoutKind.HND):
        raise BackendError(
            f"{op}: the hip backend serves the NHD and HND layouts, not {buffers.layout}",
            context={"op": op, "argument": "buffers"},
        )
    if buffers.codec not in _CODEC_DTYPES:
        raise BackendError(
            f"{op}: the hip backend stores the {RAW_CODEC!r} and {FP8_E4M3_CODEC!r} codecs, "
            f"not {buffers.codec!r}",
            context={"op": op, "argument": "buffers"},
        )
    k = buffers.k
    if k.dtype not in _CODEC_DTYPES[buffers.codec]:
        allowed = ", ".join(dtype_name(d) for d in _CODEC_DTYPES[buffers.codec])
        what = "computes in" if buffers.codec == RAW_CODEC else f"stores the {buffers.codec!r} codec as"
        raise BackendError(
            f"{op}: buffers.k is {dtype_name(k.dtype)}; the hip backend {what} {allowed}",
            context={"op": op, "argument": "buffers.k"},
        )
    if k.ndim != 4:
        raise BackendError(
            f"{op}: buffers.k must have four dimensions, got {list(k.shape)}",
            context={"op": op, "argument": "buffers"},
        )
    if tuple(buffers.v.shape) != tuple(k.shape) or buffers.v.dtype != k.dtype:
        raise BackendError(
            f"{op}: buffers.v must be {dtype_name(k.dtype)} {list(k.shape)}, "
            f"got {dtype_name(buffers.v.dtype)} {list(buffers.v.shape)}",
            context={"op": op, "argument": "buffers.v"},
        )
    if not (k.is_contiguous() and buffers.v.is_contiguous()):
        raise BackendError(
            f"{op}: buffers.k and buffers.v must be contiguous",
            context={"op": op, "argument": "buffers"},
        )
    if not k.is_cuda or buffers.v.device != k.device:
        raise BackendError(
            f"{op}: the hip backend runs on a HIP device; buffers are on {k.device} "
            f"and {buffers.v.device}",
            context={"op": op, "argument": "buffers"},
        )
