"""Repeated launches without repeated host checks.

An engine calls ``attend`` and ``store`` once per layer per step with the same tensors every
time (its per-layer q/out buffers and caches, one step's metadata). The first call of a
combination checks everything and records the library call it made; later calls with the same
objects replay that call on the current stream. A record is found by the identity of the
long-lived objects (the KV buffers and the step metadata, which it holds, so their ids cannot be
reused while it lives) and by the data pointer, shape, strides and dtype of every tensor the call
reads or writes: everything the first call's checks depended on. It holds no activation tensor,
so an engine that allocates fresh q/out (or k/v) per layer keeps nothing alive by calling; the
caching allocator hands such tensors the same addresses from step to step, so those calls still
hit. The records live in the step's plan (a planned step, or a graph bucket's fixed record) and
go with it. This cuts the host time of a decode layer's two calls, which bounds small eager
steps.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import torch

from ayaka_amd.hip import _lib

__all__ = ["Launch", "Recorder", "lookup", "remember"]

#: Most records one plan keeps (an engine has one or two per layer); past it the cache starts
#: over. Large enough for a benchmark that rotates a step over hundreds of pool copies.
MAX_RECORDS = 4096


@dataclass(slots=True)
class Launch:
    """One library call: ``fn(*args, stream)``, kept as a pointer to the same export with no
    declared argument types and the arguments converted once to the declared ones, so that a
    replay skips ctypes' per-argument conversion; ``keep`` are the tensors its pointers come
    and metadata objects its arguments were checked against."""

    op: str
    fn: Any
    args: tuple
    stream_arg: Any  # the stream handle's conversion: ctypes.c_void_p for a library export
    keep: tuple
    device: torch.device
    scratch: bool  # it uses the device's shared v2 scratch, ordered across streams


class Recorder:
    """Collects the launch a checked call makes, for :func:`remember`."""

    __slots__ = ("launch",)

    def __init__(self) -> None:
        self.launch: tuple | None = None

    def __call__(self, op: str, fn: Any, args: tuple, device: torch.device, scratch: bool) -> None:
        self.launch = (op, fn, args, device, scratch)


def signature(tensors: tuple) -> tuple:
    """Where and how each tensor lies: data pointer, shape, strides and dtype."""
    if len(tensors) == 4:  # every call site of the library: unrolled, a few hundred ns cheaper
        a, b, c, d = tensors
        return (a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), a.shape, b.shape, c.shape,
                d.shape, a.stride(), b.stride(), c.stride(), d.stride(), a.dtype, b.dtype, c.dtype,
                d.dtype)
    return (tuple(t.data_ptr() for t in tensors) + tuple(t.shape for t in tensors)
            + tuple(t.stride() for t in tensors) + tuple(t.dtype for t in tensors))


def convert(types: list, args: tuple) -> tuple:
    """``args`` as instances of the ctypes ``types`` a library export declares (the same values
    ctypes would pass for them; numpy scalars included)."""
    out = []
    for t, a in zip(types, args, strict=True):
        if isinstance(a, t):
            out.append(a)
        elif t is ctypes.c_float:
            out.append(t(float(a)))
        elif t is ctypes.c_void_p:
            out.append(t(None if a is None else int(a)))
        else:
            out.append(t(int(a)))
    return tuple(out)


def lookup(cache: dict, key: tuple) -> Launch | None:
    """The recorded launch for ``key`` (the objects' ids plus :func:`signature` of the tensors)."""
    return cache.get(key)


def remember(cache: dict, key: tuple, keep: tuple, recorder: Recorder) -> None:
    if recorder.launch is None:
        return
    if len(cache) >= MAX_RECORDS:
        cache.clear()
    op, fn, args, device, scratch = recorder.launch
    stream_arg: Any = int
    types = getattr(fn, "argtypes", None)
    if types is not None:  # a library export (its last argument is the stream)
        untyped = _lib.lib()[fn.__name__]  # a new function object: fn keeps its declared types
        untyped.restype = fn.restype
        fn, args, stream_arg = untyped, convert(types[:-1], args), ctypes.c_void_p
    cache[key] = Launch(op, fn, args, stream_arg, keep, device, scratch)


def run(launch: Launch, stream: int) -> None:
    _lib.check(launch.op, launch.fn(*launch.args, launch.stream_arg(stream)))
