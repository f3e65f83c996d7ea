"""ctypes binding of ``libayaka_hip.so`` (the C ABI declared in ``include/ayaka_hip.h``).

The library is built in-tree by :mod:`ayaka_amd._build`. There is no fallback:
if it is missing or does not load, :func:`lib` raises
:class:`~ayaka_amd.errors.CapabilityError`, and the ``hip`` backend is
unavailable.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from ayaka_amd.errors import BackendError, CapabilityError

__all__ = ["ABI_VERSION", "EXPORTS", "LIB_PATH", "check", "lib"]

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libayaka_hip.so"
ABI_VERSION = 18

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

#: name -> (restype, argtypes), one entry per function of include/ayaka_hip.h.
EXPORTS: dict[str, tuple[object, list[object]]] = {
    "ayk_abi_version": (ctypes.c_int, []),
    "ayk_last_error": (ctypes.c_char_p, []),
    "ayk_reshape_and_cache": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "ayk_reshape_and_cache_e4m3": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _P],
    ),
    "ayk_paged_attention_v1": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _P, _P,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _F32, _I32, _P],
    ),
    "ayk_paged_attention_v2_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "ayk_paged_attention_v2": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _P, _P,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _F32,
         _I32, _I32, _P, _I32, _P, _P, _SZ, _P, _I32, _P],
    ),
    "ayk_paged_attention_v2_static": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _P, _P,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _F32,
         _I32, _I32, _P, _I32, _P, _I32, _P],
    ),
    "ayk_paged_attention_v2_static_counters": (ctypes.c_int, [ctypes.POINTER(_P), ctypes.POINTER(_I64)]),
    "ayk_paged_prefill_tile_pairs": (ctypes.c_int, [_I32]),
    "ayk_paged_prefill": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I32, _I32, _I32,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _F32, _I32, _P, _SZ, _P],
    ),
    "ayk_paged_attention_windows": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _F32, _F32, _I32, _P, _SZ, _P],
    ),
    "ayk_split_model": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _P, _P]),
    "ayk_work_list": (ctypes.c_int64, [_P, _I32, _I32, _P]),
    "ayk_best_split": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _P]),
    "ayk_dispatch_makespan": (ctypes.c_int, [_P, _I64, _I32, _P]),
    "ayk_debug_kv_reach_begin": (ctypes.c_int, [_I64]),
    "ayk_debug_kv_reach_end": (ctypes.c_int, [_P]),
    "ayk_gather_blocks": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I64, _I32, _I64, _P]),
    "ayk_copy_blocks": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I64, _I32, _I64, _P]),
    "ayk_zero_blocks": (ctypes.c_int, [_P, _P, _P, _I32, _I64, _I32, _I64, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library, with every export's signature declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise CapabilityError(
                    "ops.hip",
                    detail=f"{LIB_PATH} is not built",
                    remedy="run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python -m ayaka_amd._build`",
                )
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                raise CapabilityError(
                    "ops.hip", detail=f"{LIB_PATH} does not load: {exc}", remedy="rebuild it"
                ) from exc
            for name, (restype, argtypes) in EXPORTS.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            version = handle.ayk_abi_version()
            if version != ABI_VERSION:
                raise CapabilityError(
                    "ops.hip",
                    detail=f"{LIB_PATH} has ABI {version}, this package expects {ABI_VERSION}",
                    remedy="rebuild it",
                )
            _lib = handle
    return _lib


def check(op: str, code: int) -> None:
    """Turn a non-zero return code of the library into :class:`BackendError`."""
    if code != 0:
        message = (lib().ayk_last_error() or b"").decode(errors="replace")
        raise BackendError(f"{op}: {message} (code {code})", context={"op": op, "code": code})
