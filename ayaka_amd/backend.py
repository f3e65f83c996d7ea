"""Backend registry for the op families of the decode hot path.

Same contract as the reference's registry (``python/ayaka/ops/backend.py``):
a backend is registered with a :class:`BackendCaps` record and a loader
(``register_backend``, reference ``:179-195``); :func:`load_backend` takes
backend names in priority order and picks, family by family, the first one that
implements the family, runs on this platform, device and dtype, has the
capabilities asked for, and loads (reference ``:207-291``). A loader raising
:class:`CapabilityError` marks its backend unavailable; the next listed one is
tried. Attention is taken only from a backend with ``multi_row_attention``; with
``cuda_graph`` every family must be in the backend's ``graph_safe``.

The families here are the two the hot path uses, ``kvcache`` and
``attention``; the reference's other families (norm, linear, sampling, ...)
are outside this package.

The ``hip`` backend (MI355X kernels through ``libayaka_hip.so``) is registered
on import.
"""

from __future__ import annotations

import logging
import sys
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass
from types import MappingProxyType
from typing import Any

from ayaka_amd.enums import DType
from ayaka_amd.errors import BackendError, CapabilityError, ConfigError

__all__ = [
    "FAMILIES",
    "BackendCaps",
    "OpsBackend",
    "available_backends",
    "load_backend",
    "register_backend",
]

logger = logging.getLogger(__name__)

#: The op families of the hot path, in the order messages list them.
FAMILIES: tuple[str, ...] = ("kvcache", "attention")

_CONFIG_PATH = "ops.backends"
_NOT_IMPLEMENTED = "does not implement this family"


@dataclass(frozen=True, slots=True)
class BackendCaps:
    """What one backend implements, where it runs and what it can do (reference ``:101-152``)."""

    name: str
    families: frozenset[str]
    platforms: frozenset[str]
    devices: frozenset[str]
    dtypes: frozenset[DType]
    graph_safe: frozenset[str] = frozenset()
    multi_row_attention: bool = False

    def __post_init__(self) -> None:
        if not self.name or not self.name.strip():
            raise ValueError("name must be a non-empty string")
        unknown = sorted(self.families.difference(FAMILIES))
        if unknown:
            raise ValueError(f"unknown op families {unknown}; known families: {list(FAMILIES)}")
        outside = sorted(self.graph_safe.difference(self.families))
        if outside:
            raise ValueError(f"graph_safe names families the backend does not implement: {outside}")


@dataclass(frozen=True, slots=True)
class OpsBackend:
    """The chosen implementation of each family; ``providers`` names who supplies which."""

    kvcache: Any
    attention: Any
    providers: Mapping[str, str]
    graph_safe: bool = False


_registry: dict[str, tuple[BackendCaps, Callable[[], Mapping[str, object]]]] = {}


def register_backend(caps: BackendCaps, loader: Callable[[], Mapping[str, object]]) -> None:
    """Add a backend; its loader runs only when the backend is first chosen."""
    if caps.name in _registry:
        raise ValueError(f"ops backend {caps.name!r} is already registered")
    _registry[caps.name] = (caps, loader)


def available_backends() -> tuple[BackendCaps, ...]:
    """Every registered backend's record (registered is not the same as loadable)."""
    return tuple(caps for caps, _ in _registry.values())


def _rejection(caps: BackendCaps, family: str, device: str, dtype: DType, cuda_graph: bool) -> str | None:
    if family not in caps.families:
        return _NOT_IMPLEMENTED
    problems: list[str] = []
    if sys.platform not in caps.platforms:
        problems.append(f"does not run on {sys.platform}")
    if device not in caps.devices:
        problems.append(f"has no {device} support")
    if dtype not in caps.dtypes:
        problems.append(f"has no {dtype.label} support")
    if family == "attention" and not caps.multi_row_attention:
        problems.append("serves only one query row per request")
    if cuda_graph and family not in caps.graph_safe:
        problems.append("cannot run inside a CUDA graph")
    return ", ".join(problems) or None


def load_backend(
    names: Sequence[str], *, device: str, dtype: DType, cuda_graph: bool = False
) -> OpsBackend:
    """Build the ops for one device from backends listed in priority order.

    Raises:
        ConfigError: ``names`` is empty, repeats or names an unregistered
            backend, or some family is left without a backend (the message says
            why each listed backend was rejected).
        BackendError: A loader did not return a family its record declares.
    """
    if isinstance(names, str):
        raise TypeError("names must be a sequence of backend names, not one string")
    if not names:
        raise ConfigError(_CONFIG_PATH, "BACKEND_LIST_EMPTY", "at least one backend must be listed")
    repeated = sorted({name for name in names if list(names).count(name) > 1})
    if repeated:
        raise ConfigError(_CONFIG_PATH, "BACKEND_DUPLICATE", f"listed more than once: {repeated}")
    unknown = [name for name in names if name not in _registry]
    if unknown:
        raise ConfigError(
            _CONFIG_PATH,
            "BACKEND_UNKNOWN",
            f"not registered: {unknown}; registered backends: {sorted(_registry)}",
        )

    loaded: dict[str, Mapping[str, object]] = {}
    unavailable: dict[str, str] = {}
    chosen: dict[str, object] = {}
    providers: dict[str, str] = {}
    missing: dict[str, tuple[str, ...]] = {}
    for family in FAMILIES:
        rejections: list[str] = []
        for name in names:
            caps, loader = _registry[name]
            reason = _rejection(caps, family, device, dtype, cuda_graph)
            if reason is None and name not in loaded and name not in unavailable:
                try:
                    families = loader()
                except CapabilityError as exc:
                    unavailable[name] = f"is unavailable ({exc.detail}; {exc.remedy})"
                    logger.warning("ops backend %r %s", name, unavailable[name])
                else:
                    absent = sorted(caps.families - set(families))
                    if absent:
                        raise BackendError(
                            f"ops backend {name!r} declares {absent} but its loader did not "
                            "return them",
                            context={"backend": name, "families": absent},
                        )
                    loaded[name] = families
            if reason is None:
                reason = unavailable.get(name)
            if reason is None:
                chosen[family] = loaded[name][family]
                providers[family] = name
                break
            rejections.append(f"{name} {reason}")
        else:
            missing[family] = tuple(rejections)

    if missing:
        details = "".join(f"\n  {fam}: {'; '.join(why)}" for fam, why in missing.items())
        graph = " inside a CUDA graph" if cuda_graph else ""
        raise ConfigError(
            _CONFIG_PATH,
            "BACKEND_CAPABILITY_MISSING",
            f"no backend in {list(names)} provides {', '.join(missing)} "
            f"for device {device!r} and dtype {dtype.label}{graph}:{details}",
            context={"missing": missing},
        )
    logger.info(
        "ops backends for %s %s: %s",
        device,
        dtype.label,
        ", ".join(f"{family}={name}" for family, name in providers.items()),
    )
    return OpsBackend(
        kvcache=chosen["kvcache"],
        attention=chosen["attention"],
        providers=MappingProxyType(providers),
        graph_safe=cuda_graph,
    )


def _load_hip() -> Mapping[str, object]:
    from ayaka_amd.hip import load

    return load()


register_backend(
    BackendCaps(
        name="hip",
        families=frozenset(FAMILIES),
        platforms=frozenset({"linux"}),
        devices=frozenset({"cuda"}),  # ROCm torch names HIP devices "cuda"
        dtypes=frozenset({DType.FP16, DType.BF16}),
        graph_safe=frozenset(FAMILIES),
        multi_row_attention=True,
    ),
    _load_hip,
)
