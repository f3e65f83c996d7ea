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
from collections import Counter
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


def _shortfalls(caps: BackendCaps, family: str, device: str, dtype: DType, cuda_graph: bool) -> list[str]:
    """Why ``caps`` cannot serve ``family`` here, in the reference's words (empty: it can)."""
    needs = (
        (sys.platform in caps.platforms, f"does not run on {sys.platform}"),
        (device in caps.devices, f"has no {device} support"),
        (dtype in caps.dtypes, f"has no {dtype.label} support"),
        (family != "attention" or caps.multi_row_attention, "serves only one query row per request"),
        (not cuda_graph or family in caps.graph_safe, "cannot run inside a CUDA graph"),
    )
    return [why for met, why in needs if not met]


class _Candidates:
    """The listed backends of one :func:`load_backend` call. A loader runs the first time its
    backend is the best fit for some family, and at most once; its result (the families, or
    why the backend is unavailable) serves every later family."""

    def __init__(self, device: str, dtype: DType, cuda_graph: bool) -> None:
        self.device, self.dtype, self.cuda_graph = device, dtype, cuda_graph
        self.families: dict[str, Mapping[str, object]] = {}
        self.unavailable: dict[str, str] = {}

    def _load(self, name: str) -> str | None:
        if name in self.families or name in self.unavailable:
            return self.unavailable.get(name)
        caps, loader = _registry[name]
        try:
            families = loader()
        except CapabilityError as exc:
            self.unavailable[name] = f"is unavailable ({exc.detail}; {exc.remedy})"
            logger.warning("ops backend %r %s", name, self.unavailable[name])
            return self.unavailable[name]
        absent = sorted(caps.families - set(families))
        if absent:
            raise BackendError(
                f"ops backend {name!r} declares {absent} but its loader did not return them",
                context={"backend": name, "families": absent},
            )
        self.families[name] = families
        return None

    def verdict(self, name: str, family: str) -> str | None:
        """None if ``name`` serves ``family``, else the reason it does not."""
        caps = _registry[name][0]
        if family not in caps.families:
            return _NOT_IMPLEMENTED
        shortfalls = _shortfalls(caps, family, self.device, self.dtype, self.cuda_graph)
        return ", ".join(shortfalls) if shortfalls else self._load(name)


def _check_names(names: Sequence[str]) -> None:
    if isinstance(names, str):
        raise TypeError("names must be a sequence of backend names, not one string")
    if not names:
        raise ConfigError(_CONFIG_PATH, "BACKEND_LIST_EMPTY", "at least one backend must be listed")
    repeated = sorted(name for name, count in Counter(names).items() if count > 1)
    if repeated:
        raise ConfigError(_CONFIG_PATH, "BACKEND_DUPLICATE", f"listed more than once: {repeated}")
    unknown = [name for name in names if name not in _registry]
    if unknown:
        raise ConfigError(
            _CONFIG_PATH,
            "BACKEND_UNKNOWN",
            f"not registered: {unknown}; registered backends: {sorted(_registry)}",
        )


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
    _check_names(names)
    candidates = _Candidates(device, dtype, cuda_graph)
    providers: dict[str, str] = {}
    refusals: dict[str, tuple[str, ...]] = {}
    for family in FAMILIES:
        verdicts: list[str] = []
        for name in names:
            why = candidates.verdict(name, family)
            if why is None:
                providers[family] = name
                break
            verdicts.append(f"{name} {why}")
        if family not in providers:
            refusals[family] = tuple(verdicts)

    if refusals:
        lines = "".join(f"\n  {family}: {'; '.join(why)}" for family, why in refusals.items())
        inside = " inside a CUDA graph" if cuda_graph else ""
        raise ConfigError(
            _CONFIG_PATH,
            "BACKEND_CAPABILITY_MISSING",
            f"no backend in {list(names)} provides {', '.join(refusals)} "
            f"for device {device!r} and dtype {dtype.label}{inside}:{lines}",
            context={"missing": refusals},
        )
    logger.info("ops backends for %s %s: %s", device, dtype.label,
                ", ".join(f"{family}={name}" for family, name in providers.items()))
    ops = {family: candidates.families[name][family] for family, name in providers.items()}
    return OpsBackend(providers=MappingProxyType(providers), graph_safe=cuda_graph, **ops)


def _load_hip() -> Mapping[str, object]:
    from ayaka_amd.hip import load

    return load()


register_backend(
    BackendCaps(
        name="hip",
        families=frozenset(FAMILIES),
        platforms=frozenset({"linux"}),
        devices=frozenset({"cuda"}),  # ROCm torch names HIP devices "cuda"
        dtypes=frozenset({DType.FP16, DType.BF16, DType.FP32}),
        graph_safe=frozenset(FAMILIES),
        multi_row_attention=True,
    ),
    _load_hip,
)
