"""The ``hip`` backend: MI355X kernels behind the ``attention`` and ``kvcache`` contracts.

Laid out like the reference's backends (``python/ayaka/ops/backends/torch/__init__.py``):
each family is a module of module-level functions. :func:`load` is the registry
loader; it refuses (``CapabilityError``) when no HIP device is visible or the
library is not built, so the engine never silently runs something else.
"""

from __future__ import annotations

from collections.abc import Mapping

from ayaka_amd.errors import CapabilityError

__all__ = ["load"]


def load() -> Mapping[str, object]:
    try:
        import torch
    except ImportError as exc:  # pragma: no cover - torch is part of the image
        raise CapabilityError("ops.hip", detail="torch is not importable", remedy="install torch") from exc
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise CapabilityError(
            "ops.hip",
            detail="no HIP device is visible to torch",
            remedy="run on a ROCm build of torch with an MI355X (gfx950) visible",
        )
    from ayaka_amd.hip import _lib, attention, kvcache

    _lib.lib()  # fails loudly if the kernels are not built
    return {"attention": attention, "kvcache": kvcache}
