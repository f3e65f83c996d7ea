"""ayaka_amd: an MI355X-native paged-attention decode path for the Ayaka engine.

The package mirrors the part of Ayaka's ``ops`` contract that the decode hot
path uses (reference ``python/ayaka/ops/attention.py``, ``ops/kvcache.py``,
``ops/backend.py``) and implements it with hand-written HIP kernels for gfx950,
reached through the C ABI in ``include/ayaka_hip.h``:

* :mod:`ayaka_amd.attention`, :mod:`ayaka_amd.kvcache` -- the contract records
  (``AttentionMetadata``, ``KVBuffers``) and protocols.
* :mod:`ayaka_amd.backend` -- the backend registry (``BackendCaps``,
  ``register_backend``, ``load_backend``) with the ``hip`` backend registered.
* :mod:`ayaka_amd.hip` -- the backend: ``attention`` and ``kvcache`` modules of
  module-level functions, as the reference's backends are laid out.

Importing this package does not import torch.
"""

__all__ = ["__version__"]

__version__ = "0.1.0"
