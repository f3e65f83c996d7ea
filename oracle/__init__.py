"""CPU oracle of the paged-attention decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or, for the baseline, as
the timed restatement of the reference's CPU algorithm). The product path
(``ayaka_amd``) never imports it and has no CPU fallback.

Modules:

* :mod:`oracle.paged` -- numpy restatement of the reference's torch backend:
  ``plan`` (``python/ayaka/ops/backends/torch/attention.py:64-164``), the
  decode gather-then-softmax (``:237-271``), the row-causal multi-row path
  (``:209-234``), and the cache ops (``python/ayaka/ops/backends/torch/kvcache.py:65-115``).
* :mod:`oracle.numerics` -- fp16/bf16 bit conversions and the parity metrics.

How each function is pinned (checked against something other than itself) is
listed in each function's docstring; the checks live in ``tests/test_oracle.py``.
No function here is "parity unpinned".
"""
