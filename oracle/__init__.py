"""CPU oracle for the MatMulNBits family: test infrastructure, never the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package.
"""
from . import oracle  # noqa: F401
