"""ironpangu_amd — MI355X-native continuous-batching attention path.

The product is the gfx950 shared library ``libifattn_hip.so`` (C ABI in
``include/``). This package holds its sources (``csrc/``), the build recipe,
the ctypes binding, host-side mirrors of the reference's metadata classes
(``host``), torch-tensor convenience wrappers for the kernels (``ops``) and the
seeded workload generators used by tests and the benchmark (``workloads``).
"""
from ._native import IfattnError, lib  # noqa: F401

__all__ = ["lib", "IfattnError"]
