"""dpep -- DREAMPlace's electric-potential step (density scatter, DCT Poisson
solve, field maps, per-cell field gather) on MI355X through libdpep.so.

Public pieces:
  dpep.Context                 in-process ctypes binding of the C ABI
  dpep.scatter_ttnn_client     drop-in mirror of the reference's
                               integration/scatter_ttnn_client.py
  dpep.shm                     the shared-memory wire format (v1 + v2)
  dpep.workloads               seeded synthetic placements for the five
                               benchmark configurations
"""
from ._lib import (  # noqa: F401
    Context,
    DpepError,
    EXPORTED_SYMBOLS,
    KERNEL_KEYS,
    LIB_PATH,
    TIMING_KEYS,
    last_error,
    load_library,
)

__all__ = [
    "Context",
    "DpepError",
    "EXPORTED_SYMBOLS",
    "KERNEL_KEYS",
    "LIB_PATH",
    "TIMING_KEYS",
    "last_error",
    "load_library",
]
