"""vernondsl_amd - MI355X (gfx950) HIP backend for VernonDSL's tensor-op hot path.

The compute lives in libvdsl.so (HIP device + hand-written gfx950 kernels) behind the C ABI of
include/vdsl.h; this package is its Python front end: ctypes binding (_lib), RHI objects
(rhi), op-class calls (kernels), the map-chain compiler (mapchain), the execution graph with
autodiff (graph), and the seeded workloads (spec, rng).  Importing it without a built
libvdsl.so raises ImportError: there is no CPU fallback.
"""
from . import _lib  # noqa: F401  (loads libvdsl.so; raises ImportError if it is not built)
from ._lib import VdslError  # noqa: F401
from .rhi import Buffer, Device, Event, Graph, Queue, Tensor, device_count  # noqa: F401

__all__ = ["Buffer", "Device", "Event", "Graph", "Queue", "Tensor", "VdslError", "device_count"]
