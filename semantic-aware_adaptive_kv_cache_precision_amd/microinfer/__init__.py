"""MicroInfer's paged mixed-precision KV-cache hot path, MI355X-native.

`_microinfer` re-presents the reference's native module (its pybind11
`_microinfer` and `_microinfer.device`) over the C ABI of
libmicroinfer_hip.so: HIP kernels for gfx950 and the cache runtime around
them. Importing this package loads that library; nothing here computes on the
CPU in its place.
"""

from . import _microinfer  # noqa: F401  (loads libmicroinfer_hip.so or raises)

__all__ = ["_microinfer"]
