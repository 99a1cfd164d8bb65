"""yirage_amd -- the MI355X-native `hip` backend of YiRage.

Mirrors the reference's public API for the hot path:
  new_kernel_graph() / KNGraph ops / graph.superoptimize(backend='hip') / graph(inputs=...)
  PersistentKernel(...).*_layer(...) / compile() / __call__()
  get_available_backends() & co.
Compute runs only through libyirage_hip.so (hand-written gfx950 kernels).
"""
from ._lib import YirageHipError, W_KN, W_NK
from .backend_api import (
    get_available_backends,
    get_backend_info,
    get_default_backend,
    get_registered_backends,
    is_backend_available,
)

__version__ = "0.1.0"
