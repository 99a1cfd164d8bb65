"""yirage_amd -- the MI355X-native `hip` backend of YiRage.

Mirrors the reference's public API for the hot path:
  new_kernel_graph() / KNGraph ops / graph.superoptimize(backend='hip') / graph(inputs=...)
  new_threadblock_graph() / TBGraph (bodies of `customized` ops)
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
from .dtypes import (
    bfloat16,
    convert_dtype_to_torch_type,
    dtype,
    float16,
    float32,
    float64,
    int8,
    int32,
    int64,
    uint8,
)
from .graph_dataset import graph_dataset
from .kernel import DTensor, KNGraph, check_stride, from_reference_graph, new_kernel_graph
from .threadblock import STensor, TBGraph, new_threadblock_graph

__version__ = "0.2.0"


def __getattr__(name):
    # the persistent kernel pulls in more of torch; load it on first use
    if name in ("PersistentKernel", "get_configurations_from_gpu"):
        from . import persistent_kernel

        return getattr(persistent_kernel, name)
    raise AttributeError(name)
