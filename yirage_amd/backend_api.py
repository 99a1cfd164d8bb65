"""Backend query API (python/yirage/backend_api.py:18-153), answered by the
C++ BackendRegistry inside libyirage_hip.so, where `hip` is registered."""
from __future__ import annotations

import ctypes
from typing import Any, Dict, List, Optional

from . import _lib

# Priority order of the reference (backend_api.py:80-87) with 'hip' first.
PRIORITY = ["hip", "cuda", "maca", "ascend", "mps", "cpu"]


def get_registered_backends() -> List[str]:
    L = _lib.lib()
    out = []
    for i in range(L.yr_backend_num_registered()):
        buf = ctypes.create_string_buffer(64)
        L.yr_backend_registered_name(i, buf, 64)
        out.append(buf.value.decode())
    return out


def get_available_backends() -> List[str]:
    L = _lib.lib()
    return [n for n in get_registered_backends() if L.yr_backend_is_available(n.encode())]


def is_backend_available(backend: str) -> bool:
    return bool(_lib.lib().yr_backend_is_available(backend.encode()))


def get_default_backend() -> Optional[str]:
    avail = get_available_backends()
    for b in PRIORITY:
        if b in avail:
            return b
    return avail[0] if avail else None


def get_backend_info(backend: str) -> Dict[str, Any]:
    L = _lib.lib()
    buf = ctypes.create_string_buffer(512)
    rc = L.yr_backend_compile_flags(backend.encode(), buf, 512)
    if rc != 0:
        return {"name": backend, "available": False}
    info: Dict[str, Any] = {
        "name": backend,
        "type": L.yr_backend_type_from_name(backend.encode()),
        "available": is_backend_available(backend),
        "compile_flags": buf.value.decode(),
    }
    if info["available"]:
        di = _lib.DeviceInfo()
        if L.yr_hip_device_info(0, ctypes.byref(di)) == 0:
            info.update(
                num_compute_units=di.num_compute_units,
                compute_capability=di.compute_capability,
                total_memory=di.total_memory,
                max_shared_memory=di.max_shared_memory,
                arch=di.arch_name.decode(),
            )
    return info
