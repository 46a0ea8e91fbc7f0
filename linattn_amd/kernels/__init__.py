"""Kernel entry points of the HIP backend.

The reference dispatches between triton, flex and torch backends
(src/linattn/kernels/__init__.py:36-95).  This package has exactly one backend,
``hip``: GPU tensors run the gfx950 kernels, anything else raises.
"""

from __future__ import annotations

import platform
from typing import Dict

import torch

__all__ = ["describe_backends", "backend_for", "has_hip"]


def has_hip() -> bool:
    return bool(torch.cuda.is_available()) and torch.version.hip is not None


def describe_backends() -> Dict[str, object]:
    """Environment block for reports (mirrors kernels/__init__.py:66-84)."""
    from linattn_amd._native import LIB_PATH

    info: Dict[str, object] = {
        "platform": f"{platform.system()} {platform.machine()}",
        "torch": torch.__version__,
        "hip_runtime": torch.version.hip,
        "threads": torch.get_num_threads(),
        "gpu": has_hip(),
        "hip_library": str(LIB_PATH),
        "hip_library_built": LIB_PATH.exists(),
    }
    if has_hip():
        p = torch.cuda.get_device_properties(0)
        info["device"] = p.name
        info["gcn_arch"] = getattr(p, "gcnArchName", "")
        info["compute_units"] = p.multi_processor_count
    return info


def backend_for(preferred: str = "auto") -> str:
    """The reference picks triton/flex/torch (kernels/__init__.py:87-95); here
    the only backend is ``hip``."""
    if preferred not in ("auto", "hip"):
        raise ValueError(f"backend {preferred!r} is not provided by linattn_amd (only 'hip')")
    return "hip"
