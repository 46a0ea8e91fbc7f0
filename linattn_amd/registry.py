"""``<backend>_<variant>`` registry of the HIP backend.

Mirrors the reference's ``KERNEL_VARIANTS`` / ``build`` routing
(src/linattn/registry.py:139-146, 225-236): names ``hip_quest``, ``hip_dsa``, ``hip_moba``, ``hip_xattention``,
``hip_sliding_window`` and ``hip_streaming_sink`` map to the torch variant
they implement; unknown names raise ``KeyError`` like the reference.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

from linattn_amd.core import AttnConfig, AttentionVariant
from linattn_amd.variants import SUPPORTED

__all__ = ["KERNEL_VARIANTS", "build", "build_any", "list_kernel_variants", "describe_kernel"]

KERNEL_VARIANTS: Dict[str, str] = {f"hip_{name}": name for name in SUPPORTED}


def build(name: str, cfg: Optional[AttnConfig] = None, **kw: Any) -> AttentionVariant:
    """Instantiate a ``hip_<variant>``."""
    if name in KERNEL_VARIANTS:
        backend, _, base = name.partition("_")
        return SUPPORTED[base](cfg, **kw)
    raise KeyError(f"unknown variant {name!r}; known: {sorted(KERNEL_VARIANTS)}")


def build_any(name: str, cfg: Optional[AttnConfig] = None, **kw: Any) -> AttentionVariant:
    return build(name, cfg, **kw)


def list_kernel_variants() -> List[str]:
    return list(KERNEL_VARIANTS)


def describe_kernel(name: str) -> Dict[str, Any]:
    """Metadata of a backend variant (registry.py:298-310)."""
    if name not in KERNEL_VARIANTS:
        raise KeyError(f"unknown kernel variant {name!r}; known: {sorted(KERNEL_VARIANTS)}")
    base = KERNEL_VARIANTS[name]
    cls = SUPPORTED[base]
    return {"name": name, "class": cls.__name__, "family": "hip", "reference": base,
            "docstring": (cls.__doc__ or "").strip().split("\n\n")[0].replace("\n", " ")}
