"""Runtime selection (reference ``eas/runtime/__init__.py:18-44``).

``EAS_BACKEND`` / ``get_runtime(backend)``: ``auto`` and ``hip`` (aliases
``rocm``, ``gpu``) select the MI355X HIP runtime.  This build has no Metal
backend and, like the reference, no CPU execution path.
"""

from __future__ import annotations

import os
from typing import TYPE_CHECKING

from .base import Runtime

__all__ = ["get_runtime", "Runtime"]

_hip_runtime = None

if TYPE_CHECKING:  # pragma: no cover
    from .hip import HipRuntime

_HIP_NAMES = ("auto", "hip", "rocm", "gpu")


def get_runtime(backend: str | None = None) -> Runtime:
    name = (backend or os.environ.get("EAS_BACKEND", "auto")).lower()
    if name in _HIP_NAMES:
        rt = _get_hip()
        if not rt.is_available():
            raise RuntimeError(
                "HIP runtime is not available: no usable MI355X (gfx950) GPU, or the native extension is not "
                "built (run `python -m easy_as_amd.build`)."
            )
        return rt
    if name == "cpu":
        raise ValueError("unsupported backend: 'cpu' (there is no CPU runtime for eas kernels; use 'hip' or 'auto')")
    if name in ("mps", "metal"):
        raise ValueError(f"unsupported backend: {name!r} (this build targets MI355X; use 'hip' or 'auto')")
    raise ValueError(f"unsupported backend: {name!r} (expected 'auto'|'hip')")


def _get_hip() -> "HipRuntime":
    global _hip_runtime
    if _hip_runtime is None:
        from .hip import HipRuntime

        _hip_runtime = HipRuntime()
    return _hip_runtime
