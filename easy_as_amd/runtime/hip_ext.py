"""Loader for the native module ``easy_as_amd._hip`` (reference: ``eas/runtime/metal_ext.py:10-42``)."""

from __future__ import annotations

import importlib
import importlib.util
from typing import Any

REQUIRED_API = (
    "is_available",
    "compile",
    "launch",
    "synchronize",
    "alloc_buffer",
    "copy_from_host",
    "copy_to_host",
    "dlpack_import",
    "dlpack_export",
    "queue_synchronize",
    # HIP additions used by the runtime
    "compile_to_code",
    "load",
    "launch_async",
    "launch_timed",
    "wrap_pointer",
    "device_props",
)

_BUILD_HINT = "Build it with `python -m easy_as_amd.build` (hipcc + g++, no GPU needed)."


def load_hip_ext(*, require: bool) -> Any | None:
    """Import ``easy_as_amd._hip`` and check its API; ``None`` if absent and not required."""
    if importlib.util.find_spec("easy_as_amd._hip") is None:
        if require:
            raise RuntimeError(f"HIP backend is not built: `easy_as_amd._hip` is missing. {_BUILD_HINT}")
        return None
    mod = importlib.import_module("easy_as_amd._hip")
    missing = [n for n in REQUIRED_API if not callable(getattr(mod, n, None))]
    if missing:
        raise RuntimeError(f"HIP extension `easy_as_amd._hip` is missing required API: {', '.join(missing)}. {_BUILD_HINT}")
    return mod
