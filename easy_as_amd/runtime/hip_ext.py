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
    "launch_tg",
    "launch_tg_async",
    "launch_groups",
    "launch_groups_async",
    "launch_timed",
    "wrap_pointer",
    "device_props",
)

_BUILD_HINT = "Build it with `python -m easy_as_amd.build` (hipcc + g++, no GPU needed)."


def _share_process_hip_runtime() -> None:
    """Load PyTorch-ROCm (when installed) before ``libeas_hip.so``.

    PyTorch-ROCm ships its own ``libamdhip64.so`` with the same SONAME
    (``libamdhip64.so.7``) as ``/opt/rocm``'s.  Loaded after torch, our library
    binds to torch's copy, so the process has one HIP runtime and device
    pointers and streams are shared.  Loaded first, torch would later bring a
    second runtime and fail to initialise its GPU.  ``EAS_HIP_STANDALONE=1``
    skips this (processes without torch).
    """
    import os

    if os.environ.get("EAS_HIP_STANDALONE", "") not in ("", "0"):
        return
    try:
        import torch  # type: ignore  # noqa: F401
    except Exception:
        pass


def load_hip_ext(*, require: bool) -> Any | None:
    """Import ``easy_as_amd._hip`` and check its API; ``None`` if absent and not required."""
    _share_process_hip_runtime()
    if importlib.util.find_spec("easy_as_amd._hip") is None:
        if require:
            raise RuntimeError(f"HIP backend is not built: `easy_as_amd._hip` is missing. {_BUILD_HINT}")
        return None
    mod = importlib.import_module("easy_as_amd._hip")
    missing = [n for n in REQUIRED_API if not callable(getattr(mod, n, None))]
    if missing:
        raise RuntimeError(f"HIP extension `easy_as_amd._hip` is missing required API: {', '.join(missing)}. {_BUILD_HINT}")
    return mod
