"""DLPack interop (reference ``eas/dlpack.py:16-82``): kDLCPU through NumPy,
kDLROCM zero-copy through ``easy_as_amd._hip``."""

from __future__ import annotations

from typing import Any

import numpy as np

from .tensor import Tensor, _ext, _from_capsule, _normalize_device, tensor as _tensor


def from_dlpack(x: Any, *, device: Any = None) -> Tensor:
    """``eas.Tensor`` from a DLPack producer (object with ``__dlpack__`` or a raw capsule)."""
    dev = _normalize_device(device)
    if dev == "hip":
        cap = x
        if type(cap).__name__ != "PyCapsule":
            fn = getattr(cap, "__dlpack__", None)
            if not callable(fn):
                raise TypeError("object does not implement the DLPack protocol (__dlpack__)")
            cap = fn()
        return _from_capsule(_ext(), cap)
    try:
        arr = np.from_dlpack(x)
    except Exception as e:
        raise TypeError("object does not support DLPack import via numpy.from_dlpack") from e
    if arr.dtype not in (np.float16, np.float32):
        raise TypeError("only float16/float32 tensors are supported")
    return _tensor(np.ascontiguousarray(arr), device=dev)


def to_dlpack(x: Tensor) -> Any:
    """Raw DLPack capsule of an ``eas.Tensor`` (torch-style ``to_dlpack``)."""
    if not isinstance(x, Tensor):
        raise TypeError(f"to_dlpack expects eas.Tensor, got {type(x)!r}")
    return x.__dlpack__()
