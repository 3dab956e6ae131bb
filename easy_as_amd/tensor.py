"""``eas.Tensor``: a contiguous f16/f32 array on the host (``cpu``) or an MI355X (``hip``).

Surface and semantics follow the reference (``eas/tensor.py:61-365``) with the
Apple device ``mps`` replaced by ``hip``.  ``cuda`` and ``rocm`` are accepted as
spellings of ``hip`` because that is how PyTorch-ROCm names the GPU.  GPU
tensors interoperate zero-copy with PyTorch-ROCm through DLPack (kDLROCM).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Literal

import numpy as np

from .runtime.hip_ext import load_hip_ext

Device = Literal["cpu", "hip"]

_DEVICE_ALIASES = {"cpu": "cpu", "hip": "hip", "cuda": "hip", "rocm": "hip", "gpu": "hip"}
KDL_CPU = 1
KDL_ROCM = 10


def _torch() -> Any | None:
    try:
        import torch  # type: ignore

        return torch
    except Exception:
        return None


def _is_torch_tensor(x: Any) -> bool:
    torch = _torch()
    return torch is not None and isinstance(x, torch.Tensor)


def _normalize_device(device: Any) -> Device:
    if device is None:
        return "cpu"
    name = str(device).lower().split(":")[0]
    if name not in _DEVICE_ALIASES:
        raise ValueError(f"unsupported device: {device!r} (expected 'cpu'|'hip')")
    return _DEVICE_ALIASES[name]  # type: ignore[return-value]


def _require_supported_dtype(dtype: Any) -> np.dtype:
    dt = np.dtype(dtype)
    if dt not in (np.float16, np.float32):
        raise TypeError(f"only float16/float32 tensors are supported (got {dt})")
    return dt


def _numel(shape: tuple[int, ...]) -> int:
    n = 1
    for d in shape:
        if d < 0:
            raise ValueError("negative dimensions are not allowed")
        n *= int(d)
    return n


def _ext() -> Any:
    mod = load_hip_ext(require=True)
    if not mod.is_available():
        raise RuntimeError("HIP device is not available")
    return mod


@dataclass(frozen=True, slots=True)
class _HipStorage:
    buf: object  # buffer capsule of easy_as_amd._hip
    nbytes: int


class Tensor:
    __eas_tensor__ = True

    def __init__(self, *, shape: tuple[int, ...], dtype: Any, device: Device,
                 cpu: np.ndarray | None = None, hip: _HipStorage | None = None) -> None:
        self._dtype = _require_supported_dtype(dtype)
        self._shape = tuple(int(d) for d in shape)
        self._device: Device = device
        self._cpu = cpu
        self._hip = hip
        if device == "cpu":
            if cpu is None or hip is not None:
                raise ValueError("cpu tensor requires cpu storage only")
        elif hip is None or cpu is not None:
            raise ValueError("hip tensor requires hip storage only")

    @property
    def device(self) -> Device:
        return self._device

    @property
    def dtype(self) -> np.dtype:
        return self._dtype

    @property
    def shape(self) -> tuple[int, ...]:
        return self._shape

    @property
    def nbytes(self) -> int:
        return _numel(self._shape) * int(self._dtype.itemsize)

    def __repr__(self) -> str:  # pragma: no cover
        return f"eas.Tensor(shape={self._shape}, dtype={self._dtype.name}, device={self._device!r})"

    def __array__(self, dtype: Any | None = None, copy: Any | None = None) -> np.ndarray:
        if self._device != "cpu":
            raise TypeError("cannot convert a hip tensor to numpy without .numpy()")
        arr = self._cpu
        assert arr is not None
        return arr if dtype is None else arr.astype(dtype, copy=False)

    def __dlpack__(self, stream: Any | None = None, **_: Any) -> Any:
        _ = stream
        if self._device == "cpu":
            assert self._cpu is not None
            return self._cpu.__dlpack__()
        assert self._hip is not None
        return _ext().dlpack_export(self._hip.buf, self._shape, int(self._dtype.itemsize) * 8)

    def __dlpack_device__(self) -> tuple[int, int]:
        return (KDL_CPU, 0) if self._device == "cpu" else (KDL_ROCM, 0)

    def numpy(self) -> np.ndarray:
        if self._device == "cpu":
            assert self._cpu is not None
            return self._cpu
        assert self._hip is not None
        out = np.empty(self._shape, dtype=self._dtype)
        if out.nbytes:
            _ext().copy_to_host(self._hip.buf, out)
        return out

    def to_torch(self, device: str | None = None) -> Any:
        torch = _torch()
        if torch is None:
            raise RuntimeError("torch is not available; install it to use Tensor.to_torch()")
        dev = self._device if device is None else _normalize_device(device)
        if dev == "cpu":
            return torch.from_numpy(self.numpy())
        if self._device == "hip":
            from torch.utils import dlpack  # type: ignore

            return dlpack.from_dlpack(self)
        return torch.from_numpy(self.numpy()).to("cuda")

    def to(self, device: Any) -> "Tensor":
        dev = _normalize_device(device)
        if dev == self._device:
            return self
        if dev == "cpu":
            return Tensor(shape=self._shape, dtype=self._dtype, device="cpu", cpu=self.numpy())
        mod = _ext()
        buf = mod.alloc_buffer(max(self.nbytes, 1), "private")
        assert self._cpu is not None
        if self.nbytes:
            mod.copy_from_host(buf, np.ascontiguousarray(self._cpu))
        return Tensor(shape=self._shape, dtype=self._dtype, device="hip", hip=_HipStorage(buf, self.nbytes))

    def _hip_buffer(self) -> object:
        if self._device != "hip":
            raise TypeError("expected a hip tensor")
        assert self._hip is not None
        return self._hip.buf


def _from_capsule(mod: Any, capsule: Any) -> Tensor:
    buf, shape, bits = mod.dlpack_import(capsule)
    if int(bits) not in (16, 32):
        raise TypeError(f"unsupported dlpack dtype bits: {bits}")
    dt = np.float16 if int(bits) == 16 else np.float32
    shp = tuple(int(d) for d in shape)
    return Tensor(shape=shp, dtype=dt, device="hip", hip=_HipStorage(buf, _numel(shp) * np.dtype(dt).itemsize))


def tensor(data: Any, *, device: Any = None, dtype: Any = None) -> Tensor:
    dev = _normalize_device(device)
    if _is_torch_tensor(data):
        torch = _torch()
        assert torch is not None
        t = data.detach()
        if dtype is not None:
            want = torch.float16 if _require_supported_dtype(dtype) == np.float16 else torch.float32
            if t.dtype != want:
                t = t.to(dtype=want)
        elif t.dtype not in (torch.float16, torch.float32):
            t = t.to(dtype=torch.float32)
        if dev == "hip" and t.device.type == "cuda":
            # Zero-copy: the capsule keeps the torch storage alive.
            return _from_capsule(_ext(), t.contiguous().__dlpack__())
        if t.device.type != "cpu":
            t = t.to("cpu")
        arr = t.contiguous().numpy()
        return Tensor(shape=arr.shape, dtype=arr.dtype, device="cpu", cpu=arr).to(dev)
    if isinstance(data, Tensor):
        out = data
        if dtype is not None and np.dtype(dtype) != out.dtype:
            host = out.numpy().astype(_require_supported_dtype(dtype), copy=True)
            out = Tensor(shape=out.shape, dtype=host.dtype, device="cpu", cpu=host)
        return out.to(dev)
    if dtype is None:
        arr = np.asarray(data)
        if arr.dtype not in (np.float16, np.float32):
            arr = arr.astype(np.float32)
    else:
        arr = np.asarray(data, dtype=_require_supported_dtype(dtype))
    arr = np.ascontiguousarray(arr)
    return Tensor(shape=arr.shape, dtype=arr.dtype, device="cpu", cpu=arr).to(dev)


def empty(shape: int | tuple[int, ...], *, device: Any = None, dtype: Any = None) -> Tensor:
    dev = _normalize_device(device)
    dt = _require_supported_dtype(np.float32 if dtype is None else dtype)
    shp = (int(shape),) if isinstance(shape, int) else tuple(int(d) for d in shape)
    if dev == "cpu":
        return Tensor(shape=shp, dtype=dt, device="cpu", cpu=np.empty(shp, dtype=dt))
    nbytes = _numel(shp) * dt.itemsize
    buf = _ext().alloc_buffer(max(nbytes, 1), "private")
    return Tensor(shape=shp, dtype=dt, device="hip", hip=_HipStorage(buf, nbytes))


def empty_like(x: Tensor, *, device: Any = None) -> Tensor:
    return empty(x.shape, device=x.device if device is None else device, dtype=x.dtype)
