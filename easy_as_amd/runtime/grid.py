"""Launch-geometry inference (reference ``eas/runtime/grid.py:11-130``).

The reference semantics are kept exactly: a 1-D launch is sized from
``_nthreads`` or a scalar arg ``N``; kernels that use ``program_id``/
``thread_id`` on axis 1 or 2 get a 2-D/3-D grid of ``(ceil(W/BLOCK), H, D)``
from ``_shape`` or scalar args ``H``/``W``/``D``.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

from ..ir import IRModule


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def infer_nthreads(runtime_args: Mapping[str, Any], *, nthreads: int | None = None) -> int:
    """Total 1-D extent: ``_nthreads`` if given, else the scalar argument ``N``."""
    if nthreads is None:
        if "N" not in runtime_args:
            raise ValueError(
                "1-D launches need either `_nthreads=...` or a scalar argument named 'N' for grid sizing"
            )
        nthreads = int(runtime_args["N"])
    n = int(nthreads)
    if n < 0:
        raise ValueError("nthreads must be >= 0")
    return n


def infer_1d_grid(runtime_args: Mapping[str, Any], threadgroup_size: int, *, nthreads: int | None = None) -> int:
    """Number of BLOCK-sized groups covering the 1-D extent."""
    n = infer_nthreads(runtime_args, nthreads=nthreads)
    if threadgroup_size <= 0:
        raise ValueError("threadgroup_size must be > 0")
    return _cdiv(n, threadgroup_size)


_NDIM: dict[int, tuple[IRModule, int]] = {}


def grid_ndim(ir: IRModule) -> int:
    """Highest axis used by ``program_id``/``thread_id`` plus one.  An IR never changes
    after tracing, so the scan runs once per IR (the entry holds the IR, keeping its id
    unique); an unrolled matmul has tens of thousands of instructions."""
    hit = _NDIM.get(id(ir))
    if hit is not None and hit[0] is ir:
        return hit[1]
    axes = [int(i.args[0]) for i in ir.insts if i.op in ("program_id", "thread_id")]
    ndim = max(axes, default=-1) + 1
    if len(_NDIM) >= 4096:
        _NDIM.clear()
    _NDIM[id(ir)] = (ir, ndim)
    return ndim


def infer_grid(
    ir: IRModule,
    runtime_args: Mapping[str, Any],
    threadgroup_size: int,
    *,
    shape: tuple[int, ...] | None = None,
) -> tuple[int, int, int] | None:
    """2-D/3-D group grid ``(ceil(W/BLOCK), H, D)``, or ``None`` for 1-D kernels.

    The dimensionality is the highest axis used by ``program_id``/``thread_id``
    plus one.  Sources, in priority order: the trailing 2/3 dims of ``shape``,
    then scalar runtime args ``H``, ``W`` (and ``D``).
    """
    ndim = grid_ndim(ir)
    if ndim <= 1:
        return None
    if ndim > 3:
        raise ValueError("only 1D/2D/3D grids are supported")
    if threadgroup_size <= 0:
        raise ValueError("threadgroup_size must be > 0")
    if shape is not None:
        if len(shape) < ndim:
            raise ValueError(f"_shape must have >= {ndim} dims for this kernel")
        dims = [int(d) for d in shape]
        if any(d < 0 for d in dims):
            raise ValueError("_shape dims must be >= 0")
        d, h, w = (1, dims[-2], dims[-1]) if ndim == 2 else (dims[-3], dims[-2], dims[-1])
    else:
        need = ("H", "W") if ndim == 2 else ("D", "H", "W")
        if any(k not in runtime_args for k in need):
            names = ", ".join(f"'{k}'" for k in need)
            raise ValueError(
                f"{ndim}D grid inference requires either `_shape=...` or scalar runtime args named {names} "
                "(or pass `_grid=...` explicitly)"
            )
        h, w = int(runtime_args["H"]), int(runtime_args["W"])
        d = int(runtime_args["D"]) if ndim == 3 else 1
    if h < 0 or w < 0 or d < 0:
        raise ValueError("shape dims must be >= 0")
    return (_cdiv(w, threadgroup_size) if w else 0, h, d)
