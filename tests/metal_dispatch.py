"""The sizes the reference runtime hands its native ``launch`` (test helper).

``MetalRuntime.run`` (eas/runtime/metal.py:244-346) turns a kernel call into
``mod.launch(pipeline, argv, writable, tpg, tptg)``: for a thread-mode kernel
``tpg`` counts threads (``N`` for a 1-D launch, ``groups * BLOCK`` per axis for an
explicit or inferred grid) and ``tptg`` is ``BLOCK`` (an int for 1-D, a tuple
otherwise); for an SPMD kernel ``tpg`` counts programs and ``tptg`` is
``(1, 1, 1)``.  ``reference_dispatch`` restates those rules so the tests can drive
``eas._hip.launch`` exactly as the reference's runtime would.
"""

from __future__ import annotations

from typing import Any, Mapping

from easy_as_amd.runtime.grid import infer_grid, infer_nthreads


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def reference_dispatch(ck: Any, runtime_args: Mapping[str, Any], *, nthreads: int | None = None,
                       grid: tuple[int, int, int] | None = None,
                       shape: tuple[int, ...] | None = None) -> tuple[Any, Any] | None:
    """``(threads_per_grid, threads_per_threadgroup)`` as metal.py:256-326 computes them
    (``None``: the reference launches nothing)."""
    block = int(ck.block_size)
    thread = ck.launch_mode == "thread"
    if grid is None:
        inferred = infer_grid(ck.ir, runtime_args, block, shape=shape)
        if inferred is None:
            n = infer_nthreads(runtime_args, nthreads=nthreads)
            if n == 0:
                return None
            if thread:
                return int(n), block
            return _cdiv(int(n), block), (1, 1, 1)
        gx, gy, gz = (int(g) for g in inferred)
    else:
        gx, gy, gz = (int(g) for g in grid)
    if 0 in (gx, gy, gz):
        return None
    if thread:
        return (gx * block, gy, gz), (block, 1, 1)
    return (gx, gy, gz), (1, 1, 1)
