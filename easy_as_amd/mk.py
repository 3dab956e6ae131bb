"""The ``mk`` kernel DSL: tracing-only primitives used inside ``@eas.kernel``.

Every function records an IR instruction on the builder of the trace that is
active on the calling thread; nothing executes eagerly.  The surface (names,
argument order, the operators ``+ * // % < & | ~`` of ``val``) is the
reference's (``eas/mk.py:37-201``) so user kernels trace unchanged.
"""

from __future__ import annotations

import contextlib
import threading
from collections.abc import Iterator
from dataclasses import dataclass
from typing import Any

from .ir import DType, ValueRef


class _TraceState(threading.local):
    builder: Any | None = None


_state = _TraceState()


@contextlib.contextmanager
def _trace(builder: Any) -> Iterator[None]:
    """Make ``builder`` the target of ``mk.*`` calls on this thread for the block."""
    prev, _state.builder = _state.builder, builder
    try:
        yield
    finally:
        _state.builder = prev


def _b() -> Any:
    builder = _state.builder
    if builder is None:
        raise RuntimeError("eas.mk is only valid inside an @eas.kernel trace/launch")
    return builder


def _binary(method: str, *, reflected: bool) -> Any:
    def op(self: "val", other: Any) -> "val":
        fn = getattr(_b(), method)
        return fn(other, self) if reflected else fn(self, other)

    op.__name__ = f"__{'r' if reflected else ''}{method.rstrip('_')}__"
    return op


@dataclass(frozen=True, slots=True)
class val:
    """A traced SSA value.  Only the operators the IR can express are defined."""

    ref: ValueRef

    @property
    def dtype(self) -> DType:
        return self.ref.dtype

    __add__ = _binary("add", reflected=False)
    __radd__ = _binary("add", reflected=True)
    __mul__ = _binary("mul", reflected=False)
    __rmul__ = _binary("mul", reflected=True)
    __floordiv__ = _binary("floordiv", reflected=False)
    __rfloordiv__ = _binary("floordiv", reflected=True)
    __mod__ = _binary("mod", reflected=False)
    __rmod__ = _binary("mod", reflected=True)
    __lt__ = _binary("lt", reflected=False)
    __and__ = _binary("and_", reflected=False)
    __rand__ = _binary("and_", reflected=True)
    __or__ = _binary("or_", reflected=False)
    __ror__ = _binary("or_", reflected=True)

    def __invert__(self) -> "val":
        return _b().not_(self)


# -- ids ------------------------------------------------------------------

def program_id(axis: int) -> val:
    """Index of this program (SPMD) / threadgroup (thread mode) along ``axis``."""
    return _b().program_id(axis)


def local_id(axis: int) -> val:
    """Thread index inside the threadgroup along ``axis`` (thread mode)."""
    return _b().local_id(axis)


def lane_id() -> val:
    """Lane inside the 32-wide simdgroup: ``local_id % 32``."""
    return _b().lane_id()


def sg_id() -> val:
    """Index of the 32-wide simdgroup inside the threadgroup: ``local_id // 32``."""
    return _b().sg_id()


def arange(start: int, size: int) -> val:
    """SPMD lane vector ``[start, start + size)``; makes the kernel an SPMD kernel."""
    return _b().arange(start, size)


def tid(start: int, size: int) -> val:
    """Scalar thread id ``start + local_id(0)``; makes the kernel a thread-mode
    kernel with ``size`` threads per threadgroup (the reference's old ``arange``)."""
    return _b().tid(start, size)


# -- threadgroup memory ---------------------------------------------------

def alloc_tg(size: int) -> val:
    """Threadgroup (LDS) array of ``size`` f32."""
    return _b().alloc_tg(size)


def alloc_tg_f16(size: int) -> val:
    """Threadgroup (LDS) array of ``size`` f16."""
    return _b().alloc_tg(size, dtype=DType.F16)


def alloc_tg_bf16(size: int) -> val:
    """Threadgroup (LDS) array of ``size`` bf16 (an addition to the reference's DSL)."""
    return _b().alloc_tg(size, dtype=DType.BF16)


def barrier() -> None:
    """Threadgroup barrier with threadgroup-memory ordering."""
    _b().barrier()


# -- memory ----------------------------------------------------------------

def load(buffer: Any, offset: Any, mask: Any | None = None) -> val:
    """``buffer[offset]`` where ``mask`` holds, else 0."""
    return _b().load(buffer, offset, mask)


def store(buffer: Any, offset: Any, value: Any, mask: Any | None = None) -> None:
    """``buffer[offset] = value`` where ``mask`` holds."""
    _b().store(buffer, offset, value, mask)


# -- arithmetic -------------------------------------------------------------

def where(cond: Any, a: Any, b: Any) -> val:
    return _b().where(cond, a, b)


def fma(a: Any, b: Any, c: Any) -> val:
    """Fused multiply-add ``a * b + c`` with a single rounding."""
    return _b().fma(a, b, c)


def to_f32(x: Any) -> val:
    return _b().cast(x, DType.F32)


def to_f16(x: Any) -> val:
    return _b().cast(x, DType.F16)


def to_bf16(x: Any) -> val:
    """Round to bfloat16 (nearest-even; an addition to the reference's DSL)."""
    return _b().cast(x, DType.BF16)


def to_u32(x: Any) -> val:
    return _b().cast(x, DType.U32)


def and_(a: Any, b: Any) -> val:
    return _b().and_(a, b)


def or_(a: Any, b: Any) -> val:
    return _b().or_(a, b)


def not_(x: Any) -> val:
    return _b().not_(x)


# -- contractions -------------------------------------------------------------

def dot(a_buffer: Any, a_base: Any, a_stride: Any, b_buffer: Any, b_base: Any, b_stride: Any, K: Any) -> val:
    """Per-thread f32 dot product ``sum_k A[a_base + k*a_stride] * B[b_base + k*b_stride]``
    accumulated with one fma per k, k ascending from 0."""
    return _b().dot(a_buffer, a_base, a_stride, b_buffer, b_base, b_stride, K)


def mma_zero() -> val:
    """A zero 8x8 f32 simdgroup accumulator fragment."""
    return _b().mma_zero()


def mma(a_buffer: Any, a_base: Any, a_stride: Any, b_buffer: Any, b_base: Any, b_stride: Any, acc: Any) -> val:
    """Simdgroup ``acc + A(8x8) @ B(8x8)``; A and B are row-major at ``base`` with row ``stride``."""
    return _b().mma(a_buffer, a_base, a_stride, b_buffer, b_base, b_stride, acc)


def mma_store(buffer: Any, base: Any, stride: Any, frag: Any) -> None:
    """Store an 8x8 f32 fragment row-major at ``buffer + base`` with row ``stride``."""
    _b().mma_store(buffer, base, stride, frag)
