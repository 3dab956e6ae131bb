"""Tracer (Python kernel -> eas IR), IR optimisation passes and ``compile``.

``compile(fn, runtime_args, meta)`` traces ``fn`` with ``mk`` bound to an IR
builder, runs the pass pipeline, verifies the IR and lowers it with the gfx950
emitter.  The tracing rules and the pass semantics follow the reference
(``eas/compiler.py:132-617`` builder/tracer, ``:648-1272`` passes); each pass
below cites the lines it restates.
"""

from __future__ import annotations

import os
import types
from dataclasses import dataclass, field
from typing import Any, Callable, Mapping

import numpy as np

from . import mk
from .analysis import infer_writes
from .ir import Arg, ArgKind, DType, IRModule, Inst, ValueRef, broadcast, validate_ir

U32_LIMIT = 1 << 32

# ---------------------------------------------------------------------------
# runtime-argument classification and the specialisation signature
# ---------------------------------------------------------------------------

_torch_mod: Any = None
_torch_probed = False


def _torch() -> Any | None:
    global _torch_mod, _torch_probed
    if not _torch_probed:
        _torch_probed = True
        try:
            import torch  # type: ignore

            _torch_mod = torch
        except Exception:
            _torch_mod = None
    return _torch_mod


@dataclass(frozen=True, slots=True)
class RuntimeArgSig:
    kind: ArgKind
    dtype: DType
    device: str | None = None


def _np_buffer_dtype(dt: Any) -> DType:
    dt = np.dtype(dt)
    if dt == np.float32:
        return DType.F32
    if dt == np.float16:
        return DType.F16
    raise TypeError(f"unsupported dtype: {dt} (expected float32 or float16)")


def _is_eas_tensor(v: Any) -> bool:
    return bool(getattr(v, "__eas_tensor__", False))


def _is_torch_tensor(v: Any) -> bool:
    torch = _torch()
    return torch is not None and isinstance(v, torch.Tensor)


_TORCH_BUFFER_DTYPES: dict[Any, DType] = {}


def _torch_buffer_dtype(v: Any) -> DType:
    dt = _TORCH_BUFFER_DTYPES.get(v.dtype)
    if dt is not None:
        return dt
    torch = _torch()
    assert torch is not None
    _TORCH_BUFFER_DTYPES.update({torch.float32: DType.F32, torch.float16: DType.F16, torch.bfloat16: DType.BF16})
    dt = _TORCH_BUFFER_DTYPES.get(v.dtype)
    if dt is None:
        raise TypeError(f"unsupported torch dtype: {v.dtype} (expected float32, float16 or bfloat16)")
    return dt


def _scalar_dtype(v: Any) -> DType:
    if isinstance(v, (bool, np.bool_)):
        return DType.BOOL
    if isinstance(v, (int, np.integer)):
        return DType.U32
    if isinstance(v, np.float16):
        return DType.F16
    if isinstance(v, (float, np.floating)):
        return DType.F32
    raise TypeError(f"unsupported scalar type: {type(v)!r}")


def classify_arg(v: Any) -> RuntimeArgSig:
    """Kind/dtype/device of one runtime argument (reference ``compiler.py:113-129``)."""
    if isinstance(v, np.ndarray):
        return RuntimeArgSig("buffer", _np_buffer_dtype(v.dtype), "cpu")
    if _is_eas_tensor(v):
        dev = getattr(v, "device", None)
        return RuntimeArgSig("buffer", _np_buffer_dtype(getattr(v, "dtype")), str(dev) if dev else None)
    if _is_torch_tensor(v):
        return RuntimeArgSig("buffer", _torch_buffer_dtype(v), str(v.device.type))
    return RuntimeArgSig("scalar", _scalar_dtype(v), None)


_NP_BUFFER_KEYS = {np.dtype(np.float32): ("buffer", DType.F32, "cpu"), np.dtype(np.float16): ("buffer", DType.F16, "cpu")}
_SCALAR_KEYS = {int: ("scalar", DType.U32, None), float: ("scalar", DType.F32, None), bool: ("scalar", DType.BOOL, None)}


def _arg_key(v: Any) -> tuple[str, DType, str | None]:
    """``(kind, dtype, device)`` of ``classify_arg``, with the per-launch common cases
    (NumPy f32/f16 arrays, torch tensors, Python scalars) answered without building a
    ``RuntimeArgSig``."""
    t = type(v)
    if t is np.ndarray:
        key = _NP_BUFFER_KEYS.get(v.dtype)
        if key is not None:
            return key
    elif t in _SCALAR_KEYS:
        return _SCALAR_KEYS[t]
    else:
        torch = _torch()
        if torch is not None and isinstance(v, torch.Tensor):
            return ("buffer", _torch_buffer_dtype(v), "cuda" if v.is_cuda else v.device.type)
    s = classify_arg(v)
    return (s.kind, s.dtype, s.device)


def runtime_arg_signature(runtime_args: Mapping[str, Any]) -> tuple[tuple[str, Any], ...]:
    """Cache key part for runtime args: ``(name, (kind, dtype, device))`` sorted by name.

    Scalar *values* are deliberately not part of it: they are kernel arguments,
    not trace-time constants (reference ``compiler.py:41-54``).
    """
    return tuple(sorted((name, _arg_key(value)) for name, value in runtime_args.items()))


# ---------------------------------------------------------------------------
# the IR builder behind mk.*
# ---------------------------------------------------------------------------


class _IRBuilder:
    """Records ``mk`` calls as SSA instructions (reference ``compiler.py:132-550``)."""

    def __init__(self, name: str) -> None:
        self.name = name
        self.args: list[Arg] = []
        self.insts: list[Inst] = []
        self.buffer_ids: set[int] = set()
        self._next = 0

    # -- plumbing -----------------------------------------------------------
    def new(self, dtype: DType, lanes: int = 1) -> mk.val:
        ref = ValueRef(self._next, dtype, int(lanes))
        self._next += 1
        return mk.val(ref)

    def emit(self, op: str, dtype: DType, args: tuple[Any, ...], lanes: int = 1) -> mk.val:
        v = self.new(dtype, lanes)
        self.insts.append(Inst(op, v.ref, args))  # type: ignore[arg-type]
        return v

    def value(self, x: Any) -> mk.val:
        """Coerce a traced value or a Python literal to a traced value."""
        if isinstance(x, mk.val):
            return x
        if isinstance(x, bool):
            return self.emit("const", DType.BOOL, (bool(x),))
        if isinstance(x, (int, np.integer)):
            if int(x) < 0:
                raise ValueError("invalid IR: u32 const must be a non-negative Python int")
            return self.emit("const", DType.U32, (int(x),))
        if isinstance(x, (float, np.floating)):
            return self.emit("const", DType.F32, (float(x),))
        raise TypeError(f"unsupported literal: {type(x)!r}")

    def _buffer(self, x: Any, what: str) -> mk.val:
        if not isinstance(x, mk.val) or x.ref.id not in self.buffer_ids:
            raise TypeError(f"{what} expects a buffer (arg or alloc_tg)")
        return x

    def _index(self, x: Any, what: str) -> mk.val:
        v = self.value(x)
        if v.dtype != DType.U32:
            raise TypeError(f"{what} must be u32, got {v.dtype}")
        if v.ref.lanes != 1:
            raise TypeError(f"{what} must be scalar (lanes=1), got lanes={v.ref.lanes}")
        return v

    @staticmethod
    def _lanes(op: str, *vals: mk.val) -> int:
        lanes = 1
        for v in vals:
            n = broadcast(lanes, v.ref.lanes)
            if n is None:
                raise TypeError(f"{op} lanes mismatch: {lanes} vs {v.ref.lanes}")
            lanes = n
        return lanes

    def _binary(self, op: str, a: Any, b: Any, *, operand: tuple[DType, ...] | None, result: DType | None) -> mk.val:
        av, bv = self.value(a), self.value(b)
        if operand == (DType.BOOL,):
            if av.dtype != DType.BOOL or bv.dtype != DType.BOOL:
                raise TypeError("and/or/not expect bool operands")
        else:
            if av.dtype != bv.dtype:
                raise TypeError(f"{op} dtype mismatch: {av.dtype} vs {bv.dtype}")
            if operand is not None and av.dtype not in operand:
                raise TypeError(f"{op} expects u32, got {av.dtype}")
        lanes = self._lanes(op, av, bv)
        return self.emit(op, result or av.dtype, (av.ref, bv.ref), lanes)

    # -- ids ---------------------------------------------------------------
    def program_id(self, axis: int) -> mk.val:
        return self.emit("program_id", DType.U32, (int(axis),))

    def local_id(self, axis: int) -> mk.val:
        if not isinstance(axis, int):
            raise TypeError("local_id(axis) requires an int axis")
        if axis not in (0, 1, 2):
            raise ValueError("local_id axis must be 0/1/2")
        return self.emit("local_id", DType.U32, (axis,))

    def lane_id(self) -> mk.val:
        return self.emit("lane_id", DType.U32, ())

    def sg_id(self) -> mk.val:
        return self.emit("sg_id", DType.U32, ())

    def _range(self, op: str, start: Any, size: Any) -> mk.val:
        if not isinstance(start, int) or not isinstance(size, int):
            raise TypeError(f"{op}(start, size) requires Python ints (compile-time constants)")
        if size <= 0:
            raise ValueError(f"{op}(size) must be > 0")
        return self.emit(op, DType.U32, (start, size), lanes=size if op == "arange" else 1)

    def arange(self, start: int, size: int) -> mk.val:
        return self._range("arange", start, size)

    def tid(self, start: int, size: int) -> mk.val:
        return self._range("tid", start, size)

    # -- threadgroup memory ------------------------------------------------
    def alloc_tg(self, size: int, *, dtype: DType = DType.F32) -> mk.val:
        if not isinstance(size, int):
            raise TypeError("alloc_tg(size) requires a Python int (compile-time constant)")
        if size <= 0:
            raise ValueError("alloc_tg(size) must be > 0")
        if dtype not in (DType.F16, DType.BF16, DType.F32):
            raise TypeError(f"alloc_tg(dtype=...) must be f16/bf16/f32, got {dtype}")
        v = self.emit("alloc_tg", dtype, (size,))
        self.buffer_ids.add(v.ref.id)
        return v

    def barrier(self) -> None:
        self.insts.append(Inst("barrier", None, ()))

    # -- arithmetic ------------------------------------------------------------
    def add(self, a: Any, b: Any) -> mk.val:
        return self._binary("add", a, b, operand=None, result=None)

    def mul(self, a: Any, b: Any) -> mk.val:
        return self._binary("mul", a, b, operand=None, result=None)

    def floordiv(self, a: Any, b: Any) -> mk.val:
        return self._binary("floordiv", a, b, operand=(DType.U32,), result=None)

    def mod(self, a: Any, b: Any) -> mk.val:
        return self._binary("mod", a, b, operand=(DType.U32,), result=None)

    def lt(self, a: Any, b: Any) -> mk.val:
        return self._binary("lt", a, b, operand=None, result=DType.BOOL)

    def and_(self, a: Any, b: Any) -> mk.val:
        return self._binary("and", a, b, operand=(DType.BOOL,), result=DType.BOOL)

    def or_(self, a: Any, b: Any) -> mk.val:
        return self._binary("or", a, b, operand=(DType.BOOL,), result=DType.BOOL)

    def not_(self, x: Any) -> mk.val:
        xv = self.value(x)
        if xv.dtype != DType.BOOL:
            raise TypeError("and/or/not expect bool operands")
        return self.emit("not", DType.BOOL, (xv.ref,), xv.ref.lanes)

    def fma(self, a: Any, b: Any, c: Any) -> mk.val:
        av, bv, cv = self.value(a), self.value(b), self.value(c)
        if not (av.dtype == bv.dtype == cv.dtype):
            raise TypeError(f"fma dtype mismatch: {av.dtype} vs {bv.dtype} vs {cv.dtype}")
        return self.emit("fma", av.dtype, (av.ref, bv.ref, cv.ref), self._lanes("fma", av, bv, cv))

    def where(self, cond: Any, a: Any, b: Any) -> mk.val:
        cv, av, bv = self.value(cond), self.value(a), self.value(b)
        if cv.dtype != DType.BOOL:
            raise TypeError(f"where(cond, ...) expects bool condition, got {cv.dtype}")
        if av.dtype != bv.dtype:
            raise TypeError(f"where value dtype mismatch: {av.dtype} vs {bv.dtype}")
        return self.emit("where", av.dtype, (cv.ref, av.ref, bv.ref), self._lanes("where", av, bv, cv))

    def cast(self, x: Any, dtype: DType) -> mk.val:
        xv = self.value(x)
        if not isinstance(dtype, DType):
            raise TypeError("cast(x, dtype) expects dtype to be a DType")
        if xv.dtype == dtype:
            return xv
        return self.emit("cast", dtype, (xv.ref, dtype), xv.ref.lanes)

    # -- contractions ----------------------------------------------------------
    def _contraction_operands(self, op: str, a_buffer: Any, a_base: Any, a_stride: Any, b_buffer: Any,
                              b_base: Any, b_stride: Any) -> tuple[ValueRef, ...]:
        a = self._buffer(a_buffer, f"{op} a_buffer")
        b = self._buffer(b_buffer, f"{op} b_buffer")
        for buf, what in ((a, "a_buffer"), (b, "b_buffer")):
            if buf.dtype not in (DType.F16, DType.BF16, DType.F32):
                raise TypeError(f"{op} {what} must be f16/bf16/f32")
        if op == "mma" and DType.BF16 in (a.dtype, b.dtype) and a.dtype != b.dtype:
            raise TypeError(f"mma a/b buffers must both be bf16 or neither, got {a.dtype} and {b.dtype}")
        idx = [self._index(v, f"{op} {n}") for v, n in ((a_base, "a_base"), (a_stride, "a_stride"),
                                                        (b_base, "b_base"), (b_stride, "b_stride"))]
        return (a.ref, idx[0].ref, idx[1].ref, b.ref, idx[2].ref, idx[3].ref)

    def dot(self, a_buffer: Any, a_base: Any, a_stride: Any, b_buffer: Any, b_base: Any, b_stride: Any, K: Any) -> mk.val:
        ops = self._contraction_operands("dot", a_buffer, a_base, a_stride, b_buffer, b_base, b_stride)
        k = self._index(K, "dot K")
        return self.emit("dot", DType.F32, ops + (k.ref,))

    def mma_zero(self) -> mk.val:
        return self.emit("mma_zero", DType.SG_F32_8X8, ())

    def mma(self, a_buffer: Any, a_base: Any, a_stride: Any, b_buffer: Any, b_base: Any, b_stride: Any, acc: Any) -> mk.val:
        ops = self._contraction_operands("mma", a_buffer, a_base, a_stride, b_buffer, b_base, b_stride)
        accv = self.value(acc)
        if accv.dtype != DType.SG_F32_8X8:
            raise TypeError(f"mma acc must be sg_f32_8x8, got {accv.dtype}")
        return self.emit("mma", DType.SG_F32_8X8, ops + (accv.ref,))

    def mma_store(self, buffer: Any, base: Any, stride: Any, frag: Any) -> None:
        buf = self._buffer(buffer, "mma_store(buffer, ...)")
        if buf.dtype != DType.F32:
            raise TypeError("mma_store currently supports float32 buffers only")
        basev = self._index(base, "mma_store base")
        stridev = self._index(stride, "mma_store stride")
        fragv = self.value(frag)
        if fragv.dtype != DType.SG_F32_8X8 or fragv.ref.lanes != 1:
            raise TypeError(f"mma_store frag must be sg_f32_8x8, got {fragv.dtype}")
        self.insts.append(Inst("mma_store", None, (buf.ref, basev.ref, stridev.ref, fragv.ref)))

    # -- memory ------------------------------------------------------------------
    def _mask(self, mask: Any, off: mk.val, what: str) -> mk.val:
        m = self.value(True if mask is None else mask)
        if m.dtype != DType.BOOL:
            raise TypeError(f"{what} mask must be bool, got {m.dtype}")
        if m.ref.lanes not in (1, off.ref.lanes):
            raise TypeError(f"{what} mask lanes must be 1 or match offset lanes, got {m.ref.lanes} vs {off.ref.lanes}")
        return m

    def load(self, buffer: Any, offset: Any, mask: Any | None) -> mk.val:
        buf = self._buffer(buffer, "load(buffer, ...)")
        off = self.value(offset)
        if off.dtype != DType.U32:
            raise TypeError(f"load offset must be u32, got {off.dtype}")
        m = self._mask(mask, off, "load")
        return self.emit("load", buf.dtype, (buf.ref, off.ref, m.ref), off.ref.lanes)

    def store(self, buffer: Any, offset: Any, value: Any, mask: Any | None) -> None:
        buf = self._buffer(buffer, "store(buffer, ...)")
        off = self.value(offset)
        val = self.value(value)
        if off.dtype != DType.U32:
            raise TypeError(f"store offset must be u32, got {off.dtype}")
        m = self._mask(mask, off, "store")
        if val.dtype != buf.dtype:
            raise TypeError(f"store dtype mismatch: {buf.dtype} vs {val.dtype}")
        if val.ref.lanes not in (1, off.ref.lanes):
            raise TypeError(f"store value lanes must be 1 or match offset lanes, got {val.ref.lanes} vs {off.ref.lanes}")
        self.insts.append(Inst("store", None, (buf.ref, off.ref, val.ref, m.ref)))


# ---------------------------------------------------------------------------
# tracing
# ---------------------------------------------------------------------------


def _with_globals(fn: Callable[..., Any], extra: Mapping[str, Any]) -> Callable[..., Any]:
    """A copy of ``fn`` whose globals also hold the meta parameters."""
    if not extra:
        return fn
    g = dict(fn.__globals__)
    g.update(extra)
    return types.FunctionType(fn.__code__, g, fn.__name__, fn.__defaults__, fn.__closure__)


def trace_to_ir(fn: Callable[..., Any], runtime_args: Mapping[str, Any], meta: Mapping[str, Any]) -> IRModule:
    """Run ``fn`` once with ``mk`` recording into a fresh builder.

    Runtime args become ``arg`` instructions in call order (buffers for arrays /
    tensors, scalars otherwise); meta params are bound as Python literals, so
    Python control flow over them (``range`` loops, ``if ... raise``) runs at
    trace time (reference ``compiler.py:553-601``).
    """
    b = _IRBuilder(fn.__name__)
    kwargs: dict[str, Any] = {}
    for name, value in runtime_args.items():
        sig = classify_arg(value)
        b.args.append(Arg(name, sig.dtype, sig.kind))
        v = b.emit("arg", sig.dtype, (name, sig.kind, sig.dtype))
        if sig.kind == "buffer":
            b.buffer_ids.add(v.ref.id)
        kwargs[name] = v
    lit: dict[str, Any] = {}
    for k, v in meta.items():
        if isinstance(v, np.integer):
            v = int(v)
        elif isinstance(v, np.floating):
            v = float(v)
        if not isinstance(v, (bool, int, float)):
            raise TypeError(f"meta parameter {k!r} must be a Python literal, got {type(v)!r}")
        lit[k] = v
    kwargs.update(lit)
    with mk._trace(b):
        _with_globals(fn, lit)(**kwargs)
    return IRModule(fn.__name__, tuple(b.args), tuple(b.insts))


# ---------------------------------------------------------------------------
# pass utilities
# ---------------------------------------------------------------------------


def _defs(ir: IRModule) -> dict[int, Inst]:
    return {inst.out.id: inst for inst in ir.insts if inst.out is not None}


def _use_counts(insts: tuple[Inst, ...] | list[Inst]) -> dict[int, int]:
    counts: dict[int, int] = {}
    for inst in insts:
        for a in inst.args:
            if isinstance(a, ValueRef):
                counts[a.id] = counts.get(a.id, 0) + 1
    return counts


class _Remap:
    """Value substitution while rebuilding an instruction list."""

    def __init__(self) -> None:
        self.to: dict[int, ValueRef] = {}

    def __call__(self, a: Any) -> Any:
        return self.to.get(a.id, a) if isinstance(a, ValueRef) else a

    def args(self, inst: Inst) -> tuple[Any, ...]:
        return tuple(self(a) for a in inst.args)


def _const_of(defs: Mapping[int, Inst], ref: Any) -> Any:
    inst = defs.get(ref.id) if isinstance(ref, ValueRef) else None
    return inst.args[0] if inst is not None and inst.op == "const" else None


# ---------------------------------------------------------------------------
# passes (run in the order of the reference's _optimize_ir, compiler.py:648-655)
# ---------------------------------------------------------------------------


def _thread_id_rewrite_disabled() -> bool:
    return os.environ.get("EAS_DISABLE_THREAD_ID_REWRITE", "") not in ("", "0", "false", "False")


def _single_tid_size(ir: IRModule) -> int | None:
    sizes = {int(inst.args[1]) for inst in ir.insts if inst.op == "tid"}
    return sizes.pop() if len(sizes) == 1 else None


def _rewrite_thread_id(ir: IRModule) -> IRModule:
    """``program_id(0) * S + tid(0, S)`` -> ``thread_id(0)`` (global thread index).

    Applies only when every ``tid`` in the kernel has the same size S; disabled
    by ``EAS_DISABLE_THREAD_ID_REWRITE`` (reference ``compiler.py:937-1016``).
    """
    if _thread_id_rewrite_disabled():
        return ir
    size = _single_tid_size(ir)
    if size is None:
        return ir
    defs = _defs(ir)

    def is_op(ref: Any, op: str) -> Inst | None:
        inst = defs.get(ref.id) if isinstance(ref, ValueRef) else None
        return inst if inst is not None and inst.op == op else None

    def is_pid_times_size(ref: Any) -> bool:
        mul = is_op(ref, "mul")
        if mul is None:
            return False
        x, y = mul.args
        for p, c in ((x, y), (y, x)):
            pid = is_op(p, "program_id")
            const = is_op(c, "const")
            if pid is not None and pid.args[0] == 0 and const is not None and const.args[0] == size:
                return True
        return False

    def is_tid0(ref: Any) -> bool:
        t = is_op(ref, "tid")
        return t is not None and t.args[0] == 0 and t.args[1] == size

    out: list[Inst] = []
    for inst in ir.insts:
        if inst.op == "add" and inst.out is not None:
            a, b = inst.args
            if (is_pid_times_size(a) and is_tid0(b)) or (is_pid_times_size(b) and is_tid0(a)):
                out.append(Inst("thread_id", inst.out, (0,)))
                continue
        out.append(inst)
    return IRModule(ir.name, ir.args, tuple(out))


def _fuse_fma(ir: IRModule) -> IRModule:
    """f32 ``add(mul(x, y), z)`` -> ``fma(x, y, z)`` when the mul has no other user.

    The first operand of the add that is defined by a ``mul`` is the candidate
    (reference ``compiler.py:1019-1096``); if that mul has other users nothing
    fuses.  This changes rounding (one rounding instead of two) and is the only
    source of FMAs besides ``mk.fma``: kernels are compiled with
    ``-ffp-contract=off``.
    """
    defs = _defs(ir)
    uses = _use_counts(ir.insts)
    dropped: set[int] = set()
    fused: list[Inst] = []
    for inst in ir.insts:
        if inst.op == "add" and inst.out is not None and inst.out.dtype == DType.F32:
            a, b = inst.args
            for m_ref, other in ((a, b), (b, a)):
                mul = defs.get(m_ref.id)
                if mul is not None and mul.op == "mul" and mul.out is not None:
                    if mul.out.dtype == DType.F32 and uses.get(mul.out.id, 0) == 1:
                        x, y = mul.args
                        fused.append(Inst("fma", inst.out, (x, y, other)))
                        dropped.add(mul.out.id)
                        break
                    fused.append(inst)
                    break
            else:
                fused.append(inst)
            continue
        fused.append(inst)
    out = [i for i in fused if not (i.op == "mul" and i.out is not None and i.out.id in dropped)]
    return IRModule(ir.name, ir.args, tuple(out))


def _fold_static_lts(ir: IRModule) -> IRModule:
    """Fold u32 ``lt`` to a constant when integer intervals decide it.

    Intervals come from u32 consts, ``arange``/``tid`` (``[start, start+size)``)
    and ``add``/``mul`` of intervals (reference ``compiler.py:658-795``).  Two
    deliberate differences keep the fold sound: ``thread_id`` (a global index)
    gets no interval, and an interval that could exceed 2^32 (u32 wraparound) is
    dropped.
    """
    iv: dict[int, tuple[int, int]] = {}
    for inst in ir.insts:
        out = inst.out
        if out is None or out.dtype != DType.U32 or out.id in iv:
            continue
        if inst.op == "const" and isinstance(inst.args[0], int) and not isinstance(inst.args[0], bool):
            iv[out.id] = (inst.args[0], inst.args[0])
        elif inst.op in ("arange", "tid"):
            start, size = int(inst.args[0]), int(inst.args[1])
            iv[out.id] = (start, start + size - 1)
        elif inst.op in ("add", "mul"):
            x, y = iv.get(inst.args[0].id), iv.get(inst.args[1].id)
            if x is None or y is None:
                continue
            if inst.op == "add":
                lo, hi = x[0] + y[0], x[1] + y[1]
            else:
                prods = (x[0] * y[0], x[0] * y[1], x[1] * y[0], x[1] * y[1])
                lo, hi = min(prods), max(prods)
            if hi < U32_LIMIT:
                iv[out.id] = (lo, hi)
    out_insts: list[Inst] = []
    for inst in ir.insts:
        if inst.op == "lt" and inst.out is not None:
            x, y = iv.get(inst.args[0].id), iv.get(inst.args[1].id)
            if x is not None and y is not None:
                if x[1] < y[0]:
                    out_insts.append(Inst("const", inst.out, (True,)))
                    continue
                if x[0] >= y[1]:
                    out_insts.append(Inst("const", inst.out, (False,)))
                    continue
        out_insts.append(inst)
    return IRModule(ir.name, ir.args, tuple(out_insts))


_KEEP_AS_IS = frozenset({"arg", "store", "load", "dot", "mma", "mma_store", "alloc_tg", "barrier"})


def _simplify_bools(ir: IRModule) -> IRModule:
    """Constant-fold boolean logic and lower bool ``where`` to ``and``/``or``.

    ``where(c, x, False) -> c && x``, ``where(c, True, b) -> c || b``, constant
    conditions select an operand, ``and``/``or``/``not`` with constant operands
    fold (reference ``compiler.py:798-934``).  Folding sees the constants this
    pass creates, and an operand is only substituted for a value of the same
    lane count.
    """
    remap = _Remap()
    consts: dict[int, bool] = {}
    out: list[Inst] = []

    def cbool(ref: ValueRef) -> bool | None:
        return consts.get(ref.id)

    def emit(inst: Inst) -> None:
        out.append(inst)
        if inst.op == "const" and inst.out is not None and isinstance(inst.args[0], bool):
            consts[inst.out.id] = inst.args[0]

    def alias(dst: ValueRef, src: ValueRef, fallback: Inst) -> None:
        if dst.lanes == src.lanes:
            remap.to[dst.id] = src
        else:
            emit(fallback)

    for inst in ir.insts:
        args = remap.args(inst)
        res = inst.out
        if inst.op in _KEEP_AS_IS or res is None:
            emit(Inst(inst.op, res, args))
            continue
        kept = Inst(inst.op, res, args)
        if inst.op == "where" and res.dtype == DType.BOOL:
            c, a, b = args
            cb, ab, bb = cbool(c), cbool(a), cbool(b)
            if cb is not None:
                alias(res, a if cb else b, kept)
            elif bb is False:
                if ab is True:
                    alias(res, c, kept)
                elif ab is False:
                    emit(Inst("const", res, (False,)))
                else:
                    emit(Inst("and", res, (c, a)))
            elif ab is True and bb is True:
                emit(Inst("const", res, (True,)))
            elif ab is True:
                emit(Inst("or", res, (c, b)))
            else:
                emit(kept)
            continue
        if inst.op in ("and", "or"):
            a, b = args
            av, bv = cbool(a), cbool(b)
            absorbing = inst.op == "or"  # True absorbs `or`, False absorbs `and`
            if av is absorbing or bv is absorbing:
                emit(Inst("const", res, (absorbing,)))
            elif av is not None:
                alias(res, b, kept)
            elif bv is not None:
                alias(res, a, kept)
            else:
                emit(kept)
            continue
        if inst.op == "not":
            xv = cbool(args[0])
            emit(Inst("const", res, (not xv,)) if xv is not None else kept)
            continue
        emit(kept)
    return IRModule(ir.name, ir.args, tuple(out))


def _cse_key(inst: Inst) -> tuple[Any, ...] | None:
    out = inst.out
    assert out is not None
    op, a = inst.op, inst.args
    head = (op, out.dtype, out.lanes)
    if op == "const":
        return head + (type(a[0]) is bool, a[0])
    if op in ("program_id", "thread_id", "local_id", "arange", "tid"):
        return head + tuple(int(x) for x in a)
    if op in ("lane_id", "sg_id"):
        return head
    if op in ("add", "mul", "and", "or"):
        return head + tuple(sorted((a[0].id, a[1].id)))
    if op in ("floordiv", "mod", "lt", "not", "where"):
        return head + tuple(x.id for x in a)
    if op == "cast":
        return head + (a[0].id, a[1])
    if op == "fma":
        return head + tuple(sorted((a[0].id, a[1].id))) + (a[2].id,)
    return None


def _cse_pure(ir: IRModule) -> IRModule:
    """Value-number pure instructions (commutative operands sorted) and reuse
    the first equivalent definition (reference ``compiler.py:1099-1200``)."""
    remap = _Remap()
    table: dict[tuple[Any, ...], ValueRef] = {}
    out: list[Inst] = []
    for inst in ir.insts:
        cur = Inst(inst.op, inst.out, remap.args(inst))
        if inst.op in _KEEP_AS_IS or inst.out is None:
            out.append(cur)
            continue
        key = _cse_key(cur)
        if key is not None:
            hit = table.get(key)
            if hit is not None:
                remap.to[inst.out.id] = hit
                continue
            table[key] = inst.out
        out.append(cur)
    return IRModule(ir.name, ir.args, tuple(out))


def _dce(ir: IRModule) -> IRModule:
    """Drop values that no store, ``mma_store`` or kept id depends on.

    ``arg``, ``arange``, ``tid``, ``store``, ``barrier`` and ``mma_store`` always
    stay: ``arange``/``tid`` define the launch shape even when unused
    (reference ``compiler.py:1203-1272``).
    """
    defs = _defs(ir)
    live: set[int] = set()
    work: list[ValueRef] = []
    for inst in ir.insts:
        if inst.op in ("store", "mma_store"):
            work.extend(a for a in inst.args if isinstance(a, ValueRef))
        elif inst.op in ("arg", "arange", "tid") and inst.out is not None:
            work.append(inst.out)
    while work:
        ref = work.pop()
        if ref.id in live:
            continue
        live.add(ref.id)
        d = defs.get(ref.id)
        if d is not None:
            work.extend(a for a in d.args if isinstance(a, ValueRef) and a.id not in live)
    keep_ops = ("arg", "store", "arange", "tid", "barrier")
    out = [i for i in ir.insts if i.op in keep_ops or i.out is None or i.out.id in live]
    return IRModule(ir.name, ir.args, tuple(out))


PASSES: tuple[Callable[[IRModule], IRModule], ...] = (
    _rewrite_thread_id,
    _fuse_fma,
    _fold_static_lts,
    _simplify_bools,
    _cse_pure,
    _dce,
)


def optimize_ir(ir: IRModule) -> IRModule:
    for p in PASSES:
        ir = p(ir)
    return ir


_optimize_ir = optimize_ir


# ---------------------------------------------------------------------------
# compile
# ---------------------------------------------------------------------------


@dataclass(frozen=True, slots=True)
class CompiledKernel:
    """A traced, optimised and lowered kernel specialisation.

    ``src`` is gfx950 HIP C++ (the reference's field is ``msl``); ``geometry``
    tells the runtime how the reference's launch grid maps onto HIP blocks.
    """

    ir: IRModule
    src: str
    block_size: int
    launch_mode: str
    writes: frozenset[str]
    geometry: Any = field(default=None, compare=False)


def compile(fn: Callable[..., Any], runtime_args: Mapping[str, Any], meta: Mapping[str, Any]) -> CompiledKernel:
    ir = optimize_ir(trace_to_ir(fn, runtime_args, meta))
    validate_ir(ir)
    from .codegen.hip import ir_to_hip

    lowered = ir_to_hip(ir)
    return CompiledKernel(
        ir=ir,
        src=lowered.src,
        block_size=int(lowered.block_size),
        launch_mode=str(lowered.launch_mode),
        writes=infer_writes(ir),
        geometry=lowered.geometry,
    )
