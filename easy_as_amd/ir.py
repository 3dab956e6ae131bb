"""eas IR: dtypes, SSA values, instructions, modules and the verifier.

The IR is the contract between the tracer (``compiler.py``) and the gfx950
emitter (``codegen/hip.py``).  Its types, op set and typing rules are the
reference's (``eas/ir.py:10-83`` for the data model, ``eas/ir.py:86-518`` for
the rules ``validate_ir`` enforces), so kernels trace to the same IR.  One
addition: the ``bf16`` dtype (buffers, threadgroup arrays, casts, MMA operands).
The verifier here is table driven: every op maps to one checker function.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Any, Callable, Iterable, Literal, TypeAlias


class DType(str, Enum):
    BOOL = "bool"
    F16 = "f16"
    # bfloat16: an addition to the reference's dtypes (buffers from torch.bfloat16
    # tensors, threadgroup tiles, casts and MMA operands); values convert to f32
    # for arithmetic and round back to nearest-even.
    BF16 = "bf16"
    F32 = "f32"
    U32 = "u32"
    # Opaque 8x8 f32 matrix fragment owned by one 32-lane simdgroup.
    SG_F32_8X8 = "sg_f32_8x8"


ArgKind: TypeAlias = Literal["buffer", "scalar"]

Op: TypeAlias = Literal[
    "arg",
    "const",
    "program_id",
    "thread_id",
    "local_id",
    "lane_id",
    "sg_id",
    "arange",
    "tid",
    "alloc_tg",
    "add",
    "mul",
    "floordiv",
    "mod",
    "lt",
    "and",
    "or",
    "not",
    "where",
    "cast",
    "dot",
    "mma_zero",
    "mma",
    "mma_store",
    "load",
    "store",
    "fma",
    "barrier",
]

ALL_OPS: frozenset[str] = frozenset(Op.__args__)  # type: ignore[attr-defined]


@dataclass(frozen=True, slots=True)
class ValueRef:
    id: int
    dtype: DType
    lanes: int = 1


@dataclass(frozen=True, slots=True)
class Arg:
    name: str
    dtype: DType
    kind: ArgKind


@dataclass(frozen=True, slots=True)
class Inst:
    op: Op
    out: ValueRef | None
    args: tuple[Any, ...]


@dataclass(frozen=True, slots=True)
class IRModule:
    name: str
    args: tuple[Arg, ...]
    insts: tuple[Inst, ...]

    def buffer_args(self) -> Iterable[Arg]:
        return (arg for arg in self.args if arg.kind == "buffer")

    def scalar_args(self) -> Iterable[Arg]:
        return (arg for arg in self.args if arg.kind == "scalar")


NUMERIC = (DType.U32, DType.F16, DType.BF16, DType.F32)
FLOATS = (DType.F16, DType.BF16, DType.F32)
CASTABLE = (DType.BOOL, DType.U32, DType.F16, DType.BF16, DType.F32)


def broadcast(a: int, b: int) -> int | None:
    """Lane count of a binary op over operands of ``a`` and ``b`` lanes (1 broadcasts)."""
    if a == b or b == 1:
        return a
    if a == 1:
        return b
    return None


class _Verifier:
    """State of one ``validate_ir`` walk (definitions seen so far, buffer ids)."""

    def __init__(self, ir: IRModule) -> None:
        self.ir = ir
        self.args_by_name = {a.name: a for a in ir.args}
        self.seen_args: set[str] = set()
        self.defined: dict[int, ValueRef] = {}
        self.buffers: set[int] = set()

    # -- helpers ---------------------------------------------------------
    @staticmethod
    def check(cond: bool, msg: str) -> None:
        if not cond:
            raise ValueError(f"invalid IR: {msg}")

    def define(self, ref: ValueRef) -> None:
        self.check(ref.id not in self.defined, f"duplicate SSA value id: {ref.id}")
        self.check(isinstance(ref.dtype, DType), f"invalid dtype for v{ref.id}: {ref.dtype!r}")
        self.check(isinstance(ref.lanes, int) and ref.lanes >= 1, f"invalid lanes for v{ref.id}: {ref.lanes!r}")
        self.defined[ref.id] = ref

    def use(self, x: Any, what: str) -> ValueRef:
        self.check(isinstance(x, ValueRef), f"{what} must be a ValueRef, got {type(x)!r}")
        d = self.defined.get(x.id)
        self.check(d is not None, f"use of undefined value id {x.id} for {what}")
        assert d is not None
        self.check(d.dtype == x.dtype, f"{what} dtype mismatch for v{x.id}: {d.dtype} vs {x.dtype}")
        self.check(d.lanes == x.lanes, f"{what} lanes mismatch for v{x.id}: {d.lanes} vs {x.lanes}")
        return x

    def nargs(self, inst: Inst, n: int) -> None:
        self.check(len(inst.args) == n, f"{inst.op} expects {n} args, got {len(inst.args)}")

    def out(self, inst: Inst) -> ValueRef:
        self.check(inst.out is not None, f"{inst.op} must produce a value")
        assert inst.out is not None
        return inst.out

    def no_out(self, inst: Inst) -> None:
        self.check(inst.out is None, f"{inst.op} must not produce a value")

    def lanes2(self, a: ValueRef, b: ValueRef, what: str) -> int:
        n = broadcast(a.lanes, b.lanes)
        if n is None:
            raise ValueError(f"invalid IR: {what} lanes mismatch: {a.lanes} vs {b.lanes} (no broadcast)")
        return n

    def buffer(self, x: Any, what: str) -> ValueRef:
        ref = self.use(x, what)
        self.check(ref.id in self.buffers, f"{what} must be a buffer (arg or alloc_tg)")
        return ref

    def scalar_u32(self, x: Any, what: str) -> ValueRef:
        ref = self.use(x, what)
        self.check(ref.dtype == DType.U32, f"{what} must be u32")
        self.check(ref.lanes == 1, f"{what} must be scalar (lanes=1)")
        return ref

    # -- per-op rules ----------------------------------------------------
    def op_arg(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 3)
        name, kind, dtype = str(inst.args[0]), inst.args[1], inst.args[2]
        decl = self.args_by_name.get(name)
        self.check(decl is not None, f"arg references unknown name {name!r}")
        assert decl is not None
        self.check(kind == decl.kind, f"arg kind mismatch for {name!r}")
        self.check(dtype == decl.dtype, f"arg dtype mismatch for {name!r}")
        self.check(name not in self.seen_args, f"duplicate arg inst for {name!r}")
        self.seen_args.add(name)
        self.define(out)
        if decl.kind == "buffer":
            self.buffers.add(out.id)

    def op_const(self, inst: Inst) -> None:
        out = self.out(inst)
        self.check(out.lanes == 1, "const output lanes must be 1")
        self.nargs(inst, 1)
        v = inst.args[0]
        if out.dtype == DType.BOOL:
            self.check(isinstance(v, bool), "bool const must be a Python bool")
        elif out.dtype == DType.U32:
            self.check(isinstance(v, int) and not isinstance(v, bool) and v >= 0,
                       "u32 const must be a non-negative Python int")
        elif out.dtype == DType.F32:
            self.check(isinstance(v, (int, float)), "f32 const must be an int/float")
        else:
            self.check(False, f"unsupported const dtype: {out.dtype}")
        self.define(out)

    def op_alloc_tg(self, inst: Inst) -> None:
        out = self.out(inst)
        self.check(out.lanes == 1, "alloc_tg output lanes must be 1")
        self.nargs(inst, 1)
        size = inst.args[0]
        self.check(isinstance(size, int) and size > 0, "alloc_tg(size) requires a positive Python int size")
        self.check(out.dtype in FLOATS, f"alloc_tg output must be f16/bf16/f32, got {out.dtype}")
        self.define(out)
        self.buffers.add(out.id)

    def op_axis_id(self, inst: Inst) -> None:
        out = self.out(inst)
        self.check(out.lanes == 1, f"{inst.op} output lanes must be 1")
        self.check(out.dtype == DType.U32, f"{inst.op} output must be u32")
        self.nargs(inst, 1)
        self.check(isinstance(inst.args[0], int) and inst.args[0] in (0, 1, 2), f"{inst.op} axis must be 0/1/2")
        self.define(out)

    def op_lane_sg(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 0)
        self.check(out.dtype == DType.U32, f"{inst.op} output must be u32")
        self.check(out.lanes == 1, f"{inst.op} output lanes must be 1")
        self.define(out)

    def op_range(self, inst: Inst) -> None:
        out = self.out(inst)
        self.check(out.dtype == DType.U32, f"{inst.op} output must be u32")
        self.nargs(inst, 2)
        start, size = inst.args
        self.check(isinstance(start, int) and isinstance(size, int),
                   f"{inst.op}(start, size) requires Python int literals")
        self.check(size > 0, f"{inst.op}(size) must be > 0")
        want = size if inst.op == "arange" else 1
        self.check(out.lanes == want, f"{inst.op} output lanes must be {want}")
        self.define(out)

    def op_arith(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 2)
        a = self.use(inst.args[0], f"{inst.op} lhs")
        b = self.use(inst.args[1], f"{inst.op} rhs")
        self.check(a.dtype == b.dtype, f"{inst.op} dtype mismatch: {a.dtype} vs {b.dtype}")
        self.check(a.dtype in NUMERIC, f"{inst.op} operands must be u32/f16/bf16/f32, got {a.dtype}")
        self.check(out.dtype == a.dtype, f"{inst.op} output dtype must match operands")
        self.check(out.lanes == self.lanes2(a, b, f"{inst.op} operands"), f"{inst.op} output lanes must broadcast operands")
        if inst.op in ("floordiv", "mod"):
            self.check(a.dtype == DType.U32, f"{inst.op} operands must be u32")
        self.define(out)

    def op_lt(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 2)
        a = self.use(inst.args[0], "lt lhs")
        b = self.use(inst.args[1], "lt rhs")
        self.check(a.dtype == b.dtype, f"lt dtype mismatch: {a.dtype} vs {b.dtype}")
        self.check(a.dtype in NUMERIC, f"lt operands must be u32/f16/bf16/f32, got {a.dtype}")
        self.check(out.dtype == DType.BOOL, "lt output must be bool")
        self.check(out.lanes == self.lanes2(a, b, "lt operands"), "lt output lanes mismatch")
        self.define(out)

    def op_logic(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 2)
        a = self.use(inst.args[0], f"{inst.op} lhs")
        b = self.use(inst.args[1], f"{inst.op} rhs")
        self.check(out.dtype == DType.BOOL, f"{inst.op} output must be bool")
        self.check(a.dtype == DType.BOOL and b.dtype == DType.BOOL, f"{inst.op} operands must be bool")
        self.check(out.lanes == self.lanes2(a, b, f"{inst.op} operands"), f"{inst.op} output lanes mismatch")
        self.define(out)

    def op_not(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 1)
        x = self.use(inst.args[0], "not input")
        self.check(out.dtype == DType.BOOL and x.dtype == DType.BOOL, "not input/output must be bool")
        self.check(out.lanes == x.lanes, "not output lanes must match input")
        self.define(out)

    def op_where(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 3)
        c = self.use(inst.args[0], "where cond")
        a = self.use(inst.args[1], "where a")
        b = self.use(inst.args[2], "where b")
        self.check(c.dtype == DType.BOOL, "where cond must be bool")
        self.check(a.dtype == b.dtype, f"where dtype mismatch: {a.dtype} vs {b.dtype}")
        self.check(out.dtype == a.dtype, "where output dtype must match values")
        n = self.lanes2(a, b, "where values")
        n2 = broadcast(c.lanes, n)
        if n2 is None:
            raise ValueError(f"invalid IR: where cond vs values lanes mismatch: {c.lanes} vs {n} (no broadcast)")
        self.check(out.lanes == n2, "where output lanes mismatch")
        self.define(out)

    def op_cast(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 2)
        x = self.use(inst.args[0], "cast input")
        dst = inst.args[1]
        self.check(isinstance(dst, DType), "cast target must be a DType")
        self.check(out.dtype == dst, "cast output dtype must match target dtype")
        self.check(out.lanes == x.lanes, "cast output lanes must match input")
        self.check(x.dtype in CASTABLE and dst in CASTABLE, "cast only supports bool/u32/f16/bf16/f32")
        self.define(out)

    def op_fma(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 3)
        x = self.use(inst.args[0], "fma x")
        y = self.use(inst.args[1], "fma y")
        z = self.use(inst.args[2], "fma z")
        self.check(x.dtype == y.dtype == z.dtype, "fma operands must have same dtype")
        self.check(x.dtype in FLOATS, f"fma operands must be f16/bf16/f32, got {x.dtype}")
        self.check(out.dtype == x.dtype, "fma output dtype must match operands")
        n = self.lanes2(x, y, "fma x/y")
        n2 = broadcast(z.lanes, n)
        if n2 is None:
            raise ValueError(f"invalid IR: fma z vs x/y lanes mismatch: {z.lanes} vs {n} (no broadcast)")
        self.check(out.lanes == n2, "fma output lanes mismatch")
        self.define(out)

    def op_load(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 3)
        buf = self.buffer(inst.args[0], "load buffer")
        off = self.use(inst.args[1], "load offset")
        mask = self.use(inst.args[2], "load mask")
        self.check(buf.dtype in FLOATS, f"load buffer dtype must be f16/bf16/f32, got {buf.dtype}")
        self.check(off.dtype == DType.U32, "load offset must be u32")
        self.check(mask.dtype == DType.BOOL, "load mask must be bool")
        self.check(out.dtype == buf.dtype, "load output dtype must match buffer dtype")
        self.check(out.lanes == off.lanes, "load output lanes must match offset lanes")
        self.check(mask.lanes in (1, off.lanes), "load mask lanes must be 1 or match offset lanes")
        self.define(out)

    def op_store(self, inst: Inst) -> None:
        self.no_out(inst)
        self.nargs(inst, 4)
        buf = self.buffer(inst.args[0], "store buffer")
        off = self.use(inst.args[1], "store offset")
        val = self.use(inst.args[2], "store value")
        mask = self.use(inst.args[3], "store mask")
        self.check(buf.dtype in FLOATS, f"store buffer dtype must be f16/bf16/f32, got {buf.dtype}")
        self.check(off.dtype == DType.U32, "store offset must be u32")
        self.check(mask.dtype == DType.BOOL, "store mask must be bool")
        self.check(val.dtype == buf.dtype, "store value dtype must match buffer dtype")
        self.check(val.lanes in (1, off.lanes), "store value lanes must be 1 or match offset lanes")
        self.check(mask.lanes in (1, off.lanes), "store mask lanes must be 1 or match offset lanes")

    def op_dot(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 7)
        a_buf, a_base, a_stride, b_buf, b_base, b_stride, k = inst.args
        for ref, what in ((a_buf, "dot a_buffer"), (b_buf, "dot b_buffer")):
            r = self.buffer(ref, what)
            self.check(r.dtype in FLOATS, f"{what} must be f16/bf16/f32")
        for ref, what in ((a_base, "dot a_base"), (a_stride, "dot a_stride"), (b_base, "dot b_base"),
                          (b_stride, "dot b_stride"), (k, "dot K")):
            self.scalar_u32(ref, what)
        self.check(out.dtype == DType.F32, "dot output must be f32")
        self.check(out.lanes == 1, "dot output lanes must be 1")
        self.define(out)

    def op_mma_zero(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 0)
        self.check(out.dtype == DType.SG_F32_8X8, "mma_zero currently produces sg_f32_8x8 only")
        self.check(out.lanes == 1, "mma_zero output lanes must be 1")
        self.define(out)

    def op_mma(self, inst: Inst) -> None:
        out = self.out(inst)
        self.nargs(inst, 7)
        a_buf, a_base, a_stride, b_buf, b_base, b_stride, acc = inst.args
        bufs = []
        for ref, what in ((a_buf, "mma a_buffer"), (b_buf, "mma b_buffer")):
            r = self.buffer(ref, what)
            self.check(r.dtype in FLOATS, f"{what} must be f16/bf16/f32")
            bufs.append(r.dtype)
        # bf16 fragments multiply bf16 fragments only: the MFMA takes one operand type
        self.check((DType.BF16 in bufs) <= (bufs[0] == bufs[1]), "mma a/b buffers must both be bf16 or neither")
        for ref, what in ((a_base, "mma a_base"), (a_stride, "mma a_stride"), (b_base, "mma b_base"),
                          (b_stride, "mma b_stride")):
            self.scalar_u32(ref, what)
        acc_ref = self.use(acc, "mma acc")
        self.check(acc_ref.dtype == DType.SG_F32_8X8 and acc_ref.lanes == 1, "mma acc must be a scalar sg_f32_8x8")
        self.check(out.dtype == DType.SG_F32_8X8 and out.lanes == 1, "mma currently produces sg_f32_8x8 only")
        self.define(out)

    def op_mma_store(self, inst: Inst) -> None:
        self.no_out(inst)
        self.nargs(inst, 4)
        c_buf, c_base, c_stride, frag = inst.args
        c = self.buffer(c_buf, "mma_store c_buffer")
        self.check(c.dtype == DType.F32, "mma_store c_buffer must be f32")
        self.scalar_u32(c_base, "mma_store c_base")
        self.scalar_u32(c_stride, "mma_store c_stride")
        f = self.use(frag, "mma_store frag")
        self.check(f.dtype == DType.SG_F32_8X8 and f.lanes == 1, "mma_store frag must be a scalar sg_f32_8x8")

    def op_barrier(self, inst: Inst) -> None:
        self.no_out(inst)
        self.nargs(inst, 0)

    def run(self) -> None:
        for inst in self.ir.insts:
            rule = _RULES.get(inst.op)
            self.check(rule is not None, f"unknown op: {inst.op!r}")
            assert rule is not None
            rule(self, inst)
        missing = set(self.args_by_name) - self.seen_args
        self.check(not missing, "missing arg inst(s): " + ", ".join(sorted(missing)))


_RULES: dict[str, Callable[[_Verifier, Inst], None]] = {
    "arg": _Verifier.op_arg,
    "const": _Verifier.op_const,
    "alloc_tg": _Verifier.op_alloc_tg,
    "program_id": _Verifier.op_axis_id,
    "thread_id": _Verifier.op_axis_id,
    "local_id": _Verifier.op_axis_id,
    "lane_id": _Verifier.op_lane_sg,
    "sg_id": _Verifier.op_lane_sg,
    "arange": _Verifier.op_range,
    "tid": _Verifier.op_range,
    "add": _Verifier.op_arith,
    "mul": _Verifier.op_arith,
    "floordiv": _Verifier.op_arith,
    "mod": _Verifier.op_arith,
    "lt": _Verifier.op_lt,
    "and": _Verifier.op_logic,
    "or": _Verifier.op_logic,
    "not": _Verifier.op_not,
    "where": _Verifier.op_where,
    "cast": _Verifier.op_cast,
    "fma": _Verifier.op_fma,
    "load": _Verifier.op_load,
    "store": _Verifier.op_store,
    "dot": _Verifier.op_dot,
    "mma_zero": _Verifier.op_mma_zero,
    "mma": _Verifier.op_mma,
    "mma_store": _Verifier.op_mma_store,
    "barrier": _Verifier.op_barrier,
}


def validate_ir(ir: IRModule) -> None:
    """Raise ``ValueError("invalid IR: ...")`` unless ``ir`` is well formed.

    Rules follow ``eas/ir.py:86-518`` of the reference: SSA single definition,
    dtype/lane agreement at every use, 1-vs-L lane broadcasting, buffers are
    args or ``alloc_tg`` results, ``mma_store`` targets f32 buffers only.
    """
    _Verifier(ir).run()
