"""Thread-mode kernels that are plain element streams, emitted as lanes of one program per threadgroup.

A thread-mode kernel (``mk.tid``) runs one Metal thread per element (reference ``msl.py:353-1022``):
emitted one HIP thread per Metal thread, each stream moves 4 bytes per lane, which caps such a
kernel near 73 % of HBM on MI355X (the reference's own fma kernel, ``tests/test_fma.py:13-23``,
at N = 2^28).  When the kernel uses nothing that ties a Metal thread to a HIP thread (no barrier,
threadgroup memory, local/lane/simdgroup id, dot or MMA), the threads of one threadgroup are
independent element computations, and the SPMD emitter's mapping applies: the threadgroup
becomes a program of BLOCK lanes (``tid`` becomes ``arange``, ``thread_id(0)`` becomes
``program_id(0) * BLOCK + arange``; a thread's position in its threadgroup is its lane, so
``local_id(0)`` is the lane, ``lane_id`` the lane mod 32 and ``sg_id`` the lane / 32, the
32-lane simdgroups of the Metal model), each HIP thread carries 16-byte vectors of several lanes,
and small workgroups keep every HBM stream in short chunks.

What a launch means does not change: the grid counts threadgroups (or a 1-D thread count), the
threads per threadgroup must be (BLOCK, 1, 1), and only the first ``__eas_nthreads`` threads
along x exist.  That count is the kernel's hidden argument, as for the one-thread-per-thread
emitter; every lane-varying load and store is masked with ``x < __eas_nthreads`` (x the Metal
thread's global index), so the lanes past the count read and write nothing.  Accesses at an
offset that is the same for every thread of a threadgroup are performed once per program.  That
program runs only when its first thread exists, and that thread would perform the access too.

``EAS_HIP_THREAD_LANES=0`` keeps every thread-mode kernel on the one-thread-per-thread emitter.
"""

from __future__ import annotations

import os

from ..ir import Arg, DType, Inst, IRModule, ValueRef, validate_ir

# ops a Metal thread of such a kernel may use: element arithmetic, its ids, its own loads/stores
_ALLOWED = frozenset({"arg", "const", "tid", "thread_id", "program_id", "local_id", "lane_id", "sg_id", "add",
                      "mul", "floordiv", "mod", "lt", "and", "or", "not", "where", "cast", "fma", "load", "store"})
# each lane-varying instruction is emitted once per lane a HIP thread carries
_MAX_INSTS = 256
NTHREADS = "__eas_nthreads"


def enabled() -> bool:
    """``EAS_HIP_THREAD_LANES``: 1 (default) or 0, read each time a source is emitted."""
    v = os.environ.get("EAS_HIP_THREAD_LANES", "1").strip() or "1"
    if v not in ("0", "1"):
        raise ValueError(f"EAS_HIP_THREAD_LANES must be 0 or 1, got {v!r}")
    return v == "1"


def as_lanes(ir: IRModule, block: int) -> IRModule | None:
    """The program-of-lanes form of thread-mode ``ir`` (one program per threadgroup of ``block``
    threads, an extra u32 argument ``__eas_nthreads`` last), or None when the kernel does not
    qualify.  That is when it uses an op outside the element-stream set (a barrier,
    threadgroup memory, dot or MMA), is longer than the emitter unrolls, has no lane-varying
    store, or reads or writes a shared address under a per-thread mask or value."""
    if not enabled() or block < 2 or block > 1024 or len(ir.insts) > _MAX_INSTS:
        return None  # (a BLOCK above 1024 is the thread emitter's error to raise)
    if any(i.op not in _ALLOWED for i in ir.insts) or any(a.name == NTHREADS for a in ir.args):
        return None
    next_id = 1 + max((r.id for i in ir.insts for r in (i.out, *i.args) if isinstance(r, ValueRef)), default=-1)

    def fresh(dtype: DType, lanes: int) -> ValueRef:
        nonlocal next_id
        ref = ValueRef(next_id, dtype, lanes)
        next_id += 1
        return ref

    insts: list[Inst] = []
    c32 = fresh(DType.U32, 1)
    c0 = fresh(DType.U32, 1)
    nth = fresh(DType.U32, 1)
    pid = fresh(DType.U32, 1)
    cb = fresh(DType.U32, 1)
    base = fresh(DType.U32, 1)
    lane = fresh(DType.U32, block)
    x = fresh(DType.U32, block)
    live = fresh(DType.BOOL, block)
    head = [Inst("arg", nth, (NTHREADS, "scalar", DType.U32)),
            Inst("program_id", pid, (0,)),
            Inst("const", cb, (block,)),
            Inst("mul", base, (pid, cb)),
            Inst("arange", lane, (0, block)),
            Inst("add", x, (base, lane)),
            Inst("lt", live, (x, nth)),
            Inst("const", c32, (32,)),
            Inst("const", c0, (0,))]
    new: dict[int, ValueRef] = {}
    consts_true: set[int] = set()
    live_masks: dict[int, ValueRef] = {}  # mask id -> mask && live, made once

    def m(a):
        return new[a.id] if isinstance(a, ValueRef) else a

    def masked(mask: ValueRef) -> ValueRef:
        if mask.id in consts_true:
            return live
        out = live_masks.get(mask.id)
        if out is None:
            out = live_masks[mask.id] = fresh(DType.BOOL, block)
            insts.append(Inst("and", out, (mask, live)))
        return out

    lane_store = False
    for inst in ir.insts:
        op, out = inst.op, inst.out
        args = tuple(m(a) for a in inst.args)
        if op == "arg":
            new[out.id] = out
            insts.append(inst)
            continue
        if op == "tid":
            ref = ValueRef(out.id, DType.U32, block)
            insts.append(Inst("arange", ref, (int(inst.args[0]), block)))
            new[out.id] = ref
            continue
        if op in ("local_id", "lane_id", "sg_id"):
            if op == "local_id" and int(inst.args[0]) != 0:  # threadgroups are (BLOCK, 1, 1)
                ref = ValueRef(out.id, DType.U32, 1)
                insts.append(Inst("const", ref, (0,)))
            else:  # the lane (its own SSA value: lane + 0), lane mod 32, lane / 32
                ref = ValueRef(out.id, DType.U32, block)
                src = {"local_id": ("add", c0), "lane_id": ("mod", c32), "sg_id": ("floordiv", c32)}[op]
                insts.append(Inst(src[0], ref, (lane, src[1])))
            new[out.id] = ref
            continue
        if op == "thread_id":
            d = int(inst.args[0])
            if d == 0:
                new[out.id] = x
            else:  # one thread per threadgroup along y and z: the threadgroup's index
                ref = ValueRef(out.id, DType.U32, 1)
                insts.append(Inst("program_id", ref, (d,)))
                new[out.id] = ref
            continue
        if op == "load":
            buf, off, mask = args
            if off.lanes > 1:
                mask = masked(mask)
            elif mask.lanes > 1:  # a shared address under a per-thread mask: not a stream
                return None
            ref = ValueRef(out.id, out.dtype, off.lanes)
            insts.append(Inst("load", ref, (buf, off, mask)))
            new[out.id] = ref
            continue
        if op == "store":
            buf, off, val, mask = args
            if off.lanes > 1:
                insts.append(Inst("store", None, (buf, off, val, masked(mask))))
                lane_store = True
            elif val.lanes > 1 or mask.lanes > 1:
                return None
            else:
                insts.append(Inst("store", None, args))
            continue
        lanes = max((a.lanes for a in args if isinstance(a, ValueRef)), default=1)
        ref = None if out is None else ValueRef(out.id, out.dtype, lanes)
        if op == "const" and inst.args[0] is True:
            consts_true.add(out.id)
        insts.append(Inst(op, ref, args))
        if ref is not None:
            new[out.id] = ref
    if not lane_store:
        return None
    first_op = next((k for k, i in enumerate(insts) if i.op != "arg"), len(insts))
    lanes_ir = IRModule(ir.name, ir.args + (Arg(NTHREADS, DType.U32, "scalar"),),
                        tuple(insts[:first_op] + head + insts[first_op:]))
    try:
        validate_ir(lanes_ir)
    except ValueError:  # a form this conversion does not cover: the thread emitter takes the kernel
        return None
    return lanes_ir
