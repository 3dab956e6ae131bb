"""Oracle: a numpy interpreter of eas kernels with the reference's semantics.

TEST INFRASTRUCTURE ONLY (imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg as the checker; never by the product).

``run_kernel(kernel, *args, **meta_and_options)`` traces the kernel with the
backend's tracer but executes the *unoptimised* trace, applying on its own the
one pass of the reference that changes results — FMA fusion
(eas/compiler.py:1019-1096: an f32 ``add`` whose first ``mul``-defined operand
is a single-use f32 ``mul`` becomes one correctly rounded fma).  Every other
reference pass is value-preserving, so the backend's pass pipeline is checked
rather than trusted.

Execution model restated from the reference:

* SPMD (``mk.arange``): one program per Metal thread with BLOCK lanes
  (eas/codegen/msl.py:98-350); masked loads give 0, masked stores write nothing.
* thread mode (``mk.tid``): threadgroups of BLOCK threads; a 1-D launch without
  ``_grid`` starts exactly N threads (Metal ``dispatchThreads``,
  eas/runtime/metal.py:286-288); ``lane_id = local % 32``, ``sg_id = local // 32``
  (tests/test_local_and_lane_id.py:53,73); ``dot`` is one fma per k, k ascending
  from 0.0 (msl.py:920-952); ``mma`` is ``acc + A(8x8) @ B(8x8)`` per 32-lane
  simdgroup with A/B row-major at base/stride (msl.py:953-1002; summation order
  unspecified by Metal, so it is evaluated in float64 and rounded once).
* The IR is straight-line, so executing each instruction for all threads in
  lockstep is a valid schedule for any race-free kernel; barriers are no-ops.
* Launch geometry follows eas/runtime/grid.py:11-130 and metal.py:256-326.
"""

from __future__ import annotations

from typing import Any, Mapping

import numpy as np

from . import ops

_NP = {"f32": np.float32, "f16": np.float16, "u32": np.uint32, "bool": np.bool_}


class OracleError(RuntimeError):
    pass


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _fusable_adds(insts: tuple) -> dict[int, tuple]:
    """out-id of an ``add`` -> (x, y, z) operand refs it computes as fma(x, y, z)."""
    defs = {i.out.id: i for i in insts if i.out is not None}
    uses: dict[int, int] = {}
    for i in insts:
        for a in i.args:
            if hasattr(a, "id") and hasattr(a, "lanes"):
                uses[a.id] = uses.get(a.id, 0) + 1
    fused = {}
    for i in insts:
        if i.op != "add" or i.out is None or i.out.dtype.value != "f32":
            continue
        a, b = i.args
        for m, other in ((a, b), (b, a)):
            d = defs.get(m.id)
            if d is not None and d.op == "mul":
                if d.out.dtype.value == "f32" and uses.get(m.id, 0) == 1:
                    fused[i.out.id] = (d.args[0], d.args[1], other)
                break
    return fused


class _Exec:
    def __init__(self, ir: Any, mode: str, block: int, nthreads_total: int, groups: tuple[int, int, int],
                 live_threads: int | None, buffers: dict[str, np.ndarray], scalars: dict[str, Any]) -> None:
        self.ir = ir
        self.mode = mode
        self.block = block
        gx, gy, gz = groups
        if mode == "spmd":
            n = gx * gy * gz
            idx = np.arange(n)
            self.pid = (idx % gx, (idx // gx) % gy, idx // (gx * gy))
            self.lanes = block
            self.exists = np.ones((n, 1), bool)
            self.group = idx  # each program owns its own threadgroup memory
            self.ngroups = n
        else:
            n = gx * gy * gz * block
            idx = np.arange(n)
            g = idx // block
            self.local = idx % block
            self.pid = (g % gx, (g // gx) % gy, g // (gx * gy))
            self.lanes = 1
            self.group = g
            self.ngroups = gx * gy * gz
            gid_x = self.pid[0] * block + self.local
            live = np.ones(n, bool) if live_threads is None else gid_x < live_threads
            self.exists = live[:, None]
        self.n = n
        self.vals: dict[int, Any] = {}
        self.buffers = buffers
        self.scalars = scalars
        self.tg: dict[int, np.ndarray] = {}
        self.fused = _fusable_adds(ir.insts)

    # -- helpers --------------------------------------------------------------
    def col(self, x: np.ndarray) -> np.ndarray:
        return np.asarray(x).reshape(self.n, 1)

    def v(self, ref: Any) -> np.ndarray:
        return self.vals[ref.id]

    def bcast(self, *arrs: np.ndarray) -> list[np.ndarray]:
        return list(np.broadcast_arrays(*arrs))

    def _target(self, buf_ref: Any) -> tuple[np.ndarray, bool]:
        if buf_ref.id in self.tg:
            return self.tg[buf_ref.id], True
        return self.vals[buf_ref.id], False

    def gather(self, buf_ref: Any, off: np.ndarray, mask: np.ndarray, dtype: Any) -> np.ndarray:
        data, is_tg = self._target(buf_ref)
        off, mask = self.bcast(off, mask & self.exists)
        out = np.zeros(off.shape, dtype=dtype)
        rows = np.broadcast_to(self.col(self.group), off.shape)
        sel = mask
        o = off[sel].astype(np.int64)
        limit = data.shape[1] if is_tg else data.size
        if o.size and (o.max() >= limit):
            raise OracleError(f"out-of-bounds load at offset {int(o.max())} (size {limit})")
        out[sel] = data[rows[sel], o] if is_tg else data[o]
        return out

    def scatter(self, buf_ref: Any, off: np.ndarray, val: np.ndarray, mask: np.ndarray) -> None:
        data, is_tg = self._target(buf_ref)
        off, val, mask = self.bcast(off, val, mask & self.exists)
        sel = mask
        o = off[sel].astype(np.int64)
        limit = data.shape[1] if is_tg else data.size
        if o.size and o.max() >= limit:
            raise OracleError(f"out-of-bounds store at offset {int(o.max())} (size {limit})")
        if is_tg:
            rows = np.broadcast_to(self.col(self.group), off.shape)
            data[rows[sel], o] = val[sel]
        else:
            data[o] = val[sel]

    # -- execution ---------------------------------------------------------------
    def run(self) -> None:
        with np.errstate(all="ignore"):
            for inst in self.ir.insts:
                self.step(inst)

    def step(self, inst: Any) -> None:
        op, out, a = inst.op, inst.out, inst.args
        V = self.v
        if op == "arg":
            name, kind, _ = a
            if kind == "buffer":
                self.vals[out.id] = self.buffers[name]
            else:
                self.vals[out.id] = np.full((self.n, 1), self.scalars[name], dtype=_NP[out.dtype.value])
            return
        if op == "const":
            self.vals[out.id] = np.full((self.n, 1), a[0], dtype=_NP[out.dtype.value])
            return
        if op == "alloc_tg":
            self.tg[out.id] = np.zeros((self.ngroups, int(a[0])), dtype=_NP[out.dtype.value])
            self.vals[out.id] = None
            return
        if op == "program_id":
            self.vals[out.id] = self.col(self.pid[int(a[0])]).astype(np.uint32)
            return
        if op == "thread_id":
            ax = int(a[0])
            base = self.pid[ax] * (self.block if ax == 0 and self.mode == "thread" else 1)
            extra = self.local if ax == 0 and self.mode == "thread" else 0
            self.vals[out.id] = self.col(base + extra).astype(np.uint32)
            return
        if op == "local_id":
            self.vals[out.id] = self.col(self.local if int(a[0]) == 0 else np.zeros(self.n)).astype(np.uint32)
            return
        if op == "lane_id":
            self.vals[out.id] = self.col(self.local % 32).astype(np.uint32)
            return
        if op == "sg_id":
            self.vals[out.id] = self.col(self.local // 32).astype(np.uint32)
            return
        if op == "tid":
            self.vals[out.id] = self.col(self.local + int(a[0])).astype(np.uint32)
            return
        if op == "arange":
            start, size = int(a[0]), int(a[1])
            self.vals[out.id] = np.broadcast_to(np.arange(start, start + size, dtype=np.uint32), (self.n, size)).copy()
            return
        if op == "add" and out.id in self.fused:
            x, y, z = self.fused[out.id]
            xv, yv, zv = self.bcast(V(x), V(y), V(z))
            self.vals[out.id] = ops.fmaf(xv, yv, zv).reshape(xv.shape)
            return
        if op in ("add", "mul", "floordiv", "mod", "lt", "and", "or"):
            x, y = V(a[0]), V(a[1])
            if op == "add":
                r = x + y
            elif op == "mul":
                r = x * y
            elif op == "floordiv":
                r = np.where(y == 0, 0, x // np.where(y == 0, 1, y))
            elif op == "mod":
                r = np.where(y == 0, 0, x % np.where(y == 0, 1, y))
            elif op == "lt":
                r = x < y
            elif op == "and":
                r = x & y
            else:
                r = x | y
            self.vals[out.id] = np.asarray(r).astype(_NP[out.dtype.value])
            return
        if op == "not":
            self.vals[out.id] = ~V(a[0])
            return
        if op == "where":
            self.vals[out.id] = np.where(V(a[0]), V(a[1]), V(a[2])).astype(_NP[out.dtype.value])
            return
        if op == "cast":
            x = V(a[0])
            dst = out.dtype.value
            if dst == "u32" and x.dtype.kind == "f":
                xf = x.astype(np.float64)
                r = np.where(np.isnan(xf), 0, np.clip(np.trunc(xf), 0, 4294967295)).astype(np.uint32)
            elif dst == "bool":
                r = x != 0
            else:
                r = x.astype(np.float32).astype(_NP[dst]) if x.dtype == np.bool_ else x.astype(_NP[dst])
            self.vals[out.id] = r
            return
        if op == "fma":
            x, y, z = self.bcast(V(a[0]), V(a[1]), V(a[2]))
            r = ops.fmaf(x.astype(np.float32), y.astype(np.float32), z.astype(np.float32)).reshape(x.shape)
            self.vals[out.id] = r.astype(_NP[out.dtype.value])
            return
        if op == "load":
            buf, off, mask = a
            self.vals[out.id] = self.gather(buf, V(off), V(mask), _NP[out.dtype.value])
            return
        if op == "store":
            buf, off, val, mask = a
            self.scatter(buf, V(off), V(val), V(mask))
            return
        if op == "barrier":
            return
        if op == "dot":
            a_buf, a_base, a_st, b_buf, b_base, b_st, k = a
            K = V(k).astype(np.int64)
            acc = np.zeros((self.n, 1), np.float32)
            ab, bb = V(a_base).astype(np.int64), V(b_base).astype(np.int64)
            ast, bst = V(a_st).astype(np.int64), V(b_st).astype(np.int64)
            for kk in range(int(K.max(initial=0))):
                act = (kk < K) & self.exists
                xa = self.gather(a_buf, (ab + kk * ast).astype(np.uint32), act, np.float32).astype(np.float32)
                xb = self.gather(b_buf, (bb + kk * bst).astype(np.uint32), act, np.float32).astype(np.float32)
                acc = np.where(act, ops.fmaf(xa, xb, acc).reshape(acc.shape), acc)
            self.vals[out.id] = acc
            return
        if op == "mma_zero":
            self.vals[out.id] = np.zeros((self.n, 8, 8), np.float32)
            return
        if op == "mma":
            a_buf, a_base, a_st, b_buf, b_base, b_st, acc = a
            r8 = np.arange(8)
            aoff = V(a_base).reshape(self.n, 1, 1).astype(np.int64) + r8[:, None] * V(a_st).reshape(self.n, 1, 1) + r8[None, :]
            boff = V(b_base).reshape(self.n, 1, 1).astype(np.int64) + r8[:, None] * V(b_st).reshape(self.n, 1, 1) + r8[None, :]
            A = self.gather(a_buf, aoff.reshape(self.n, 64).astype(np.uint32), np.ones((self.n, 1), bool), np.float32)
            B = self.gather(b_buf, boff.reshape(self.n, 64).astype(np.uint32), np.ones((self.n, 1), bool), np.float32)
            prod = np.einsum("nik,nkj->nij", A.reshape(self.n, 8, 8).astype(np.float64), B.reshape(self.n, 8, 8).astype(np.float64))
            self.vals[out.id] = (V(acc).astype(np.float64) + prod).astype(np.float32)
            return
        if op == "mma_store":
            c_buf, c_base, c_st, frag = a
            r8 = np.arange(8)
            off = V(c_base).reshape(self.n, 1, 1).astype(np.int64) + r8[:, None] * V(c_st).reshape(self.n, 1, 1) + r8[None, :]
            writer = (self.local % 32 == 0)[:, None]
            self.scatter(c_buf, off.reshape(self.n, 64).astype(np.uint32), V(frag).reshape(self.n, 64), writer)
            return
        raise OracleError(f"oracle cannot execute op {op!r}")


def run_kernel(kernel: Any, *args: Any, **kwargs: Any) -> dict[str, np.ndarray]:
    """Execute ``kernel`` on host copies of its buffers; returns ``{name: output array}``.

    Takes the same arguments as a kernel call (runtime args, meta, ``_grid`` /
    ``_shape`` / ``_nthreads`` / ``_tptg``); numpy inputs are not modified.
    """
    from easy_as_amd.compiler import trace_to_ir
    from easy_as_amd.codegen.hip import infer_block_and_mode
    from easy_as_amd.runtime.grid import infer_grid, infer_nthreads

    kw = dict(kwargs)
    opts = kernel._extract_runtime_options(kw)
    meta, rargs = kernel._bind_and_split(*args, **kw)
    opts = kernel._normalize_runtime_options(opts, meta, rargs)
    ir = trace_to_ir(kernel.fn, rargs, meta)
    block, mode = infer_block_and_mode(ir)
    buffers: dict[str, np.ndarray] = {}
    scalars: dict[str, Any] = {}
    for arg in ir.args:
        val = rargs[arg.name]
        if arg.kind == "buffer":
            arr = val.numpy() if hasattr(val, "numpy") and not isinstance(val, np.ndarray) else val
            arr = np.asarray(arr)
            buffers[arg.name] = np.array(arr, dtype=_NP[arg.dtype.value]).reshape(-1)
        else:
            scalars[arg.name] = val
    live = None
    grid = opts["grid"]
    if grid is None:
        inferred = infer_grid(ir, rargs, block, shape=opts["shape"])
        if inferred is None:
            n = infer_nthreads(rargs, nthreads=opts["nthreads"])
            grid = (_cdiv(n, block), 1, 1)
            live = n if mode == "thread" else None
        else:
            grid = inferred
    if any(int(g) == 0 for g in grid):
        return buffers
    ex = _Exec(ir, mode, block, 0, tuple(int(g) for g in grid), live, buffers, scalars)
    ex.run()
    return buffers
