"""Lift tile-GEMM kernels written with ``mk.mma`` to a tuned gfx950 MFMA GEMM.

The reference's simdgroup-MMA matmul (``examples/matmul_simdgroup.py:29-127``)
computes one 8x8 fragment per 32-lane simdgroup with tiny tiles
(``NT = (BM/8)(BN/8)*32 <= 1024``); lowered literally it cannot feed MI355X's
matrix cores.  This module *proves* that a kernel's IR computes a dense GEMM and,
only then, replaces it with hand-written MFMA kernels (``codegen/gemm_kernels.py``):
``v_mfma_f32_16x16x32_f16`` (or ``_bf16``) by default, A and B moved HBM -> LDS by
``buffer_load ... lds`` DMA rings in their row-major layouts, B transposed on its
way out of LDS by ``ds_read_b64_tr_b16``; operands the DMA cannot take (f32
inputs, rows not 4-byte aligned) run a register-staged body instead.  The fp32
tiled ``dot`` pattern lifts to ``v_mfma_f32_32x32x2_f32`` the same way.

Proof method (no pattern matching on source text): the IR is executed
symbolically for all NT threads of one threadgroup at once.  Thread ids are
concrete; ``program_id`` values and u32 scalar arguments stay symbolic, so every
index is a polynomial in those symbols with per-thread integer coefficients,
and every mask is a concrete per-thread part plus affine atoms ``p < 0``.
Threadgroup memory is tracked slot by slot (which load, for which thread, last
wrote it).  At each ``mma`` the fragment slots are resolved to global loads and
decoded into (row, k) / (k, col) positions; at the end every copied-out output
element is matched to its fragment.  The kernel is lifted only if, for every
output element of the threadgroup's tile,

    C[row*ldc + col] = sum_{k in [0, K)} f16(A[row*K + k]) * f16(B[k*ldb + col])

with rows/cols of the tile ``TM*pid_r + r`` / ``TN*pid_c + c`` (r < TM, c < TN),
each k exactly once, A/B elements masked only by ``row < M`` / ``col < N`` and
stores masked only by those, ``ldb == ldc`` the same scalar as the column bound.
Anything else (other side effects, symbolic K, data-dependent indices, stale or
uninitialised tile slots) leaves the kernel to the literal lowering.  The lifted
kernel computes exactly the rectangle the launched grid covers, so partial grids
(``_grid`` smaller than the matrix) keep their meaning; it needs M*K, K*N and
M*N below 2^32 (the u32 index range the reference computes in).
"""

from __future__ import annotations

import os

from dataclasses import dataclass
from typing import Any

import numpy as np

from ..ir import DType, IRModule, Inst, ValueRef

Mono = tuple[str, ...]


class Unsupported(Exception):
    """The kernel is not (provably) a dense tile GEMM."""


# ---------------------------------------------------------------------------
# symbolic integers: polynomials with per-thread coefficients
# ---------------------------------------------------------------------------


class Poly:
    __slots__ = ("t",)

    def __init__(self, terms: dict[Mono, np.ndarray]) -> None:
        self.t = {m: c for m, c in terms.items() if np.any(c)}

    @staticmethod
    def const(v: Any, n: int) -> "Poly":
        return Poly({(): np.full(n, int(v), dtype=np.int64)})

    def concrete(self) -> np.ndarray | None:
        keys = set(self.t)
        if keys <= {()}:
            c = self.t.get(())
            return c if c is not None else None
        return None

    def add(self, o: "Poly", sign: int = 1) -> "Poly":
        out = dict(self.t)
        for m, c in o.t.items():
            out[m] = out[m] + sign * c if m in out else sign * c
        return Poly(out)

    def mul(self, o: "Poly") -> "Poly":
        out: dict[Mono, np.ndarray] = {}
        for m1, c1 in self.t.items():
            for m2, c2 in o.t.items():
                m = tuple(sorted(m1 + m2))
                out[m] = out[m] + c1 * c2 if m in out else c1 * c2
        if any(len(m) > 3 for m in out):
            raise Unsupported("index polynomial of degree > 3")
        return Poly(out)


def _concrete_of(p: Poly, n: int) -> np.ndarray:
    c = p.concrete()
    if c is None:
        if p.t:
            raise Unsupported("symbolic value where a thread-only value is required")
        return np.zeros(n, dtype=np.int64)
    return c


@dataclass
class Cond:
    """Mask: ``base`` (per thread) AND every atom ``poly < 0``."""

    base: np.ndarray
    atoms: list[Poly]


@dataclass
class Rec:
    """A float value produced by one instruction for all threads."""

    kind: str            # "gload" | "lds" | "frag"
    buf: str = ""        # global buffer name (gload)
    off: Poly | None = None
    cond: Cond | None = None
    rnd: str = ""        # rounded to "f16" or "bf16" after the load ("": as loaded)
    src_rec: np.ndarray | None = None   # lds: record id per thread
    src_thr: np.ndarray | None = None   # lds: writer thread per thread
    frag: Any = None                    # frag: (sg, i, j) arrays per thread


@dataclass
class Frag:
    steps: list[tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]]  # (A rec, A thr, B rec, B thr) per step


@dataclass(frozen=True)
class GemmSpec:
    a: str
    b: str
    c: str
    m_sym: str | None      # row bound (None: rows bounded by the launched grid only)
    n_sym: str
    K: int
    TM: int
    TN: int
    row_axis: int          # program_id axis indexing tile rows (the other indexes cols)
    a_dtype: DType
    b_dtype: DType
    c_dtype: DType
    c_f16: bool            # output rounded from the f32 accumulator to C's 16-bit type (f16 or bf16)
    f32: bool = False      # fp32 products and sums (the `mk.dot` tiled pattern); else 16-bit MFMA operands
    row_base: str | None = None   # tile rows start at TM * (program_id + row_base) when set
    col_base: str | None = None
    col_masked: bool = True       # outputs/operands bounded by col < N (else by the launched grid)
    op_dtype: DType = DType.F16   # MFMA operand type: the dtype of the threadgroup tiles A and B pass through


# ---------------------------------------------------------------------------
# symbolic execution
# ---------------------------------------------------------------------------


class _SymExec:
    def __init__(self, ir: IRModule, nt: int) -> None:
        self.ir = ir
        self.n = nt
        self.ints: dict[int, Poly] = {}
        self.bools: dict[int, Cond] = {}
        self.floats: dict[int, int] = {}   # value id -> record id
        self.recs: list[Rec] = []
        self.frags: dict[int, Frag] = {}
        self.op_dtype: DType | None = None   # threadgroup tile dtype of the mma operands
        self.tg: dict[int, tuple[np.ndarray, np.ndarray, DType]] = {}
        self.global_bufs: dict[int, str] = {}
        self.scalars: dict[int, str] = {}
        self.stores: list[tuple[str, Poly, Cond, int]] = []
        self.frag_stores: list[tuple[int, int, np.ndarray, np.ndarray]] = []  # (tg id, frag id, base, stride)
        self.loaded: set[str] = set()
        self.stored: set[str] = set()
        # f32 values that are sums of products of threadgroup slots (`dot` chains): value id -> terms,
        # each term (A rec, A writer thread, B rec, B writer thread), arrays of shape (threads, k)
        self.sums: dict[int, list[tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]]] = {}
        self.dot_stores: list[tuple[str, Poly, Cond, list]] = []

    def run(self) -> None:
        for inst in self.ir.insts:
            self.step(inst)

    # -- helpers ------------------------------------------------------------
    def ip(self, ref: ValueRef) -> Poly:
        p = self.ints.get(ref.id)
        if p is None:
            raise Unsupported(f"u32 value v{ref.id} is not an index expression")
        return p

    def bc(self, ref: ValueRef) -> Cond:
        c = self.bools.get(ref.id)
        if c is None:
            raise Unsupported(f"bool value v{ref.id} is not a mask expression")
        return c

    def uniform_sg(self, arr: np.ndarray, what: str) -> np.ndarray:
        per = arr.reshape(-1, 32)
        if np.any(per != per[:, :1]):
            raise Unsupported(f"{what} differs across a simdgroup")
        return per[:, 0]

    def new_rec(self, r: Rec) -> int:
        self.recs.append(r)
        return len(self.recs) - 1

    # -- instructions ------------------------------------------------------------
    def step(self, inst: Inst) -> None:
        op, out, a = inst.op, inst.out, inst.args
        n = self.n
        tids = np.arange(n, dtype=np.int64)
        if op == "arg":
            name, kind, dt = a
            if kind == "buffer":
                self.global_bufs[out.id] = name
            elif dt == DType.U32:
                self.ints[out.id] = Poly({(name,): np.ones(n, np.int64)})
                self.scalars[out.id] = name
            return
        if op == "const":
            v = a[0]
            if out.dtype == DType.U32:
                self.ints[out.id] = Poly.const(v, n)
            elif out.dtype == DType.BOOL:
                self.bools[out.id] = Cond(np.full(n, bool(v)), [])
            elif out.dtype == DType.F32 and float(v) == 0.0:
                self.sums[out.id] = []
            return  # other float consts only matter if used, which is unsupported below
        if op == "program_id":
            self.ints[out.id] = Poly({(f"%p{int(a[0])}",): np.ones(n, np.int64)})
            return
        if op == "thread_id":
            raise Unsupported("global thread ids are not tile-GEMM indexing")
        if op == "tid":
            self.ints[out.id] = Poly({(): tids + int(a[0])})
            return
        if op == "local_id":
            self.ints[out.id] = Poly({(): tids if int(a[0]) == 0 else np.zeros(n, np.int64)})
            return
        if op == "lane_id":
            self.ints[out.id] = Poly({(): tids % 32})
            return
        if op == "sg_id":
            self.ints[out.id] = Poly({(): tids // 32})
            return
        if op in ("add", "mul") and out.dtype == DType.U32:
            x, y = self.ip(a[0]), self.ip(a[1])
            self.ints[out.id] = x.add(y) if op == "add" else x.mul(y)
            return
        if op == "add" and out.dtype == DType.F32:
            if a[0].id not in self.sums or a[1].id not in self.sums:
                raise Unsupported("f32 add of values that are not dot sums")
            self.sums[out.id] = self.sums[a[0].id] + self.sums[a[1].id]
            return
        if op == "dot":
            a_buf, a_base, a_st, b_buf, b_base, b_st, kref = a
            if a_buf.id not in self.tg or b_buf.id not in self.tg:
                raise Unsupported("dot operands must come from threadgroup memory")
            if self.tg[a_buf.id][2] != DType.F32 or self.tg[b_buf.id][2] != DType.F32:
                raise Unsupported("only f32 threadgroup tiles are lifted for dot")
            kd = _concrete_of(self.ip(kref), n)
            if np.any(kd != kd[0]) or kd[0] <= 0:
                raise Unsupported("dot length differs across threads")
            kk = np.arange(int(kd[0]), dtype=np.int64)
            a_slots = _concrete_of(self.ip(a_base), n)[:, None] + _concrete_of(self.ip(a_st), n)[:, None] * kk[None, :]
            b_slots = _concrete_of(self.ip(b_base), n)[:, None] + _concrete_of(self.ip(b_st), n)[:, None] * kk[None, :]
            ar, at, _ = self.tg[a_buf.id]
            br, bt, _ = self.tg[b_buf.id]
            if a_slots.min() < 0 or b_slots.min() < 0 or a_slots.max() >= ar.size or b_slots.max() >= br.size:
                raise Unsupported("dot reads outside its threadgroup tile")
            if np.any(ar[a_slots] < 0) or np.any(br[b_slots] < 0):
                raise Unsupported("dot reads an unwritten threadgroup slot")
            self.sums[out.id] = [(ar[a_slots].copy(), at[a_slots].copy(), br[b_slots].copy(), bt[b_slots].copy())]
            return
        if op in ("floordiv", "mod"):
            x, y = _concrete_of(self.ip(a[0]), n), _concrete_of(self.ip(a[1]), n)
            if np.any(y <= 0) or np.any(x < 0):
                raise Unsupported("division by zero / negative in index math")
            self.ints[out.id] = Poly({(): x // y if op == "floordiv" else x % y})
            return
        if op == "lt" and a[0].dtype == DType.U32:
            d = self.ip(a[0]).add(self.ip(a[1]), -1)
            c = d.concrete()
            if c is not None or not d.t:
                self.bools[out.id] = Cond((c if c is not None else np.zeros(n, np.int64)) < 0, [])
            else:
                self.bools[out.id] = Cond(np.ones(n, bool), [d])
            return
        if op == "and":
            x, y = self.bc(a[0]), self.bc(a[1])
            self.bools[out.id] = Cond(x.base & y.base, x.atoms + y.atoms)
            return
        if op == "or":
            x, y = self.bc(a[0]), self.bc(a[1])
            if x.atoms or y.atoms:
                raise Unsupported("disjunction of symbolic conditions")
            self.bools[out.id] = Cond(x.base | y.base, [])
            return
        if op == "not":
            x = self.bc(a[0])
            if x.atoms:
                raise Unsupported("negated symbolic condition")
            self.bools[out.id] = Cond(~x.base, [])
            return
        if op == "where" and out.dtype == DType.U32:
            c = self.bc(a[0])
            if c.atoms:
                raise Unsupported("data-dependent select in index math")
            x, y = _concrete_of(self.ip(a[1]), n), _concrete_of(self.ip(a[2]), n)
            self.ints[out.id] = Poly({(): np.where(c.base, x, y)})
            return
        if op == "cast":
            src = a[0]
            if out.dtype in (DType.F16, DType.BF16) and src.dtype == DType.F32 and src.id in self.floats:
                r = self.recs[self.floats[src.id]]
                if r.kind != "gload" and r.kind != "lds":
                    raise Unsupported("cast of a computed float")
                self.floats[out.id] = self.new_rec(Rec(**{**r.__dict__, "rnd": out.dtype.value}))
                return
            raise Unsupported(f"cast {src.dtype}->{out.dtype} in a GEMM kernel")
        if op == "alloc_tg":
            size = int(a[0])
            self.tg[out.id] = (np.full(size, -1, np.int64), np.zeros(size, np.int64), out.dtype)
            return
        if op == "barrier":
            return
        if op == "load":
            buf, off, mask = a
            cond = self.bc(mask)
            if buf.id in self.global_bufs:
                name = self.global_bufs[buf.id]
                self.loaded.add(name)
                self.floats[out.id] = self.new_rec(Rec("gload", buf=name, off=self.ip(off), cond=cond))
                return
            if buf.id in self.tg:
                if cond.atoms:
                    raise Unsupported("symbolic mask on a threadgroup load")
                slots = _concrete_of(self.ip(off), n)
                recs, thrs, _ = self.tg[buf.id]
                if np.any(slots >= recs.size):
                    raise Unsupported("threadgroup load out of range")
                sr = np.where(cond.base, recs[slots], -2)
                st = thrs[slots]
                if np.any(sr == -1):
                    raise Unsupported("read of an unwritten threadgroup slot")
                self.floats[out.id] = self.new_rec(Rec("lds", src_rec=sr, src_thr=st))
                return
            raise Unsupported("load from an unknown buffer")
        if op == "store":
            buf, off, val, mask = a
            cond = self.bc(mask)
            if val.id in self.sums and buf.id in self.global_bufs:
                name = self.global_bufs[buf.id]
                self.stored.add(name)
                self.dot_stores.append((name, self.ip(off), cond, self.sums[val.id]))
                return
            if val.id not in self.floats:
                raise Unsupported("stored value is not a tracked float")
            rid = self.floats[val.id]
            if buf.id in self.tg:
                if cond.atoms:
                    raise Unsupported("symbolic mask on a threadgroup store")
                if self.recs[rid].kind != "gload":
                    raise Unsupported("threadgroup store of a non-load value")
                slots = _concrete_of(self.ip(off), n)
                recs, thrs, _ = self.tg[buf.id]
                w = np.nonzero(cond.base)[0]
                if np.any(slots[w] >= recs.size):
                    raise Unsupported("threadgroup store out of range")
                if np.unique(slots[w]).size != w.size:
                    raise Unsupported("two threads store one threadgroup slot")
                recs[slots[w]] = rid
                thrs[slots[w]] = w
                return
            if buf.id in self.global_bufs:
                name = self.global_bufs[buf.id]
                self.stored.add(name)
                self.stores.append((name, self.ip(off), cond, rid))
                return
            raise Unsupported("store to an unknown buffer")
        if op == "mma_zero":
            self.frags[out.id] = Frag([])
            return
        if op == "mma":
            a_buf, a_base, a_st, b_buf, b_base, b_st, acc = a
            if a_buf.id not in self.tg or b_buf.id not in self.tg:
                raise Unsupported("mma operands must come from threadgroup memory")
            tile_dts = (self.tg[a_buf.id][2], self.tg[b_buf.id][2])
            if tile_dts not in ((DType.F16, DType.F16), (DType.BF16, DType.BF16)):
                raise Unsupported("only f16 or bf16 threadgroup tiles (both alike) are lifted")
            if self.op_dtype not in (None, tile_dts[0]):
                raise Unsupported("mma operand type changes between steps")
            self.op_dtype = tile_dts[0]
            prev = self.frags.get(acc.id)
            if prev is None:
                raise Unsupported("mma accumulator chain not rooted at mma_zero")
            ab = self.uniform_sg(_concrete_of(self.ip(a_base), n), "mma a_base")
            ast = self.uniform_sg(_concrete_of(self.ip(a_st), n), "mma a_stride")
            bb = self.uniform_sg(_concrete_of(self.ip(b_base), n), "mma b_base")
            bst = self.uniform_sg(_concrete_of(self.ip(b_st), n), "mma b_stride")
            r8 = np.arange(8)
            a_slots = ab[:, None, None] + r8[None, :, None] * ast[:, None, None] + r8[None, None, :]  # (S, i, k)
            b_slots = bb[:, None, None] + r8[None, :, None] * bst[:, None, None] + r8[None, None, :]  # (S, k, j)
            ar, at, _ = self.tg[a_buf.id]
            br, bt, _ = self.tg[b_buf.id]
            if a_slots.max() >= ar.size or b_slots.max() >= br.size or a_slots.min() < 0:
                raise Unsupported("mma fragment outside its threadgroup tile")
            if np.any(ar[a_slots] < 0) or np.any(br[b_slots] < 0):
                raise Unsupported("mma reads an unwritten threadgroup slot")
            self.frags[out.id] = Frag(prev.steps + [(ar[a_slots].copy(), at[a_slots].copy(), br[b_slots].copy(), bt[b_slots].copy())])
            return
        if op == "mma_store":
            c_buf, c_base, c_st, frag = a
            if c_buf.id not in self.tg:
                raise Unsupported("mma_store outside threadgroup memory")
            f = self.frags.get(frag.id)
            if f is None:
                raise Unsupported("mma_store of an unknown fragment")
            base = self.uniform_sg(_concrete_of(self.ip(c_base), n), "mma_store base")
            st = self.uniform_sg(_concrete_of(self.ip(c_st), n), "mma_store stride")
            fid = self.new_rec(Rec("frag", frag=(f, base, st)))
            recs, thrs, _ = self.tg[c_buf.id]
            r8 = np.arange(8)
            slots = base[:, None, None] + r8[None, :, None] * st[:, None, None] + r8[None, None, :]  # (S, i, j)
            if slots.max() >= recs.size:
                raise Unsupported("mma_store outside its threadgroup tile")
            flat = slots.reshape(-1)
            if np.unique(flat).size != flat.size:
                raise Unsupported("overlapping fragment stores")
            recs[flat] = fid
            thrs[flat] = np.arange(flat.size)  # encodes (sg, i, j) as sg*64 + i*8 + j
            return
        raise Unsupported(f"op {op!r} is not part of a tile GEMM")


# ---------------------------------------------------------------------------
# decoding of gathered element positions
# ---------------------------------------------------------------------------


def _gather_poly(recs: list[Rec], rid: np.ndarray, thr: np.ndarray, attr: str) -> dict[Mono, np.ndarray]:
    """Coefficients of rec.<attr> (a Poly) at (record, thread) pairs, shape of ``rid``."""
    out: dict[Mono, np.ndarray] = {}
    for r in np.unique(rid):
        sel = rid == r
        p: Poly = getattr(recs[int(r)], attr)
        for m, c in p.t.items():
            arr = out.setdefault(m, np.zeros(rid.shape, np.int64))
            arr[sel] = c[thr[sel]]
    return out


def _poly_sub(x: dict[Mono, np.ndarray], y: dict[Mono, np.ndarray], shape: tuple[int, ...]) -> dict[Mono, np.ndarray]:
    out = {m: c.copy() for m, c in x.items()}
    for m, c in y.items():
        out[m] = out.get(m, np.zeros(shape, np.int64)) - c
    return {m: c for m, c in out.items() if np.any(c)}


def _uniform_step(d: dict[Mono, np.ndarray]) -> dict[Mono, int]:
    """A difference that must be the same integer polynomial for every element."""
    out = {}
    for m, c in d.items():
        if np.any(c != c.flat[0]):
            raise Unsupported("non-uniform stride between fragment elements")
        out[m] = int(c.flat[0])
    return out


def _split(off: dict[Mono, np.ndarray], stride: dict[Mono, int], shape) -> tuple[dict[Mono, np.ndarray], dict[Mono, np.ndarray]]:
    """Decompose ``off = stride * major + minor``.

    A literal stride L splits the constant term by div/mod (minor in [0, L))
    and requires every symbolic term to be a multiple of L (it belongs to the
    major index).  A scalar-argument stride X moves the terms containing X to
    the major index (X removed) and leaves the rest as the minor index.
    """
    zero = np.zeros(shape, np.int64)
    if set(stride) == {()}:
        L = stride[()]
        if L <= 0:
            raise Unsupported("non-positive row stride")
        c0 = off.get((), zero)
        major = {(): c0 // L}
        for m, c in off.items():
            if m == ():
                continue
            if np.any(c % L):
                raise Unsupported("index not a multiple of the row stride")
            major[m] = c // L
        return {m: c for m, c in major.items() if np.any(c)}, {(): c0 % L}
    if len(stride) == 1:
        (sm, sc), = stride.items()
        if len(sm) != 1 or sc != 1 or sm[0].startswith("%p"):
            raise Unsupported("row stride must be a literal or one scalar argument")
        sym = sm[0]
        major: dict[Mono, np.ndarray] = {}
        minor: dict[Mono, np.ndarray] = {}
        for m, c in off.items():
            if sym in m:
                rest = list(m)
                rest.remove(sym)
                if sym in rest:
                    raise Unsupported("index quadratic in the row stride")
                major[tuple(rest)] = c
            else:
                minor[m] = c
        return major, minor
    raise Unsupported("unsupported row stride")


def _concrete_part(p: dict[Mono, np.ndarray], shape, what: str) -> np.ndarray:
    if set(p) - {()}:
        raise Unsupported(f"{what} index is symbolic")
    return p.get((), np.zeros(shape, np.int64))


def _same(p: dict[Mono, np.ndarray], q: dict[Mono, np.ndarray]) -> bool:
    keys = set(p) | set(q)
    for m in keys:
        a = p.get(m)
        b = q.get(m)
        if a is None and b is None:
            continue
        if a is None:
            a = np.zeros_like(b)
        if b is None:
            b = np.zeros_like(a)
        if not np.array_equal(a, b):
            return False
    return True


def _as_tile(p: dict[Mono, np.ndarray], what: str) -> tuple[str, int, np.ndarray, str | None]:
    """``p = T * (%p<axis> [+ base]) + r`` with r concrete and base one scalar argument;
    returns (axis symbol, T, r, base symbol or None)."""
    syms = [m for m in p if m != ()]
    pids = [m for m in syms if len(m) == 1 and m[0].startswith("%p")]
    bases = [m for m in syms if len(m) == 1 and not m[0].startswith("%p")]
    if len(pids) != 1 or len(bases) > 1 or len(pids) + len(bases) != len(syms):
        raise Unsupported(f"{what} index is not tile*(program_id + base) + offset")
    T = p[pids[0]]
    if np.any(T != T.flat[0]) or T.flat[0] <= 0:
        raise Unsupported(f"{what} tile size differs")
    base = None
    if bases:
        if not np.array_equal(p[bases[0]], T):
            raise Unsupported(f"{what} base offset is not a whole number of tiles")
        base = bases[0][0]
    r = p.get((), np.zeros(T.shape, np.int64))
    return pids[0][0], int(T.flat[0]), r, base


def _atoms_match(recs: list[Rec], rid: np.ndarray, thr: np.ndarray, expect: dict[Mono, np.ndarray], bound_sym: str | None,
                 valid: np.ndarray) -> str | None:
    """Every element's symbolic mask is empty or exactly ``expect - bound_sym < 0``;
    returns the bound symbol found (or ``bound_sym``)."""
    found = bound_sym
    for r in np.unique(rid[valid]):
        sel = (rid == r) & valid
        cond = recs[int(r)].cond
        uniq: list[Poly] = []
        for atom in cond.atoms:
            if not any(set(atom.t) == set(u.t) and all(np.array_equal(atom.t[m], u.t[m]) for m in atom.t) for u in uniq):
                uniq.append(atom)
        if len(uniq) > 1:
            raise Unsupported("more than one symbolic bound on an operand")
        for atom in uniq:
            neg = [m for m, c in atom.t.items() if len(m) == 1 and not m[0].startswith("%p") and np.all(c[thr[sel]] == -1)]
            if len(neg) != 1:
                raise Unsupported("operand bound is not `index < scalar`")
            sym = neg[0][0]
            if found is not None and sym != found:
                raise Unsupported("operand bounded by two different scalars")
            found = sym
            for m, c in atom.t.items():
                if m == neg[0]:
                    continue
                want = expect.get(m)
                got = c[thr[sel]]
                if want is None or not np.array_equal(want[sel], got):
                    raise Unsupported("operand bound differs from its row/col index")
            for m, c in expect.items():
                if m not in atom.t and np.any(c[sel]):
                    raise Unsupported("operand bound differs from its row/col index")
    return found


def analyze(ir: IRModule, block: int) -> GemmSpec:
    """Prove that ``ir`` is a dense tile GEMM; raise :class:`Unsupported` otherwise."""
    if block % 32 or block > 1024:
        raise Unsupported("threadgroup size must be a multiple of 32")
    ops = {i.op for i in ir.insts}
    if "mma" not in ops or "mma_store" not in ops:
        raise Unsupported("no simdgroup MMA")
    ex = _SymExec(ir, block)
    ex.run()
    recs = ex.recs
    frag_recs = [r for r in recs if r.kind == "frag"]
    if len(frag_recs) != 1:
        raise Unsupported("expected exactly one mma_store")
    frag, _, _ = frag_recs[0].frag
    if not frag.steps:
        raise Unsupported("empty mma chain")
    if len(ex.stored) != 1 or ex.stored & ex.loaded:
        raise Unsupported("expected one output buffer that is not read")
    c_name = next(iter(ex.stored))
    S = block // 32

    a_buf = b_buf = None
    lda = ldb = None
    row_of = col_of = None       # per (S, 8) row / col polys of the fragment
    m_sym = n_sym = None
    ks: list[np.ndarray] = []
    for ar, at, br, bt in frag.steps:
        for rid in (ar, br):
            kinds = {recs[int(r)].kind for r in np.unique(rid)}
            if kinds != {"gload"}:
                raise Unsupported("fragment slot not filled from global memory")
        an = {recs[int(r)].buf for r in np.unique(ar)}
        bn = {recs[int(r)].buf for r in np.unique(br)}
        if len(an) != 1 or len(bn) != 1:
            raise Unsupported("fragment mixes buffers")
        an, bn = an.pop(), bn.pop()
        a_buf = a_buf or an
        b_buf = b_buf or bn
        if (an, bn) != (a_buf, b_buf) or a_buf == b_buf or c_name in (a_buf, b_buf):
            raise Unsupported("operand buffers change between steps")
        shape = ar.shape
        # liveness: the concrete part of each element's load mask; masked elements are 0
        a_base = np.zeros(shape, bool)
        b_base = np.zeros(shape, bool)
        for r in np.unique(ar):
            sel = ar == r
            a_base[sel] = recs[int(r)].cond.base[at[sel]]
        for r in np.unique(br):
            sel = br == r
            b_base[sel] = recs[int(r)].cond.base[bt[sel]]
        if np.any(a_base != a_base[:, :1, :]) or np.any(b_base != b_base[:, :, :1]):
            raise Unsupported("operand liveness varies along rows/cols")
        live = a_base[:, 0, :]                                  # (S, k)
        if not np.array_equal(live, b_base[:, :, 0]) or np.any(live != live[:1]):
            raise Unsupported("operand masks do not agree along k")
        lk = live[0]
        kidx = np.nonzero(lk)[0]
        if kidx.size == 0:
            ks.append(np.full((S, 8), -1, np.int64))
            continue
        k0 = int(kidx[0])
        pairs = np.nonzero(lk[:-1] & lk[1:])[0]
        a_off = _gather_poly(recs, ar, at, "off")
        b_off = _gather_poly(recs, br, bt, "off")
        # strides between live fragment elements
        a_row = _uniform_step(_poly_sub({m: c[:, 1:, kidx] for m, c in a_off.items()},
                                        {m: c[:, :-1, kidx] for m, c in a_off.items()}, (S, 7, kidx.size)))
        if pairs.size:
            a_col = _uniform_step(_poly_sub({m: c[:, :, pairs + 1] for m, c in a_off.items()},
                                            {m: c[:, :, pairs] for m, c in a_off.items()}, (S, 8, pairs.size)))
            b_row = _uniform_step(_poly_sub({m: c[:, pairs + 1, :] for m, c in b_off.items()},
                                            {m: c[:, pairs, :] for m, c in b_off.items()}, (S, pairs.size, 8)))
            if a_col != {(): 1}:
                raise Unsupported("A fragment columns are not contiguous")
            if ldb is None:
                ldb = b_row
            if b_row != ldb:
                raise Unsupported("B row stride changes between steps")
        b_col = _uniform_step(_poly_sub({m: c[:, kidx, 1:] for m, c in b_off.items()},
                                        {m: c[:, kidx, :-1] for m, c in b_off.items()}, (S, kidx.size, 7)))
        if b_col != {(): 1}:
            raise Unsupported("B fragment columns are not contiguous")
        if lda is None:
            lda = a_row
        if a_row != lda:
            raise Unsupported("A row stride changes between steps")
        if ldb is None:
            raise Unsupported("B row stride not determined")
        a_major, a_minor = _split(a_off, lda, shape)        # A: row index, k
        b_major, b_minor = _split(b_off, ldb, shape)        # B: k, col index
        a_k = _concrete_part(a_minor, shape, "A's k")
        b_k = _concrete_part(b_major, shape, "B's k")
        for m, c in a_major.items():
            if np.any(c[:, :, kidx] != c[:, :, k0:k0 + 1]):
                raise Unsupported("A row index varies along k")
        for m, c in b_minor.items():
            if np.any(c[:, kidx, :] != c[:, k0:k0 + 1, :]):
                raise Unsupported("B column index varies along k")
        if not np.array_equal(a_k[:, 0, kidx], b_k[:, kidx, 0]):
            raise Unsupported("A and B k indices are not paired")
        ri = {m: c[:, :, k0] for m, c in a_major.items()}      # (S, i)
        col_poly = {m: c[:, k0, :] for m, c in b_minor.items()}  # (S, j)
        if row_of is None:
            row_of, col_of = ri, col_poly
        if not _same(ri, row_of):
            raise Unsupported("A rows change between steps")
        if not _same(col_poly, col_of):
            raise Unsupported("B cols change between steps")
        live3_a = np.broadcast_to(lk[None, None, :], shape)
        live3_b = np.broadcast_to(lk[None, :, None], shape)
        row_full = {m: np.repeat(c[:, :, None], 8, axis=2) for m, c in ri.items()}
        col_full = {m: np.repeat(c[:, None, :], 8, axis=1) for m, c in col_of.items()}
        m_sym = _atoms_match(recs, ar, at, row_full, m_sym, live3_a)
        n_sym = _atoms_match(recs, br, bt, col_full, n_sym, live3_b)
        ks.append(np.where(lk[None, :], a_k[:, 0, :], -1))
    assert lda is not None and ldb is not None and row_of is not None and col_of is not None
    if set(lda) != {()}:
        raise Unsupported("A's row length (K) must be a compile-time constant")
    K = lda[()]
    allk = np.concatenate(ks, axis=1)        # (S, steps*8)
    for s in range(S):
        got = np.sort(allk[s][allk[s] >= 0])
        if not np.array_equal(got, np.arange(K)):
            raise Unsupported("the k steps do not cover [0, K) exactly once")
    if len(ldb) != 1 or list(ldb)[0] == () or list(ldb.values())[0] != 1:
        raise Unsupported("B's row stride must be a scalar argument")
    ldb_sym = list(ldb)[0][0]
    if n_sym is not None and n_sym != ldb_sym:
        raise Unsupported("B's column bound differs from its row stride")
    r_axis, TM, r_off, r_base = _as_tile(row_of, "row")
    c_axis, TN, c_off, c_base = _as_tile(col_of, "col")
    if r_axis == c_axis:
        raise Unsupported("rows and cols indexed by the same program id")

    # --- copy-out: every tile element stored once to C[row*ldb + col] ---
    seen = np.zeros((S, 8, 8), np.int64)
    frag_rid = recs.index(frag_recs[0])
    c_rnd = None
    # a bound the operand loads apply must guard every output store too: the lifted kernel
    # writes only rows < M (cols < N), while a store without that mask would also write
    # the rows (cols) past it
    m_from_loads, n_from_loads = m_sym, n_sym
    for name, off, cond, rid in ex.stores:
        row_masked = col_masked = False
        r = recs[rid]
        if r.kind != "lds":
            raise Unsupported("output is not read back from the fragment tile")
        sel = cond.base & (r.src_rec >= 0)
        if np.any((r.src_rec != frag_rid) & sel):
            raise Unsupported("output element not from the accumulator")
        if c_rnd is None:
            c_rnd = r.rnd
        if r.rnd != c_rnd:
            raise Unsupported("mixed output conversions")
        t = np.nonzero(sel)[0]
        code = r.src_thr[t]
        sg, i, j = code // 64, (code // 8) % 8, code % 8
        np.add.at(seen, (sg, i, j), 1)
        offp = {m: c[t] for m, c in off.t.items()}
        major, minor = _split(offp, ldb, t.shape)
        want_row = {m: c[sg, i] for m, c in row_of.items()}
        want_col = {m: c[sg, j] for m, c in col_of.items()}
        if not (_same(major, want_row) and _same(minor, want_col)):
            raise Unsupported("output offset is not row*ldb + col of its fragment element")
        # store masks: at most `row < M` and `col < N`
        for atom in cond.atoms:
            at = {m: c[t] for m, c in atom.t.items()}
            neg = [m for m, c in at.items() if len(m) == 1 and not m[0].startswith("%p") and np.all(c == -1)]
            if len(neg) != 1:
                raise Unsupported("output mask is not `index < scalar`")
            rest = {m: c for m, c in at.items() if m != neg[0]}
            sym = neg[0][0]
            is_row = _same(rest, want_row)
            is_col = _same(rest, want_col)
            if is_row and (m_sym is None or m_sym == sym):
                m_sym = sym
                row_masked = True
            elif is_col and sym == ldb_sym:
                col_masked = True
            else:
                raise Unsupported("output mask is not row < M / col < N")
        if m_from_loads is not None and not row_masked:
            raise Unsupported("row bound applied inconsistently (the loads have it, an output store does not)")
        if n_from_loads is not None and not col_masked:
            raise Unsupported("column bound applied inconsistently (the loads have it, an output store does not)")
    if np.any(seen != 1):
        raise Unsupported("the tile is not stored exactly once")
    # the tile is the full rectangle [0,TM) x [0,TN)
    rows = r_off.reshape(-1)
    cols = c_off.reshape(-1)
    if sorted(set(rows.tolist())) != list(range(TM)) or sorted(set(cols.tolist())) != list(range(TN)):
        raise Unsupported("the fragments do not tile a TM x TN rectangle")
    if m_sym is None:
        raise Unsupported("no row bound found (M)")
    args = {a.name: a for a in ir.args}
    if m_sym not in args or ldb_sym not in args:
        raise Unsupported("bounds are not kernel arguments")
    a_dt, b_dt, c_dt = args[a_buf].dtype, args[b_buf].dtype, args[c_name].dtype
    if c_rnd != ("" if c_dt == DType.F32 else c_dt.value):
        raise Unsupported(f"{c_dt.value} output without an explicit conversion")
    assert ex.op_dtype is not None
    return GemmSpec(a=a_buf, b=b_buf, c=c_name, m_sym=m_sym, n_sym=ldb_sym, K=int(K), TM=TM, TN=TN,
                    row_axis=int(r_axis[2:]), a_dtype=a_dt, b_dtype=b_dt, c_dtype=c_dt, c_f16=bool(c_rnd),
                    row_base=r_base, col_base=c_base, op_dtype=ex.op_dtype)


def analyze_dot(ir: IRModule, block: int) -> GemmSpec:
    """Prove that a thread-mode kernel built from ``mk.dot`` over threadgroup tiles
    (``examples/matmul_tiled.py:27-131``) is a dense fp32 GEMM.

    Every stored output must be, for its thread, the sum over k in [0, K) (each k
    once) of A[row*K + k] * B[k*ldb + col] with f32 threadgroup tiles filled from
    global loads masked only by ``row < M`` / ``col < N`` (k beyond K masked to
    zero), stored to C[row*ldb + col] under ``row < M`` / ``col < N``, and the
    outputs of one threadgroup must cover a TM x TN rectangle exactly once.
    """
    ops = {i.op for i in ir.insts}
    if "dot" not in ops or ops & {"mma", "mma_zero", "mma_store"}:
        raise Unsupported("not a dot-tile kernel")
    ex = _SymExec(ir, block)
    ex.run()
    recs = ex.recs
    if ex.stores or not ex.dot_stores:
        raise Unsupported("outputs are not dot sums")
    if len(ex.stored) != 1 or ex.stored & ex.loaded:
        raise Unsupported("expected one output buffer that is not read")
    c_name = next(iter(ex.stored))
    a_buf = b_buf = ldb_sym = m_sym = None
    col_masked: bool | None = None
    row_masked_out: list[bool] = []
    K = None
    rows_all: list[np.ndarray] = []
    cols_all: list[np.ndarray] = []
    tile = None
    for name, off, cond, terms in ex.dot_stores:
        t = np.nonzero(cond.base)[0]
        if t.size == 0 or not terms:
            raise Unsupported("empty output or empty sum")
        AR = np.concatenate([x[0] for x in terms], axis=1)[t]
        AT = np.concatenate([x[1] for x in terms], axis=1)[t]
        BR = np.concatenate([x[2] for x in terms], axis=1)[t]
        BT = np.concatenate([x[3] for x in terms], axis=1)[t]
        for rid in (AR, BR):
            if {recs[int(r)].kind for r in np.unique(rid)} != {"gload"}:
                raise Unsupported("tile slot not filled from global memory")
        an = {recs[int(r)].buf for r in np.unique(AR)}
        bn = {recs[int(r)].buf for r in np.unique(BR)}
        if len(an) != 1 or len(bn) != 1:
            raise Unsupported("an operand mixes buffers")
        an, bn = an.pop(), bn.pop()
        a_buf, b_buf = a_buf or an, b_buf or bn
        if (an, bn) != (a_buf, b_buf) or a_buf == b_buf or c_name in (a_buf, b_buf):
            raise Unsupported("operand buffers differ between outputs")
        # concrete liveness of each product (a masked load is 0, so the product is 0)
        a_live = np.zeros(AR.shape, bool)
        b_live = np.zeros(BR.shape, bool)
        for r in np.unique(AR):
            sel = AR == r
            a_live[sel] = recs[int(r)].cond.base[AT[sel]]
        for r in np.unique(BR):
            sel = BR == r
            b_live[sel] = recs[int(r)].cond.base[BT[sel]]
        live = a_live & b_live
        a_off = _gather_poly(recs, AR, AT, "off")
        b_off = _gather_poly(recs, BR, BT, "off")
        # B: k * ldb + col with ldb one scalar argument: the scalar whose coefficient runs
        # through [0, K) over each thread's live products (a tile-base scalar's does not)
        def k_cover(sym: str) -> tuple[dict, np.ndarray, int]:
            b_k, b_col_ = _split(b_off, {(sym,): 1}, AR.shape)
            kB_ = _concrete_part(b_k, AR.shape, "B's k")
            kk: int | None = K
            for i in range(t.size):
                ks = np.sort(kB_[i][live[i]])
                if kk is None:
                    kk = int(ks.size)
                if ks.size != kk or not np.array_equal(ks, np.arange(kk)):
                    raise Unsupported("the dot chain does not cover k in [0, K) exactly once")
            return b_col_, kB_, int(kk or 0)

        cands = sorted({m[0] for m in b_off if len(m) == 1 and not m[0].startswith("%p")})
        if ldb_sym is not None:
            cands = [ldb_sym] if ldb_sym in cands else []
        found = None
        for sym in cands:
            try:
                found = (sym, *k_cover(sym))
                break
            except Unsupported:
                continue
        if found is None:
            raise Unsupported("B's row stride is not a scalar argument walking k over [0, K)")
        ldb_sym, b_col, kB, K = found
        if K == 0:
            raise Unsupported("empty reduction")
        # A: row * K + k (row length K, a compile-time constant)
        a_rest = _poly_sub(a_off, {(): kB}, AR.shape)
        row = {}
        for m, cf in a_rest.items():
            if np.any(cf[live] % K):
                raise Unsupported("A's row length is not the reduction length K")
            row[m] = cf // K
        # row / col uniform along k (over the live products)
        def first_live(d: dict) -> dict:
            out = {}
            j0 = np.argmax(live, axis=1)
            for m, cf in d.items():
                v = cf[np.arange(t.size), j0]
                if np.any((cf != v[:, None]) & live):
                    raise Unsupported("operand row/col varies along k")
                out[m] = v
            return out
        row1 = first_live(row)
        col1 = first_live(b_col)
        m_sym = _atoms_match(recs, AR, AT, {m: np.repeat(c[:, None], AR.shape[1], 1) for m, c in row1.items()},
                             m_sym, live)
        n_found = _atoms_match(recs, BR, BT, {m: np.repeat(c[:, None], BR.shape[1], 1) for m, c in col1.items()},
                               None, live)
        if n_found is not None and n_found != ldb_sym:
            raise Unsupported("B's column bound differs from its row stride")
        # output offset row * ldb + col, masks row < M / col < N
        offp = {m: c[t] for m, c in off.t.items()}
        o_row, o_col = _split(offp, {(ldb_sym,): 1}, t.shape)
        if not (_same(o_row, row1) and _same(o_col, col1)):
            raise Unsupported("output offset is not row*ldb + col of its products")
        out_row = out_col = False
        for atom in cond.atoms:
            at_ = {m: c[t] for m, c in atom.t.items()}
            neg = [m for m, c in at_.items() if len(m) == 1 and not m[0].startswith("%p") and np.all(c == -1)]
            if len(neg) != 1:
                raise Unsupported("output mask is not `index < scalar`")
            rest = {m: c for m, c in at_.items() if m != neg[0]}
            sym = neg[0][0]
            if _same(rest, row1) and (m_sym is None or m_sym == sym):
                m_sym, out_row = sym, True
            elif _same(rest, col1) and sym == ldb_sym:
                out_col = True
            else:
                raise Unsupported("output mask is not row < M / col < N")
        # a bound is either applied to the operand and the output, or nowhere (a full-tile kernel)
        masks = (n_found is not None, out_col)
        if masks[0] != masks[1] or (col_masked is not None and col_masked != masks[0]):
            raise Unsupported("column bound applied inconsistently")
        col_masked = masks[0]
        r_axis, TM, r_off, r_base = _as_tile(row1, "row")
        c_axis, TN, c_off, c_base = _as_tile(col1, "col")
        if r_axis == c_axis:
            raise Unsupported("rows and cols indexed by the same program id")
        if tile is None:
            tile = (r_axis, TM, c_axis, TN, r_base, c_base)
        if tile != (r_axis, TM, c_axis, TN, r_base, c_base):
            raise Unsupported("outputs use different tilings")
        row_masked_out.append(out_row)
        rows_all.append(r_off)
        cols_all.append(c_off)
    assert tile is not None and K is not None
    r_axis, TM, c_axis, TN, r_base, c_base = tile
    pos = np.concatenate(rows_all) * TN + np.concatenate(cols_all)
    if pos.size != TM * TN or not np.array_equal(np.sort(pos), np.arange(TM * TN)):
        raise Unsupported("the outputs do not cover a TM x TN tile exactly once")
    # the row bound, when there is one, guards the A loads and every output store
    if m_sym is not None and not all(row_masked_out):
        raise Unsupported("row bound applied inconsistently")
    args = {x.name: x for x in ir.args}
    if (m_sym is not None and m_sym not in args) or ldb_sym not in args:
        raise Unsupported("bounds are not kernel arguments")
    dts = (args[a_buf].dtype, args[b_buf].dtype, args[c_name].dtype)
    if dts != (DType.F32, DType.F32, DType.F32):
        raise Unsupported("the fp32 GEMM lift takes f32 A, B and C")
    return GemmSpec(a=a_buf, b=b_buf, c=c_name, m_sym=m_sym, n_sym=ldb_sym, K=int(K), TM=TM, TN=TN,
                    row_axis=int(r_axis[2:]), a_dtype=DType.F32, b_dtype=DType.F32, c_dtype=DType.F32,
                    c_f16=False, f32=True, row_base=r_base, col_base=c_base, col_masked=bool(col_masked))


# ---------------------------------------------------------------------------
# lowering and launch planning
# ---------------------------------------------------------------------------


def try_lift(ir: IRModule, block: int) -> Any:
    """Lowered MFMA GEMM for ``ir`` if it provably is one, else ``None``."""
    import os

    if os.environ.get("EAS_HIP_DISABLE_GEMM_LIFT", "") not in ("", "0"):
        return None
    ops = {i.op for i in ir.insts}
    try:
        if "mma" in ops:
            spec = analyze(ir, block)
        elif "dot" in ops:
            spec = analyze_dot(ir, block)
        else:
            return None
    except Unsupported:
        return None
    from .gemm_kernels import emit_gemm

    return emit_gemm(ir, block, spec)


def _numel(v: Any) -> int | None:
    """Element count of a buffer argument (numpy array, torch tensor, eas.Tensor)."""
    numel = getattr(v, "numel", None)
    if callable(numel):
        return int(numel())
    shape = getattr(v, "shape", None)
    if shape is not None:
        n = 1
        for d in shape:
            n *= int(d)
        return n
    return None


def plan_gemm(geo: Any, groups: tuple[int, int, int], runtime_args: Any, live_x: int | None,
              compute_units: int = 256) -> Any:
    """Launch plan of a lifted GEMM for a reference grid ``groups``.

    The launch covers rows [m_lo, m_hi) and columns [n_lo, n_hi): the origin is
    TM * row_base (TN * col_base) when the kernel offsets its program ids by a
    scalar, the extent is the launched grid, clamped to M (N) when the kernel
    bounds rows (columns).  Every buffer must hold what that rectangle touches;
    a launch that would read or write past one raises instead of running.
    """
    from ..runtime.hip import LaunchPlan

    if live_x is not None:
        raise ValueError("a lifted GEMM kernel needs a 2-D grid (pass _grid=...)")
    p = geo.params
    K = int(p["K"])
    ldb = int(runtime_args[p["n_sym"]])
    g_rows = groups[p["row_axis"]]
    g_cols = groups[1 - p["row_axis"]]
    m_lo = p["TM"] * int(runtime_args[p["row_base"]]) if p.get("row_base") else 0
    n_lo = p["TN"] * int(runtime_args[p["col_base"]]) if p.get("col_base") else 0
    m_hi = m_lo + g_rows * p["TM"]
    n_hi = n_lo + g_cols * p["TN"]
    if p.get("m_sym"):
        m_hi = min(m_hi, int(runtime_args[p["m_sym"]]))
    if p.get("col_masked", True):
        n_hi = min(n_hi, ldb)
    if m_hi <= m_lo or n_hi <= n_lo:
        return None
    if max(m_hi * K, K * max(ldb, n_hi), m_hi * max(ldb, n_hi)) >= 1 << 32:
        raise ValueError("lifted GEMM: matrix too large for u32 indexing")
    need = {p["a"]: m_hi * K, p["b"]: (K - 1) * ldb + n_hi, p["c"]: (m_hi - 1) * ldb + n_hi}
    for name, n_need in need.items():
        have = _numel(runtime_args.get(name)) if name in runtime_args else None
        if have is not None and have < n_need:
            raise ValueError(f"buffer {name!r} holds {have} elements; this launch touches {n_need}")
    hidden = (m_lo, m_hi, n_lo, n_hi)
    m, n = m_hi - m_lo, n_hi - n_lo
    tiles = -(-m // p["BM"]) * -(-n // p["BN"])
    tiles128 = -(-m // 128) * -(-n // 128)
    tiles128x256 = -(-m // 128) * -(-n // 256)
    tiles128x64 = -(-m // 128) * -(-n // 64)
    tiles64 = -(-m // 64) * -(-n // 64)
    choice = _gemm_entry_choice()
    if m <= p.get("skinny_m", 0):
        # The 4-wave entry runs its skinny path for every launch of at most skinny_m rows (one
        # workgroup per skinny_n columns, all rows), so it is only ever launched on that grid.
        # Up to WIDE_M rows, a launch whose groups would take more than one round of CUs gets
        # twice the columns per workgroup (the kernel reads which from the grid).  From 17 rows
        # on, a launch whose groups still take more than one round goes to the 128 x 128 entry
        # instead (or to the entry EAS_HIP_GEMM_ENTRY names).
        groups = -(-n // p["skinny_n"])
        if m <= WIDE_M and groups > compute_units:
            groups = -(-n // (2 * p["skinny_n"]))
        other = None
        if m > SKINNY_CUT and p.get("pp_entry") and _dma_fits(p, runtime_args, K, ldb, m, n_lo, n):
            if choice == "tile128" or (choice == "auto" and groups > compute_units):
                other = LaunchPlan((tiles128, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t128_entry"])
            elif choice == "tile128x256":
                other = LaunchPlan((tiles128x256, 1, 1), (p["t128_threads"], 1, 1), hidden,
                                   entry=p["t128x256_entry"])
            elif choice == "tile128x64":
                other = LaunchPlan((tiles128x64, 1, 1), (p["t128_threads"], 1, 1), hidden,
                                   entry=p["t128x64_entry"])
            elif choice == "tile64":
                other = LaunchPlan((tiles64, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t64_entry"])
            elif choice == "8wave":
                other = LaunchPlan((tiles, 1, 1), (p["pp_threads"], 1, 1), hidden, entry=p["pp_entry"])
        return other or LaunchPlan((groups, 1, 1), (p["threads"], 1, 1), hidden)
    if p.get("f32"):
        # fp32: 128 x 128 tiles (a quarter of the DMA bytes per flop) while they still give every CU one
        if p.get("t128_entry") and _dma_fits(p, runtime_args, K, ldb, m, n_lo, n, elem=4) and (
                choice == "tile128" or (choice == "auto" and tiles128 >= compute_units)):
            return LaunchPlan((tiles128, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t128_entry"])
        return LaunchPlan((tiles, 1, 1), (p["threads"], 1, 1), hidden)
    if p.get("pp_entry") and choice != "4wave" and _dma_fits(p, runtime_args, K, ldb, m, n_lo, n):
        # When 256 x 256 tiles would fill at most half of the CUs: 128 x 128 tiles if they take one
        # round of CUs, else 128 x 256 ones (at most twice the 256 x 256 count, so one round too).
        # If even 128 x 128 would fill at most half of the CUs: 64 x 64 tiles while they need at most
        # 1.75 rounds of CUs, else 128 x 64 (twice the 128 x 128 count: one round).
        small = choice == "auto" and 2 * tiles <= compute_units
        if choice == "tile128x256" or (small and tiles128 > compute_units):
            return LaunchPlan((tiles128x256, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t128x256_entry"])
        tiny = small and 2 * tiles128 <= compute_units
        if choice == "tile64" or (tiny and 4 * tiles64 <= 7 * compute_units):
            return LaunchPlan((tiles64, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t64_entry"])
        if choice == "tile128x64" or tiny:
            return LaunchPlan((tiles128x64, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t128x64_entry"])
        if choice == "tile128" or small:
            return LaunchPlan((tiles128, 1, 1), (p["t128_threads"], 1, 1), hidden, entry=p["t128_entry"])
        return LaunchPlan((tiles, 1, 1), (p["pp_threads"], 1, 1), hidden, entry=p["pp_entry"])
    return LaunchPlan((tiles, 1, 1), (p["threads"], 1, 1), hidden)


_ENTRY_CHOICES = ("auto", "8wave", "tile128", "tile128x256", "tile128x64", "tile64", "4wave")
SKINNY_CUT = 16  # up to this many rows a launch always takes the skinny path
WIDE_M = 128  # up to this many rows the skinny path may take 128 columns per workgroup


def _gemm_entry_choice() -> str:
    """``EAS_HIP_GEMM_ENTRY``: ``auto`` (default), or one entry for every f16 launch
    the DMA takes: ``8wave``, ``tile128``, ``tile128x256``, ``tile128x64``, ``tile64`` or ``4wave``."""
    v = os.environ.get("EAS_HIP_GEMM_ENTRY", "auto").strip().lower() or "auto"
    if v not in _ENTRY_CHOICES:
        raise ValueError(f"EAS_HIP_GEMM_ENTRY must be one of {_ENTRY_CHOICES}, got {v!r}")
    return v


def _dma_fits(p: dict, runtime_args: Any, K: int, ldb: int, m: int, n_lo: int, n: int, elem: int = 2) -> bool:
    """Whether the DMA entries take this launch.  16-bit f16/bf16 (``elem`` 2): every row of A and B
    (after the move to the rectangle's origin) 4-byte aligned; fp32 (``elem`` 4): 16-byte
    aligned; each operand's extent under 2 GiB.  Device addresses are known here for
    torch tensors; numpy inputs are staged into fresh allocations, and the entries
    re-check the addresses they get (a misaligned operand takes their slow element-wise
    guard rather than a wrong result)."""
    step = 2 if elem == 2 else 4  # elements per aligned unit: 4 bytes of f16, 16 bytes of f32
    if K % step or ldb % step or n_lo % step:
        return False
    if m * K * elem >= 1 << 31 or ((K - 1) * ldb + n) * elem >= 1 << 31:
        return False
    for name in (p["a"], p["b"]):
        ptr = getattr(runtime_args.get(name), "data_ptr", None)
        if callable(ptr) and int(ptr()) % (2 * step if elem == 2 else 16):
            return False
    return True
