"""Seeded random eas kernels for differential tests: the HIP backend against the oracle interpreter.

``spmd_source(seed)`` and ``thread_source(seed)`` write the source of one random ``@eas.kernel``
over the public DSL (the ops of ``eas/mk.py`` the reference defines: ``+``, ``*``, ``//``, ``%``,
``<``, ``&``, ``|``, ``~``, ``where``, ``fma``, ``to_f16``, ``to_f32``, masked ``load`` /
``store``, and in thread mode ``tid``, ``local_id``, ``lane_id``, ``sg_id``, ``alloc_tg`` and
``barrier`` and ``dot``), with runtime f32 and u32 scalars and, for some SPMD kernels, a 2-D
grid.  ``case(seed)`` gives a kernel source and its launch, ``build(src)`` the kernel and
``inputs(seed, n)`` the arguments.  Every index a kernel computes stays inside its buffers
(gathers are reduced ``% N``, threadgroup slots ``% BLOCK``, dot windows ``% 1800`` with N >=
2048), every divisor is a literal >= 1, and the f32 values come from N(0,1) inputs, so each
program has one defined result for the oracle to give.
"""

from __future__ import annotations

import random

import numpy as np

import eas
from eas import mk

_F_LITS = ("0.5", "1.5", "2.0", "0.1", "0.003", "10000.0", "7.25", "1e-20", "3.0e5")
_U_LITS = (1, 2, 3, 5, 7, 31, 64, 1000)


class _Gen:
    """Straight-line random program: pools of named f32, f16, u32 and bool values."""

    def __init__(self, rng: random.Random):
        self.r = rng
        self.lines: list[str] = []
        self.f: list[str] = []
        self.h: list[str] = []
        self.u: list[str] = []
        self.b: list[str] = []
        self.n = 0

    def emit(self, pool: list[str], expr: str) -> str:
        name = f"t{self.n}"
        self.n += 1
        self.lines.append(f"    {name} = {expr}")
        pool.append(name)
        return name

    def pick(self, pool: list[str]) -> str:
        # favour recent values so that chains grow deep, but reuse old ones too (multi-use
        # products decide whether an add may fuse into an fma)
        k = len(pool)
        return pool[min(k - 1, int(self.r.expovariate(0.35)))] if self.r.random() < 0.3 else pool[-1 - min(
            k - 1, int(self.r.expovariate(0.5)))]

    def f_expr(self) -> str:
        r, p = self.r, self.pick
        kind = r.randrange(13)
        if kind == 0:
            return f"{p(self.f)} + {p(self.f)}"
        if kind == 1:
            return f"{p(self.f)} * {p(self.f)}"
        if kind == 2:
            return f"{p(self.f)} * {p(self.f)} + {p(self.f)}"  # fuses (single-use product)
        if kind == 3:
            return f"{p(self.f)} + {p(self.f)} * {p(self.f)}"  # product second: fuses too
        if kind == 4:
            return f"mk.fma({p(self.f)}, {p(self.f)}, {p(self.f)})"
        if kind == 5:
            lit = r.choice(_F_LITS)
            return f"{p(self.f)} * {lit}" if r.random() < 0.5 else f"{lit} + {p(self.f)}"
        if kind == 6:
            return f"mk.where({p(self.b)}, {p(self.f)}, {p(self.f)})"
        if kind == 7 and self.h:
            return f"mk.to_f32({p(self.h)})"
        if kind == 8:
            return f"mk.to_f32(mk.to_f16({p(self.f)}))"
        if kind == 9 and self.u:
            return f"mk.to_f32({p(self.u)} % {r.choice((1000, 4096, 65536))})"
        if kind == 11 and self.b:
            return f"mk.to_f32({p(self.b)}) * {p(self.f)}"
        if kind == 10 and len(self.f) >= 2:
            # a product used twice: neither add may fuse it
            prod = self.emit(self.f, f"{p(self.f)} * {p(self.f)}")
            self.emit(self.f, f"{prod} + {p(self.f)}")
            return f"{p(self.f)} + {prod}"
        return f"{p(self.f)} + {r.choice(_F_LITS)}"

    def h_expr(self) -> str:
        r, p = self.r, self.pick
        kind = r.randrange(8)
        if kind == 0:
            return f"{p(self.h)} + {p(self.h)}"
        if kind == 1:
            return f"{p(self.h)} * {p(self.h)}"
        if kind == 2:
            return f"mk.fma({p(self.h)}, {p(self.h)}, {p(self.h)})"
        if kind == 3:
            return f"mk.where({p(self.b)}, {p(self.h)}, {p(self.h)})"
        if kind == 4:
            # f32 values can be large (products of products): scale before narrowing
            return f"mk.to_f16({p(self.f)} * 0.001)"
        if kind == 6 and self.u:
            return f"mk.to_f16({p(self.u)} % 70000)"
        if kind == 7 and self.b:
            return f"mk.to_f16({p(self.b)}) + {p(self.h)}"
        return f"{p(self.h)} * {p(self.h)} + {p(self.h)}"  # f16: never fused, two roundings

    def b_expr(self) -> str:
        r, p = self.r, self.pick
        kind = r.randrange(7)
        if kind == 0:
            return f"{p(self.f)} < {p(self.f)}"
        if kind == 1:
            return f"{p(self.f)} < {r.choice(_F_LITS)}"
        if kind == 2 and self.u:
            return f"{p(self.u)} < {r.choice(_U_LITS) * 3}"
        if kind == 3 and len(self.b) >= 2:
            return f"{p(self.b)} & {p(self.b)}"
        if kind == 4 and len(self.b) >= 2:
            return f"{p(self.b)} | {p(self.b)}"
        if kind == 5 and self.b:
            return f"~{p(self.b)}"
        return f"{p(self.h)} < {p(self.h)}" if self.h else f"{p(self.f)} < {p(self.f)}"

    def u_expr(self) -> str:
        r, p = self.r, self.pick
        kind = r.randrange(7)
        if kind == 0:
            return f"{p(self.u)} % {r.choice(_U_LITS)}"
        if kind == 1:
            return f"{p(self.u)} // {r.choice(_U_LITS)}"
        if kind == 2:
            return f"{p(self.u)} * {r.choice(_U_LITS)} + {r.choice(_U_LITS)}"
        if kind == 3:
            return f"{p(self.u)} + {p(self.u)}"
        if kind == 4:
            return f"mk.to_u32({p(self.f)} * 100.0)"  # negative and NaN saturate to 0
        if kind == 5 and self.b:
            return f"mk.where({p(self.b)}, {p(self.u)}, {p(self.u)})"
        return f"({p(self.u)} * {r.choice(_U_LITS)}) % 4099"

    def body(self, n_stmts: int) -> None:
        for _ in range(n_stmts):
            k = self.r.random()
            if k < 0.5:
                self.emit(self.f, self.f_expr())
            elif k < 0.65:
                self.emit(self.h, self.h_expr())
            elif k < 0.85:
                self.emit(self.b, self.b_expr())
            else:
                self.emit(self.u, self.u_expr())


def _loads(g: _Gen, index: str, mask: str, nvar: str) -> None:
    g.f.append("alpha")  # runtime f32 scalar
    g.u.append("S")  # runtime u32 scalar
    g.lines += [
        f"    a = mk.load(x, {index}, {mask})",
        f"    b = mk.load(y, {index}, {mask})",
        f"    c = mk.load(z, {index}, {mask})",
        f"    hh = mk.load(h, {index}, {mask})",
        f"    gi = ({index} * 7 + 3) % {nvar}",
        f"    ga = mk.load(x, gi, {mask})",
    ]
    g.f += ["a", "b", "c", "ga"]
    g.h += ["hh"]
    g.u += [index, "gi"]
    g.b += [mask]


def _stores(g: _Gen, index: str, mask: str) -> None:
    # fold a few more values into each output so that most of the program stays live
    f_out = g.f[-1]
    for v in g.r.sample(g.f[:-1], min(3, len(g.f) - 1)):
        f_out = g.emit(g.f, f"{f_out} + {v}")
    h_out = g.h[-1]
    if len(g.h) > 1:
        h_out = g.emit(g.h, f"{h_out} + {g.r.choice(g.h[:-1])}")
    g.lines.append(f"    mk.store(out, {index}, {f_out}, {mask})")
    if g.r.random() < 0.5:
        # a second, conditional store to the same elements: program order decides
        g.lines.append(f"    mk.store(out, {index}, {g.pick(g.f)}, {mask} & {g.pick(g.b)})")
    g.lines.append(f"    mk.store(out16, {index}, {h_out}, {mask})")


SIGNATURE = "def fuzz(x, y, z, h, out, out16, N, alpha, S, BLOCK: eas.constexpr):"


def spmd_source(seed: int, n_stmts: int = 20, grid_x: int = 0) -> str:
    """An SPMD (``mk.arange``) kernel ``fuzz(x, y, z, h, out, out16, N, alpha, S, BLOCK)``.  With
    ``grid_x`` > 0 the programs form a 2-D grid of ``grid_x`` columns (launch with ``_grid``) and
    program (px, py) covers block py * grid_x + px."""
    g = _Gen(random.Random(seed))
    pid = "mk.program_id(0)" if grid_x <= 0 else f"mk.program_id(1) * {grid_x} + mk.program_id(0)"
    g.lines = [SIGNATURE,
               f"    pid = {pid}",
               "    offs = pid * BLOCK + mk.arange(0, BLOCK)",
               "    m = offs < N"]
    g.u.append("pid")
    _loads(g, "offs", "m", "N")
    g.body(n_stmts // 2)
    if g.r.random() < 0.3:
        # lanes of one program exchange a value through threadgroup memory
        g.lines += ["    lanes = mk.arange(0, BLOCK)",
                    "    tgs = mk.alloc_tg(BLOCK)",
                    f"    mk.store(tgs, lanes, {g.pick(g.f)})",
                    "    mk.barrier()",
                    f"    xs = mk.load(tgs, (lanes * {g.r.choice((1, 3, 5, 7, 33))} + {g.r.randrange(64)}) % BLOCK)"]
        g.f.append("xs")
    g.body(n_stmts - n_stmts // 2)
    _stores(g, "offs", "m")
    return "\n".join(g.lines) + "\n"


def thread_source(seed: int, n_stmts: int = 20, exchange: bool | None = None) -> str:
    """A thread-mode (``mk.tid``) kernel ``fuzz(x, y, z, h, out, out16, N, BLOCK)``; with
    ``exchange`` (default: seeded) a value goes through threadgroup memory to another thread
    of the group (``(lid * p + q) % BLOCK``) between two barriers."""
    r = random.Random(seed)
    g = _Gen(r)
    g.lines = [SIGNATURE,
               "    i = mk.tid(0, BLOCK)",
               "    m = i < N",
               "    lid = mk.local_id(0)",
               "    lane = mk.lane_id()",
               "    sg = mk.sg_id()"]
    g.u += ["lid", "lane", "sg"]
    _loads(g, "i", "m", "N")
    g.body(n_stmts // 2)
    if exchange if exchange is not None else r.random() < 0.6:
        src = g.pick(g.f)
        mult = r.choice((1, 3, 5, 7, 33))
        g.lines += ["    tg = mk.alloc_tg(BLOCK)",
                    f"    mk.store(tg, lid, {src})",
                    "    mk.barrier()",
                    f"    xr = mk.load(tg, (lid * {mult} + {r.randrange(64)}) % BLOCK)"]
        g.f.append("xr")
    for _ in range(r.randrange(3)):
        # a per-thread dot product over a strided window of two buffers (f32 or f16 operands);
        # bases are reduced % 1800 and spans stay < 200, so every index is < N (N >= 2048)
        ka, kb = r.choice(("x", "y", "z", "h")), r.choice(("x", "y", "z", "h"))
        base_a = f"({g.pick(g.u)} * {r.choice(_U_LITS)}) % 1800"
        base_b = f"({g.pick(g.u)} + {r.randrange(100)}) % 1800"
        kd = r.randrange(1, 40)
        g.emit(g.f, f"mk.dot({ka}, {base_a}, {r.randrange(1, 5)}, {kb}, {base_b}, {r.randrange(0, 5)}, {kd})")
    g.body(n_stmts - n_stmts // 2)
    _stores(g, "i", "m")
    return "\n".join(g.lines) + "\n"


def build(src: str):
    """The ``@eas.kernel`` the source defines."""
    ns: dict = {"eas": eas, "mk": mk}
    exec(compile(src, "<fuzz kernel>", "exec"), ns)  # noqa: S102 - test programs written above
    return eas.kernel(ns["fuzz"])


def inputs(seed: int, n: int) -> tuple:
    """x, y, z ~ N(0,1) f32, h ~ N(0,1) f16, out and out16 zero, then N, alpha (an f32 scalar)
    and S (a u32 scalar)."""
    rng = np.random.default_rng(seed)
    x, y, z = (rng.standard_normal(n, dtype=np.float32) for _ in range(3))
    h = rng.standard_normal(n, dtype=np.float32).astype(np.float16)
    alpha = float(np.float32(rng.uniform(0.25, 4.0)))
    return x, y, z, h, np.zeros(n, np.float32), np.zeros(n, np.float16), n, alpha, int(rng.integers(0, 5000))


def case(seed: int) -> dict:
    """Launch of fuzz case ``seed``: ``mode``, ``N``, ``BLOCK``, the kernel ``src`` and the call's
    ``options`` (``_grid`` for a 2-D SPMD grid).  Thread-mode kernels get N >= 2048 (the dot
    windows); those with a threadgroup exchange get N a multiple of BLOCK (a partial last group
    would read slots no thread wrote), the others often a partial last group."""
    r = random.Random(10_000 + seed)
    mode = "spmd" if seed % 2 == 0 else "thread"
    # seeds from 200 on also take BLOCKs that are not powers of two, and the extremes, so the
    # emitters' workgroup mappings meet thread counts their workgroup sizes do not divide
    block = r.choice((64, 128, 256)) if seed < 200 else r.choice((32, 96, 100, 200, 384, 1000, 1024))
    n = r.randrange(1, 9000)
    options: dict = {}
    if mode == "thread" and r.random() < 0.4:
        # a partial last threadgroup: exactly N threads exist, so no threadgroup exchange
        n = max(2048, n)
        src = thread_source(seed, exchange=False)
    elif mode == "thread":
        n = max(-(-2048 // block) * block, n - n % block)  # whole threadgroups, at least 2048 threads
        src = thread_source(seed)
    elif seed % 4 == 2:
        # 2-D grid: enough programs for N, laid out grid_x wide
        grid_x = r.choice((1, 2, 3, 5))
        programs = -(-n // block)
        options["_grid"] = (grid_x, -(-programs // grid_x), 1)
        src = spmd_source(seed, grid_x=grid_x)
    else:
        src = spmd_source(seed)
    return {"mode": mode, "N": n, "BLOCK": block, "src": src, "options": options}


def same_values(got: np.ndarray, want: np.ndarray) -> bool:
    """Bit-equal, except that any NaN matches any NaN (payloads are not part of the contract)."""
    got, want = np.asarray(got), np.asarray(want)
    if got.shape != want.shape or got.dtype != want.dtype:
        return False
    gn, wn = np.isnan(got), np.isnan(want)
    if not np.array_equal(gn, wn):
        return False
    bits = np.uint32 if got.dtype == np.float32 else np.uint16
    return bool(np.array_equal(got[~gn].view(bits), want[~wn].view(bits)))
