"""Lifted GEMMs at the reference's native launch convention, on the CPU.

The reference runtime launches its matmul kernels like any other pipeline:
``launch(pipeline, argv, writable, threads_per_grid, threads_per_threadgroup)``
with ``threads_per_grid = (gx * BLOCK, gy, gz)`` (eas/runtime/metal.py:307-346,
_metal.mm:1013-1222), or ``launch_tg`` with threadgroup counts
(_metal.mm:1232-1379).  Here such a kernel may have been lifted to an MFMA GEMM
with several entry points, so ``eas_hip_launch_threads/threadgroups`` plan it in
C (``eas_hip_plan_gemm``) from M, N and the tile bases in the packed arguments,
the buffers' lengths and the compute units.  ``eas._hip.plan_dispatch`` exposes
that planner without a GPU; every case below must land on what the Python
runtime's ``gemm_lift.plan_gemm`` plans for the same call: the same entry,
workgroups, block and covered rectangle, the same launches refused, the same
launches that run nothing.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

import kernels as K
from easy_as_amd.codegen.gemm_lift import plan_gemm
from easy_as_amd.codegen.hip import GEMM_ENTRY_BITS
from easy_as_amd.runtime.hip import pack_scalar, plan_launch
from easy_as_amd.runtime.hip_ext import load_hip_ext
from metal_dispatch import reference_dispatch


@pytest.fixture(scope="module")
def hip():
    return load_hip_ext(require=True)


class Buf:
    """A device buffer as both planners see it: its element count and address."""

    def __init__(self, numel: int, ptr: int, itemsize: int) -> None:
        self.n, self.ptr, self.itemsize = numel, ptr, itemsize

    def numel(self) -> int:
        return self.n

    def data_ptr(self) -> int:
        return self.ptr


_ITEMSIZE = {"f16": 2, "bf16": 2, "f32": 4}


def _args(ck, m: int, n: int, k: int, *, extra=None, short=None, misalign=None):
    """Runtime arguments of an M x N x K launch: buffers sized exactly for the matrices (one
    `short` buffer an element too small), at 256-byte aligned addresses (`misalign`: that
    buffer 2 bytes off)."""
    p = ck.geometry.params
    sizes = {p["a"]: m * k, p["b"]: k * n, p["c"]: m * n}
    args, base = {}, 1 << 20
    for a in ck.ir.args:
        if a.kind == "buffer":
            numel = sizes[a.name] - (1 if a.name == short else 0)
            ptr = base + (2 if a.name == misalign else 0)
            args[a.name] = Buf(numel, ptr, _ITEMSIZE[a.dtype.value])
            base += (numel * 4 + (1 << 20)) // 256 * 256
        elif a.name == "M":
            args[a.name] = m
        elif a.name == "N":
            args[a.name] = n
        else:
            args[a.name] = 0
    args.update(extra or {})
    return args


def _argv(hip, ck, args):
    """argv as the reference runtime builds it (metal.py:142-242): buffers, then packed scalars."""
    out = []
    for a in ck.ir.args:
        v = args[a.name]
        out.append(hip.wrap_pointer(v.ptr, v.n * v.itemsize) if a.kind == "buffer" else pack_scalar(a.dtype, v))
    return out


def _both(hip, ck, args, groups, *, cus=256, choice="auto", by_groups=True):
    """(C plan, Python plan) of a launch of `groups` threadgroups, each as (grid, block, hidden,
    entry), None when nothing runs, or the exception type and message it raised."""
    tpg = groups if by_groups else (groups[0] * ck.block_size, groups[1], groups[2])
    try:
        c = hip.plan_dispatch(ck.src, tpg, (ck.block_size, 1, 1), by_groups, argv=_argv(hip, ck, args),
                              compute_units=cus, entry_choice=choice)
    except ValueError as e:
        c = ("ValueError", str(e))
    import os

    old = os.environ.get("EAS_HIP_GEMM_ENTRY")
    os.environ["EAS_HIP_GEMM_ENTRY"] = choice
    try:
        plan = plan_gemm(ck.geometry, tuple(groups), args, None, cus)
        py = None if plan is None else (plan.grid, plan.block, plan.hidden, plan.entry)
    except ValueError as e:
        py = ("ValueError", str(e))
    finally:
        if old is None:
            del os.environ["EAS_HIP_GEMM_ENTRY"]
        else:
            os.environ["EAS_HIP_GEMM_ENTRY"] = old
    return c, py


def _agree(c, py):
    if isinstance(py, tuple) and py and py[0] == "ValueError":
        return isinstance(c, tuple) and c[0] == "ValueError"
    return c == py


def _mma(kname="matmul_mma_kernel", k=4096, a=np.float16, c=np.float32):
    return getattr(K, kname).compile(np.zeros(8, a), np.zeros(8, a), np.zeros(8, c), 64, 64, BM=32, BN=32, BK=8,
                                     K=k, NT=512)


# M x N x K: the configs' shapes, skinny launches of 1-128 rows (one and two rounds of CUs),
# each smaller-tile regime, edge tiles, K tails, K not a multiple of 4 bytes (odd K, K % 4 == 2)
_MNK = [(4096, 4096, 4096), (4096, 4096, 4100), (16, 14336, 4096), (8192, 8192, 8192), (300, 520, 200),
        (33, 17, 100), (1, 104, 72), (17, 300, 72), (65, 300, 72), (128, 16390, 200), (100, 40960, 512),
        (16, 28672, 4096), (48, 28672, 2048), (2048, 2048, 2048), (1024, 1024, 1024), (512, 14336, 1024),
        (768, 768, 768), (2048, 1024, 2048), (2560, 2560, 2560), (512, 512, 4096), (260, 264, 33),
        (300, 256, 50), (7, 101, 64), (3072, 3072, 3072), (129, 64, 64)]


@pytest.mark.parametrize("mnk", _MNK, ids=lambda s: "x".join(map(str, s)))
def test_c_plan_matches_plan_gemm_on_the_reference_grid(hip, mnk):
    m, n, k = mnk
    ck = _mma(k=k)
    args = _args(ck, m, n, k)
    groups = K.mma_grid({"BM": 32, "BN": 32}, args)
    for cus, by_groups in itertools.product((256, 80), (True, False)):
        c, py = _both(hip, ck, args, groups, cus=cus, by_groups=by_groups)
        assert c == py, (mnk, cus, by_groups, c, py)
    # the same through plan_launch, as HipRuntime.run plans the call
    plan = plan_launch(ck, args, grid=groups)
    assert hip.plan_dispatch(ck.src, groups, (512, 1, 1), True, argv=_argv(hip, ck, args)) == \
        (plan.grid, plan.block, plan.hidden, plan.entry)


@pytest.mark.parametrize("choice", ["auto", "8wave", "tile128", "tile128x256", "tile128x64", "tile64", "4wave"])
def test_every_entry_override_plans_alike(hip, choice):
    ck = _mma(k=1024)
    for m, n in ((4096, 4096), (40, 28672), (12, 4096), (1024, 1024), (200, 3000), (129, 16448)):
        args = _args(ck, m, n, 1024)
        c, py = _both(hip, ck, args, K.mma_grid({"BM": 32, "BN": 32}, args), choice=choice)
        assert c == py, (choice, m, n, c, py)


def test_partial_and_oversized_grids(hip):
    # a grid covering part of C (the launch covers its rectangle only), and one past M and N
    # (clamped to M and N, as the kernel's masks bound it)
    ck = _mma(k=512)
    args = _args(ck, 1000, 700, 512)
    for groups in ((3, 2, 1), (1, 1, 1), (22, 32, 1), (40, 50, 1), (22, 1, 4), (1, 32, 1)):
        c, py = _both(hip, ck, args, groups)
        assert c == py and c is not None, (groups, c, py)


def test_dtypes_and_output_types(hip):
    # f16 output, bf16 operands, f32 inputs rounded to f16 (the register-staged body only)
    for kname, a, c in (("matmul_mma_f16out_kernel", np.float16, np.float16),
                        ("matmul_mma_bf16_kernel", None, np.float32),
                        ("matmul_mma_kernel", np.float32, np.float32)):
        if a is None:
            import torch

            z = torch.zeros(8, dtype=torch.bfloat16)
            ck = K.matmul_mma_bf16_kernel.compile(z, z, torch.zeros(8), 64, 64, BM=32, BN=32, BK=8, K=4096, NT=512)
        else:
            ck = _mma(kname, 4096, a, c)
        for m, n in ((16, 14336), (8192, 8192), (4096, 4096), (100, 200)):
            args = _args(ck, m, n, 4096)
            cp, py = _both(hip, ck, args, K.mma_grid({"BM": 32, "BN": 32}, args))
            assert cp == py, (kname, m, n, cp, py)


@pytest.mark.parametrize("mnk,bases", [((1024, 1024, 1024), (0, 0)), ((2048, 2048, 2048), (0, 0)),
                                       ((4096, 3000, 96), (0, 0)), ((2048, 2048, 100), (0, 0)),
                                       ((1000, 1000, 64), (5, 3)), ((300, 200, 32), (9, 0)),
                                       ((300, 200, 32), (0, 6)), ((300, 200, 32), (10, 0))])
def test_tiled_fp32_with_tile_bases(hip, mnk, bases):
    # the reference's tiled fp32 matmul offsets its threadgroup ids by PID_M_BASE and PID_N_BASE;
    # (10, 0) starts past M = 300 (32-row tiles): nothing runs
    m, n, k = mnk
    f = np.zeros(8, np.float32)
    ck = K.matmul_tiled_kernel.compile(f, f, f, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
    assert ck.geometry.kind == "gemm"
    args = _args(ck, m, n, k, extra={"PID_M_BASE": bases[0], "PID_N_BASE": bases[1]})
    groups = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
    for cus in (256, 64):
        c, py = _both(hip, ck, args, groups, cus=cus)
        assert c == py, (mnk, bases, cus, c, py)
    if bases == (10, 0):
        assert c is None


def test_alignment_decides_the_dma_entries(hip):
    # an operand 2 bytes off a 4-byte boundary cannot take the DMA entries: both planners fall
    # back to the kernel's own entry (whose register-staged body reads any alignment)
    ck = _mma(k=4096)
    for misalign in ("a", "b", "c", None):
        args = _args(ck, 4096, 4096, 4096, misalign=misalign)
        c, py = _both(hip, ck, args, K.mma_grid({"BM": 32, "BN": 32}, args))
        assert c == py, (misalign, c, py)
        assert (c[3] is None) == (misalign in ("a", "b"))
    # fp32: rows of A and B must be 16-byte aligned for the 128 x 128 entry
    f = np.zeros(8, np.float32)
    ck = K.matmul_tiled_kernel.compile(f, f, f, 64, 64, 0, 0, BM=32, BN=32, BK=32, K=2048, NT=256)
    for n in (2048, 2046, 2050):
        args = _args(ck, 2048, n, 2048)
        c, py = _both(hip, ck, args, (K.cdiv(n, 32), 64, 1))
        assert c == py, (n, c, py)


def test_refusals_match(hip):
    ck = _mma(k=200)
    grid = K.mma_grid({"BM": 32, "BN": 32}, {"M": 300, "N": 520})
    # a buffer one element short of what the launch touches: both refuse, naming it
    for short in ("a", "b", "c"):
        c, py = _both(hip, ck, _args(ck, 300, 520, 200, short=short), grid)
        assert c[0] == py[0] == "ValueError" and "holds" in c[1] and "holds" in py[1], (short, c, py)
    # matrices past u32 indexing
    big = _mma(k=1 << 16)
    c, py = _both(hip, big, _args(big, 1 << 16, 64, 1 << 16), (2, 2048, 1))
    assert c[0] == py[0] == "ValueError" and "u32" in c[1], (c, py)
    argv = _argv(hip, ck, _args(ck, 300, 520, 200))
    # a partial threadgroup: the lift proved what whole threadgroups compute
    with pytest.raises(ValueError, match="whole threadgroups"):
        hip.plan_dispatch(ck.src, (17 * 512 - 1, 10, 1), (512, 1, 1), argv=argv)
    with pytest.raises(ValueError, match=r"\(512, 1, 1\)"):
        hip.plan_dispatch(ck.src, (17, 10, 1), (1, 1, 1), True, argv=argv)
    with pytest.raises(ValueError, match="must be > 0"):
        hip.plan_dispatch(ck.src, (17, 0, 1), (512, 1, 1), True, argv=argv)
    with pytest.raises(ValueError, match="EAS_HIP_GEMM_ENTRY"):
        hip.plan_dispatch(ck.src, (17, 10, 1), (512, 1, 1), True, argv=argv, entry_choice="tile32")
    # the plan reads M and N from argv: a short argv is refused, a missing one too
    with pytest.raises(ValueError, match="packed arguments"):
        hip.plan_dispatch(ck.src, (17, 10, 1), (512, 1, 1), True, argv=argv[:3])
    with pytest.raises(TypeError, match="argv"):
        hip.plan_dispatch(ck.src, (17, 10, 1), (512, 1, 1), True)


def test_entry_override_read_from_the_environment(hip, monkeypatch):
    ck = _mma(k=1024)
    args = _args(ck, 4096, 4096, 1024)
    grid = K.mma_grid({"BM": 32, "BN": 32}, args)
    argv = _argv(hip, ck, args)
    assert hip.plan_dispatch(ck.src, grid, (512, 1, 1), True, argv=argv)[3] == "matmul_mma_kernel__pp"
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", " Tile128 ")
    assert hip.plan_dispatch(ck.src, grid, (512, 1, 1), True, argv=argv)[3] == "matmul_mma_kernel__t128"
    assert plan_gemm(ck.geometry, grid, args, None).entry == "matmul_mma_kernel__t128"


def test_gemm_line_matches_the_geometry(hip):
    from easy_as_amd.codegen.gemm_lift import SKINNY_CUT, WIDE_M
    from easy_as_amd.codegen.hip import kernarg_offsets

    f = np.zeros(8, np.float32)
    for ck in (_mma(k=4100), _mma("matmul_mma_f16out_kernel", 4096, np.float16, np.float16),
               _mma(k=33), _mma(k=64, a=np.float32),
               K.matmul_tiled_kernel.compile(f, f, f, 64, 64, 0, 0, BM=32, BN=32, BK=32, K=1024, NT=256)):
        g = hip.launch_shape(ck.src)["gemm"]
        p = ck.geometry.params
        pos = {a.name: i for i, a in enumerate(ck.ir.args)}
        offs = kernarg_offsets(ck.ir)
        assert g["entry"] == ck.geometry.entry
        assert (g["K"], g["tm"], g["tn"], g["row_axis"], g["bm"], g["bn"]) == \
            (p["K"], p["TM"], p["TN"], p["row_axis"], p["BM"], p["BN"])
        assert (g["threads"], g["pp_threads"], g["t128_threads"]) == (p["threads"], p["pp_threads"], p["t128_threads"])
        assert (g["skinny_m"], g["skinny_n"], g["skinny_cut"], g["wide_m"]) == \
            (p["skinny_m"], p["skinny_n"], SKINNY_CUT, WIDE_M)
        assert (g["a_arg"], g["b_arg"], g["c_arg"]) == (pos[p["a"]], pos[p["b"]], pos[p["c"]])
        assert g["ldb_off"] == offs[pos[p["n_sym"]]]
        assert g["m_off"] == (offs[pos[p["m_sym"]]] if p.get("m_sym") else -1)
        assert g["row_base_off"] == (offs[pos[p["row_base"]]] if p.get("row_base") else -1)
        mask = 1 | sum(1 << bit for key, bit in GEMM_ENTRY_BITS if p.get(key))
        assert g["entries"] == mask


def test_malformed_gemm_lines_are_rejected(hip):
    ck = _mma(k=256)
    line = next(x for x in ck.src.splitlines() if x.startswith("// eas-gemm:"))
    head = next(x for x in ck.src.splitlines() if x.startswith("// eas-launch:"))
    assert hip.launch_shape(head + "\n" + line + "\n")["gemm"]["K"] == 256
    for old, new in (("K=256", "K=0"), ("row_axis=1", "row_axis=2"), ("entries=63", "entries=62"),
                     ("entries=63", "entries=127"), ("a_elem=2", "a_elem=3"), ("threads=256", "threads=100"),
                     ("ldb=28", "ldb=30"), ("entry=matmul_mma_kernel", "entry=mat-mul"), (" tm=32", ""),
                     ("K=256", "K=-1"), ("K=256", "K=256 warp=1")):
        assert old in line, old
        with pytest.raises(ValueError):
            hip.launch_shape(head + "\n" + line.replace(old, new) + "\n")
    with pytest.raises(ValueError, match="eas-gemm"):
        hip.launch_shape(head + "\n")


def test_reference_dispatch_of_the_lifted_kernels_is_planned(hip):
    # the sizes metal.py hands `launch` for the two matmul kernels, planned as the runtime plans them
    f, h = np.zeros(8, np.float32), np.zeros(8, np.float16)
    tiled = K.matmul_tiled_kernel.compile(f, f, f, 64, 64, 0, 0, BM=32, BN=32, BK=32, K=1024, NT=256)
    mma = K.matmul_mma_kernel.compile(h, h, f, 64, 64, BM=32, BN=32, BK=8, K=4100, NT=512)
    for ck, m, n, k, grid in ((tiled, 1024, 1024, 1024, (32, 32, 1)),
                              (mma, 4096, 4096, 4100, K.mma_grid({"BM": 32, "BN": 32}, {"M": 4096, "N": 4096})),
                              (mma, 300, 520, 4100, K.mma_grid({"BM": 32, "BN": 32}, {"M": 300, "N": 520}))):
        args = _args(ck, m, n, k)
        tpg, tptg = reference_dispatch(ck, args, grid=grid)
        plan = plan_launch(ck, args, grid=grid)
        assert hip.plan_dispatch(ck.src, tpg, tptg, argv=_argv(hip, ck, args)) == \
            (plan.grid, plan.block, plan.hidden, plan.entry)


def test_random_launches_plan_alike(hip):
    # 300 seeded random launches: kernel kind, M, N, K, partial and oversized grids, tile bases,
    # operand alignment, a short buffer now and then, CU count and entry override; both planners
    # must give the same plan, the same refusal, or both nothing
    import random

    r = random.Random(7)
    f = np.zeros(8, np.float32)
    kernels = {}
    choices = ("auto", "auto", "auto", "8wave", "tile128", "tile128x256", "tile128x64", "tile64", "4wave")
    planned = 0
    for case in range(300):
        kind = r.choice(("mma", "mma16out", "mma32in", "tiled"))
        m, n = r.choice((1, 7, 16, 17, 64, 100, 128, 129, 300, 1000, 4096)), r.choice((1, 8, 65, 130, 520, 4096, 16390))
        k = r.choice((2, 33, 36, 100, 4100))
        key = (kind, k)
        if key not in kernels:
            if kind == "tiled":
                kernels[key] = K.matmul_tiled_kernel.compile(f, f, f, 64, 64, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
            elif kind == "mma32in":
                kernels[key] = _mma(k=k, a=np.float32)
            else:
                kernels[key] = _mma("matmul_mma_f16out_kernel" if kind == "mma16out" else "matmul_mma_kernel", k,
                                    np.float16, np.float16 if kind == "mma16out" else np.float32)
        ck = kernels[key]
        if ck.geometry is None or ck.geometry.kind != "gemm":
            continue  # not lifted (the literal lowering runs it): no GEMM plan to compare
        extra = {}
        if kind == "tiled":
            extra = {"PID_M_BASE": r.choice((0, 0, 1, 5)), "PID_N_BASE": r.choice((0, 0, 2, 7))}
        args = _args(ck, m, n, k, extra=extra, short=r.choice((None,) * 8 + ("a", "b", "c")),
                     misalign=r.choice((None,) * 6 + ("a", "b")))
        full = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
        groups = r.choice((full, full, (max(1, full[0] // 2), full[1], 1), (full[0] + 3, full[1] + 2, 1),
                           (1, 1, 1)))
        c, py = _both(hip, ck, args, groups, cus=r.choice((256, 256, 80, 304)), choice=r.choice(choices),
                      by_groups=r.random() < 0.5)
        assert _agree(c, py), (case, kind, m, n, k, groups, extra, c, py)
        planned += 1
    assert planned > 200
