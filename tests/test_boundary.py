"""The reference's native launch convention at the ``eas._hip`` seam, on the CPU.

``eas._hip.launch(pipeline, argv, writable, threads_per_grid,
threads_per_threadgroup)`` takes the sizes the reference runtime passes
(eas/runtime/metal.py:341-346, _metal.mm:1013-1222) and ``launch_tg`` takes
threadgroup counts (_metal.mm:1232-1379).  Both plan their HIP workgroups with
``eas_hip_plan_dispatch`` from the launch shape on the kernel source's
``eas-launch`` line; ``plan_dispatch`` exposes that planner without a GPU.  Here
it is driven exactly as the reference runtime drives ``launch`` and must land on
the dispatch ``HipRuntime`` plans for the same call.  The GPU side
(tests/test_gpu_boundary.py) runs kernels through ``launch`` itself.
"""

from __future__ import annotations

import numpy as np
import pytest

import eas
import kernels as K
from eas import mk
from easy_as_amd.codegen.hip import kernarg_bytes
from easy_as_amd.runtime.grid import infer_grid
from easy_as_amd.runtime.hip import plan_launch
from easy_as_amd.runtime.hip_ext import load_hip_ext
from metal_dispatch import reference_dispatch


@pytest.fixture(scope="module")
def hip():
    return load_hip_ext(require=True)


def _f(n=8):
    return np.zeros(n, np.float32)


def _kernels():
    f, h = _f(), np.zeros(8, np.float16)
    return {
        "add256": (K.add_kernel.compile(f, f, f, 8, BLOCK=256), [{"N": n} for n in (1, 255, 1031, 1 << 20, 1 << 28)]),
        "add1024": (K.add_kernel.compile(f, f, f, 8, BLOCK=1024), [{"N": n} for n in (1, 1031, 1 << 28)]),
        "fill256": (K.fill_kernel.compile(f, 8, BLOCK=256), [{"N": n} for n in (1, 4099, 1 << 20)]),
        "rotate": (K.spmd_tg_rotate_kernel.compile(f, f, 8, BLOCK=256), [{"N": n} for n in (1, 1000)]),
        "add_f16": (K.add_kernel.compile(h, h, h, 8, BLOCK=256), [{"N": n} for n in (7, 4099)]),
        "fma_thread": (K.simple_fma_kernel.compile(f, f, f, f, 8, BLOCK=256), [{"N": n} for n in (1, 1000, 1 << 20)]),
        "tptg64": (K.tptg_independent_kernel.compile(f, 8, BLOCK=64), [{"N": n} for n in (1, 1000)]),
    }


CASES = [(name, i) for name, (_, args) in _kernels().items() for i in range(len(args))]


@pytest.mark.parametrize("name,i", CASES)
def test_launch_by_threads_plans_what_the_runtime_plans(hip, name, i):
    ck, arglist = _kernels()[name]
    args = arglist[i]
    tpg, tptg = reference_dispatch(ck, args)
    grid, block, hidden = hip.plan_dispatch(ck.src, tpg, tptg)
    plan = plan_launch(ck, args)
    assert (grid, block, hidden) == (plan.grid, plan.block, plan.hidden)


def test_explicit_grids_by_threads_and_by_threadgroups(hip):
    # a 2-D launch of a thread-mode kernel: the reference passes threads per axis to launch and
    # threadgroups to launch_tg; both plan one workgroup per threadgroup
    ck = K.grid_callable_kernel.compile(_f(), 5, 10, BLOCK=4)
    for grid in ((3, 5, 1), (1, 1, 1), (7, 2, 3)):
        args = {"H": grid[1], "W": 4 * grid[0]}
        tpg, tptg = reference_dispatch(ck, args, grid=grid)
        plan = plan_launch(ck, args, grid=grid)
        assert hip.plan_dispatch(ck.src, tpg, tptg) == (plan.grid, plan.block, plan.hidden)
        assert hip.plan_dispatch(ck.src, grid, tptg, by_groups=True) == (plan.grid, plan.block, plan.hidden)
    # a grid inferred from H and W: threads per axis to launch, the inferred groups to launch_tg
    ck = K.add2d_hw_kernel.compile(_f(), _f(), _f(), 17, 103, BLOCK=32)
    args = {"H": 17, "W": 103}
    tpg, tptg = reference_dispatch(ck, args)
    plan = plan_launch(ck, args)
    assert hip.plan_dispatch(ck.src, tpg, tptg) == (plan.grid, plan.block, plan.hidden)
    groups = infer_grid(ck.ir, args, ck.block_size)
    assert hip.plan_dispatch(ck.src, groups, tptg, by_groups=True) == (plan.grid, plan.block, plan.hidden)


@pytest.mark.parametrize("env", [{"EAS_HIP_SPMD_UNROLL": "4"}, {"EAS_HIP_SPMD_WG": "1024"},
                                 {"EAS_HIP_SPMD_LPT": "16", "EAS_HIP_SPMD_WG": "32"}])
def test_launch_by_threads_matches_every_spmd_mapping(hip, monkeypatch, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    f = _f()
    for block in (256, 1024):
        ck = eas.kernel(K.add_kernel.fn).compile(f, f, f, 8, BLOCK=block)
        for n in (1, 1031, 4099 + block, 1 << 20):
            tpg, tptg = reference_dispatch(ck, {"N": n})
            plan = plan_launch(ck, {"N": n})
            assert hip.plan_dispatch(ck.src, tpg, tptg) == (plan.grid, plan.block, plan.hidden), (env, block, n)


def test_random_launches_plan_alike(hip, monkeypatch):
    """400 seeded launches of SPMD, lanes and one-thread-per-thread kernels over random BLOCKs,
    workgroup mappings, sizes and explicit grids: the C planner (by threads, as `launch`, and by
    threadgroups, as `launch_tg`) gives the dispatch `plan_launch` gives."""
    import random

    r = random.Random(7)
    f = _f()
    envs = [{}, {"EAS_HIP_SPMD_WG": "64"}, {"EAS_HIP_SPMD_WG": "1024"}, {"EAS_HIP_SPMD_LPT": "16"},
            {"EAS_HIP_SPMD_UNROLL": "2"}, {"EAS_HIP_THREAD_LANES": "0"}]
    kerns = [(K.add_kernel, (f, f, f)), (K.fill_kernel, (f,)), (K.simple_fma_kernel, (f, f, f, f)),
             (K.tptg_independent_kernel, (f,)), (K.lane_id_kernel, (f,)), (K.tg_copy_kernel, (f, f))]
    for case in range(400):
        env = r.choice(envs)
        with monkeypatch.context() as mp:
            for k, v in env.items():
                mp.setenv(k, v)
            kern, bufs = r.choice(kerns)
            block = r.choice((1, 2, 3, 32, 64, 96, 100, 200, 256, 384, 1000, 1024))
            ck = eas.kernel(kern.fn).compile(*bufs, 8, BLOCK=block)
        n = r.choice((1, block - 1 or 1, block, 7 * block + 3, r.randrange(1, 1 << 22), (1 << 28) + 5))
        grid = None if r.random() < 0.6 else (r.randrange(1, 5000), r.randrange(1, 4), r.randrange(1, 3))
        args = {"N": n}
        what = (case, kern.name, block, env, n, grid)
        plan = plan_launch(ck, args, grid=grid)
        tpg, tptg = reference_dispatch(ck, args, grid=grid)
        assert hip.plan_dispatch(ck.src, tpg, tptg) == (plan.grid, plan.block, plan.hidden), what
        if ck.launch_mode == "thread" and grid is None:
            continue  # by threadgroups a 1-D launch has every thread of them live: another launch
        groups = grid or (-(-n // block), 1, 1)  # threadgroups, or SPMD programs
        assert hip.plan_dispatch(ck.src, groups, tptg, by_groups=True) == (plan.grid, plan.block, plan.hidden), what


def test_non_uniform_last_threadgroup(monkeypatch):
    # 1000 threads of BLOCK 256: four threadgroups, the hidden extent stops the last 24 threads.
    # Emitted as lanes (the default for this element stream), each threadgroup is two workgroups
    # of 32 threads carrying 16-byte vectors; one thread per Metal thread, one workgroup each.
    hip = load_hip_ext(require=True)
    ck = K.simple_fma_kernel.compile(_f(), _f(), _f(), _f(), 8, BLOCK=256)
    assert ck.geometry.params.get("lanes") and ck.launch_mode == "thread"
    assert hip.plan_dispatch(ck.src, 1000, 256) == ((8, 1, 1), (32, 1, 1), (1000,))
    assert plan_launch(ck, {"N": 1000}).grid == (8, 1, 1)
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", "0")
    one = eas.kernel(K.simple_fma_kernel.fn).compile(_f(), _f(), _f(), _f(), 8, BLOCK=256)
    assert not one.geometry.params.get("lanes")
    assert hip.plan_dispatch(one.src, 1000, 256) == ((4, 1, 1), (256, 1, 1), (1000,))
    # the int form of threads_per_threadgroup and its omission mean the same
    for c in (ck, one):
        assert hip.plan_dispatch(c.src, 1000) == hip.plan_dispatch(c.src, (1000,), (256, 1, 1))


def test_launch_convention_errors(hip):
    f = _f()
    thread = K.simple_fma_kernel.compile(f, f, f, f, 8, BLOCK=256)
    spmd = K.add_kernel.compile(f, f, f, 8, BLOCK=256)
    with pytest.raises(ValueError, match=r"\(256, 1, 1\)"):
        hip.plan_dispatch(thread.src, 1000, (1, 1, 1))  # an SPMD-shaped call to a thread kernel
    with pytest.raises(ValueError, match=r"\(1, 1, 1\)"):
        hip.plan_dispatch(spmd.src, 5, (256, 1, 1))  # a thread-shaped call to an SPMD kernel
    for bad in (0, (4, 0, 1), (0,)):
        with pytest.raises(ValueError, match="must be > 0"):
            hip.plan_dispatch(spmd.src, bad, (1, 1, 1))
    with pytest.raises(ValueError, match="2\\^32"):
        hip.plan_dispatch(thread.src, 1 << 33, 256)
    # threadgroup counts whose thread total would wrap a u64 are refused, not truncated
    for groups in ((1 << 54) // 256 * 256, (1 << 56) + 3, (1 << 32) // 256):
        with pytest.raises(ValueError, match="2\\^32"):
            hip.plan_dispatch(thread.src, groups, 256, by_groups=True)
    most = ((1 << 32) - 1) // 256
    want = plan_launch(thread, {"N": 8}, grid=(most, 1, 1))
    assert want.hidden == (most * 256,)
    assert hip.plan_dispatch(thread.src, most, 256, by_groups=True) == (want.grid, want.block, want.hidden)
    # a lifted GEMM's plan reads M, N and its buffers from argv
    h = np.zeros(8, np.float16)
    gemm = K.matmul_mma_kernel.compile(h, h, f, 300, 520, BM=32, BN=32, BK=8, K=200, NT=512)
    assert gemm.geometry.kind == "gemm"
    with pytest.raises(TypeError, match="argv"):
        hip.plan_dispatch(gemm.src, (17 * 512, 10, 1), (512, 1, 1))
    # a source without an eas-launch line has no shape
    with pytest.raises(ValueError, match="eas-launch"):
        hip.plan_dispatch('extern "C" __global__ void k() {}', 64)


def test_launch_shape_line_matches_the_geometry(hip):
    f, h = _f(), np.zeros(8, np.float16)
    for ck in (K.add_kernel.compile(f, f, f, 8, BLOCK=1024), K.axpy_kernel.compile(f, f, f, 8, 2.0, BLOCK=256),
               K.simple_fma_kernel.compile(f, f, f, f, 8, BLOCK=128),
               K.matmul_mma_kernel.compile(h, h, f, 300, 520, BM=32, BN=32, BK=8, K=200, NT=512)):
        shape = hip.launch_shape(ck.src)
        geo = ck.geometry
        assert shape["kind"] == geo.kind and shape["block_size"] == geo.block_size
        assert shape["wg_size"] == geo.wg_size and shape["split"] == geo.split
        assert shape["arg_bytes"] == kernarg_bytes(ck.ir)
        assert shape["hidden"] == (4 if geo.kind == "gemm" else 1)


def test_kernarg_bytes_follow_natural_alignment():
    @eas.kernel
    def mixed(flag, a, h, x, N, BLOCK: eas.constexpr):
        offs = mk.program_id(0) * BLOCK + mk.arange(0, BLOCK)
        mk.store(a, offs, mk.load(a, offs, offs < N) * x, offs < N)

    ck = mixed.compile(True, _f(), np.float16(1.0), 2.0, 8, BLOCK=256)
    kinds = [(a.name, a.kind, a.dtype.value) for a in ck.ir.args]
    # bool at 0, pointer at 8, f16 at 16, f32 at 20, u32 at 24 -> 28 bytes
    assert [k[0] for k in kinds] == ["flag", "a", "h", "x", "N"]
    assert kernarg_bytes(ck.ir) == 28


def test_malformed_launch_lines_are_rejected(hip):
    good = "// eas-launch: kind=spmd block=256 wg=32 ppw=1 split=2 args=28 hidden=1\n"
    assert hip.launch_shape(good)["split"] == 2
    # unrolled split programs: each group of `split` workgroups runs `ppw` programs
    unrolled = hip.launch_shape("// eas-launch: kind=spmd block=256 wg=32 ppw=4 split=2 args=28 hidden=1\n")
    assert (unrolled["programs_per_wg"], unrolled["split"]) == (4, 2)
    for bad in ("// eas-launch: block=256\n", "// eas-launch: kind=warp block=256 wg=32 hidden=1\n",
                "// eas-launch: kind=spmd block=256 wg=2048 hidden=1\n",
                "// eas-launch: kind=thread block=256 wg=128 hidden=2\n",
                "// eas-launch: kind=spmd block=256 wg=32 hidden=9\n",
                "// eas-launch: kind=spmd block=x wg=32 hidden=1\n"):
        with pytest.raises(ValueError):
            hip.launch_shape(bad)


def test_compile_defaults_are_the_runtime_options(hip):
    # compile(src, name) without options (the reference's signature) compiles as HipRuntime does
    from easy_as_amd.runtime.hip import COMPILE_OPTIONS

    assert tuple(hip.DEFAULT_OPTIONS) == COMPILE_OPTIONS
